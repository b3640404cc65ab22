"""Independent constructions of ggml blocks for the tests.

These build blocks in the FORWARD direction, from chosen codes and scales, the
way ggml's quantizers pack them (quantize_row_q4_K / quantize_row_q6_K), so a
decoder that reads a wrong nibble, quadrant, high-bit pair or scale index
fails an exact comparison.  The expected weights come from exact rational
arithmetic on the chosen values, not from the oracle's formula.
"""
from fractions import Fraction

import numpy as np


def f16_bits(x):
    return int(np.array(x, np.float16).view(np.uint16))


def pack_q4k_scales(sc, m):
    """8 six-bit scales and mins -> 12 bytes (ggml get_scale_min_k4 packing)."""
    s = [0] * 12
    for j in range(8):
        if j < 4:
            s[j] |= sc[j] & 63
            s[j + 4] |= m[j] & 63
        else:
            s[j + 4] |= (sc[j] & 0xF) | ((m[j] & 0xF) << 4)
            s[j - 4] |= (sc[j] >> 4) << 6
            s[j] |= (m[j] >> 4) << 6
    return s


def make_q4k_block(d, dmin, sc, m, q):
    """q: 256 codes 0..15 in element order.  Element e = 32*j + i is in
    sub-block j; codes of sub-blocks 2p / 2p+1 share qs bytes 32p..32p+31 as
    low / high nibbles."""
    b = np.zeros(144, np.uint8)
    b[0:2] = np.array([f16_bits(d)], np.uint16).view(np.uint8)
    b[2:4] = np.array([f16_bits(dmin)], np.uint16).view(np.uint8)
    b[4:16] = pack_q4k_scales(sc, m)
    for e in range(256):
        j, i = divmod(e, 32)
        byte = 16 + 32 * (j // 2) + i
        b[byte] |= (q[e] & 0xF) << (4 * (j % 2))
    return b


def q4k_exact(d, dmin, sc, m, q):
    """Exact weights d*sc*q - dmin*m as Fractions (d, dmin f16-representable)."""
    D, Dm = Fraction(float(np.float16(d))), Fraction(float(np.float16(dmin)))
    return [D * sc[e // 32] * q[e] - Dm * m[e // 32] for e in range(256)]


def make_q6k_block(d, sc, q):
    """q: 256 six-bit codes in element order; sc: 16 i8 scales (element e uses
    sc[e // 16]).  ggml packs element 128*n2 + l + 32*t (t = 0..3) into ql/qh:
    ql[64n2+l] = q(t=0) low | q(t=2) low << 4, ql[64n2+l+32] = q(t=1) | q(t=3) << 4,
    qh[32n2+l] = hi2(t=0) | hi2(t=1) << 2 | hi2(t=2) << 4 | hi2(t=3) << 6."""
    b = np.zeros(210, np.uint8)
    for n2 in range(2):
        for l in range(32):
            qq = [q[128 * n2 + l + 32 * t] for t in range(4)]
            b[64 * n2 + l] = (qq[0] & 0xF) | ((qq[2] & 0xF) << 4)
            b[64 * n2 + l + 32] = (qq[1] & 0xF) | ((qq[3] & 0xF) << 4)
            b[128 + 32 * n2 + l] = ((qq[0] >> 4) | ((qq[1] >> 4) << 2) | ((qq[2] >> 4) << 4)
                                    | ((qq[3] >> 4) << 6))
    b[192:208] = np.array(sc, np.int8).view(np.uint8)
    b[208:210] = np.array([f16_bits(d)], np.uint16).view(np.uint8)
    return b


def q6k_exact(d, sc, q):
    D = Fraction(float(np.float16(d)))
    return [D * sc[e // 16] * (q[e] - 32) for e in range(256)]


def make_q5k_block(d, dmin, sc, m, q):
    """q: 256 five-bit codes in element order.  Element e = 32*j + i (sub-block j):
    low nibble in qs[32*(j//2) + i] (low half for even j, high for odd j), the 5th
    bit in qh[i] bit j (block_q5_K, crates/arf-core/src/model/gguf.rs:2053-2090)."""
    b = np.zeros(176, np.uint8)
    b[0:2] = np.array([f16_bits(d)], np.uint16).view(np.uint8)
    b[2:4] = np.array([f16_bits(dmin)], np.uint16).view(np.uint8)
    b[4:16] = pack_q4k_scales(sc, m)
    for e in range(256):
        j, i = divmod(e, 32)
        b[48 + 32 * (j // 2) + i] |= (q[e] & 0xF) << (4 * (j % 2))
        b[16 + i] |= (q[e] >> 4) << j
    return b


def q5k_exact(d, dmin, sc, m, q):
    """Exact weights d*sc*q - dmin*m as Fractions (d, dmin f16-representable)."""
    D, M = Fraction(float(np.float16(d))), Fraction(float(np.float16(dmin)))
    return [D * sc[e // 32] * q[e] - M * m[e // 32] for e in range(256)]


def make_q80_block(d, q):
    b = np.zeros(34, np.uint8)
    b[0:2] = np.array([f16_bits(d)], np.uint16).view(np.uint8)
    b[2:34] = np.array(q, np.int8).view(np.uint8)
    return b


def ref_f32_to_f16_bits_test(x):
    """The reference's test helper f32_to_f16_bits_test
    (crates/arf-core/src/model/gguf.rs:2769-2779): truncating, flushes tiny to 0."""
    b = int(np.array(x, np.float32).view(np.uint32))
    sign = (b >> 16) & 0x8000
    exp = ((b >> 23) & 0xFF) - 127 + 15
    mant = (b >> 13) & 0x3FF
    if exp <= 0:
        return sign
    return sign | (exp << 10) | mant


def ref_make_q4k_block(d, dmin, scales12, qs128):
    """make_q4k_block of crates/arf-core/src/model/gguf.rs:2781-2788."""
    b = np.zeros(144, np.uint8)
    b[0:2] = np.array([ref_f32_to_f16_bits_test(d)], np.uint16).view(np.uint8)
    b[2:4] = np.array([ref_f32_to_f16_bits_test(dmin)], np.uint16).view(np.uint8)
    b[4:16] = scales12
    b[16:144] = qs128
    return b


class Lcg32:
    """x = x*1664525 + 1013904223 (mod 2^32), byte = x >> 24
    (crates/arf-core/src/model/gguf.rs:2917-2921)."""

    def __init__(self, seed):
        self.x = seed & 0xFFFFFFFF

    def byte(self):
        self.x = (self.x * 1664525 + 1013904223) & 0xFFFFFFFF
        return self.x >> 24


def lcg_q4k_blocks(seed, n_blocks, d_base, d_div, dm_base, dm_div):
    """The pseudo-random gate blocks of gguf.rs:2913-2968 (cases c and d)."""
    g = Lcg32(seed)
    raw = np.zeros(n_blocks * 144, np.uint8)
    for b in range(n_blocks):
        p = b * 144
        d_val = np.float32(d_base) + np.float32(g.byte()) / np.float32(d_div)
        dm_val = np.float32(dm_base) + np.float32(g.byte()) / np.float32(dm_div)
        raw[p:p + 2] = np.array([ref_f32_to_f16_bits_test(d_val)], np.uint16).view(np.uint8)
        raw[p + 2:p + 4] = np.array([ref_f32_to_f16_bits_test(dm_val)], np.uint16).view(np.uint8)
        for i in range(12):
            raw[p + 4 + i] = g.byte() & 63
        for i in range(128):
            raw[p + 16 + i] = g.byte()
    return raw


def moe_route_lcg_logits(count, state):
    """LCG of crates/arf-gpu/tests/moe_gpu.rs:84-89:
    s = s*6364136223846793005 + 1 (mod 2^64); v = (s >> 40) / 2^23 - 0.5."""
    out = []
    s = state
    for _ in range(count):
        s = (s * 6364136223846793005 + 1) & 0xFFFFFFFFFFFFFFFF
        out.append(np.float32(np.float32(s >> 40) / np.float32(1 << 23) - np.float32(0.5)))
    return np.array(out, np.float32), s


def moe_dequant_reference(oracle, x, raw, E, hidden, inter, logits, top_k, norm):
    """MoeMlp::forward (moe.rs:53-86) on every token from the oracle's routing
    (top_k_softmax) and bit-exact dequant, the projections as float32 BLAS products over
    each expert's tokens (quantized linear == dequant + f32 matmul, weight.rs:1693-1709),
    SwiGLU (mlp.rs:20-24) in f32 and out[t] += w_j * y_j in top-k slot order."""
    T = x.shape[0]
    x = np.asarray(x, np.float32)
    ids = np.zeros((T, top_k), np.int64)
    wts = np.zeros((T, top_k), np.float32)
    for t in range(T):
        ids[t], wts[t] = oracle.top_k_softmax(logits[t], top_k, norm)
    g_all, u_all, d_all = (r.reshape(E, -1) for r in raw)
    ys = np.zeros((T, top_k, hidden), np.float32)
    for e in range(E):
        tt, jj = np.nonzero(ids == e)
        if tt.size == 0:
            continue
        wg = oracle.dequant("q4_k", g_all[e], inter * hidden).reshape(inter, hidden)
        wu = oracle.dequant("q4_k", u_all[e], inter * hidden).reshape(inter, hidden)
        wd = oracle.dequant("q4_k", d_all[e], hidden * inter).reshape(hidden, inter)
        xe = x[tt]
        g, u = xe @ wg.T, xe @ wu.T
        with np.errstate(over="ignore"):  # exp(-g) = inf for g << 0: silu -> 0, as in f32
            h = (g / (np.float32(1) + np.exp(-g)) * u).astype(np.float32)
        ys[tt, jj] = h @ wd.T
    out = np.zeros((T, hidden), np.float32)
    for j in range(top_k):
        out += wts[:, j:j + 1] * ys[:, j]
    return out
