"""CPU tests that pin the oracle (oracle/arfq_oracle.c) before it is trusted.

Sources of truth, in order: the reference's own known-answer tests and golden
gates (quoted with file:line), then closed forms built independently of the
oracle's code (forward packing + exact rational arithmetic, IEEE conversions,
float64 matmuls).  A plausible decoder mistake (wrong nibble, quadrant, qh bit
pair, scale index, sign fold) fails at least one of these exactly.
"""
import numpy as np
import pytest

from conftest import rel_err
from formats import (f16_bits, lcg_q4k_blocks, make_q4k_block, make_q5k_block, make_q6k_block,
                     make_q80_block, moe_route_lcg_logits, pack_q4k_scales, q4k_exact, q5k_exact,
                     q6k_exact, ref_make_q4k_block)


# ---------------------------------------------------------------- f16 ----
def test_f16_known_values(oracle):
    # crates/arf-core/src/model/gguf.rs:2485-2491
    assert oracle.f16_to_f32(0x3C00) == 1.0
    assert oracle.f16_to_f32(0x4000) == 2.0
    assert oracle.f16_to_f32(0xC000) == -2.0
    assert oracle.f16_to_f32(0x0000) == 0.0
    assert abs(oracle.f16_to_f32(0x3555) - 0.333) < 1e-3


def test_f16_all_patterns_match_ieee(oracle):
    # all 65536 patterns vs numpy's IEEE binary16 -> binary32 (exact, NaN payload kept)
    import ctypes
    L = oracle.lib()
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(np.float32).view(np.uint32)
    got = np.array([L.arfo_f16_to_f32(int(h)) for h in bits], np.float32).view(np.uint32)
    nan = np.isnan(bits.view(np.float16))
    assert np.array_equal(got[~nan], want[~nan])
    # NaNs: ctypes float round trip may quiet a signalling NaN; the class must match
    assert np.all(np.isnan(got[nan].view(np.float32)))


# ------------------------------------------------------- Q4_K scale/min ----
def test_q4k_scale_min_known(oracle):
    # gguf.rs:2494-2505
    assert all(oracle.q4k_get_scale_min([0] * 12, j) == (0, 0) for j in range(8))
    s = [0] * 12
    s[0], s[4] = 0b0010_1010, 0b0001_0101
    assert oracle.q4k_get_scale_min(s, 0) == (42, 21)
    # gguf.rs:2963-2980 (j>=4 branch): sc = 51, m = 26
    s = [0] * 12
    s[0], s[4], s[8] = 0b1100_0101, 0b0100_0111, 0b1010_0011
    assert oracle.q4k_get_scale_min(s, 4) == (51, 26)


def test_q4k_scale_min_roundtrip_random(oracle):
    rng = np.random.default_rng(7)
    for _ in range(300):
        sc = rng.integers(0, 64, 8).tolist()
        m = rng.integers(0, 64, 8).tolist()
        packed = pack_q4k_scales(sc, m)
        for j in range(8):
            assert oracle.q4k_get_scale_min(packed, j) == (sc[j], m[j])


# ------------------------------------------------------------ Q4_K dequant ----
def test_dequant_q4k_known_block(oracle):
    # gguf.rs:2522-2538: d=2, dmin=1, sc0=3, m0=5, q=4 -> 19.0; next weight -> -5.0
    b = np.zeros(144, np.uint8)
    b[0:2] = np.array([0x4000], np.uint16).view(np.uint8)
    b[2:4] = np.array([0x3C00], np.uint16).view(np.uint8)
    b[4], b[8], b[16] = 3, 5, 0x04
    out = oracle.dequant("q4_k", b, 256)
    assert out[0] == 19.0 and out[1] == -5.0


def test_dequant_q4k_exact_forward_packing(oracle):
    rng = np.random.default_rng(11)
    for trial in range(40):
        d = 2.0 ** int(rng.integers(-8, 2))
        dmin = 2.0 ** int(rng.integers(-8, 2))
        sc = rng.integers(0, 64, 8).tolist()
        m = rng.integers(0, 64, 8).tolist()
        q = rng.integers(0, 16, 256).tolist()
        blk = make_q4k_block(d, dmin, sc, m, q)
        got = oracle.dequant("q4_k", blk, 256)
        want = np.array([float(v) for v in q4k_exact(d, dmin, sc, m, q)], np.float64)
        assert np.array_equal(got.astype(np.float64), want), trial


def _q4ks_bit_exact(oracle, raw, rows, cols, label):
    ggml = oracle.dequant("q4_k", raw, rows * cols)
    q4ks = oracle.q4ks_to_f32(oracle.q4ks_from_ggml(raw, rows, cols), rows, cols)
    assert np.array_equal(ggml.view(np.uint32), q4ks.view(np.uint32)), label
    return ggml


def test_from_ggml_q4k_is_bit_exact_gate(oracle):
    # crates/arf-core/src/model/gguf.rs:2862-2982, cases (a)-(e)
    sc = np.zeros(12, np.uint8); sc[0], sc[4] = 3, 5
    qs = np.zeros(128, np.uint8); qs[0] = 0x04
    out = _q4ks_bit_exact(oracle, ref_make_q4k_block(2.0, 1.0, sc, qs), 1, 256, "known_block")
    assert out[0] == 19.0
    sc = np.zeros(12, np.uint8); sc[1], sc[5] = 10, 63
    qs = np.zeros(128, np.uint8); qs[0] = 0x70
    out = _q4ks_bit_exact(oracle, ref_make_q4k_block(1.0, 0.5, sc, qs), 1, 256, "sign_fold_m63")
    assert out[32] == np.float32(10.0 * 7 - 31.5)  # sub-block 1, weight 0: 1*10*7 - 0.5*63
    raw = lcg_q4k_blocks(0x12345678, 3, 1.0, 64.0, 0.5, 128.0)
    _q4ks_bit_exact(oracle, raw, 1, 768, "pseudo_random_1row_3blocks")
    raw = lcg_q4k_blocks(0xDEADBEEF, 2, 2.0, 128.0, 1.0, 256.0)
    _q4ks_bit_exact(oracle, raw, 2, 256, "multi_row_2x256")
    sc = np.zeros(12, np.uint8)
    sc[0], sc[4], sc[8] = 0b1100_0101, 0b0100_0111, 0b1010_0011
    qs = np.zeros(128, np.uint8); qs[64] = 0x0F
    out = _q4ks_bit_exact(oracle, ref_make_q4k_block(0.25, 0.125, sc, qs), 1, 256,
                          "high_scale_path_j4")
    assert out[128] == np.float32(0.25 * 51 * 15 - 0.125 * 26)


def test_q4ks_transcode_bit_exact_random_with_subnormals(oracle):
    from arf_amd import synth
    raw = synth.weight("q4_k", 8, 1024, seed=5).reshape(-1, 144)
    raw[::7, 0:2] = np.array([1, 0], np.uint8)  # smallest f16 subnormal d
    raw[3::11, 2:4] = np.array([0x17, 0x02], np.uint8)  # subnormal dmin
    _q4ks_bit_exact(oracle, raw.reshape(-1), 8, 1024, "random_subnormal")


# ------------------------------------------------------------ Q6_K dequant ----
def test_dequant_q6k_known_block(oracle):
    # gguf.rs:2564-2575: d=0.5, sc0=4, ql0=10 -> -44.0
    b = np.zeros(210, np.uint8)
    b[192], b[0] = 4, 10
    b[208:210] = np.array([0x3800], np.uint16).view(np.uint8)
    assert oracle.dequant("q6_k", b, 256)[0] == -44.0


def test_dequant_q6k_exact_forward_packing(oracle):
    rng = np.random.default_rng(13)
    for trial in range(40):
        d = 2.0 ** int(rng.integers(-10, 1))
        sc = rng.integers(-32, 32, 16).tolist()
        q = rng.integers(0, 64, 256).tolist()
        got = oracle.dequant("q6_k", make_q6k_block(d, sc, q), 256)
        want = np.array([float(v) for v in q6k_exact(d, sc, q)], np.float64)
        assert np.array_equal(got.astype(np.float64), want), trial


def test_dequant_q6k_each_quadrant_and_qh_pair(oracle):
    # one nonzero code at a time: every (half, quadrant, qh pair, scale slot)
    for e in range(0, 256, 5):
        for hi in range(4):
            q = [32] * 256
            q[e] = (hi << 4) | (e % 16)
            sc = list(range(1, 17))
            got = oracle.dequant("q6_k", make_q6k_block(1.0, sc, q), 256)
            want = np.zeros(256)
            want[e] = sc[e // 16] * (q[e] - 32)
            assert np.array_equal(got, want), (e, hi)


# ------------------------------------------------------------ Q8_0 dequant ----
def test_dequant_q5k_known_block(oracle):
    # dequant_q5_k_known_block (gguf.rs:2541-2561): d=2, dmin=1, sc0=3, m0=5, q0=4 -> 19;
    # with the 5th bit of weight 0 set, q0 = 20 -> 115
    b = np.zeros(176, np.uint8)
    b[0:2] = np.array([f16_bits(2.0)], np.uint16).view(np.uint8)
    b[2:4] = np.array([f16_bits(1.0)], np.uint16).view(np.uint8)
    b[4], b[8], b[48] = 3, 5, 0x04
    assert oracle.dequant("q5_k", b, 256)[0] == 19.0
    b[16] = 0x01
    assert oracle.dequant("q5_k", b, 256)[0] == 115.0


def test_dequant_q5k_exact_forward_packing(oracle):
    # the dequant is exact here (d, dmin powers of two, products exact in f32)
    rng = np.random.default_rng(17)
    for trial in range(40):
        d, dmin = 2.0 ** int(rng.integers(-10, 1)), 2.0 ** int(rng.integers(-10, 1))
        sc, m = rng.integers(0, 64, 8).tolist(), rng.integers(0, 64, 8).tolist()
        q = rng.integers(0, 32, 256).tolist()
        got = oracle.dequant("q5_k", make_q5k_block(d, dmin, sc, m, q), 256)
        want = np.array([float(v) for v in q5k_exact(d, dmin, sc, m, q)], np.float64)
        assert np.array_equal(got.astype(np.float64), want), trial


def test_dequant_q5k_each_high_bit_lands_on_its_weight(oracle):
    # one 5th bit at a time: a transposed qh read puts it on another weight
    for e in range(256):
        q = [0] * 256
        q[e] = 16
        got = oracle.dequant("q5_k", make_q5k_block(1.0, 0.0, [1] * 8, [0] * 8, q), 256)
        want = np.zeros(256)
        want[e] = 16.0
        assert np.array_equal(got, want), e


def test_q5k_native_unpack_matches_dequant(oracle):
    # q5k_native_unpack_matches_the_reference_dequantizer (crates/arf-core/tests/q5k_native.rs):
    # the same deterministic bytes, rebuilt from the Q5KS unpack, against dequant_q5_k
    rows, cols = 2, 512
    nb = rows * cols // 256
    b = np.zeros(nb * 176, np.uint8)
    for blk in range(nb):
        p = blk * 176
        b[p:p + 2] = np.array([f16_bits(0.05)], np.uint16).view(np.uint8)
        b[p + 2:p + 4] = np.array([f16_bits(-0.01)], np.uint16).view(np.uint8)
        b[p + 4:p + 16] = [(blk * 13 + i * 7) % 256 for i in range(12)]
        b[p + 16:p + 48] = [(blk * 31 + i * 11) % 256 for i in range(32)]
        b[p + 48:p + 176] = [(blk * 17 + i * 3) % 256 for i in range(128)]
    want = oracle.dequant("q5_k", b, rows * cols)
    lo, hi, scales, mins, d, dmin = oracle.q5ks_from_ggml(b, rows, cols)
    pos = np.arange(rows * cols)
    code = ((lo[pos // 8] >> ((pos % 8) * 4)) & 0xF) | (((hi[pos // 32] >> (pos % 32)) & 1) << 4)
    r, c = pos // cols, pos % cols
    sub, sup = r * (cols // 32) + c // 32, r * (cols // 256) + c // 256
    got = code.astype(np.float32) * (d[sup] * scales[sub].astype(np.float32)) + \
        dmin[sup] * mins[sub].astype(np.float32)
    assert np.max(np.abs(got - want)) < 1e-5


def _iq4_block(d=1.0):
    b = np.zeros(136, np.uint8)
    b[0:2] = np.array([f16_bits(d)], np.uint16).view(np.uint8)
    return b


IQ4 = [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113]


def test_dequant_iq4_xs_known_block(oracle):
    # dequant_iq4_xs_known_block (gguf.rs:2994-3005): ls = 0 -> dl = -32
    b = _iq4_block()
    b[8] = 0x10
    out = oracle.dequant("iq4_xs", b, 256)
    assert out[0] == -32.0 * -127.0 and out[16] == -32.0 * -104.0 and out[1] == -32.0 * -127.0


def test_iq4_xs_sub_scale_32_is_the_zero_point(oracle):
    # iq4_xs_sub_scale_32_is_the_zero_point (gguf.rs:3007-3028)
    b = _iq4_block()
    b[2:4] = np.array([sum(2 << (2 * j) for j in range(8))], np.uint16).view(np.uint8)
    b[8:] = 0xFF
    assert not oracle.dequant("iq4_xs", b, 256).any()


def test_iq4_xs_each_sub_block_uses_its_own_scale_and_the_codebook(oracle):
    # iq4_xs_each_sub_block_uses_its_own_scale (gguf.rs:3030-3055), then every code of every
    # sub-block against the codebook (iq4_xs_codebook_is_not_a_linear_ramp, gguf.rs:3057-3064)
    b = _iq4_block()
    sh = 0
    for j in range(8):
        ls = 33 + j
        b[4 + j // 2] |= (ls & 0xF) << (4 * (j % 2))
        sh |= ((ls >> 4) & 3) << (2 * j)
    b[2:4] = np.array([sh], np.uint16).view(np.uint8)
    rng = np.random.default_rng(5)
    codes = rng.integers(0, 16, 256)
    for j in range(8):
        for i in range(16):
            b[8 + 16 * j + i] = codes[32 * j + i] | (codes[32 * j + 16 + i] << 4)
    out = oracle.dequant("iq4_xs", b, 256)
    want = np.array([(e // 32 + 1) * IQ4[codes[e]] for e in range(256)], np.float32)
    assert np.array_equal(out, want)
    assert IQ4 != [(c - 8) * 16 for c in range(16)]


def test_dequant_q80_closed_form(oracle):
    qs = np.arange(-128, 128, dtype=np.int32)
    for d in (1.0, 0.5, 0.001, 6.0e-8, 65504.0):
        blocks = np.concatenate([make_q80_block(d, qs[i:i + 32]) for i in range(0, 256, 32)])
        got = oracle.dequant("q8_0", blocks, 256)
        want = np.float32(np.float16(d)) * qs.astype(np.float32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), d


# --------------------------------------------------------------- matmuls ----
def test_matmul_nt_matches_float64(oracle):
    # crates/arf-ml/src/matmul.rs:516-531 (nt vs standard, k not a multiple of 8)
    for (m, k, n) in [(3, 13, 5), (64, 40, 64), (4, 300, 33)]:
        a = np.random.default_rng(m).standard_normal((m, k)).astype(np.float32)
        b = np.random.default_rng(n).standard_normal((n, k)).astype(np.float32)
        got = oracle.matmul_nt(a, b)
        want = a.astype(np.float64) @ b.astype(np.float64).T
        assert np.max(np.abs(got - want)) < 1e-4


def test_matmul_nt_integer_exact(oracle):
    # crates/arf-ml/src/matmul.rs:551-566 (parallel path == serial), integer data -> exact
    a = (np.arange(64 * 40) % 7).astype(np.float32).reshape(64, 40)
    b = (np.arange(64 * 40) % 5).astype(np.float32).reshape(64, 40)
    assert np.array_equal(oracle.matmul_nt(a, b), (a.astype(np.int64) @ b.astype(np.int64).T))


@pytest.mark.parametrize("qtype,k", [("q4_k", 512), ("q6_k", 512), ("q8_0", 256), ("q5_k", 512),
                                     ("iq4_xs", 512)])
def test_quantized_linear_equals_dequant_matmul(oracle, qtype, k):
    # weight.rs:1693-1709: quantized linear == dequant + f32 matmul
    from arf_amd import synth
    n, m = 24, 3
    blocks = synth.weight(qtype, n, k, seed=17)
    x = synth.activations(m, k, seed=18)
    w = oracle.dequant(qtype, blocks, n * k).reshape(n, k).astype(np.float64)
    want = x.astype(np.float64) @ w.T
    got = oracle.matmul_q(qtype, x, blocks, n)
    assert rel_err(got, want) < 1e-5


def test_quantized_matmul_exact_on_integer_inputs(oracle):
    # power-of-two scales + integer activations: every f32 op is exact
    rng = np.random.default_rng(3)
    n, k = 4, 512
    blocks, wexact = [], []
    for r in range(n):
        for sb in range(k // 256):
            sc = rng.integers(0, 64, 8).tolist(); m = rng.integers(0, 64, 8).tolist()
            q = rng.integers(0, 16, 256).tolist()
            blocks.append(make_q4k_block(0.25, 0.5, sc, m, q))
            wexact += [float(v) for v in q4k_exact(0.25, 0.5, sc, m, q)]
    W = np.array(wexact).reshape(n, k)
    x = rng.integers(-3, 4, (2, k)).astype(np.float32)
    got = oracle.matmul_q("q4_k", x, np.concatenate(blocks), n)
    assert np.array_equal(got.astype(np.float64), x.astype(np.float64) @ W.T)


def test_par_rows_threads_do_not_change_result(oracle):
    from arf_amd import synth
    blocks = synth.weight("q4_k", 64, 512, seed=1)
    x = synth.activations(16, 512, seed=2)
    oracle.set_threads(1)
    serial = oracle.matmul_q("q4_k", x, blocks, 64)
    oracle.set_threads(0)
    par = oracle.matmul_q("q4_k", x, blocks, 64)
    assert np.array_equal(serial, par)


# ------------------------------------------------------------ routing ----
def test_top_k_softmax_reference_cases(oracle):
    # crates/arf-core/src/model/moe.rs:134-159
    ids, w = oracle.top_k_softmax([2.0, -1.0, 3.0, 0.0], 2, True)
    assert ids.tolist() == [2, 0] and abs(w.sum() - 1.0) < 1e-6 and w[0] > w[1]
    ids, w = oracle.top_k_softmax([2.0, -1.0, 3.0, 0.0], 2, False)
    assert 0.5 < w.sum() < 1.0
    ids, _ = oracle.top_k_softmax([1.0, 1.0, 1.0, 1.0], 2, True)
    assert ids.tolist() == [0, 1]


def test_top_k_softmax_128_expert_lcg_cases(oracle):
    # crates/arf-gpu/tests/moe_gpu.rs:84-93: two 128-expert top-8 cases, seed 99
    state = 99
    for norm in (True, False):
        logits, state = moe_route_lcg_logits(128, state)
        ids, w = oracle.top_k_softmax(logits, 8, norm)
        p = np.exp(logits.astype(np.float64) - logits.max())
        p /= p.sum()
        order = sorted(range(128), key=lambda i: (-p[i], i))[:8]
        assert ids.tolist() == order
        want = p[order] / (p[order].sum() if norm else 1.0)
        assert np.max(np.abs(w - want)) < 1e-6


# ---------------------------------------------------------------- MoE ----
def _silu64(v):
    return v / (1.0 + np.exp(-v))


def test_moe_forward_matches_float64_composition(oracle):
    from arf_amd import synth
    E, hidden, inter, T, top_k = 4, 256, 256, 3, 2
    gate = synth.weight("q4_k", inter, hidden, seed=31, experts=E)
    up = synth.weight("q4_k", inter, hidden, seed=32, experts=E)
    down = synth.weight("q4_k", hidden, inter, seed=33, experts=E)
    x = synth.activations(T, hidden, seed=34)
    logits = synth.router_logits(T, E, seed=35)
    got = oracle.moe_forward(x, gate, up, down, E, inter, logits, top_k, True)
    G = oracle.dequant("q4_k", gate, E * inter * hidden).reshape(E, inter, hidden).astype(np.float64)
    U = oracle.dequant("q4_k", up, E * inter * hidden).reshape(E, inter, hidden).astype(np.float64)
    D = oracle.dequant("q4_k", down, E * hidden * inter).reshape(E, hidden, inter).astype(np.float64)
    want = np.zeros((T, hidden))
    for t in range(T):
        p = np.exp(logits[t].astype(np.float64) - logits[t].max()); p /= p.sum()
        ids = sorted(range(E), key=lambda i: (-p[i], i))[:top_k]
        wts = p[ids] / p[ids].sum()
        xt = x[t].astype(np.float64)
        for e, wt in zip(ids, wts):
            h = _silu64(G[e] @ xt) * (U[e] @ xt)
            want[t] += wt * (D[e] @ h)
    assert rel_err(got, want) < 1e-4


def test_moe_one_hot_router_is_the_expert(oracle):
    from arf_amd import synth
    E, hidden, inter = 3, 256, 256
    gate = synth.weight("q4_k", inter, hidden, seed=41, experts=E)
    up = synth.weight("q4_k", inter, hidden, seed=42, experts=E)
    down = synth.weight("q4_k", hidden, inter, seed=43, experts=E)
    x = synth.activations(1, hidden, seed=44)
    logits = np.array([[-1e4, 30.0, -1e4]], np.float32)  # all mass on expert 1
    got = oracle.moe_forward(x, gate, up, down, E, inter, logits, 1, True)
    gb = gate.reshape(E, -1)[1]; ub = up.reshape(E, -1)[1]; db = down.reshape(E, -1)[1]
    g = oracle.matmul_q("q4_k", x, gb, inter)
    u = oracle.matmul_q("q4_k", x, ub, inter)
    h = (g / (1 + np.exp(-g))) * u
    y = oracle.matmul_q("q4_k", h.astype(np.float32), db, hidden)
    assert rel_err(got, y) < 1e-6


def test_moe_dequant_reference_equals_moe_forward(oracle):
    # the full-size C5 GPU check computes MoeMlp::forward from the oracle's routing and
    # dequant with BLAS products per expert; it must agree with the oracle's own
    # restatement of moe.rs:53-86 (serial token loop, matmul_nt_q4ks per projection)
    from arf_amd import synth
    from formats import moe_dequant_reference
    E, T, k, hidden, inter = 8, 24, 2, 512, 256
    raw = [synth.weight("q4_k", inter, hidden, seed=70, experts=E),
           synth.weight("q4_k", inter, hidden, seed=71, experts=E),
           synth.weight("q4_k", hidden, inter, seed=72, experts=E)]
    x = (synth.activations(T, hidden, seed=73) * np.float32(0.05)).astype(np.float32)
    logits = synth.router_logits(T, E, seed=74)
    want = oracle.moe_forward(x, raw[0], raw[1], raw[2], E, inter, logits, k, True)
    got = moe_dequant_reference(oracle, x, raw, E, hidden, inter, logits, k, True)
    assert rel_err(got, want) < 1e-5


def test_moe_forward_accumulates_onto_shared_output(oracle):
    # MoeMlp::forward with a shared expert (moe.rs:62-67): out starts at 0, the shared
    # output s is added first, then w_j * y_j per token in slot order.  init = 0 gives the
    # plain block bit for bit; init = s gives s plus the routed sum (within f32 rounding),
    # and each token's result is ((s + w0 y0) + w1 y1) exactly
    from arf_amd import synth
    E, hidden, inter, T, top_k = 4, 256, 256, 3, 2
    gate = synth.weight("q4_k", inter, hidden, seed=51, experts=E)
    up = synth.weight("q4_k", inter, hidden, seed=52, experts=E)
    down = synth.weight("q4_k", hidden, inter, seed=53, experts=E)
    x = (synth.activations(T, hidden, seed=54) * np.float32(0.05)).astype(np.float32)
    logits = synth.router_logits(T, E, seed=55)
    plain = oracle.moe_forward(x, gate, up, down, E, inter, logits, top_k, True)
    zero = oracle.moe_forward(x, gate, up, down, E, inter, logits, top_k, True, init=np.zeros_like(plain))
    assert np.array_equal(plain.view(np.uint32), zero.view(np.uint32))
    s = synth.activations(T, hidden, seed=56)
    got = oracle.moe_forward(x, gate, up, down, E, inter, logits, top_k, True, init=s)
    assert rel_err(got, s.astype(np.float64) + plain) < 1e-5
    # slot by slot: one-expert blocks (top_k = 1 of a one-hot router) added in order
    for t in range(T):
        ids, wts = oracle.top_k_softmax(logits[t], top_k, True)
        acc = s[t].copy()
        for e, w in zip(ids, wts):
            oh = np.full((1, E), -1e4, np.float32)
            oh[0, e] = 30.0
            ye = oracle.moe_forward(x[t:t + 1], gate, up, down, E, inter, oh, 1, True)[0]
            acc = (acc + np.float32(w) * ye).astype(np.float32)
        assert np.array_equal(acc.view(np.uint32), got[t].view(np.uint32))


def _gelu64(v):
    v = np.asarray(v, np.float64)
    inner = np.clip(np.sqrt(2.0 / np.pi) * (v + 0.044715 * v ** 3), -15.0, 15.0)
    return 0.5 * v * (1.0 + np.tanh(inner))


def test_geglu_known_values_and_closed_forms(oracle):
    # GeGLU (decode_ops_msl.metal:15-27, CPU oracle selftest.rs:6091-6095): gelu_tanh(g) * u
    one = np.ones(1, np.float32)
    f = lambda g: oracle.glu(np.array([g], np.float32), one, 1)[0]
    assert f(0.0) == 0.0
    # qwen_vision.rs:1205 gelu_tanh(1.0) = 0.841192 (to 1e-5): the erf form gives 0.8413447
    # and dropping the cubic term 0.8317, both outside it
    assert abs(f(1.0) - 0.841192) < 1e-5
    # vision.rs:512-513
    assert abs(f(0.0)) < 1e-6 and f(10.0) > 9.9 and abs(f(-10.0)) < 1e-3
    # |g| >= 7: the (clamped) tanh is +-1 in f32, so gelu(g) = g and gelu(-g) = 0
    for g in (7.0, 8.5, 34.0, 1e6, 1e20):
        assert f(g) == np.float32(g)
        assert f(-g) == 0.0
    # oddness of tanh: gelu(g) - gelu(-g) = g
    g = np.linspace(-6, 6, 1201, dtype=np.float32)
    ones = np.ones_like(g)
    d = oracle.glu(g, ones, 1).astype(np.float64) - oracle.glu(-g, ones, 1).astype(np.float64)
    assert np.max(np.abs(d - g) / np.maximum(np.abs(g), 1e-3)) < 4e-7
    # the selftest's inputs (gate spans the clamp region) against float64 of the same
    # formula: within 1e-6 relative, plus the f32 rounding of tanh (2^-22 of 0.5 |g u|),
    # which 1 + tanh(inner) magnifies where gelu is near 0 (g < -3)
    i = np.arange(4096)
    gs = (((i % 29) - 14) * 0.3).astype(np.float32)
    us = (((i % 19) - 9) * 0.1).astype(np.float32)
    got = oracle.glu(gs, us, 1).astype(np.float64)
    want = _gelu64(gs) * us.astype(np.float64)
    bound = 1e-6 * np.abs(want) + 2.0 ** -22 * 0.5 * np.abs(gs.astype(np.float64) * us)
    assert np.all(np.abs(want - got) <= bound)


def test_swiglu_act_matches_float64(oracle):
    i = np.arange(4096)
    gs = (((i % 29) - 14) * 0.3).astype(np.float32)
    us = (((i % 19) - 9) * 0.1).astype(np.float32)
    got = oracle.glu(gs, us, 0).astype(np.float64)
    want = _silu64(gs.astype(np.float64)) * us.astype(np.float64)
    assert np.max(np.abs(want - got) / np.maximum(np.abs(want), 1e-4)) < 2e-6
