"""The Q6_K operand arithmetic of the skinny MFMA kernel, replayed in numpy (CPU).

arfq_skinny.h (SkQ6K::codes, SkQ6KI::frag) builds the B operand of each MFMA from the
repacked Q6_K bytes without a table: the 6-bit codes q are assembled as bytes, v_perm puts
two of them under the f16 pattern of 1024 (the value 1024 + q), and one packed f16 FMA per
two weights gives sc * (q - 32) / 2 = (1024 + q) * (sc / 2) - 528 * sc.  The scale itself
comes from the byte sc + 128 under 0x64 (1152 + sc), times 1/2, less 576.  These tests pin
the claims the kernel rests on: the codes match ggml's dequant order (dequant_q6_k,
crates/arf-core/src/model/gguf.rs:2092-2131), every step is exact in f16 for |sc| <= 62, and
the FMA's constant stops being an f16 value at |sc| = 63 -- the bound of the upload's flag
that routes a tensor to the kernel's other (f32-scaled) form.
"""
import numpy as np

f16 = np.float16


def _fma16(a, b, c):
    # v_pk_fma_f16: a * b + c with one rounding (the product of two f16 values is exact in
    # float64, and so is the sum here: every term is below 2^17 with 11-bit significands)
    return f16(np.float64(a) * np.float64(b) + np.float64(c))


def _sc_half(sc):
    v = f16(1024 + (sc + 128))             # the byte sc + 128 under 0x64: 1152 + sc
    return _fma16(v, f16(0.5), f16(-576))   # sc / 2


def test_scale_and_constant_exact_up_to_62():
    for sc in range(-64, 65):
        s = _sc_half(sc)
        assert float(s) == sc / 2
        c = f16(np.float64(s) * -1056)      # v_pk_mul_f16: -528 sc
        if abs(sc) <= 62 or abs(sc) == 64:
            assert float(c) == -528 * sc, sc
        else:
            assert float(c) != -528 * sc    # 33 * 63 = 2079 needs 12 significant bits


def test_operand_exact_for_every_code_within_62():
    q = np.arange(64)
    for sc in range(-62, 63):
        s = _sc_half(sc)
        c = f16(np.float64(s) * -1056)
        got = np.array([float(_fma16(f16(1024 + int(v)), s, c)) for v in q])
        np.testing.assert_array_equal(got, (q - 32) * sc / 2)


def test_kind4_codes_minus_32_exact():
    # the other form: (1024 + q) - 1056 = q - 32, exact
    q = np.arange(64)
    got = (q + 1024).astype(f16) + f16(-1056)
    np.testing.assert_array_equal(got.astype(np.float64), q - 32)


def _codes(qa, qb, qh, t):
    # SkQ6K::codes for one dword: quadrant t's four codes, one per byte
    lo = (qb if t & 1 else qa) >> (4 if t & 2 else 0)
    hi = [qh << 4, qh << 2, qh, qh >> 2][t]
    return ((lo & 0x0F0F0F0F) | (hi & 0x30303030)) & 0xFFFFFFFF


def test_byte_codes_follow_ggml_order():
    rng = np.random.default_rng(7)
    for _ in range(300):
        qa, qb, qh = (int(v) for v in rng.integers(0, 2**32, size=3, dtype=np.uint64))
        for t in range(4):
            got = _codes(qa, qb, qh, t)
            for i in range(4):
                la = (qa >> (8 * i)) & 0xFF
                lb = (qb >> (8 * i)) & 0xFF
                h = (qh >> (8 * i)) & 0xFF
                # ggml: q1 = ql[l] & 0xF | (qh[l] & 3) << 4, q2 = ql[l + 32] & 0xF | (qh >> 2 & 3) << 4,
                # q3 = ql[l] >> 4 | (qh >> 4 & 3) << 4, q4 = ql[l + 32] >> 4 | (qh >> 6 & 3) << 4
                l = lb if t & 1 else la
                want = ((l >> 4) if t & 2 else (l & 0xF)) | (((h >> (2 * t)) & 3) << 4)
                assert (got >> (8 * i)) & 0xFF == want
