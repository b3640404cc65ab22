"""GPU parity: the HIP path (through the C ABI) against the CPU oracle.

Dequant: bit-exact (memcmp of the f32 arrays), including f16-subnormal scales.
Matmul: max_i |g_i - c_i| / max(|c_i|, rms(c)) <= 2e-3 (fp32 accumulation).
"""
import sys

import numpy as np
import pytest

from conftest import rel_err
from formats import make_q80_block

pytestmark = pytest.mark.gpu

TOL = 2e-3


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


# ------------------------------------------------------------- dequant ----
def test_f16_conversion_exhaustive_via_q8_0(gpu_ctx, oracle):
    # q = 1 everywhere, d = every f16 pattern: dequant = f16_to_f32(d) * 1
    _say("case: f16 exhaustive")
    from arf_amd import QType
    d = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    blocks = np.zeros((65536, 34), np.uint8)
    blocks[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
    blocks[:, 2:34] = 1
    w = gpu_ctx.upload(QType.Q8_0, blocks, 2048, 1024)
    got = gpu_ctx.dequant(w).numpy().reshape(65536, 32)[:, 0]
    want = oracle.dequant("q8_0", blocks, 65536 * 32).reshape(65536, 32)[:, 0]
    finite = np.isfinite(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(np.isinf(got), np.isinf(want))


@pytest.mark.parametrize("qtype", ["q4_k", "q6_k", "q8_0", "q5_k", "iq4_xs"])
def test_dequant_bit_exact(gpu_ctx, oracle, qtype):
    _say("case: dequant", qtype)
    from arf_amd import QType, synth
    n, k, E = 40, 1024, 3
    raw = synth.weight(qtype, n, k, seed=101, experts=E)
    bb = synth.BLOCK_BYTES[qtype]
    blk = raw.reshape(-1, bb)
    # f16-subnormal and zero scales in some blocks
    dofs = {"q4_k": 0, "q8_0": 0, "q6_k": 208, "q5_k": 0, "iq4_xs": 0}[qtype]
    blk[::5, dofs:dofs + 2] = np.array([3, 0], np.uint8)
    blk[1::9, dofs:dofs + 2] = 0
    w = gpu_ctx.upload(QType[qtype.upper()], raw, n, k, E)
    got = gpu_ctx.dequant(w).numpy()
    want = oracle.dequant(qtype, raw, E * n * k)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_dequant_q80_known_closed_form(gpu_ctx):
    from arf_amd import QType
    qs = np.arange(-128, 128).reshape(8, 32)
    blocks = np.concatenate([make_q80_block(0.5, q) for q in qs])
    w = gpu_ctx.upload(QType.Q8_0, blocks, 1, 256)
    got = gpu_ctx.dequant(w).numpy()
    assert np.array_equal(got, 0.5 * np.arange(-128, 128, dtype=np.float32))


# ---------------------------------------------------------------- GEMV ----
def _matmul(ctx, qtype, n, k, m, seed, x_dtype=np.float32, experts=1, expert=0):
    from arf_amd import QType, synth
    raw = synth.weight(qtype, n, k, seed=seed, experts=experts)
    x = synth.activations(m, k, seed=seed + 1).astype(x_dtype)
    w = ctx.upload(QType[qtype.upper()], raw, n, k, experts)
    xd = ctx.to_device(x)
    y = ctx.empty((m, n), np.float32)
    ctx.matmul(w, xd, m, y, expert)
    got = y.numpy()
    per = raw.size // experts
    return got, raw[expert * per:(expert + 1) * per], x


@pytest.mark.parametrize("qtype,n,k", [
    ("q4_k", 64, 256), ("q4_k", 37, 1024), ("q4_k", 130, 5120), ("q4_k", 33, 768),
    ("q8_0", 64, 2048), ("q8_0", 31, 96), ("q8_0", 100, 512),
    ("q6_k", 64, 4352), ("q6_k", 21, 256), ("q6_k", 50, 17408),
    ("q5_k", 64, 256), ("q5_k", 37, 1024), ("q5_k", 130, 5120), ("q5_k", 33, 2816),
    ("iq4_xs", 64, 256), ("iq4_xs", 37, 1024), ("iq4_xs", 130, 5120), ("iq4_xs", 33, 2816),
])
@pytest.mark.parametrize("m", [1, 2, 3, 4])
def test_gemv_small_shapes(gpu_ctx, oracle, qtype, n, k, m):
    _say("case: gemv", qtype, n, k, m)
    got, raw, x = _matmul(gpu_ctx, qtype, n, k, m, seed=7 * n + k + m)
    want = oracle.matmul_q(qtype, x, raw, n)
    assert rel_err(got, want) <= TOL


@pytest.mark.parametrize("qtype", ["q4_k", "q6_k", "q5_k", "iq4_xs"])
@pytest.mark.parametrize("n,k", [(300, 32768), (5000, 12288)])
def test_gemv_f32_many_columns(gpu_ctx, oracle, qtype, n, k):
    # the m = 1 f32 GEMVs at 32 and 12 four-block columns: a group whose home column runs
    # out takes the next one not yet exhausted from the workgroup's mask; at n = 300 most
    # workgroups hold 1-2 rows, fewer chunks per column than groups
    _say("case: gemv f32 many columns", qtype, n, k)
    got, raw, x = _matmul(gpu_ctx, qtype, n, k, 1, seed=11 * n + k)
    want = oracle.matmul_q(qtype, x, raw, n)
    assert rel_err(got, want) <= 1e-5


@pytest.mark.parametrize("qtype,m", [("q4_k", 1), ("q6_k", 1), ("q6_k", 2), ("q5_k", 1), ("q5_k", 3),
                                     ("iq4_xs", 1), ("iq4_xs", 4)])
def test_gemv_expert_offset(gpu_ctx, oracle, qtype, m):
    _say("case: gemv expert offset", qtype, m)
    got, raw, x = _matmul(gpu_ctx, qtype, 48, 512, m, seed=5, experts=4, expert=3)
    assert rel_err(got, oracle.matmul_q(qtype, x, raw, 48)) <= TOL


def test_c1_q8_0_gemv_full(gpu_ctx, oracle):
    _say("case: C1 full")
    got, raw, x = _matmul(gpu_ctx, "q8_0", 2048, 2048, 1, seed=0xA7F00001)
    assert rel_err(got, oracle.matmul_q("q8_0", x, raw, 2048)) <= TOL


# The m = 1 Q4_K GEMV multiplies f32 x by the exact weights in f32 (only the
# order of the f32 sums differs from matmul_nt_q4ks), so it is held to 1e-5.
F32_TOL = 1e-5


def test_c2_q4_k_gemv_full(gpu_ctx, oracle):
    _say("case: C2 full")
    got, raw, x = _matmul(gpu_ctx, "q4_k", 17408, 5120, 1, seed=0xA7F00002)
    want = oracle.matmul_q("q4_k", x, raw, 17408)
    e = rel_err(got, want)
    _say("C2 rel err", e)
    assert e <= F32_TOL


def test_c2_q4_k_gemv_x16_option(gpu_ctx, oracle):
    # ARFQ_OPT_GEMV_X16: the 16-bit fixed-point x kernel, within the matmul gate
    _say("case: C2 full, x16 option")
    import arf_amd
    gpu_ctx.set_options(arf_amd.arfq.OPT_GEMV_X16)
    try:
        got, raw, x = _matmul(gpu_ctx, "q4_k", 17408, 5120, 1, seed=0xA7F00002)
    finally:
        gpu_ctx.set_options(0)
    e = rel_err(got, oracle.matmul_q("q4_k", x, raw, 17408))
    _say("C2 x16 rel err", e)
    assert e <= TOL


def _q4k_dyadic_blocks(n, k, seed):
    """Q4_K blocks with d = 2^-4, dmin = 2^-5 and random 6-bit scales / nibbles:
    every weight is a multiple of 2^-9 below 64."""
    from arf_amd import synth
    raw = synth.weight("q4_k", n, k, seed=seed).reshape(-1, 144)
    raw[:, 0:2] = np.frombuffer(np.float16(2.0 ** -4).tobytes(), np.uint8)
    raw[:, 2:4] = np.frombuffer(np.float16(2.0 ** -5).tobytes(), np.uint8)
    return raw.reshape(-1)


@pytest.mark.parametrize("n,k", [(17408, 5120), (300, 256), (64, 2048)])
def test_q4k_gemv_f32_exact_on_integer_x(gpu_ctx, oracle, n, k):
    # integer x in [-8, 8] and dyadic weights: every product, sub-block sum and
    # row sum is exact in f32 in any order, so the GEMV must equal the oracle bit
    # for bit -- any rounding of x or of the codes would show
    _say("case: q4k f32 exact", n, k)
    from arf_amd import QType
    raw = _q4k_dyadic_blocks(n, k, seed=n + k)
    rng = np.random.default_rng(k)
    x = rng.integers(-8, 9, size=(1, k)).astype(np.float32)
    w = gpu_ctx.upload(QType.Q4_K, raw, n, k)
    y = gpu_ctx.empty((1, n), np.float32)
    gpu_ctx.matmul(w, gpu_ctx.to_device(x), 1, y)
    got = y.numpy()
    want = oracle.matmul_q("q4_k", x, raw, n)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("case", ["huge", "tiny", "mixed"])
def test_q4k_gemv_f32_dynamic_range(gpu_ctx, oracle, case):
    # sub-blocks of x at very different magnitudes: above 2^76 the kernel holds x at
    # a smaller power of two; f32 subnormal x is scaled up exactly
    _say("case: q4k f32 range", case)
    from arf_amd import QType, synth
    n, k = 96, 2048
    raw = synth.weight("q4_k", n, k, seed=77)
    rng = np.random.default_rng(78)
    x = rng.standard_normal((1, k)).astype(np.float32)
    sub = x.reshape(-1, 32)
    if case == "huge":
        sub *= np.float32(2.0 ** 90)
    elif case == "tiny":
        sub *= np.float32(2.0 ** -130)  # mostly f32 subnormals
    else:
        exps = rng.integers(-60, 100, size=(sub.shape[0], 1))
        sub *= np.exp2(exps).astype(np.float32)
    x = sub.reshape(1, k)
    w = gpu_ctx.upload(QType.Q4_K, raw, n, k)
    y = gpu_ctx.empty((1, n), np.float32)
    gpu_ctx.matmul(w, gpu_ctx.to_device(x), 1, y)
    got = y.numpy()
    want = oracle.matmul_q("q4_k", x, raw, n)
    assert np.all(np.isfinite(got))
    e = rel_err(got, want)
    _say("rel err", e)
    assert e <= (1e-4 if case == "tiny" else F32_TOL)


def test_c3_q6_k_gemv_m1_full(gpu_ctx, oracle):
    # C3 at m = 1: the f32-x GEMV (exact products), held to the f32 bound
    _say("case: C3 m=1 full")
    got, raw, x = _matmul(gpu_ctx, "q6_k", 5120, 17408, 1, seed=0xA7F00003)
    e = rel_err(got, oracle.matmul_q("q6_k", x, raw, 5120))
    _say("C3 m=1 rel err", e)
    assert e <= F32_TOL


def test_c3_q6_k_gemv_x16_option(gpu_ctx, oracle):
    # ARFQ_OPT_GEMV_X16 at C3 m = 1: the integer-dot kernel (x in 16-bit fixed point)
    import arf_amd
    _say("case: C3 m=1, x16 option")
    gpu_ctx.set_options(arf_amd.arfq.OPT_GEMV_X16)
    try:
        got, raw, x = _matmul(gpu_ctx, "q6_k", 5120, 17408, 1, seed=0xA7F00003)
    finally:
        gpu_ctx.set_options(0)
    e = rel_err(got, oracle.matmul_q("q6_k", x, raw, 5120))
    _say("C3 x16 rel err", e)
    assert e <= TOL


def _dyadic_blocks(qtype, n, k, seed):
    """Q6_K and IQ4_XS blocks with d = 2^-4, Q5_K blocks with d = 2^-4 and dmin = 2^-5
    (random codes and scales): every weight is a multiple of 2^-5 below 256."""
    from arf_amd import synth
    bb = {"q6_k": 210, "q5_k": 176, "iq4_xs": 136}[qtype]
    raw = synth.weight(qtype, n, k, seed=seed).reshape(-1, bb)
    if qtype == "q6_k":
        raw[:, 208:210] = np.frombuffer(np.float16(2.0 ** -4).tobytes(), np.uint8)
    elif qtype == "iq4_xs":
        raw[:, 0:2] = np.frombuffer(np.float16(2.0 ** -4).tobytes(), np.uint8)
    else:
        raw[:, 0:2] = np.frombuffer(np.float16(2.0 ** -4).tobytes(), np.uint8)
        raw[:, 2:4] = np.frombuffer(np.float16(2.0 ** -5).tobytes(), np.uint8)
    return raw.reshape(-1)


@pytest.mark.parametrize("qtype,n,k", [("q6_k", 512, 4096), ("q6_k", 300, 256), ("q5_k", 512, 4096),
                                       ("q5_k", 64, 2048), ("iq4_xs", 512, 4096), ("iq4_xs", 70, 1024)])
def test_dot_gemv_f32_exact_on_integer_x(gpu_ctx, oracle, qtype, n, k):
    # the f32-x Q6_K / Q5_K / IQ4_XS GEMV (m = 1): integer x in [-8, 8] and dyadic weights keep
    # every product and sum exact in f32 in any order, so the result equals the
    # oracle's bit for bit -- any rounding of x or of the codes would show
    _say("case: dot f32 exact", qtype, n, k)
    from arf_amd import QType
    raw = _dyadic_blocks(qtype, n, k, seed=n + k)
    rng = np.random.default_rng(k + 1)
    x = rng.integers(-8, 9, size=(1, k)).astype(np.float32)
    w = gpu_ctx.upload(QType[qtype.upper()], raw, n, k)
    y = gpu_ctx.empty((1, n), np.float32)
    gpu_ctx.matmul(w, gpu_ctx.to_device(x), 1, y)
    assert np.array_equal(y.numpy(), oracle.matmul_q(qtype, x, raw, n))


@pytest.mark.parametrize("qtype", ["q5_k", "iq4_xs"])
def test_next_formats_gemv_c2_shape(gpu_ctx, oracle, qtype):
    # Q5_K / IQ4_XS at C2's shape (the survey's next row: no benchmark config of its own)
    _say("case: C2 shape", qtype)
    got, raw, x = _matmul(gpu_ctx, qtype, 17408, 5120, 1, seed=0xA7F00005)
    e = rel_err(got, oracle.matmul_q(qtype, x, raw, 17408))
    _say(qtype, "rel err", e)
    assert e <= F32_TOL  # m = 1: the f32-x GEMV


@pytest.mark.parametrize("qtype", ["q5_k", "iq4_xs"])
@pytest.mark.parametrize("m,n,k,x16", [(1, 130, 1024, True), (4, 64, 256, True), (5, 130, 1024, False),
                                       (8, 37, 2816, True), (32, 200, 5120, False),
                                       (33, 130, 1024, False), (64, 256, 2816, True),
                                       (100, 130, 1024, False), (130, 64, 512, True)])
def test_next_formats_skinny_and_prefill(gpu_ctx, oracle, qtype, m, n, k, x16):
    # Q5_K / IQ4_XS beyond the decode GEMV: the skinny MFMA kernel (m <= 64) and the
    # prefill above 64 rows; f16 x (the x16 cases) is what the oracle sees.  Exact
    # weights with x in f16 parts hold 2e-5: Q5_K everywhere at f32 x, IQ4_XS on the skinny
    # kernel; the IQ4_XS prefill at f32 x runs the tile loop with weights rounded to f16
    _say("case: next-format skinny", qtype, m, n, k, "f16" if x16 else "f32")
    dt = np.float16 if x16 else np.float32
    got, raw, x = _matmul(gpu_ctx, qtype, n, k, m, seed=11 * m + n, x_dtype=dt)
    e = rel_err(got, oracle.matmul_q(qtype, x.astype(np.float32), raw, n))
    _say("rel err", e)
    exact = not x16 and (qtype == "q5_k" or m <= 64)
    assert e <= (2e-5 if exact else TOL)


@pytest.mark.parametrize("m,lim", [(1, 128), (8, 128), (64, 128), (130, 128), (8, 64), (64, 64),
                                   (130, 64), (8, 62), (64, 62)])
def test_q6_k_full_range_scales(gpu_ctx, oracle, m, lim):
    # quantizers put each block's largest sub-block scale near +-127, where sc * (q - 32)
    # passes 2048 and would round in f16; the skinny kernel (m = 5..64) multiplies the exact
    # codes q - 32 and scales each sub-block's product by d * sc in f32, the prefill GEMM
    # (m = 130) holds sc * (q - 32) as f16 hi + lo operands (exact) against x as f16
    # hi + lo.  The synthetic blocks keep scales in [-32, 31], so this test draws them from
    # all of i8 (lim 128).  Scales within +-64 keep the prefill's one operand; within +-62
    # the skinny kernel's integer operands sc * (q - 32) / 2, whose FMA constant -528 sc is
    # an f16 value only up to |sc| = 62: lim 64 and 62 put +-lim and +-(lim - 1) into every
    # block, so both sides of each threshold run.  At m = 8 (three f16 parts of x), 64 and
    # 130 (hi + lo) every output is held to 2e-5
    from arf_amd import QType, synth
    _say("case: q6_k full-range scales", m, lim)
    n, k = 384, 4096
    raw = synth.weight("q6_k", n, k, seed=0xA7F0000C)
    blk = raw.reshape(-1, 210)
    rng = np.random.default_rng(0xA7F0000D)
    if lim == 128:
        blk[:, 192:208] = rng.integers(-128, 128, size=(blk.shape[0], 16)).astype(np.int8).view(np.uint8)
    else:
        sc = rng.integers(-lim, lim + 1, size=(blk.shape[0], 16))
        sc[:, :4] = [lim, -lim, lim - 1, 1 - lim]
        blk[:, 192:208] = rng.permuted(sc, axis=1).astype(np.int8).view(np.uint8)
    x = synth.activations(m, k, seed=0xA7F0000E)
    w = gpu_ctx.upload(QType.Q6_K, raw, n, k)
    y = gpu_ctx.empty((m, n), np.float32)
    gpu_ctx.matmul(w, gpu_ctx.to_device(x), m, y)
    e = rel_err(y.numpy(), oracle.matmul_q("q6_k", x, raw, n))
    _say("rel err", e)
    assert e <= (2e-5 if m > 1 else TOL)


@pytest.mark.parametrize("qtype", ["q4_k", "q6_k", "q8_0"])
def test_vocab_wide_lm_head_gemv(gpu_ctx, oracle, qtype):
    # the survey's next row: the lm_head GEMV over a 151936-token vocabulary at K = 5120
    # (the bench's shape; Q4_K as the reference prefers the GGUF's own Q4_K blocks,
    # island.rs:557-570); every logit against the oracle's bit-exact dequant + BLAS (in row
    # chunks), and the first and last 2048 rows against the oracle's own matmul (the f32
    # GEMVs to 1e-5 there)
    _say("case: lm_head", qtype)
    n, k = 151936, 5120
    got, raw, x = _matmul(gpu_ctx, qtype, n, k, 1, seed=0xA7F0000A)
    assert np.all(np.isfinite(got))
    rb = raw.reshape(n, -1)
    want = np.concatenate([_dequant_matmul(oracle, qtype, x, rb[i:i + 16384].reshape(-1), min(16384, n - i))
                           for i in range(0, n, 16384)], axis=1)
    e = rel_err(got, want)
    _say("lm_head rel err (all rows)", e)
    assert e <= TOL
    for r0 in (0, n - 2048):
        part = oracle.matmul_q(qtype, x, rb[r0:r0 + 2048].reshape(-1), 2048)
        assert rel_err(got[:, r0:r0 + 2048], part) <= (TOL if qtype == "q8_0" else F32_TOL)


# ---- f32 x over the batched decode range ----
# m = 2..8 multiply f32 x in f32 terms: Q4_K / Q5_K / IQ4_XS on the skinny MFMA kernel
# with x as three f16 parts (hi + mid + lo, which represent every f32 value within 2^15 of
# its row's max |x| exactly; the exact codes times each part, f32 sums), Q6_K on the f32
# GEMV at m <= 4, Q8_0 on its f32 GEMV at m <= 4.  m = 9..64: the skinny kernel with x as
# f16 hi + lo (~22 bits).  Held to 2e-5 against the oracle.
SMALL_M_TOL = 2e-5


_SMALL_M_CASES = [(m, q, 200, 2048) for m in (2, 3, 4, 5, 8, 33, 48, 64)
                  for q in ("q4_k", "q5_k", "iq4_xs", "q6_k", "q8_0")] + \
                 [(m, "q4_k", 17408, 5120) for m in (2, 4, 64)]  # C2's shape


@pytest.mark.parametrize("m,qtype,n,k", _SMALL_M_CASES)
def test_small_m_f32_x(gpu_ctx, oracle, qtype, n, k, m):
    _say("case: small-m f32 x", qtype, n, k, m)
    got, raw, x = _matmul(gpu_ctx, qtype, n, k, m, seed=13 * m + n + k)
    e = rel_err(got, oracle.matmul_q(qtype, x, raw, n))
    _say("rel err", e)
    assert e <= SMALL_M_TOL


@pytest.mark.parametrize("qtype,n,k", [("q4_k", 300, 2048), ("q4_k", 17408, 5120), ("q5_k", 300, 2048),
                                       ("iq4_xs", 300, 2048), ("q6_k", 300, 2048)])
@pytest.mark.parametrize("m", [2, 3, 4])
def test_small_m_exact_on_integer_x(gpu_ctx, oracle, qtype, n, k, m):
    # integer x in [-8, 8] and dyadic weights: every product and sum is exact in f32 in
    # any order, so m = 2..4 must equal the oracle bit for bit, as m = 1 does
    _say("case: small-m exact", qtype, n, k, m)
    from arf_amd import QType
    raw = _q4k_dyadic_blocks(n, k, seed=n + k + m) if qtype == "q4_k" else _dyadic_blocks(qtype, n, k, seed=n + k + m)
    rng = np.random.default_rng(k + m)
    x = rng.integers(-8, 9, size=(m, k)).astype(np.float32)
    w = gpu_ctx.upload(QType[qtype.upper()], raw, n, k)
    y = gpu_ctx.empty((m, n), np.float32)
    gpu_ctx.matmul(w, gpu_ctx.to_device(x), m, y)
    assert np.array_equal(y.numpy(), oracle.matmul_q(qtype, x, raw, n))


@pytest.mark.parametrize("qtype", ["q4_k", "q5_k", "iq4_xs"])
def test_x16_option_long_k_keeps_working(gpu_ctx, oracle, qtype):
    # ARFQ_OPT_GEMV_X16 at a 70B-class ffn_down (n = 8192, k = 28672): the 16-bit kernels'
    # LDS would pass 64 KiB there (Q4_K 66.3 KB, Q5_K / IQ4_XS 68 KB), so these shapes keep
    # the f32 kernels and must still run
    import arf_amd
    _say("case: x16 long k", qtype)
    gpu_ctx.set_options(arf_amd.arfq.OPT_GEMV_X16)
    try:
        got, raw, x = _matmul(gpu_ctx, qtype, 8192, 28672, 1, seed=29)
    finally:
        gpu_ctx.set_options(0)
    e = rel_err(got, oracle.matmul_q(qtype, x, raw, 8192))
    _say("rel err", e)
    assert e <= F32_TOL


def test_x16_option_long_k_ffn(gpu_ctx, oracle):
    # the FFN's fused activation-into-down GEMV under ARFQ_OPT_GEMV_X16 with k = 28672
    import arf_amd
    from arf_amd import QType, synth
    _say("case: x16 long k ffn")
    hidden, inter = 8192, 28672
    shapes = [(inter, hidden), (inter, hidden), (hidden, inter)]
    raws = [synth.weight("q4_k", n, k, seed=41 + i) for i, (n, k) in enumerate(shapes)]
    ws = [gpu_ctx.upload(QType.Q4_K, r, n, k) for r, (n, k) in zip(raws, shapes)]
    x = (synth.activations(1, hidden, seed=47) * np.float32(0.005)).astype(np.float32)
    y = gpu_ctx.empty((1, hidden), np.float32)
    gpu_ctx.set_options(arf_amd.arfq.OPT_GEMV_X16)
    try:
        gpu_ctx.ffn(ws[0], ws[1], ws[2], gpu_ctx.to_device(x), 1, y)
    finally:
        gpu_ctx.set_options(0)
    g = oracle.matmul_q("q4_k", x, raws[0], inter)
    u = oracle.matmul_q("q4_k", x, raws[1], inter)
    want = oracle.matmul_q("q4_k", oracle.glu(g, u, 0).reshape(g.shape), raws[2], hidden)
    e = rel_err(y.numpy(), want)
    _say("rel err", e)
    assert e <= TOL


def test_shape_errors_raise(gpu_ctx):
    from arf_amd import QType, synth
    raw = synth.weight("q4_k", 4, 256, seed=1)
    with pytest.raises(ValueError):
        gpu_ctx.upload(QType.Q4_K, raw[:-1], 4, 256)
    with pytest.raises(ValueError):
        gpu_ctx.upload(QType.Q4_K, raw, 4, 255)
    w = gpu_ctx.upload(QType.Q4_K, raw, 4, 256)
    x = gpu_ctx.to_device(np.zeros((1, 256), np.float32))
    y = gpu_ctx.empty((1, 4), np.float32)
    with pytest.raises(ValueError):
        gpu_ctx.matmul(w, x, 1, y, expert=1)


# ---------------------------------------------------------------- GEMM ----
@pytest.mark.parametrize("m,n,k", [(8, 64, 256), (130, 200, 512), (300, 128, 1024),
                                   (64, 17, 768), (257, 129, 5120)])
def test_gemm_q4k_f16_small(gpu_ctx, oracle, m, n, k):
    _say("case: gemm q4k f16", m, n, k)
    got, raw, x = _matmul(gpu_ctx, "q4_k", n, k, m, seed=3 * m + n + k, x_dtype=np.float16)
    want = oracle.matmul_q("q4_k", x.astype(np.float32), raw, n)
    e = rel_err(got, want)
    _say("rel err", e)
    assert e <= TOL


@pytest.mark.parametrize("m", [5, 16, 64, 65, 200])
@pytest.mark.parametrize("qtype,n,k", [("q4_k", 96, 2048), ("q6_k", 130, 1792), ("q8_0", 77, 1216),
                                       ("q8_0", 100, 2048)])
def test_gemm_f32_x(gpu_ctx, oracle, qtype, n, k, m):
    # m > 4 goes through the MFMA kernels: f32 x scaled per row into f16 range, then
    # split into f16 parts (three at m <= 8, hi + lo above) on the skinny kernel and the
    # direct-operand prefill, whose weights are exact: 2e-5.  Q8_0 with k not a multiple
    # of 256 runs the tile loop (x hi + lo, weights d * q rounded to f16): 2e-3
    _say("case: gemm f32 x", qtype, n, k, m)
    got, raw, x = _matmul(gpu_ctx, qtype, n, k, m, seed=91 + m + n)
    e = rel_err(got, oracle.matmul_q(qtype, x, raw, n))
    _say("rel err", e)
    assert e <= (2e-5 if k % 256 == 0 else TOL)


@pytest.mark.parametrize("m", [5, 8, 32, 64, 130])
@pytest.mark.parametrize("qtype", ["q4_k", "q5_k", "q6_k", "q8_0", "iq4_xs"])
def test_mfma_paths_f32_x_beyond_f16_range(gpu_ctx, oracle, qtype, m):
    # m >= 5 runs the MFMA kernels on f16 operands: an f32 x is scaled per row by a power
    # of two into f16 range first (and the output rows back), so x blocks up to 1e6 -- far
    # past f16's 65504 -- stay finite.  x goes in as f16 hi + mid + lo (m <= 8) or hi + lo
    # (~22 bits), so even sub-blocks spread over 9 decades stay close to the f32 reference;
    # above 64 rows (the prefill kernels) checked on N(0,1) x with 1 block in 8 at 1e6.
    # IQ4_XS above 64 rows at f32 x runs the tile loop, whose weights are rounded to f16.
    _say("case: mfma f32 x range", qtype, m)
    from arf_amd import QType, synth
    n, k = 96, 2048
    raw = synth.weight(qtype, n, k, seed=11 * m + len(qtype))
    rng = np.random.default_rng(m)
    x = rng.standard_normal((m, k)).astype(np.float32)
    sub = x.reshape(m, -1, 32)
    if m <= 64:
        sub *= (10.0 ** rng.uniform(-3, 6, size=(m, sub.shape[1], 1))).astype(np.float32)
    else:
        f = np.ones((m, sub.shape[1], 1), np.float32)
        f[rng.random(f.shape) < 0.125] = 1e6
        f[:, 0] = 1e6  # every row has one
        sub *= f
    x = sub.reshape(m, k)
    assert np.abs(x).max() > 65504
    w = gpu_ctx.upload(QType[qtype.upper()], raw, n, k)
    y = gpu_ctx.empty((m, n), np.float32)
    gpu_ctx.matmul(w, gpu_ctx.to_device(x), m, y)
    got = y.numpy()
    assert np.all(np.isfinite(got))
    e = rel_err(got, oracle.matmul_q(qtype, x, raw, n))
    _say("rel err", e)
    assert e <= (1e-4 if m <= 64 or qtype != "iq4_xs" else TOL)


@pytest.mark.parametrize("qtype,m,n,k", [("q6_k", 33, 64, 4096), ("q8_0", 129, 300, 640),
                                         ("q6_k", 256, 136, 512)])
def test_gemm_f16_x_other_formats(gpu_ctx, oracle, qtype, m, n, k):
    _say("case: gemm f16 x", qtype, m, n, k)
    got, raw, x = _matmul(gpu_ctx, qtype, n, k, m, seed=5 * m + n, x_dtype=np.float16)
    e = rel_err(got, oracle.matmul_q(qtype, x.astype(np.float32), raw, n))
    _say("rel err", e)
    assert e <= TOL


@pytest.mark.parametrize("n,k,m", [(256, 8192, 8), (200, 5120, 130)])
def test_gemm_split_k_is_deterministic(gpu_ctx, n, k, m):
    # both shapes run split-K (the skinny kernel at m = 8, the prefill kernel's
    # split tail at m = 130); the ordered reduction gives the same bits twice
    from arf_amd import QType, synth
    raw = synth.weight("q4_k", n, k, seed=17)
    w = gpu_ctx.upload(QType.Q4_K, raw, n, k)
    x = gpu_ctx.to_device(synth.activations(m, k, seed=18))
    y1 = gpu_ctx.empty((m, n), np.float32)
    y2 = gpu_ctx.empty((m, n), np.float32)
    gpu_ctx.matmul(w, x, m, y1)
    gpu_ctx.matmul(w, x, m, y2)
    assert np.array_equal(y1.numpy().view(np.uint32), y2.numpy().view(np.uint32))


@pytest.mark.parametrize("m,n,k,xdt", [(1024, 16896, 1024, np.float16), (256, 66048, 512, np.float32),
                                        (512, 33280, 768, np.float16)])
def test_gemm_q4k_prefill_split_tail(gpu_ctx, oracle, m, n, k, xdt):
    # Q4_K prefill with more tiles than CUs and a remainder: the tiles past the
    # last whole round are cut into K ranges whose partials are added in order
    # (XCD tile order at m = 1024); every output is checked, and a repeat gives
    # the same bits.  The f32 case holds f16 values times 2^20 (the prefill
    # rounds f32 x to f16 after its per-row power-of-two scaling, which this x
    # survives exactly), so it checks the row scales on the split tiles
    _say("case: gemm q4k prefill split tail", m, n, k, xdt.__name__)
    from arf_amd import QType, synth
    raw = synth.weight("q4_k", n, k, seed=m + n)
    x = synth.activations(m, k, seed=k + 7).astype(np.float16).astype(xdt)
    if xdt == np.float32:
        x *= np.float32(2.0 ** 20)
    w = gpu_ctx.upload(QType.Q4_K, raw, n, k)
    xd = gpu_ctx.to_device(x)
    outs = []
    for _ in range(2):
        y = gpu_ctx.empty((m, n), np.float32)
        gpu_ctx.matmul(w, xd, m, y)
        outs.append(y.numpy())
    e = rel_err(outs[0], _dequant_matmul(oracle, "q4_k", x.astype(np.float32), raw, n))
    _say("rel err (all rows)", e)
    assert e <= TOL
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    rows = np.array([0, m // 2, m - 1])
    assert rel_err(outs[0][rows], oracle.matmul_q("q4_k", x[rows].astype(np.float32), raw, n)) <= TOL


def test_skinny_split_k_repeats(gpu_ctx, oracle):
    # skinny products split over K store their partials and a second launch adds
    # each output's splits in split order: interleaved shapes (split counts 16, 3
    # and 8; column counts a multiple of 4 and not) give the oracle's result, and
    # the same bits, on every repeat
    from arf_amd import QType, synth
    cases = [("q6_k", 512, 8192, 8), ("q6_k", 130, 1792, 16), ("q8_0", 1000, 4096, 24)]
    runs = []
    for qtype, n, k, m in cases:
        raw = synth.weight(qtype, n, k, seed=n + m)
        x = synth.activations(m, k, seed=k + m)
        runs.append((gpu_ctx.upload(QType[qtype.upper()], raw, n, k), gpu_ctx.to_device(x),
                     oracle.matmul_q(qtype, x, raw, n), None))
    for rep in range(3):
        for i, (qtype, n, k, m) in enumerate(cases):
            _say("case: skinny split repeat", rep, qtype, n, k, m)
            w, xd, want, first = runs[i]
            y = gpu_ctx.empty((m, n), np.float32)
            gpu_ctx.matmul(w, xd, m, y)
            got = y.numpy()
            assert rel_err(got, want) <= TOL
            if first is None:
                runs[i] = (w, xd, want, got)
            else:
                assert np.array_equal(got.view(np.uint32), first.view(np.uint32))


def _dequant_matmul(oracle, qtype, x, raw, n):
    """Every row of x . W^T from the oracle's bit-exact dequant and a float32 BLAS product:
    quantized linear == dequant + f32 matmul (weight.rs:1693-1709), pinned against the
    oracle's own matmuls by test_quantized_linear_equals_dequant_matmul."""
    k = x.shape[1]
    w = oracle.dequant(qtype, raw, n * k).reshape(n, k)
    return np.asarray(x, np.float32) @ w.T


@pytest.mark.parametrize("m", [8, 32, 64])
def test_c3_q6_k_batched_decode_full(gpu_ctx, oracle, m):
    # C3: Q6_K K=17408 N=5120 at decode batch m, every output checked
    _say("case: C3 full m =", m)
    n, k = 5120, 17408
    got, raw, x = _matmul(gpu_ctx, "q6_k", n, k, m, seed=0xA7F00003 + m)
    e = rel_err(got, _dequant_matmul(oracle, "q6_k", x, raw, n))
    _say("C3 rel err (all rows)", e)
    assert e <= TOL
    # spot rows against the oracle's own matmul_nt as well
    rows = np.array([0, m - 1])
    assert rel_err(got[rows], oracle.matmul_q("q6_k", x[rows], raw, n)) <= TOL


def test_c4_q4_k_gemm_full(gpu_ctx, oracle):
    # full C4 shape (2048 x 5120 f16 x, 17408 Q4_K rows), every output checked
    _say("case: C4 full")
    m, n, k = 2048, 17408, 5120
    got, raw, x = _matmul(gpu_ctx, "q4_k", n, k, m, seed=0xA7F00004, x_dtype=np.float16)
    assert np.all(np.isfinite(got))
    e = rel_err(got, _dequant_matmul(oracle, "q4_k", x.astype(np.float32), raw, n))
    _say("C4 rel err (all rows)", e)
    assert e <= TOL
    rows = np.r_[0:4, 2044:2048]
    assert rel_err(got[rows], oracle.matmul_q("q4_k", x[rows].astype(np.float32), raw, n)) <= TOL


@pytest.mark.parametrize("qtype", ["q5_k", "iq4_xs", "q6_k", "q8_0"])
def test_prefill_tile_full(gpu_ctx, oracle, qtype):
    # the rounded-weight prefill tile (m > 64) at 2048 f16 x rows: every output against the
    # oracle's exact dequant + BLAS; the tile holds each weight rounded once to f16
    # (2^-11), which the k-sums average down
    _say("case: prefill tile full", qtype)
    m, n, k = 2048, 640, 5120
    got, raw, x = _matmul(gpu_ctx, qtype, n, k, m, seed=0xA7F00010 + len(qtype), x_dtype=np.float16)
    assert np.all(np.isfinite(got))
    e = rel_err(got, _dequant_matmul(oracle, qtype, x.astype(np.float32), raw, n))
    _say("rel err (all rows)", e)
    assert e <= TOL
    rows = np.r_[0:2, 2046:2048]
    assert rel_err(got[rows], oracle.matmul_q(qtype, x[rows].astype(np.float32), raw, n)) <= TOL


@pytest.mark.parametrize("case", ["q6_k_full_range_scales", "q6_k", "q8_0"])
def test_prefill_exact_weights(gpu_ctx, oracle, case):
    # the prefill GEMM at 2048 f16 x rows multiplies exact weights: Q8_0's d * q as two f16
    # operands (hi + lo), Q6_K's sc * (q - 32) in units of d as one operand while every
    # |sc| <= 64 (the synthetic scales) and as hi + lo once the upload has seen a scale
    # beyond +-64 (here every scale drawn from all of i8, as quantizers produce them).
    # x is f16, so the only difference from the oracle's exact dequant + BLAS is the order
    # of the f32 sums: every output is held to 1e-4
    from arf_amd import QType, synth
    qtype = case[:4]
    _say("case: prefill exact weights", case)
    m, n, k = 2048, 640, 5120
    raw = synth.weight(qtype, n, k, seed=0xA7F00020 + len(case)).copy()
    if case.endswith("full_range_scales"):
        blk = raw.reshape(-1, 210)
        rng = np.random.default_rng(0xA7F00021)
        blk[:, 192:208] = rng.integers(-128, 128, size=(blk.shape[0], 16)).astype(np.int8).view(np.uint8)
    x = synth.activations(m, k, seed=0xA7F00022).astype(np.float16)
    w = gpu_ctx.upload(QType[qtype.upper()], raw, n, k)
    y = gpu_ctx.empty((m, n), np.float32)
    gpu_ctx.matmul(w, gpu_ctx.to_device(x), m, y)
    got = y.numpy()
    w.free()
    assert np.all(np.isfinite(got))
    e = rel_err(got, _dequant_matmul(oracle, qtype, x.astype(np.float32), raw, n))
    _say("rel err (all rows)", e)
    assert e <= 1e-4


# (bytes per block, offset of the f16 block scale d) of the direct-operand prefill formats,
# and their elements per block
_D_FIELD = {"q4_k": (144, 0), "q5_k": (176, 0), "q6_k": (210, 208), "q8_0": (34, 0), "iq4_xs": (136, 0)}
QK_OF = {"q4_k": 256, "q5_k": 256, "q6_k": 256, "q8_0": 32, "iq4_xs": 256}


@pytest.mark.parametrize("qtype", ["q4_k", "q5_k", "q6_k", "q8_0", "iq4_xs"])
def test_prefill_direct_operand_block_units(gpu_ctx, oracle, qtype):
    # the direct-operand prefill kernel with work items that run the whole K range (136
    # tiles of 128 x 512 rows: no split) over weight blocks whose d spans 2^-4 .. 2^2 of
    # the generator's, every 5th one dead (d = 0): the accumulators change unit at every
    # block, and the per-block (Q4_K, IQ4_XS, Q8_0) and per-group (Q6_K) scales must belong
    # to the block being multiplied.  Every output against BLAS on the weights the
    # operands hold, where only the f32 sums differ: the oracle's exact dequant for Q4_K,
    # Q5_K and Q8_0 (d * q as f16 hi + lo); for the formats whose operands are in units of
    # d and rounded to f16 past 2048, that dequant rounded the same way (Q6_K, IQ4_XS: the
    # dequant at d = 1, sc * (q - 32) and (ls - 32) * kv, rounded, times d; the synthetic
    # Q6_K scales keep sc * (q - 32) within 2048, so its rounding is none).
    from arf_amd import QType, synth
    m, n, k = 1024, 8704, 1024
    _say("case: direct-operand block units", qtype)
    rng = np.random.default_rng(0xB10C + len(qtype))
    raw = synth.weight(qtype, n, k, seed=0xB10D).copy()
    bb, off = _D_FIELD[qtype]
    blocks = raw.reshape(-1, bb)
    d = np.ascontiguousarray(blocks[:, off:off + 2]).view(np.float16).astype(np.float32).reshape(-1)
    d *= np.exp2(rng.integers(-4, 3, size=d.shape)).astype(np.float32)
    d[::5] = 0.0
    dh = d.astype(np.float16)
    blocks[:, off:off + 2] = dh.reshape(-1, 1).view(np.uint8)
    x = synth.activations(m, k, seed=0xB10E).astype(np.float16)
    if qtype in ("q4_k", "q5_k", "q8_0"):
        wref = oracle.dequant(qtype, raw, n * k).reshape(n, k)
    else:
        one = raw.copy()
        one.reshape(-1, bb)[:, off:off + 2] = np.full((1, 1), 1.0, np.float16).view(np.uint8)
        unit = oracle.dequant(qtype, one, n * k).reshape(-1, QK_OF[qtype])
        wref = (unit.astype(np.float16).astype(np.float32) * dh.astype(np.float32)[:, None]).reshape(n, k)
    w = gpu_ctx.upload(QType[qtype.upper()], raw, n, k)
    y = gpu_ctx.empty((m, n), np.float32)
    gpu_ctx.matmul(w, gpu_ctx.to_device(x), m, y)
    got = y.numpy()
    w.free()
    assert np.all(np.isfinite(got))
    e = rel_err(got, x.astype(np.float32) @ wref.T)
    _say("rel err against the operands' weights (all rows)", e)
    assert e <= 1e-4


# ------------------------------------------------------ edge cases ----
def _run(ctx, qtype, raw, x, n):
    from arf_amd import QType
    m, k = x.shape
    w = ctx.upload({"q4_k": QType.Q4_K, "q6_k": QType.Q6_K, "q8_0": QType.Q8_0}[qtype], raw, n, k)
    y = ctx.empty((m, n), np.float32)
    ctx.matmul(w, ctx.to_device(x), m, y)
    got = y.numpy()
    w.free()
    return got


def _dead_blocks(qtype, raw, every):
    """Zero the block scale d of every `every`-th block (dmin stays: the min term remains)."""
    raw = raw.copy()
    bb = {"q4_k": 144, "q6_k": 210}[qtype]
    off = {"q4_k": 0, "q6_k": 208}[qtype]
    blocks = raw.reshape(-1, bb)
    blocks[::every, off:off + 2] = 0
    return blocks.reshape(-1)


@pytest.mark.parametrize("qtype", ["q4_k", "q6_k"])
@pytest.mark.parametrize("m", [1, 2, 200])
def test_x_dynamic_range_and_dead_blocks(gpu_ctx, oracle, qtype, m):
    # x blocks of 32 scaled over 12 decades, some all zero; weight blocks with d = 0.
    # m = 1, 2 run the decode GEMVs (the f32 Q4_K GEMV scales x per sub-block, the
    # integer GEMVs quantize x per 32-element block); m = 200 runs the prefill path
    # (Q4_K: the direct-operand kernel with its d = 0 handling) on x scaled per row
    # into f16 range, with no clipping: the largest blocks are far beyond 65504.
    from arf_amd import synth
    n, k = 96, 2048
    _say("case: dynamic range / dead blocks", qtype, m)
    rng = np.random.default_rng(1234 + m)
    raw = _dead_blocks(qtype, synth.weight(qtype, n, k, seed=77 + m), every=3)
    x = synth.activations(m, k, seed=78 + m)
    scale = 10.0 ** rng.uniform(-6, 6, size=(m, k // 32)).astype(np.float32)
    scale[rng.random(size=scale.shape) < 0.1] = 0.0
    x = (x.reshape(m, k // 32, 32) * scale[..., None]).reshape(m, k).astype(np.float32)
    # the oracle sees x as given (at m = 200 the prefill kernel splits x into f16 hi + lo
    # after the row's power-of-two scale: blocks far below the row's largest lose their
    # low bits or fall out, and the gate measures what that costs against f32 x)
    got = _run(gpu_ctx, qtype, raw, x, n)
    want = oracle.matmul_q(qtype, x, raw, n)
    e = rel_err(got, want)
    _say("rel err", e)
    assert np.all(np.isfinite(got))
    assert e <= TOL


@pytest.mark.parametrize("qtype", ["q4_k", "q6_k"])
def test_zero_x_gives_zero(gpu_ctx, qtype):
    from arf_amd import synth
    n, k = 64, 1024
    raw = synth.weight(qtype, n, k, seed=5)
    for m in (1, 2, 8, 100):
        got = _run(gpu_ctx, qtype, raw, np.zeros((m, k), np.float32), n)
        assert np.array_equal(got, np.zeros_like(got)), (qtype, m)


@pytest.mark.parametrize("m", [16, 64])
def test_x16_option_skinny_one_part(gpu_ctx, oracle, m):
    # ARFQ_OPT_GEMV_X16 on the skinny kernel: an f32 x enters as one f16 part (11 bits);
    # within the matmul gate, and measurably different from the default's hi + lo
    import arf_amd
    _say("case: x16 skinny", m)
    gpu_ctx.set_options(arf_amd.arfq.OPT_GEMV_X16)
    try:
        got16, raw, x = _matmul(gpu_ctx, "q6_k", 256, 4096, m, seed=53)
    finally:
        gpu_ctx.set_options(0)
    got, _, _ = _matmul(gpu_ctx, "q6_k", 256, 4096, m, seed=53)
    want = oracle.matmul_q("q6_k", x, raw, 256)
    e16, e = rel_err(got16, want), rel_err(got, want)
    _say("rel err x16", e16, "default", e)
    assert e16 <= TOL and e <= SMALL_M_TOL and e16 > e


@pytest.mark.parametrize("qtype,n,k", [("q8_0", 16384, 4096), ("q6_k", 3000, 27648)])
def test_upload_in_staging_chunks_bit_exact(gpu_ctx, oracle, qtype, n, k):
    # host uploads pass through the context's staging buffer 64 MB of whole blocks at a
    # time: rows on both sides of each chunk boundary (and the first and last rows)
    # dequantize bit-exactly
    from arf_amd import QType, synth
    _say("case: chunked upload", qtype, n, k)
    raw = synth.weight(qtype, n, k, seed=611)
    bb, qk = synth.BLOCK_BYTES[qtype], synth.QK[qtype]
    assert raw.size > (64 << 20)
    w = gpu_ctx.upload(QType[qtype.upper()], raw, n, k)
    got = gpu_ctx.dequant(w).numpy().reshape(n, k)
    per = (64 << 20) // bb  # blocks per chunk
    bpr = k // qk           # blocks per row
    rows = {0, n - 1}
    for c in range(1, raw.size // bb // per + 1):
        r = c * per // bpr
        rows.update(range(max(0, r - 2), min(n, r + 3)))
    rb = raw.reshape(n, -1)
    for r in sorted(rows):
        want = oracle.dequant(qtype, rb[r], k)
        assert np.array_equal(got[r].view(np.uint32), want.view(np.uint32)), r
    w.free()
