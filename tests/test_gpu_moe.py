"""GPU parity of the MoE path (routing, grouping, grouped SwiGLU GEMMs, combine)
against the CPU oracle, through the C ABI.

Routing: expert ids identical to the oracle's top_k_softmax (crates/arf-core/src/
model/moe.rs:89-121); weights within 1e-6 (only the exp's last bit may differ).
MoE block: max|g - c| / max(|c|, rms(c)) <= 2e-3 against MoeMlp::forward
(moe.rs:53-86) on the same f16-valued x.
"""
import sys

import numpy as np
import pytest

from conftest import rel_err
from formats import moe_dequant_reference, moe_route_lcg_logits

pytestmark = pytest.mark.gpu

TOL = 2e-3


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _route(ctx, logits, top_k, norm):
    T, E = logits.shape
    lg = ctx.to_device(logits)
    ids = ctx.empty((T, top_k), np.int32)
    w = ctx.empty((T, top_k), np.float32)
    ctx.moe_route(lg, T, E, top_k, norm, ids, w)
    return ids.numpy(), w.numpy()


def _check_route(oracle, logits, top_k, norm, got_ids, got_w):
    for t in range(logits.shape[0]):
        ids, w = oracle.top_k_softmax(logits[t], top_k, norm)
        assert got_ids[t].tolist() == ids.tolist(), f"token {t}"
        assert np.max(np.abs(got_w[t] - w)) <= 1e-6, f"token {t}"


# ------------------------------------------------------------- routing ----
def test_route_reference_cases(gpu_ctx, oracle):
    # crates/arf-core/src/model/moe.rs:134-159 (incl. the tie case -> lower index)
    _say("case: route reference cases")
    lg = np.array([[2.0, -1.0, 3.0, 0.0], [1.0, 1.0, 1.0, 1.0]], np.float32)
    for norm in (True, False):
        ids, w = _route(gpu_ctx, lg, 2, norm)
        assert ids[0].tolist() == [2, 0] and ids[1].tolist() == [0, 1]
        _check_route(oracle, lg, 2, norm, ids, w)
        if norm:
            assert abs(float(w[0].sum()) - 1.0) < 1e-6


def test_route_128_expert_lcg_cases(gpu_ctx, oracle):
    # crates/arf-gpu/tests/moe_gpu.rs:84-93: 128 experts, top-8, LCG seed 99
    _say("case: route 128-expert LCG")
    state = 99
    rows = []
    for _ in range(2):
        lg, state = moe_route_lcg_logits(128, state)
        rows.append(lg)
    lg = np.stack(rows)
    for norm in (True, False):
        ids, w = _route(gpu_ctx, lg, 8, norm)
        _check_route(oracle, lg, 8, norm, ids, w)


@pytest.mark.parametrize("T,E,k", [(512, 128, 8), (37, 8, 2), (5, 1000, 64), (3, 64, 1),
                                   (1, 200, 7)])
def test_route_random(gpu_ctx, oracle, T, E, k):
    from arf_amd import synth
    _say("case: route random", T, E, k)
    lg = synth.router_logits(T, E, seed=T * 1000 + E + k)
    ids, w = _route(gpu_ctx, lg, k, True)
    _check_route(oracle, lg, k, True, ids, w)


def test_route_shape_errors(gpu_ctx):
    lg = gpu_ctx.to_device(np.zeros((2, 8), np.float32))
    ids = gpu_ctx.empty((2, 9), np.int32)
    w = gpu_ctx.empty((2, 9), np.float32)
    with pytest.raises(ValueError):
        gpu_ctx.moe_route(lg, 2, 8, 9, True, ids, w)  # top_k > n_experts
    with pytest.raises(ValueError):
        gpu_ctx.moe_route(lg, 2, 8, 0, True, ids, w)


# ---------------------------------------------------------------- block ----
def _weights(ctx, E, hidden, inter, seed, qd="q4_k", qg="q4_k"):
    from arf_amd import QType, synth
    gate = synth.weight(qg, inter, hidden, seed=seed, experts=E)
    up = synth.weight(qg, inter, hidden, seed=seed + 1, experts=E)
    down = synth.weight(qd, hidden, inter, seed=seed + 2, experts=E)
    wg = ctx.upload(QType[qg.upper()], gate, inter, hidden, E)
    wu = ctx.upload(QType[qg.upper()], up, inter, hidden, E)
    wd = ctx.upload(QType[qd.upper()], down, hidden, inter, E)
    return (gate, up, down), (wg, wu, wd)


def _moe_gpu(ctx, ws, x, logits, top_k, norm):
    T, hidden = x.shape
    y = ctx.empty((T, hidden), np.float32)
    ctx.moe(ws[0], ws[1], ws[2], ctx.to_device(logits), T, top_k, norm, ctx.to_device(x), y)
    return y.numpy()


@pytest.mark.parametrize("T", [1, 4, 16])
def test_moe_decode_small_T_at_c5_experts(gpu_ctx, oracle, T):
    # the survey's next row (small-T MoE decode) on C5's expert shapes: 128 experts, top-8
    from arf_amd import synth
    E, k, hidden, inter = 128, 8, 2048, 768
    _say("case: moe decode T =", T)
    raw, ws = _weights(gpu_ctx, E, hidden, inter, seed=900 + T)
    x = synth.activations(T, hidden, seed=T + 17, dtype=np.float16)
    logits = synth.router_logits(T, E, seed=T + 18)
    got = _moe_gpu(gpu_ctx, ws, x, logits, k, True)
    want = oracle.moe_forward(x.astype(np.float32), raw[0], raw[1], raw[2], E, inter, logits, k,
                              True)
    e = rel_err(got, want)
    _say("rel err", e)
    assert e <= TOL


@pytest.mark.parametrize("T,E,k,hidden,inter", [(5, 8, 2, 256, 256), (70, 16, 4, 512, 768),
                                                (1, 4, 4, 256, 512), (129, 6, 2, 768, 256),
                                                (70, 16, 4, 512, 256), (70, 8, 4, 256, 1024)])
def test_moe_block_small(gpu_ctx, oracle, T, E, k, hidden, inter):
    # synthetic Q4_K experts give |silu(g) * u| up to ~1e5 at hidden >= 512: the
    # intermediate must not overflow f16 on the way to the down projection.  inter = 1024
    # is past the x-stationary down kernel's LDS (the tile x 128-column kernel runs)
    from arf_amd import synth
    _say("case: moe block", T, E, k, hidden, inter)
    raw, ws = _weights(gpu_ctx, E, hidden, inter, seed=T + E + k)
    x = synth.activations(T, hidden, seed=T + 7, dtype=np.float16)
    logits = synth.router_logits(T, E, seed=T + 8)
    got = _moe_gpu(gpu_ctx, ws, x, logits, k, True)
    want = oracle.moe_forward(x.astype(np.float32), raw[0], raw[1], raw[2], E, inter, logits, k,
                              True)
    e = rel_err(got, want)
    _say("rel err", e)
    assert e <= TOL


def test_moe_f32_x_and_no_renorm(gpu_ctx, oracle):
    # f32 x is rounded to f16 for the grouped GEMM tiles; the oracle sees the f32 x
    # itself (MoeMlp::forward's arithmetic), so the gate covers that rounding
    from arf_amd import synth
    _say("case: moe f32 x")
    T, E, k, hidden, inter = 33, 8, 3, 512, 256
    raw, ws = _weights(gpu_ctx, E, hidden, inter, seed=300)
    x = synth.activations(T, hidden, seed=301)
    logits = synth.router_logits(T, E, seed=302)
    got = _moe_gpu(gpu_ctx, ws, x, logits, k, False)
    want = oracle.moe_forward(x, raw[0], raw[1], raw[2], E, inter, logits, k, False)
    e = rel_err(got, want)
    _say("rel err", e)
    assert e <= TOL


@pytest.mark.parametrize("qg,qd", [("q4_k", "q6_k"), ("q5_k", "q5_k"), ("iq4_xs", "iq4_xs"),
                                   ("q5_k", "iq4_xs"), ("q8_0", "q8_0"), ("q6_k", "q4_k")])
def test_moe_expert_formats(gpu_ctx, oracle, qg, qd):
    # down projection in Q6_K (as Q4_K_M GGUFs ship ffn_down_exps), Q5_K / IQ4_XS / Q8_0
    # experts and Q6_K gate|up through the grouped GEMMs; composed from oracle parts on
    # the f32 intermediate (the GPU's down GEMM reads it rounded to f16: the gate covers
    # that)
    from arf_amd import synth
    _say("case: moe experts", qg, qd)
    T, E, k, hidden, inter = 9, 4, 2, 256, 512
    raw, ws = _weights(gpu_ctx, E, hidden, inter, seed=400, qd=qd, qg=qg)
    x = synth.activations(T, hidden, seed=401, dtype=np.float16)
    logits = synth.router_logits(T, E, seed=402)
    got = _moe_gpu(gpu_ctx, ws, x, logits, k, True)
    g_e = raw[0].reshape(E, -1)
    u_e = raw[1].reshape(E, -1)
    d_e = raw[2].reshape(E, -1)
    want = np.zeros((T, hidden), np.float32)
    xf = x.astype(np.float32)
    for t in range(T):
        ids, w = oracle.top_k_softmax(logits[t], k, True)
        for e, wt in zip(ids, w):
            g = oracle.matmul_q(qg, xf[t:t + 1], g_e[e], inter)
            u = oracle.matmul_q(qg, xf[t:t + 1], u_e[e], inter)
            with np.errstate(over="ignore"):  # exp(-g) = inf for g << 0: silu -> 0, as in f32
                h = ((g / (1.0 + np.exp(-g))) * u).astype(np.float32)
            want[t] += wt * oracle.matmul_q(qd, h, d_e[e], hidden)[0]
    e = rel_err(got, want)
    _say("rel err", e)
    assert e <= TOL


def test_moe_ids_matches_moe_and_drops_invalid(gpu_ctx, oracle):
    from arf_amd import synth
    _say("case: moe_ids")
    T, E, k, hidden, inter = 20, 8, 2, 256, 256
    raw, ws = _weights(gpu_ctx, E, hidden, inter, seed=500)
    x = synth.activations(T, hidden, seed=501, dtype=np.float16)
    logits = synth.router_logits(T, E, seed=502)
    ref = _moe_gpu(gpu_ctx, ws, x, logits, k, True)
    ids = np.zeros((T, k), np.int32)
    w = np.zeros((T, k), np.float32)
    for t in range(T):
        ids[t], w[t] = oracle.top_k_softmax(logits[t], k, True)
    y = gpu_ctx.empty((T, hidden), np.float32)
    gpu_ctx.moe_ids(ws[0], ws[1], ws[2], gpu_ctx.to_device(ids), gpu_ctx.to_device(w), T, k,
                    gpu_ctx.to_device(x), y)
    assert rel_err(y.numpy(), ref) <= 1e-6
    # an out-of-range id drops that (token, slot) pair; the others are unchanged
    bad = ids.copy()
    bad[3, 1] = E + 5
    bad[7, 0] = -1
    gpu_ctx.moe_ids(ws[0], ws[1], ws[2], gpu_ctx.to_device(bad), gpu_ctx.to_device(w), T, k,
                    gpu_ctx.to_device(x), y)
    got = y.numpy()
    keep = np.ones(T, bool)
    keep[[3, 7]] = False
    assert rel_err(got[keep], ref[keep]) <= 1e-6
    assert np.all(np.isfinite(got))
    # a dropped pair adds nothing: the same bits as a valid id with weight 0
    # (acc + 0 * o = acc), so tokens 3 and 7 hold their other slot alone
    fix, w0 = bad.copy(), w.copy()
    fix[3, 1], fix[7, 0] = 0, 0
    w0[3, 1], w0[7, 0] = 0.0, 0.0
    z = gpu_ctx.empty((T, hidden), np.float32)
    gpu_ctx.moe_ids(ws[0], ws[1], ws[2], gpu_ctx.to_device(fix), gpu_ctx.to_device(w0), T, k,
                    gpu_ctx.to_device(x), z)
    assert np.array_equal(got.view(np.uint32), z.numpy().view(np.uint32))
    # (T * k = 40 pairs: the decode path, whose down GEMV combines through counters)
    # the counters are left at zero: a repeat of the first call gives its bits
    gpu_ctx.moe_ids(ws[0], ws[1], ws[2], gpu_ctx.to_device(ids), gpu_ctx.to_device(w), T, k,
                    gpu_ctx.to_device(x), y)
    first = y.numpy().copy()
    gpu_ctx.moe_ids(ws[0], ws[1], ws[2], gpu_ctx.to_device(ids), gpu_ctx.to_device(w), T, k,
                    gpu_ctx.to_device(x), y)
    assert np.array_equal(first.view(np.uint32), y.numpy().view(np.uint32))


def test_moe_deterministic(gpu_ctx):
    from arf_amd import synth
    T, E, k, hidden, inter = 300, 16, 4, 256, 256
    _, ws = _weights(gpu_ctx, E, hidden, inter, seed=600)
    x = synth.activations(T, hidden, seed=601, dtype=np.float16)
    logits = synth.router_logits(T, E, seed=602)
    a = _moe_gpu(gpu_ctx, ws, x, logits, k, True)
    b = _moe_gpu(gpu_ctx, ws, x, logits, k, True)
    assert np.all(np.isfinite(a))
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_moe_shape_errors(gpu_ctx):
    from arf_amd import QType, synth
    _, ws = _weights(gpu_ctx, 4, 256, 256, seed=700)
    x = gpu_ctx.to_device(np.zeros((2, 256), np.float16))
    lg = gpu_ctx.to_device(np.zeros((2, 4), np.float32))
    y = gpu_ctx.empty((2, 256), np.float32)
    with pytest.raises(ValueError):
        gpu_ctx.moe(ws[0], ws[1], ws[2], lg, 2, 5, True, x, y)  # top_k > experts
    down_bad = gpu_ctx.upload(QType.Q4_K, synth.weight("q4_k", 512, 256, seed=1, experts=4),
                              512, 256, 4)
    with pytest.raises(ValueError):
        gpu_ctx.moe(ws[0], ws[1], down_bad, lg, 2, 2, True, x, y)


def test_c5_moe_full(gpu_ctx, oracle):
    # C5: 128 experts, top-8, T=512, hidden 2048, inter 768; every token checked
    from arf_amd import synth
    _say("case: C5 full")
    cfg = synth.CONFIGS["c5_moe"]
    T, E, k, hidden, inter = cfg["tokens"], cfg["experts"], cfg["top_k"], cfg["hidden"], cfg["inter"]
    raw, ws = _weights(gpu_ctx, E, hidden, inter, seed=0xA7F00005)
    x = synth.activations(T, hidden, seed=0xA7F00008, dtype=np.float16)
    logits = synth.router_logits(T, E, seed=0xA7F00009)
    got = _moe_gpu(gpu_ctx, ws, x, logits, k, True)
    assert np.all(np.isfinite(got))
    want = moe_dequant_reference(oracle, x, raw, E, hidden, inter, logits, k, True)
    e = rel_err(got, want)
    _say("C5 rel err (all 512 tokens)", e)
    assert e <= TOL
    # and a few tokens against the oracle's own MoeMlp::forward
    rows = np.r_[0:2, 510:512]
    assert rel_err(got[rows], oracle.moe_forward(x[rows].astype(np.float32), raw[0], raw[1], raw[2],
                                                 E, inter, logits[rows], k, True)) <= TOL


# ------------------------------------------------------------------- FFN ----
def _ffn_oracle(oracle, x, raws, qts, inter, hidden):
    g = oracle.matmul_q(qts[0], x, raws[0], inter)
    u = oracle.matmul_q(qts[1], x, raws[1], inter)
    with np.errstate(over="ignore"):  # exp(-g) overflows to inf for g << 0: silu -> 0, as in f32
        h = (g / (np.float32(1.0) + np.exp(-g)) * u).astype(np.float32)
    return oracle.matmul_q(qts[2], h, raws[2], hidden), g


@pytest.mark.parametrize("qts,hidden,inter,m,xscale", [
    (("q4_k", "q4_k", "q4_k"), 512, 768, 1, 1.0), (("q4_k", "q4_k", "q4_k"), 512, 768, 3, 1.0),
    (("q4_k", "q4_k", "q4_k"), 512, 768, 8, 1.0), (("q4_k", "q4_k", "q6_k"), 1024, 512, 1, 1.0),
    (("q8_0", "q8_0", "q5_k"), 768, 256, 2, 1.0), (("q4_k", "q4_k", "q4_k"), 5120, 17408, 1, 1.0),
    # m = 8 at C2's shape: gate/up on the skinny MFMA kernel, h = silu(g) * u far above f16's
    # range into the down GEMM's f32 x (row-scaled into f16 range)
    (("q4_k", "q4_k", "q4_k"), 5120, 17408, 8, 1.0),
    # x scaled down so that most g fall in [-10, 10], where silu is neither 0 nor the identity
    (("q4_k", "q4_k", "q4_k"), 512, 768, 1, 0.02), (("q4_k", "q4_k", "q6_k"), 512, 768, 8, 0.02),
    (("q5_k", "q5_k", "iq4_xs"), 1024, 512, 5, 0.02)])
def test_ffn_matches_mlp_forward(gpu_ctx, oracle, qts, hidden, inter, m, xscale):
    # ffn_dispatch / Mlp::forward (island.rs:13436-13529, mlp.rs:20-24): the fused SwiGLU-into-
    # down GEMV (Q4_K down, m <= 4) and the SwiGLU kernel + matmul path
    from arf_amd import QType, synth
    _say("case: ffn", qts, hidden, inter, m, xscale)
    shapes = [(inter, hidden), (inter, hidden), (hidden, inter)]
    raws = [synth.weight(q, n, k, seed=31 + i) for i, (q, (n, k)) in enumerate(zip(qts, shapes))]
    ws = [gpu_ctx.upload(QType[q.upper()], r, n, k) for q, r, (n, k) in zip(qts, raws, shapes)]
    x = (synth.activations(m, hidden, seed=37) * np.float32(xscale)).astype(np.float32)
    y = gpu_ctx.empty((m, hidden), np.float32)
    gpu_ctx.ffn(ws[0], ws[1], ws[2], gpu_ctx.to_device(x), m, y)
    want, g = _ffn_oracle(oracle, x, raws, qts, inter, hidden)
    got = y.numpy()
    assert np.all(np.isfinite(got))
    e = rel_err(got, want)
    _say("rel err", e, "share of g in [-10, 10]", float(np.mean(np.abs(g) <= 10)))
    if xscale < 1:
        assert np.mean(np.abs(g) <= 10) > 0.5
    assert e <= TOL


def test_ffn_shape_errors(gpu_ctx):
    from arf_amd import QType, synth
    g = gpu_ctx.upload(QType.Q4_K, synth.weight("q4_k", 256, 512, seed=1), 256, 512)
    d = gpu_ctx.upload(QType.Q4_K, synth.weight("q4_k", 256, 512, seed=2), 256, 512)  # not [512, 256]
    x = gpu_ctx.to_device(np.zeros((1, 512), np.float32))
    y = gpu_ctx.empty((1, 512), np.float32)
    with pytest.raises(ValueError):
        gpu_ctx.ffn(g, g, d, x, 1, y)


# ------------------------------------------------------------ GeGLU FFN ----
def _glu_oracle(oracle, x, raws, qts, inter, hidden, act):
    g = oracle.matmul_q(qts[0], x, raws[0], inter)
    u = oracle.matmul_q(qts[1], x, raws[1], inter)
    h = oracle.glu(g, u, act).reshape(g.shape)
    return oracle.matmul_q(qts[2], h, raws[2], hidden), g


@pytest.mark.parametrize("qts,hidden,inter,m,xscale,x16", [
    # m = 1, Q4_K: gate and up in one launch, GeGLU applied as the down GEMV reads its x
    (("q4_k", "q4_k", "q4_k"), 512, 768, 1, 0.02, False),
    (("q4_k", "q4_k", "q4_k"), 5120, 17408, 1, 0.005, False),
    # inter 28672: the activation as a launch of its own, the down GEMV's x in four rounds
    (("q4_k", "q4_k", "q4_k"), 512, 28672, 1, 0.02, False),
    # the 16-bit-x GEMV option (gate and up as two launches)
    (("q4_k", "q4_k", "q4_k"), 512, 768, 1, 0.02, True),
    # m = 3: the integer-dot GEMV with GeGLU fused; m = 8: skinny GEMMs + the GeGLU kernel
    (("q4_k", "q4_k", "q4_k"), 512, 768, 3, 0.02, False),
    (("q4_k", "q4_k", "q6_k"), 512, 768, 8, 0.02, False),
    (("q4_k", "q4_k", "q6_k"), 1024, 512, 1, 0.02, False)])
def test_ffn_geglu_matches_reference(gpu_ctx, oracle, qts, hidden, inter, m, xscale, x16):
    # ffn_dispatch's gate GEMV, up GEMV, geglu, down GEMV (island.rs:13436-13529,
    # decode_ops_msl.metal:15-27); x scaled so that most g fall where gelu is curved
    import arf_amd.arfq as A
    from arf_amd import QType, synth
    _say("case: ffn geglu", qts, hidden, inter, m, xscale, x16)
    shapes = [(inter, hidden), (inter, hidden), (hidden, inter)]
    raws = [synth.weight(q, n, k, seed=61 + i) for i, (q, (n, k)) in enumerate(zip(qts, shapes))]
    ws = [gpu_ctx.upload(QType[q.upper()], r, n, k) for q, r, (n, k) in zip(qts, raws, shapes)]
    x = (synth.activations(m, hidden, seed=67) * np.float32(xscale)).astype(np.float32)
    y = gpu_ctx.empty((m, hidden), np.float32)
    gpu_ctx.set_options(A.OPT_GEMV_X16 if x16 else 0)
    try:
        gpu_ctx.ffn(ws[0], ws[1], ws[2], gpu_ctx.to_device(x), m, y, act=A.ACT_GELU_TANH)
    finally:
        gpu_ctx.set_options(0)
    want, g = _glu_oracle(oracle, x, raws, qts, inter, hidden, 1)
    got = y.numpy()
    assert np.all(np.isfinite(got))
    e = rel_err(got, want)
    _say("rel err", e, "share of g in [-6, 6]", float(np.mean(np.abs(g) <= 6)))
    assert np.mean(np.abs(g) <= 6) > 0.5
    assert e <= TOL
    # the same weights through SwiGLU differ (the activation is not cosmetic)
    y2 = gpu_ctx.empty((m, hidden), np.float32)
    gpu_ctx.ffn(ws[0], ws[1], ws[2], gpu_ctx.to_device(x), m, y2, act=A.ACT_SILU)
    assert rel_err(y2.numpy(), want) > 10 * TOL


def _q80_identity(n):
    """Q8_0 blocks of the n x n identity: d = 1.0, one code 1 per row."""
    nb = n // 32
    blk = np.zeros((n, nb, 34), np.uint8)
    blk[:, :, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    r = np.arange(n)
    blk[r, r // 32, 2 + r % 32] = 1
    return blk.reshape(-1)


@pytest.mark.parametrize("act", [0, 1])
@pytest.mark.parametrize("m", [1, 2])
def test_ffn_activation_exact_through_identity(gpu_ctx, oracle, act, m):
    # gate = up = down = the identity in Q8_0, whose f32 GEMV adds exactly one nonzero term
    # per output: y = act(x) * x elementwise, so the GPU's activation is compared with the
    # oracle's directly (to the last bits of exp / tanh), over the selftest's inputs
    # (selftest.rs:6049-6052) including the clamp region and |x| >= 7
    from arf_amd import QType
    n = 256
    raw = _q80_identity(n)
    w = gpu_ctx.upload(QType.Q8_0, raw, n, n)
    i = np.arange(m * n)
    x = (((i % 29) - 14) * 0.3).astype(np.float32).reshape(m, n)
    x[0, :6] = [7.0, -7.0, 20.0, -20.0, 0.0, 1.0]
    y = gpu_ctx.empty((m, n), np.float32)
    gpu_ctx.ffn(w, w, w, gpu_ctx.to_device(x), m, y, act=act)
    got = y.numpy().reshape(-1).astype(np.float64)
    want = oracle.glu(x, x, act).astype(np.float64)
    # a few ulps of exp / tanh apart; for GeGLU at g < -3 the tanh's rounding is magnified
    # by 1 + tanh(inner) ~ 0 (2^-21 of 0.5 |g u| bounds it)
    xx = x.reshape(-1).astype(np.float64)
    bound = 2e-6 * np.abs(want) + (2.0 ** -21 * 0.5 * xx * xx if act else 0.0) + 1e-30
    _say("max err / bound", float(np.max(np.abs(got - want) / bound)))
    assert np.all(np.abs(got - want) <= bound)


# ---------------------------------------------------- MoE shared expert ----
@pytest.mark.parametrize("T,E,k", [(2, 16, 4), (40, 16, 4)])
def test_moe_add_onto_shared_expert(gpu_ctx, oracle, T, E, k):
    # MoeMlp::forward with a shared expert (moe.rs:62-67): y = shared Mlp (arfq_ffn), then
    # the routed block added on top (arfq_moe_add), on the decode path (8 pairs) and the
    # grouped path (160 pairs); arfq_moe_add onto zeros gives arfq_moe's bits
    from arf_amd import QType, synth
    hidden, inter = 512, 256
    _say("case: moe add", T, E, k)
    raw, ws = _weights(gpu_ctx, E, hidden, inter, seed=500 + T)
    sh_raw = [synth.weight("q4_k", inter, hidden, seed=510), synth.weight("q4_k", inter, hidden, seed=511),
              synth.weight("q4_k", hidden, inter, seed=512)]
    sh = [gpu_ctx.upload(QType.Q4_K, sh_raw[0], inter, hidden), gpu_ctx.upload(QType.Q4_K, sh_raw[1], inter, hidden),
          gpu_ctx.upload(QType.Q4_K, sh_raw[2], hidden, inter)]
    x = (synth.activations(T, hidden, seed=T + 520) * np.float32(0.05)).astype(np.float16)
    xf = x.astype(np.float32)
    logits = synth.router_logits(T, E, seed=T + 521)
    xd, lg = gpu_ctx.to_device(xf), gpu_ctx.to_device(logits)
    y = gpu_ctx.empty((T, hidden), np.float32)
    gpu_ctx.ffn(sh[0], sh[1], sh[2], xd, T, y)
    s_gpu = y.numpy()
    gpu_ctx.moe(ws[0], ws[1], ws[2], lg, T, k, True, gpu_ctx.to_device(x), y, accumulate=True)
    got = y.numpy()
    s_want, _ = _ffn_oracle(oracle, xf, sh_raw, ("q4_k",) * 3, inter, hidden)
    assert rel_err(s_gpu, s_want) <= TOL
    want = oracle.moe_forward(xf, raw[0], raw[1], raw[2], E, inter, logits, k, True, init=s_want)
    e = rel_err(got, want)
    _say("rel err", e)
    assert e <= TOL
    # accumulate onto zeros == overwrite
    z = gpu_ctx.to_device(np.zeros((T, hidden), np.float32))
    gpu_ctx.moe(ws[0], ws[1], ws[2], lg, T, k, True, gpu_ctx.to_device(x), z, accumulate=True)
    plain = _moe_gpu(gpu_ctx, ws, x, logits, k, True)
    assert np.array_equal(z.numpy().view(np.uint32), plain.view(np.uint32))
