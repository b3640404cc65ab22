"""Golden vectors (tests/golden/fixtures.npz, written by tests/golden/make_fixtures.py).

CPU: the oracle still reproduces every fixture bit for bit, and the fixtures hold
the reference's known answers (gguf.rs:2522-2538 -> 19.0 / -5.0,
gguf.rs:2564-2575 -> -44.0, the sign-fold and high-scale gate values of
gguf.rs:2862-2982, the route ties of moe.rs:134-159).
GPU: the HIP path through the C ABI against the same fixtures: dequant bit-exact,
route ids identical and weights within 1e-6, matmul and MoE within the 2e-3 gate.
"""
import os

import numpy as np
import pytest

from conftest import rel_err

FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "fixtures.npz")
TOL = 2e-3

_QT = {"q4k": "q4_k", "q80": "q8_0", "q6k": "q6_k", "q4k_f16": "q4_k"}


@pytest.fixture(scope="module")
def fx():
    with np.load(FIX, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def _dequant_cases(fx):
    out = [("q4_k", fx["dq_q4k_known_raw"], fx["dq_q4k_known_y"], (1, 256))]
    for name in ("known", "signfold", "lcg_a", "lcg_b", "highj"):
        r, c = fx[f"dq_q4k_gate_{name}_shape"].tolist()
        out.append(("q4_k", fx[f"dq_q4k_gate_{name}_raw"], fx[f"dq_q4k_gate_{name}_y"], (r, c)))
    out.append(("q6_k", fx["dq_q6k_known_raw"], fx["dq_q6k_known_y"], (1, 256)))
    q = fx["dq_q6k_quads_raw"]
    out.append(("q6_k", q, fx["dq_q6k_quads_y"], (q.size // 210, 256)))
    q = fx["dq_q80_closed_raw"]
    out.append(("q8_0", q, fx["dq_q80_closed_y"], (q.size // 34 // 8, 256)))
    return out


# ------------------------------------------------------------------ CPU ----
def test_fixtures_hold_reference_known_answers(fx):
    assert fx["dq_q4k_known_y"][0] == 19.0 and fx["dq_q4k_known_y"][1] == -5.0
    assert fx["dq_q4k_gate_known_y"][0] == 19.0
    assert fx["dq_q4k_gate_signfold_y"][32] == np.float32(10.0 * 7 - 31.5)
    assert fx["dq_q4k_gate_highj_y"][128] == np.float32(0.25 * 51 * 15 - 0.125 * 26)
    assert fx["dq_q6k_known_y"][0] == -44.0
    w = fx["route_lcg128_norm1_w"]
    assert np.all(np.abs(w.sum(axis=1) - 1.0) < 1e-6)


def test_oracle_reproduces_dequant_fixtures(fx, oracle):
    for qtype, raw, y, (r, c) in _dequant_cases(fx):
        got = oracle.dequant(qtype, raw, r * c)
        assert np.array_equal(got.view(np.uint32), y.view(np.uint32)), qtype


def test_oracle_reproduces_matmul_fixtures(fx, oracle):
    for name, qt in _QT.items():
        x, raw, y = fx[f"mm_{name}_x"], fx[f"mm_{name}_raw"], fx[f"mm_{name}_y"]
        got = oracle.matmul_q(qt, x.astype(np.float32), raw, y.shape[1])
        assert np.array_equal(got.view(np.uint32), y.view(np.uint32)), name


def test_oracle_reproduces_route_and_moe_fixtures(fx, oracle):
    lg = fx["route_lcg128_logits"]
    for norm in (0, 1):
        for t in range(lg.shape[0]):
            ids, w = oracle.top_k_softmax(lg[t], 8, bool(norm))
            assert ids.tolist() == fx[f"route_lcg128_norm{norm}_ids"][t].tolist()
            assert np.array_equal(w.astype(np.float32), fx[f"route_lcg128_norm{norm}_w"][t])
    T, E, k, hidden, inter = fx["moe_small_dims"].tolist()
    got = oracle.moe_forward(fx["moe_small_x"].astype(np.float32), fx["moe_small_gate"],
                             fx["moe_small_up"], fx["moe_small_down"], E, inter,
                             fx["moe_small_logits"], k, True)
    assert np.array_equal(got.view(np.uint32), fx["moe_small_y"].view(np.uint32))


# ------------------------------------------------------------------ GPU ----
@pytest.mark.gpu
def test_gpu_dequant_matches_fixtures(fx, gpu_ctx):
    from arf_amd import QType
    qt = {"q4_k": QType.Q4_K, "q6_k": QType.Q6_K, "q8_0": QType.Q8_0}
    for qtype, raw, y, (r, c) in _dequant_cases(fx):
        print("case: golden dequant", qtype, r, c, flush=True)
        w = gpu_ctx.upload(qt[qtype], raw, r, c)
        got = gpu_ctx.dequant(w).numpy()
        w.free()
        assert np.array_equal(got.view(np.uint32), y.view(np.uint32)), qtype


@pytest.mark.gpu
def test_gpu_matmul_matches_fixtures(fx, gpu_ctx):
    from arf_amd import QType
    qt = {"q4_k": QType.Q4_K, "q6_k": QType.Q6_K, "q8_0": QType.Q8_0}
    for name, qtn in _QT.items():
        x, raw, y = fx[f"mm_{name}_x"], fx[f"mm_{name}_raw"], fx[f"mm_{name}_y"]
        m, n = y.shape
        print("case: golden matmul", name, m, n, x.shape[1], flush=True)
        w = gpu_ctx.upload(qt[qtn], raw, n, x.shape[1])
        xd = gpu_ctx.to_device(x)
        yd = gpu_ctx.empty((m, n), np.float32)
        gpu_ctx.matmul(w, xd, m, yd)
        got = yd.numpy()
        w.free()
        assert rel_err(got, y) <= TOL, name


@pytest.mark.gpu
def test_gpu_route_matches_fixtures(fx, gpu_ctx):
    print("case: golden route", flush=True)
    lg = fx["route_lcg128_logits"]
    T, E = lg.shape
    for norm in (0, 1):
        ids = gpu_ctx.empty((T, 8), np.int32)
        w = gpu_ctx.empty((T, 8), np.float32)
        gpu_ctx.moe_route(gpu_ctx.to_device(lg), T, E, 8, bool(norm), ids, w)
        assert np.array_equal(ids.numpy(), fx[f"route_lcg128_norm{norm}_ids"])
        assert np.max(np.abs(w.numpy() - fx[f"route_lcg128_norm{norm}_w"])) <= 1e-6


@pytest.mark.gpu
def test_gpu_moe_matches_fixture(fx, gpu_ctx):
    from arf_amd import QType
    print("case: golden moe", flush=True)
    T, E, k, hidden, inter = fx["moe_small_dims"].tolist()
    g = gpu_ctx.upload(QType.Q4_K, fx["moe_small_gate"], inter, hidden, E)
    u = gpu_ctx.upload(QType.Q4_K, fx["moe_small_up"], inter, hidden, E)
    d = gpu_ctx.upload(QType.Q4_K, fx["moe_small_down"], hidden, inter, E)
    y = gpu_ctx.empty((T, hidden), np.float32)
    gpu_ctx.moe(g, u, d, gpu_ctx.to_device(fx["moe_small_logits"]), T, k, True,
                gpu_ctx.to_device(fx["moe_small_x"]), y)
    got = y.numpy()
    for wt in (g, u, d):
        wt.free()
    assert rel_err(got, fx["moe_small_y"]) <= TOL
