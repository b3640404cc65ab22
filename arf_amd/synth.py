"""Seeded synthetic GGUF weights and activations for the benchmark configs.

Block contents follow the generation rules the benchmark is quoted on:
  Q8_0  d = f16(|N(0,1)| * 0.002), 32 i8 codes uniform in [-127, 127]
  Q4_K  d, dmin = f16(|N(0,1)| * 0.01), 12 scale bytes and 128 qs bytes uniform
  Q6_K  ql[128], qh[64] uniform bytes, 16 i8 scales uniform in [-32, 31],
        d = f16(|N(0,1)| * 0.005)
f16 rounding is IEEE round-to-nearest-even with subnormals kept (numpy).
Everything is drawn from numpy's PCG64 seeded per call, so the CPU oracle and
the GPU read the same bytes.
"""
import numpy as np

BLOCK_BYTES = {"q8_0": 34, "q4_k": 144, "q6_k": 210}
QK = {"q8_0": 32, "q4_k": 256, "q6_k": 256}


def _f16_bytes(v):
    return np.asarray(v, np.float16).view(np.uint8).reshape(-1, 2)


def q8_0_blocks(rng, nblk):
    out = np.empty((nblk, 34), np.uint8)
    out[:, 0:2] = _f16_bytes(np.abs(rng.standard_normal(nblk)) * 0.002)
    out[:, 2:34] = rng.integers(-127, 128, size=(nblk, 32), dtype=np.int16).astype(np.int8).view(np.uint8)
    return out


def q4_k_blocks(rng, nblk):
    out = np.empty((nblk, 144), np.uint8)
    out[:, 0:2] = _f16_bytes(np.abs(rng.standard_normal(nblk)) * 0.01)
    out[:, 2:4] = _f16_bytes(np.abs(rng.standard_normal(nblk)) * 0.01)
    out[:, 4:144] = rng.integers(0, 256, size=(nblk, 140), dtype=np.uint8)
    return out


def q6_k_blocks(rng, nblk):
    out = np.empty((nblk, 210), np.uint8)
    out[:, 0:192] = rng.integers(0, 256, size=(nblk, 192), dtype=np.uint8)
    out[:, 192:208] = rng.integers(-32, 32, size=(nblk, 16), dtype=np.int16).astype(np.int8).view(np.uint8)
    out[:, 208:210] = _f16_bytes(np.abs(rng.standard_normal(nblk)) * 0.005)
    return out


_GEN = {"q8_0": q8_0_blocks, "q4_k": q4_k_blocks, "q6_k": q6_k_blocks}


def weight(qtype, n, k, seed, experts=1):
    """Raw ggml blocks for `experts` stacked [n, k] matrices, flat uint8."""
    qtype = qtype.lower()
    assert k % QK[qtype] == 0
    rng = np.random.default_rng(seed)
    nblk = experts * n * (k // QK[qtype])
    return _GEN[qtype](rng, nblk).reshape(-1)


def activations(m, k, seed, dtype=np.float32):
    rng = np.random.default_rng(seed)
    return rng.standard_normal((m, k), dtype=np.float32).astype(dtype)


def router_logits(tokens, n_experts, seed):
    rng = np.random.default_rng(seed)
    return rng.standard_normal((tokens, n_experts), dtype=np.float32)


# The benchmark configurations (name -> description used by bench.py and tests)
CONFIGS = {
    "c1_q8_0_gemv": dict(qtype="q8_0", m=1, k=2048, n=2048),
    "c2_q4_k_gemv": dict(qtype="q4_k", m=1, k=5120, n=17408),
    "c3_q6_k_gemv": dict(qtype="q6_k", m=(1, 8, 32, 64), k=17408, n=5120),
    "c4_q4_k_gemm": dict(qtype="q4_k", m=2048, k=5120, n=17408),
    "c5_moe": dict(qtype="q4_k", experts=128, top_k=8, tokens=512, hidden=2048, inter=768),
}
