"""ctypes view of the CPU restatement of Arf's reference arithmetic (liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, where it is the checker.  The product library
(arf_amd / libarfq.so) never imports or calls it.

Each wrapper names the reference function it restates; the C source
(oracle/arfq_oracle.c) cites the reference file:line for each.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_i8p = ctypes.POINTER(ctypes.c_int8)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i64 = ctypes.c_int64


def build():
    """Compile liboracle.so from oracle/arfq_oracle.c (always rebuilds)."""
    subprocess.run(["make", "-B", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.arfo_f16_to_f32.restype = ctypes.c_float
        L.arfo_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.arfo_q4k_get_scale_min.argtypes = [_u8p, ctypes.c_int, _u8p, _u8p]
        for name in ("arfo_dequant_q8_0", "arfo_dequant_q4_k", "arfo_dequant_q6_k",
                     "arfo_dequant_q5_k", "arfo_dequant_iq4_xs"):
            getattr(L, name).argtypes = [_u8p, _i64, _f32p]
        L.arfo_q4ks_from_ggml.argtypes = [_u8p, _i64, _i64, _u32p, _u8p, _i8p, _f32p, _f32p]
        L.arfo_q5ks_from_ggml.argtypes = [_u8p, _i64, _i64, _u32p, _u32p, _u8p, _i8p, _f32p,
                                          _f32p]
        L.arfo_q4ks_to_f32.argtypes = [_u32p, _u8p, _i8p, _f32p, _f32p, _i64, _i64, _f32p]
        L.arfo_matmul_nt.argtypes = [_f32p, _i64, _i64, _f32p, _i64, _f32p]
        for name in ("arfo_matmul_nt_q8_0", "arfo_matmul_nt_q4_k", "arfo_matmul_nt_q6_k",
                     "arfo_matmul_nt_q5_k", "arfo_matmul_nt_iq4_xs"):
            getattr(L, name).argtypes = [_f32p, _i64, _i64, _u8p, _i64, _f32p]
        L.arfo_matmul_nt_q4ks.argtypes = [_f32p, _i64, _i64, _u32p, _u8p, _i8p, _f32p, _f32p,
                                          _i64, _f32p]
        L.arfo_top_k_softmax.argtypes = [_f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                         _i32p, _f32p]
        L.arfo_moe_forward.argtypes = [_f32p, _i64, _i64, _i64, _u8p, _u8p, _u8p, ctypes.c_int,
                                       _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p]
        L.arfo_glu.argtypes = [_f32p, _f32p, _i64, ctypes.c_int, _f32p]
        L.arfo_set_threads.argtypes = [ctypes.c_int]
        L.arfo_threads.restype = ctypes.c_int
        _lib = L
    return _lib


def _p(a, t):
    return a.ctypes.data_as(t)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def set_threads(t):
    """Worker count for par_rows (0 = hardware concurrency, the reference's choice)."""
    lib().arfo_set_threads(int(t))


def threads():
    return lib().arfo_threads()


def f16_to_f32(h):
    """crates/arf-ml/src/dtype.rs:41-70"""
    return lib().arfo_f16_to_f32(int(h))


def q4k_get_scale_min(scales12, j):
    """crates/arf-ml/src/weight.rs:1353-1365"""
    s = _c(scales12, np.uint8)
    sc = ctypes.c_uint8()
    m = ctypes.c_uint8()
    lib().arfo_q4k_get_scale_min(_p(s, _u8p), int(j), ctypes.byref(sc), ctypes.byref(m))
    return sc.value, m.value


_BLOCK = {"q8_0": (32, 34), "q4_k": (256, 144), "q6_k": (256, 210), "q5_k": (256, 176),
          "iq4_xs": (256, 136)}


def dequant(qtype, blocks, n):
    """dequant_q8_0 / dequant_q4_k / dequant_q6_k / dequant_q5_k / dequant_iq4_xs
    (crates/arf-core/src/model/gguf.rs:1633-1649, 2004-2035, 2092-2131, 2053-2090, 1937-1976):
    raw ggml block bytes -> n f32 values."""
    qk, bb = _BLOCK[qtype]
    b = _c(blocks, np.uint8).reshape(-1)
    assert n % qk == 0 and b.size == n // qk * bb, "block byte count mismatch"
    out = np.empty(n, dtype=np.float32)
    getattr(lib(), "arfo_dequant_" + qtype)(_p(b, _u8p), n, _p(out, _f32p))
    return out


def q4ks_from_ggml(blocks, rows, cols):
    """Q4KSMatrix::from_ggml_q4k (crates/arf-ml/src/weight.rs:1000-1080)."""
    b = _c(blocks, np.uint8).reshape(-1)
    assert cols % 256 == 0 and b.size == rows * cols // 256 * 144
    codes = np.zeros(rows * cols // 8, np.uint32)
    scales = np.zeros(rows * cols // 32, np.uint8)
    mins = np.zeros(rows * cols // 32, np.int8)
    d = np.zeros(rows * cols // 256, np.float32)
    dmin = np.zeros(rows * cols // 256, np.float32)
    lib().arfo_q4ks_from_ggml(_p(b, _u8p), rows, cols, _p(codes, _u32p), _p(scales, _u8p),
                              _p(mins, _i8p), _p(d, _f32p), _p(dmin, _f32p))
    return codes, scales, mins, d, dmin


def q5ks_from_ggml(blocks, rows, cols):
    """Q5KSMatrix::from_ggml_q5k (crates/arf-ml/src/weight.rs:551-632)."""
    b = _c(blocks, np.uint8).reshape(-1)
    assert cols % 256 == 0 and b.size == rows * cols // 256 * 176
    lo = np.zeros(rows * cols // 8, np.uint32)
    hi = np.zeros(rows * cols // 32, np.uint32)
    scales = np.zeros(rows * cols // 32, np.uint8)
    mins = np.zeros(rows * cols // 32, np.int8)
    d = np.zeros(rows * cols // 256, np.float32)
    dmin = np.zeros(rows * cols // 256, np.float32)
    lib().arfo_q5ks_from_ggml(_p(b, _u8p), rows, cols, _p(lo, _u32p), _p(hi, _u32p),
                              _p(scales, _u8p), _p(mins, _i8p), _p(d, _f32p), _p(dmin, _f32p))
    return lo, hi, scales, mins, d, dmin


def q4ks_to_f32(q4ks, rows, cols):
    """Q4KSMatrix::to_f32 (crates/arf-ml/src/weight.rs:1110-1136)."""
    codes, scales, mins, d, dmin = q4ks
    out = np.empty(rows * cols, np.float32)
    lib().arfo_q4ks_to_f32(_p(codes, _u32p), _p(scales, _u8p), _p(mins, _i8p), _p(d, _f32p),
                           _p(dmin, _f32p), rows, cols, _p(out, _f32p))
    return out


def matmul_nt(a, b):
    """matmul_nt (crates/arf-ml/src/matmul.rs:84-99): a [m,k] x b[n,k]^T -> [m,n]."""
    a = _c(a, np.float32)
    b = _c(b, np.float32)
    m, k = a.shape
    n = b.shape[0]
    assert b.shape[1] == k
    out = np.empty((m, n), np.float32)
    lib().arfo_matmul_nt(_p(a, _f32p), m, k, _p(b, _f32p), n, _p(out, _f32p))
    return out


def matmul_q4ks(a, q4ks, n):
    """matmul_nt_q4ks (crates/arf-ml/src/matmul.rs:363-400) on an already transcoded
    weight (the reference transcodes at load time, weights.rs:478-500)."""
    a = _c(a, np.float32)
    if a.ndim == 1:
        a = a.reshape(1, -1)
    m, k = a.shape
    codes, scales, mins, d, dmin = q4ks
    out = np.empty((m, n), np.float32)
    lib().arfo_matmul_nt_q4ks(_p(a, _f32p), m, k, _p(codes, _u32p), _p(scales, _u8p),
                              _p(mins, _i8p), _p(d, _f32p), _p(dmin, _f32p), n, _p(out, _f32p))
    return out


def matmul_q(qtype, a, blocks, n):
    """The reference CPU matmul for a ggml-quantized weight [n, k]:
    q8_0 -> matmul_nt_q8_0 (matmul.rs:174-204); q4_k -> from_ggml_q4k + matmul_nt_q4ks
    (weight.rs:1000-1080, matmul.rs:322-400); q6_k / q5_k / iq4_xs -> dequant + matmul_nt."""
    a = _c(a, np.float32)
    if a.ndim == 1:
        a = a.reshape(1, -1)
    m, k = a.shape
    qk, bb = _BLOCK[qtype]
    b = _c(blocks, np.uint8).reshape(-1)
    assert k % qk == 0 and b.size == n * (k // qk) * bb, "block byte count mismatch"
    out = np.empty((m, n), np.float32)
    getattr(lib(), "arfo_matmul_nt_" + qtype)(_p(a, _f32p), m, k, _p(b, _u8p), n,
                                              _p(out, _f32p))
    return out


def top_k_softmax(logits, top_k, norm_topk):
    """crates/arf-core/src/model/moe.rs:89-121 for one row."""
    lg = _c(logits, np.float32).reshape(-1)
    k = min(top_k, lg.size)
    ids = np.zeros(k, np.int32)
    w = np.zeros(k, np.float32)
    lib().arfo_top_k_softmax(_p(lg, _f32p), lg.size, int(top_k), int(bool(norm_topk)),
                             _p(ids, _i32p), _p(w, _f32p))
    return ids, w


def glu(g, u, act):
    """h = act(g) * u elementwise: act 0 SwiGLU (mlp.rs:20-24), 1 GeGLU with the reference's
    inner clamp (decode_ops_msl.metal:15-27, selftest.rs:6091-6095)."""
    g = _c(g, np.float32).reshape(-1)
    u = _c(u, np.float32).reshape(-1)
    assert g.size == u.size
    out = np.empty(g.size, np.float32)
    lib().arfo_glu(_p(g, _f32p), _p(u, _f32p), g.size, int(act), _p(out, _f32p))
    return out


def moe_forward(x, gate, up, down, n_experts, inter, logits, top_k, norm_topk, init=None):
    """MoeMlp::forward with Q4_K SwiGLU experts (crates/arf-core/src/model/moe.rs:53-86,
    mlp.rs:20-24).  x [T, hidden] f32; gate/up: n_experts x [inter, hidden] Q4_K blocks;
    down: n_experts x [hidden, inter] Q4_K blocks; logits [T, n_experts].  init [T, hidden]:
    the shared experts' output, which the routed contributions are added to (moe.rs:62-67)."""
    x = _c(x, np.float32)
    T, hidden = x.shape
    lg = _c(logits, np.float32)
    assert lg.shape == (T, n_experts)
    g = _c(gate, np.uint8).reshape(-1)
    u = _c(up, np.uint8).reshape(-1)
    d = _c(down, np.uint8).reshape(-1)
    assert g.size == u.size == n_experts * inter * hidden // 256 * 144
    assert d.size == n_experts * hidden * inter // 256 * 144
    out = np.empty((T, hidden), np.float32) if init is None else np.array(init, np.float32, copy=True)
    assert out.shape == (T, hidden)
    lib().arfo_moe_forward(_p(x, _f32p), T, hidden, inter, _p(g, _u8p), _p(u, _u8p),
                           _p(d, _u8p), int(n_experts), _p(lg, _f32p), int(top_k),
                           int(bool(norm_topk)), int(init is not None), _p(out, _f32p))
    return out
