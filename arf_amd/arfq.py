"""Python host side of the arfq C ABI (include/arfq.h), through ctypes.

Mirrors the shape of Arf's GPU matmul interface so a caller written against
`add_matmul_m(m, a, weight, out, n, kdim)` (crates/arf-gpu/src/gpu/dispatch.rs:
191-202) and `GpuMatWeight` (crates/arf-gpu/src/gpu/types.rs:15-61) finds the
same names and argument meaning:

    ctx = Context(0)                       # GpuContext::new
    w = ctx.upload(QType.Q4_K, blocks, n, k)   # GpuMatWeight upload
    a = ctx.to_device(x)                   # activation buffer
    out = ctx.empty((m, n), np.float32)
    add_matmul_m(ctx, m, a, w, out, n, k)  # records the matmul on the stream
    y = out.numpy()                        # readback (synchronises)

There is no CPU fallback: if libarfq.so is missing or no GPU is present the
calls raise.  Shape mismatches raise ValueError where the reference panics
(crates/arf-ml/src/matmul.rs:180-183,374-386).
"""
import ctypes
import enum
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libarfq.so")

ARFQ_OK = 0
ARFQ_E_INVALID = -1
ARFQ_E_SHAPE = -2
ARFQ_E_DEVICE = -3
ARFQ_E_NOMEM = -4
ARFQ_E_UNSUPPORTED = -5
ARFQ_E_FORMAT = -6
ARFQ_E_IO = -7
ARFQ_E_NOT_FOUND = -8

# context options (include/arfq.h ARFQ_OPT_*)
OPT_GEMV_X16 = 1
# arfq_act: the FFN's gate activation (GateAct)
ACT_SILU = 0
ACT_GELU_TANH = 1


class QType(enum.IntEnum):
    """ggml type ids (crates/arf-core/src/model/gguf.rs:36-90)."""
    Q8_0 = 8
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14
    IQ4_XS = 23


class DType(enum.IntEnum):
    F32 = 0
    F16 = 1


# (weights per block, bytes per block): crates/arf-core/src/model/gguf.rs:1657-1673
BLOCK = {QType.Q8_0: (32, 34), QType.Q4_K: (256, 144), QType.Q6_K: (256, 210),
         QType.Q5_K: (256, 176), QType.IQ4_XS: (256, 136)}

# the C ABI, by name -> (restype, argtypes); tests check every name is exported
_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_SIGS = {
    "arfq_version": (_int, []),
    "arfq_status_string": (ctypes.c_char_p, [_int]),
    "arfq_ctx_create": (_int, [_int, _vp, ctypes.POINTER(_vp)]),
    "arfq_ctx_destroy": (_int, [_vp]),
    "arfq_ctx_stream": (_vp, [_vp]),
    "arfq_last_error": (ctypes.c_char_p, [_vp]),
    "arfq_ctx_sync": (_int, [_vp]),
    "arfq_ctx_set_options": (_int, [_vp, ctypes.c_uint]),
    "arfq_weight_upload": (_int, [_vp, _int, _vp, ctypes.c_size_t, _i64, _i64, _int,
                                  ctypes.POINTER(_vp)]),
    "arfq_weight_upload_device": (_int, [_vp, _int, _vp, ctypes.c_size_t, _i64, _i64, _int,
                                         ctypes.POINTER(_vp)]),
    "arfq_weight_free": (_int, [_vp]),
    "arfq_weight_info": (_int, [_vp, ctypes.POINTER(_int), ctypes.POINTER(_i64),
                                ctypes.POINTER(_i64), ctypes.POINTER(_int),
                                ctypes.POINTER(ctypes.c_size_t)]),
    "arfq_matmul": (_int, [_vp, _vp, _int, _i64, _vp, _int, _vp]),
    "arfq_matmul_noalloc": (_int, [_vp, _vp, _int, _i64, _vp, _int, _vp]),
    "arfq_dequant_f32": (_int, [_vp, _vp, _vp]),
    "arfq_moe_route": (_int, [_vp, _vp, _i64, _int, _int, _int, _vp, _vp]),
    "arfq_moe": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _int, _int, _vp, _int, _vp]),
    "arfq_moe_ids": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _int, _vp, _int, _vp]),
    "arfq_moe_add": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _int, _int, _vp, _int, _vp]),
    "arfq_moe_ids_add": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _int, _vp, _int, _vp]),
    "arfq_dev_malloc": (_int, [_vp, ctypes.c_size_t, ctypes.POINTER(_vp)]),
    "arfq_dev_free": (_int, [_vp, _vp]),
    "arfq_copy_h2d": (_int, [_vp, _vp, _vp, ctypes.c_size_t]),
    "arfq_copy_d2h": (_int, [_vp, _vp, _vp, ctypes.c_size_t]),
    "arfq_copy_d2d": (_int, [_vp, _vp, _vp, ctypes.c_size_t]),
    "arfq_stream_read": (_int, [_vp, _vp, ctypes.c_size_t, _vp, _int]),
    "arfq_ctx_device_info": (_int, [_vp, ctypes.POINTER(_int), ctypes.POINTER(_int), ctypes.POINTER(_int)]),
    "arfq_ctx_memory": (_int, [_vp, ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t),
                               ctypes.POINTER(ctypes.c_size_t)]),
    "arfq_timer_start": (_int, [_vp]),
    "arfq_timer_stop": (_int, [_vp, ctypes.POINTER(ctypes.c_float)]),
    "arfq_matmul_repeat": (_int, [_vp, ctypes.POINTER(_vp), _int, _int, _i64, _vp, _int, _vp]),
    "arfq_ffn": (_int, [_vp, _vp, _vp, _vp, _i64, _vp, _vp]),
    "arfq_ffn_act": (_int, [_vp, _vp, _vp, _vp, _i64, _vp, _vp, _int]),
    "arfq_gguf_is_gguf": (_int, [ctypes.c_char_p]),
    "arfq_gguf_open": (_int, [ctypes.c_char_p, ctypes.POINTER(_vp)]),
    "arfq_gguf_close": (_int, [_vp]),
    "arfq_gguf_last_error": (ctypes.c_char_p, [_vp]),
    "arfq_gguf_tensor_count": (_int, [_vp, ctypes.POINTER(_i64)]),
    "arfq_gguf_tensor_info": (_int, [_vp, _i64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_int),
                                     ctypes.POINTER(_int), ctypes.POINTER(_i64), _int,
                                     ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)]),
    "arfq_gguf_find": (_int, [_vp, ctypes.c_char_p, ctypes.POINTER(_i64)]),
    "arfq_gguf_blocks": (_int, [_vp, ctypes.c_char_p, _int, ctypes.POINTER(_vp),
                                ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(_i64),
                                ctypes.POINTER(_i64)]),
    "arfq_gguf_upload": (_int, [_vp, _vp, ctypes.c_char_p, _i64, _i64, ctypes.POINTER(_vp)]),
}

_lib = None


def load_library(path=LIB_PATH):
    """Load libarfq.so.  Raises if it has not been built: there is no fallback."""
    global _lib
    if _lib is None:
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is missing: build it with `python -m arf_amd.build`")
        L = ctypes.CDLL(path)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def exported_symbols():
    return sorted(_SIGS)


class ArfqError(RuntimeError):
    def __init__(self, status, msg):
        super().__init__(f"arfq error {status}: {msg}")
        self.status = status


def _check(ctx_handle, status):
    if status != ARFQ_OK:
        L = load_library()
        msg = L.arfq_last_error(ctx_handle)
        msg = msg.decode() if msg else L.arfq_status_string(status).decode()
        if status == ARFQ_E_SHAPE:
            raise ValueError(msg)
        raise ArfqError(status, msg)


class DeviceArray:
    """A device allocation with a numpy-like shape/dtype (the buffer the
    reference binds as a wgpu BindingResource)."""

    def __init__(self, ctx, shape, dtype):
        self.ctx = ctx
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = ctypes.c_void_p()
        _check(ctx.handle, load_library().arfq_dev_malloc(ctx.handle, self.nbytes, ctypes.byref(p)))
        self.ptr = p.value

    def upload(self, host):
        host = np.ascontiguousarray(host, dtype=self.dtype)
        if host.nbytes != self.nbytes:
            raise ValueError(f"upload: {host.nbytes} bytes into a {self.nbytes}-byte buffer")
        _check(self.ctx.handle,
               load_library().arfq_copy_h2d(self.ctx.handle, self.ptr, host.ctypes.data, host.nbytes))
        return self

    def numpy(self):
        out = np.empty(self.shape, self.dtype)
        _check(self.ctx.handle,
               load_library().arfq_copy_d2h(self.ctx.handle, out.ctypes.data, self.ptr, self.nbytes))
        return out

    def free(self):
        if self.ptr:
            load_library().arfq_dev_free(self.ctx.handle, self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            if self.ptr and self.ctx.handle:
                self.free()
        except Exception:
            pass


class Weight:
    """An uploaded GGUF weight: n_experts x [n rows, k cols] (GpuMatWeight /
    PackedExperts, crates/arf-gpu/src/gpu/types.rs:15-61,89-112)."""

    def __init__(self, ctx, handle, qtype, n, k, experts):
        self.ctx, self.handle = ctx, handle
        self.qtype, self.n, self.k, self.experts = QType(qtype), n, k, experts

    @property
    def bytes_num(self):
        """Bytes one full matmul over one expert streams (types.rs:69-82)."""
        sz = ctypes.c_size_t()
        _check(self.ctx.handle, load_library().arfq_weight_info(self.handle, None, None, None,
                                                                None, ctypes.byref(sz)))
        return sz.value

    def free(self):
        if self.handle:
            load_library().arfq_weight_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Context:
    """One HIP device + one stream (GpuContext + CommandPass)."""

    def __init__(self, device=0):
        L = load_library()
        h = ctypes.c_void_p()
        st = L.arfq_ctx_create(int(device), None, ctypes.byref(h))
        if st != ARFQ_OK:
            raise ArfqError(st, (L.arfq_last_error(None) or b"").decode())
        self.handle = h.value
        self.device = device

    def close(self):
        if self.handle:
            load_library().arfq_ctx_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    # -- memory --
    def empty(self, shape, dtype):
        return DeviceArray(self, shape, dtype)

    def to_device(self, host, dtype=None):
        host = np.asarray(host)
        return DeviceArray(self, host.shape, dtype or host.dtype).upload(host)

    def sync(self):
        _check(self.handle, load_library().arfq_ctx_sync(self.handle))

    def set_options(self, options):
        """ARFQ_OPT_* bits (OPT_GEMV_X16: 16-bit fixed-point x in the m = 1 Q4_K GEMV)."""
        _check(self.handle, load_library().arfq_ctx_set_options(self.handle, int(options)))

    # -- weights --
    def upload(self, qtype, blocks, n_rows, k_cols, n_experts=1):
        qtype = QType(qtype)
        b = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1)
        h = ctypes.c_void_p()
        _check(self.handle, load_library().arfq_weight_upload(
            self.handle, int(qtype), b.ctypes.data, b.nbytes, int(n_rows), int(k_cols),
            int(n_experts), ctypes.byref(h)))
        return Weight(self, h.value, qtype, int(n_rows), int(k_cols), int(n_experts))

    def upload_gguf(self, gguf, name, row0=0, n_rows=-1):
        """Upload GGUF tensor `name`: a 2-D matrix (or its rows [row0, row0 + n_rows)) or a
        3-D `*_exps` tensor as n_experts experts (arfq_gguf_upload)."""
        L = load_library()
        h = ctypes.c_void_p()
        st = L.arfq_gguf_upload(self.handle, gguf.handle, name.encode(), int(row0), int(n_rows),
                                ctypes.byref(h))
        if st != ARFQ_OK:
            msg = (L.arfq_gguf_last_error(gguf.handle) or b"").decode()
            if not msg or st in (ARFQ_E_DEVICE, ARFQ_E_NOMEM):
                msg = (L.arfq_last_error(self.handle) or b"").decode() or msg
            raise (ValueError(msg) if st == ARFQ_E_SHAPE else ArfqError(st, msg))
        qt, n, k, e = _weight_shape(h.value)
        return Weight(self, h.value, QType(qt), n, k, e)

    # -- compute --
    def matmul(self, w, x, m, y, expert=0):
        """y[m, w.n] = x[m, w.k] . W_expert^T  (x: DeviceArray f32/f16, y: DeviceArray f32)."""
        xd = {np.dtype(np.float32): DType.F32, np.dtype(np.float16): DType.F16}.get(x.dtype)
        if xd is None:
            raise ValueError(f"matmul: x dtype {x.dtype} (want f32 or f16)")
        if x.nbytes < m * w.k * x.dtype.itemsize:
            raise ValueError("matmul: a shape")
        if y.dtype != np.float32 or y.nbytes < m * w.n * 4:
            raise ValueError("matmul: out shape")
        _check(self.handle, load_library().arfq_matmul(self.handle, w.handle, int(expert), int(m),
                                                       x.ptr, int(xd), y.ptr))

    def dequant(self, w):
        out = self.empty((w.experts * w.n * w.k,), np.float32)
        _check(self.handle, load_library().arfq_dequant_f32(self.handle, w.handle, out.ptr))
        return out

    def moe_route(self, logits, tokens, n_experts, top_k, norm_topk, ids, weights):
        _check(self.handle, load_library().arfq_moe_route(
            self.handle, logits.ptr, int(tokens), int(n_experts), int(top_k), int(bool(norm_topk)),
            ids.ptr, weights.ptr))

    def ffn(self, gate, up, down, x, m, y, act=None):
        """y[m, hidden] = down . (act(gate . x) * (up . x)) (ffn_dispatch / Mlp::forward);
        act ACT_SILU (default: arfq_ffn) or ACT_GELU_TANH (arfq_ffn_act)."""
        L = load_library()
        if act is None:
            _check(self.handle, L.arfq_ffn(self.handle, gate.handle, up.handle, down.handle, int(m), x.ptr,
                                           y.ptr))
        else:
            _check(self.handle, L.arfq_ffn_act(self.handle, gate.handle, up.handle, down.handle, int(m),
                                               x.ptr, y.ptr, int(act)))

    def moe(self, gate, up, down, logits, tokens, top_k, norm_topk, x, y, accumulate=False):
        """MoE block into y (accumulate: added to y, which holds the shared experts' output)."""
        xd = DType.F16 if x.dtype == np.float16 else DType.F32
        fn = load_library().arfq_moe_add if accumulate else load_library().arfq_moe
        _check(self.handle, fn(self.handle, gate.handle, up.handle, down.handle, logits.ptr, int(tokens),
                               int(top_k), int(bool(norm_topk)), x.ptr, int(xd), y.ptr))

    def moe_ids(self, gate, up, down, ids, weights, tokens, top_k, x, y, accumulate=False):
        xd = DType.F16 if x.dtype == np.float16 else DType.F32
        fn = load_library().arfq_moe_ids_add if accumulate else load_library().arfq_moe_ids
        _check(self.handle, fn(self.handle, gate.handle, up.handle, down.handle, ids.ptr, weights.ptr,
                               int(tokens), int(top_k), x.ptr, int(xd), y.ptr))

    def copy_d2d(self, dst, src, nbytes=None):
        """Enqueue dst <- src (device arrays) on the context's stream."""
        nb = src.nbytes if nbytes is None else int(nbytes)
        if nb > dst.nbytes or nb > src.nbytes:
            raise ValueError("copy_d2d: size")
        _check(self.handle, load_library().arfq_copy_d2d(self.handle, dst.ptr, src.ptr, nb))

    def stream_read(self, src, nbytes=None, stamps=None):
        """Enqueue one read-only pass over nbytes of src (arfq_stream_read); `stamps`
        (a uint64 device array of 4 * g entries) receives workgroup g's
        (realtime, clock) at start and end for the first g workgroups."""
        nb = src.nbytes if nbytes is None else int(nbytes)
        if nb > src.nbytes:
            raise ValueError("stream_read: size")
        ns = 0 if stamps is None else stamps.nbytes // 32
        _check(self.handle, load_library().arfq_stream_read(
            self.handle, src.ptr, nb, None if stamps is None else stamps.ptr, ns))

    def device_info(self):
        """(compute units, peak shader clock kHz, s_memrealtime frequency kHz)."""
        cus, sclk, wclk = _int(), _int(), _int()
        _check(self.handle, load_library().arfq_ctx_device_info(
            self.handle, ctypes.byref(cus), ctypes.byref(sclk), ctypes.byref(wclk)))
        return cus.value, sclk.value, wclk.value

    def memory(self):
        """(context scratch bytes, device free bytes, device total bytes)."""
        sb, fr, tot = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_size_t()
        _check(self.handle, load_library().arfq_ctx_memory(
            self.handle, ctypes.byref(sb), ctypes.byref(fr), ctypes.byref(tot)))
        return sb.value, fr.value, tot.value

    # -- timing --
    def timer_start(self):
        _check(self.handle, load_library().arfq_timer_start(self.handle))

    def timer_stop(self):
        ms = ctypes.c_float()
        _check(self.handle, load_library().arfq_timer_stop(self.handle, ctypes.byref(ms)))
        return ms.value

    def matmul_repeat(self, ws, iters, m, x, y):
        arr = (ctypes.c_void_p * len(ws))(*[w.handle for w in ws])
        xd = DType.F16 if x.dtype == np.float16 else DType.F32
        _check(self.handle, load_library().arfq_matmul_repeat(
            self.handle, arr, len(ws), int(iters), int(m), x.ptr, int(xd), y.ptr))


def _weight_shape(handle):
    L = load_library()
    qt, n, k, e = _int(), _i64(), _i64(), _int()
    _check(None, L.arfq_weight_info(handle, ctypes.byref(qt), ctypes.byref(n), ctypes.byref(k),
                                    ctypes.byref(e), None))
    return qt.value, n.value, k.value, e.value


class GgufTensor:
    """One tensor table entry: ggml dims fastest-varying first, type id, absolute byte offset,
    ggml_byte_len bytes (TensorDesc, crates/arf-core/src/model/gguf.rs:92-100)."""

    def __init__(self, name, ggml_type, dims, offset, nbytes):
        self.name, self.ggml_type, self.dims = name, ggml_type, tuple(dims)
        self.offset, self.nbytes = offset, nbytes

    def __repr__(self):
        return f"GgufTensor({self.name!r}, type={self.ggml_type}, dims={self.dims}, offset={self.offset})"


class Gguf:
    """A GGUF v3 file opened read-only and memory-mapped by the library (LazyGguf::open_raw,
    crates/arf-core/src/model/gguf.rs:509-564).  Raises ArfqError on a malformed file."""

    def __init__(self, path):
        L = load_library()
        h = ctypes.c_void_p()
        st = L.arfq_gguf_open(os.fsencode(path), ctypes.byref(h))
        if st != ARFQ_OK:
            raise ArfqError(st, (L.arfq_gguf_last_error(None) or b"").decode())
        self.handle = h.value
        n = _i64()
        L.arfq_gguf_tensor_count(self.handle, ctypes.byref(n))
        self.tensors = []
        for i in range(n.value):
            name, ty, nd = ctypes.c_char_p(), _int(), _int()
            dims = (_i64 * 8)()
            off, nb = ctypes.c_uint64(), ctypes.c_uint64()
            self._check(L.arfq_gguf_tensor_info(self.handle, i, ctypes.byref(name), ctypes.byref(ty),
                                                ctypes.byref(nd), dims, 8, ctypes.byref(off),
                                                ctypes.byref(nb)))
            self.tensors.append(GgufTensor(name.value.decode(), ty.value, dims[:min(nd.value, 8)],
                                           off.value, nb.value))

    @staticmethod
    def is_gguf(path):
        """is_gguf_file (gguf.rs:1115-1125): a regular file starting with the magic."""
        return bool(load_library().arfq_gguf_is_gguf(os.fsencode(path)))

    def _check(self, st):
        if st != ARFQ_OK:
            L = load_library()
            raise ArfqError(st, (L.arfq_gguf_last_error(self.handle) or b"").decode())

    def tensor_names(self):
        return [t.name for t in self.tensors]

    def find(self, name):
        i = _i64()
        self._check(load_library().arfq_gguf_find(self.handle, name.encode(), ctypes.byref(i)))
        return self.tensors[i.value]

    def blocks(self, name, ggml_type):
        """(bytes, rows, cols) of a tensor stored as `ggml_type` (get_q4k_blocks_raw /
        get_q8_0_blocks_raw, gguf.rs:774-828); None when it is stored as another type."""
        L = load_library()
        p, nb, r, c = ctypes.c_void_p(), ctypes.c_size_t(), _i64(), _i64()
        st = L.arfq_gguf_blocks(self.handle, name.encode(), int(ggml_type), ctypes.byref(p),
                                ctypes.byref(nb), ctypes.byref(r), ctypes.byref(c))
        if st == ARFQ_E_UNSUPPORTED:
            return None
        self._check(st)
        buf = (ctypes.c_uint8 * nb.value).from_address(p.value) if nb.value else b""
        return np.frombuffer(buf, np.uint8).copy(), r.value, c.value

    def close(self):
        if self.handle:
            load_library().arfq_gguf_close(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def add_matmul_m(ctx, m, a, weight, out, n, kdim, expert=0):
    """`add_matmul_m(cp, k, uni, m, a, weight, out, n, kdim, cache)` of
    crates/arf-gpu/src/gpu/dispatch.rs:191-202 with the wgpu recording state
    folded into `ctx`: records out[m, n] = a[m, kdim] . weight^T on the stream.
    The kernel is chosen by (weight kind, m) inside the library."""
    if weight.n != n or weight.k != kdim:
        raise ValueError(f"add_matmul_m: weight is [{weight.n}, {weight.k}], asked [{n}, {kdim}]")
    ctx.matmul(weight, a, m, out, expert)


def add_matmul(ctx, a, weight, out, n, kdim):
    """m = 1 wrapper (dispatch.rs:169-181)."""
    add_matmul_m(ctx, 1, a, weight, out, n, kdim)
