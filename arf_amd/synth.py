"""Seeded synthetic GGUF weights and activations for the benchmark configs.

Block contents follow the generation rules the benchmark is quoted on:
  Q8_0  d = f16(|N(0,1)| * 0.002), 32 i8 codes uniform in [-127, 127]
  Q4_K  d, dmin = f16(|N(0,1)| * 0.01), 12 scale bytes and 128 qs bytes uniform
  Q6_K  ql[128], qh[64] uniform bytes, 16 i8 scales uniform in [-32, 31],
        d = f16(|N(0,1)| * 0.005)
  Q5_K  as Q4_K, plus 32 uniform bytes of 5th bits (no benchmark config; the
        survey's next row)
  IQ4_XS d = f16(|N(0,1)| * 0.0005), scale and code bytes uniform (likewise)
f16 rounding is IEEE round-to-nearest-even with subnormals kept (numpy).
Everything is drawn from numpy's PCG64 seeded per call, so the CPU oracle and
the GPU read the same bytes.  gguf_write() lays such tensors out as a GGUF v3
model file.
"""
import struct

import numpy as np

BLOCK_BYTES = {"q8_0": 34, "q4_k": 144, "q6_k": 210, "q5_k": 176, "iq4_xs": 136}
QK = {"q8_0": 32, "q4_k": 256, "q6_k": 256, "q5_k": 256, "iq4_xs": 256}


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


def q5_k_blocks(rng, nblk):
    """Q5_K as Q4_K (d, dmin, scale bytes) plus 32 uniform bytes of 5th bits."""
    out = np.empty((nblk, 176), np.uint8)
    out[:, 0:2] = _f16_bytes(np.abs(rng.standard_normal(nblk)) * 0.01)
    out[:, 2:4] = _f16_bytes(np.abs(rng.standard_normal(nblk)) * 0.01)
    out[:, 4:176] = rng.integers(0, 256, size=(nblk, 172), dtype=np.uint8)
    return out


def iq4_xs_blocks(rng, nblk):
    """IQ4_XS: d = f16(|N(0,1)| * 0.0005), scale and code bytes uniform."""
    out = np.empty((nblk, 136), np.uint8)
    out[:, 0:2] = _f16_bytes(np.abs(rng.standard_normal(nblk)) * 0.0005)
    out[:, 2:136] = rng.integers(0, 256, size=(nblk, 134), dtype=np.uint8)
    return out


_GEN = {"q8_0": q8_0_blocks, "q4_k": q4_k_blocks, "q6_k": q6_k_blocks, "q5_k": q5_k_blocks,
        "iq4_xs": iq4_xs_blocks}


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


# ---- synthetic GGUF v3 files ------------------------------------------------------
# Value types: 0 u8, 1 i8, 2 u16, 3 i16, 4 u32, 5 i32, 6 f32, 7 bool, 8 string,
# 9 array (element type, values), 10 u64, 11 i64, 12 f64
# (crates/arf-core/src/model/gguf.rs:323-360).
_GGUF_FMT = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q",
             11: "<q", 12: "<d"}


def _gguf_string(s):
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _gguf_value(vty, v):
    if vty in _GGUF_FMT:
        return struct.pack(_GGUF_FMT[vty], v)
    if vty == 8:
        return _gguf_string(v)
    if vty == 9:
        ety, items = v
        return struct.pack("<IQ", ety, len(items)) + b"".join(_gguf_value(ety, x) for x in items)
    raise ValueError(f"GGUF value type {vty}")


def gguf_kv(key, vty, value):
    """One key/value record."""
    return _gguf_string(key) + struct.pack("<I", vty) + _gguf_value(vty, value)


def gguf_header(kvs, tensors, alignment=32, version=3, magic=b"GGUF", raw_kv=None):
    """Header, key/values and tensor table of a GGUF file, padded to the alignment.
    kvs: [(key, vty, value)]; tensors: [(name, ggml dims, ggml type id, byte length)].
    Returns (header bytes, [absolute data offset of each tensor]); each tensor's data
    starts at an aligned offset, as ggml's writer places it."""
    head = magic + struct.pack("<IQQ", version, len(tensors), len(kvs) + (1 if raw_kv else 0))
    head += b"".join(gguf_kv(*x) for x in kvs) + (raw_kv or b"")
    table, offs, off = b"", [], 0
    for name, dims, ty, nbytes in tensors:
        off = -(-off // alignment) * alignment
        offs.append(off)
        table += _gguf_string(name) + struct.pack("<I", len(dims))
        table += b"".join(struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", ty, off)
        off += nbytes
    body = head + table
    data_start = -(-len(body) // alignment) * alignment
    return body + b"\0" * (data_start - len(body)), [data_start + o for o in offs]


def gguf_bytes(kvs, tensors, alignment=32, **kw):
    """A whole GGUF file image; tensors: [(name, ggml dims, ggml type id, data bytes)].
    Returns (file bytes, [absolute data offset of each tensor])."""
    head, offs = gguf_header(kvs, [(n, d, t, len(b)) for n, d, t, b in tensors], alignment, **kw)
    out = bytearray(head)
    for (_, _, _, data), o in zip(tensors, offs):
        out += b"\0" * (o - len(out)) + data
    return bytes(out), offs


def gguf_write(path, kvs, tensors, alignment=32):
    """Write a GGUF file; tensors: [(name, ggml dims, ggml type id, byte length, fill)] where
    fill(f) writes exactly that many bytes to the open file (large tensors stream to disk).
    Returns the absolute data offset of each tensor."""
    head, offs = gguf_header(kvs, [t[:4] for t in tensors], alignment)
    with open(path, "wb") as f:
        f.write(head)
        for (_, _, _, nbytes, fill), o in zip(tensors, offs):
            f.write(b"\0" * (o - f.tell()))
            fill(f)
            if f.tell() != o + nbytes:
                raise ValueError("gguf_write: fill wrote the wrong byte count")
    return offs
