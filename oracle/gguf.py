"""Pure-Python restatement of Arf's GGUF v3 table reader, the checker for the
library's C++ reader (arfq_gguf_open and friends).

TEST INFRASTRUCTURE ONLY: imported by tests/, never by arf_amd/.

Follows crates/arf-core/src/model/gguf.rs:
- LazyGguf::open_raw (:509-564): magic "GGUF", version 3, u64 tensor and
  key/value counts; key/value pairs (u64-length string key, u32 value type,
  value) where only general.alignment (u32, default 32) is kept; the tensor
  table (string name, u32 n_dims, u64 dims fastest-varying first, u32 ggml type,
  u64 offset); data_start = header end rounded up to the alignment.
- Reader::skip_value (:323-360): the value-type sizes 0/1/7 -> 1, 2/3 -> 2,
  4/5/6 -> 4, 10/11/12 -> 8, 8 = u64-length string, 9 = u32 element type +
  u64 count + elements.
- GgmlType::from_id (:60-90) for the accepted type ids and ggml_block_bytes /
  ggml_byte_len (:1657-1705) for the byte length of a tensor.
- get_q4k_blocks_raw / get_q8_0_blocks_raw (:774-828): rows = elements / ne0,
  cols = ne0.
"""
import struct

# ggml type id -> (elements per block, bytes per block); gguf.rs:60-90,1657-1673
TYPE_GEOM = {0: (1, 4), 1: (1, 2), 30: (1, 2), 2: (32, 18), 3: (32, 20), 8: (32, 34),
             20: (32, 18), 12: (256, 144), 13: (256, 176), 14: (256, 210), 11: (256, 110),
             21: (256, 110), 23: (256, 136)}
_FIXED = {0: 1, 1: 1, 7: 1, 2: 2, 3: 2, 4: 4, 5: 4, 6: 4, 10: 8, 11: 8, 12: 8}


class GgufError(ValueError):
    pass


def byte_len(ggml_type, n):
    """ggml_byte_len (gguf.rs:1678-1705)."""
    qk, nb = TYPE_GEOM[ggml_type]
    return (n // qk) * nb


class _Reader:
    def __init__(self, buf):
        self.buf, self.pos = buf, 0

    def take(self, n):
        if n < 0 or self.pos + n > len(self.buf):
            raise GgufError("GGUF truncated")
        s = self.buf[self.pos:self.pos + n]
        self.pos += n
        return s

    def u32(self):
        return struct.unpack("<I", self.take(4))[0]

    def u64(self):
        return struct.unpack("<Q", self.take(8))[0]

    def string(self):
        return self.take(self.u64()).decode("utf-8", "replace")

    def skip_value(self, vty):
        if vty in _FIXED:
            self.take(_FIXED[vty])
        elif vty == 8:
            self.take(self.u64())
        elif vty == 9:
            ety = self.u32()
            n = self.u64()
            for _ in range(n):
                self.skip_value(ety)
        else:
            raise GgufError(f"unknown GGUF value type {vty}")


def parse(buf):
    """Parse a GGUF file image: returns (alignment, data_start, tensors) with tensors a list of
    dicts name, dims, type, offset (relative to data_start), nbytes."""
    r = _Reader(buf)
    if r.take(4) != b"GGUF":
        raise GgufError("not a GGUF file (bad magic)")
    version = r.u32()
    if version != 3:
        raise GgufError(f"GGUF version {version} unsupported (only v3)")
    n_tensors, n_kv = r.u64(), r.u64()
    alignment = 32
    for _ in range(n_kv):
        key = r.string()
        vty = r.u32()
        if key == "general.alignment":
            alignment = r.u32()
        else:
            r.skip_value(vty)
    tensors = []
    for _ in range(n_tensors):
        name = r.string()
        n_dims = r.u32()
        dims = [r.u64() for _ in range(n_dims)]
        ty = r.u32()
        if ty not in TYPE_GEOM:
            raise GgufError(f"unsupported ggml tensor type {ty}")
        offset = r.u64()
        n = 1
        for d in dims:
            n *= d
        tensors.append({"name": name, "dims": dims, "type": ty, "offset": offset,
                        "nbytes": byte_len(ty, n)})
    data_start = -(-r.pos // alignment) * alignment
    return alignment, data_start, tensors


def blocks(buf, name, ggml_type):
    """(bytes, rows, cols) of a tensor stored as ggml_type, else None (gguf.rs:774-828)."""
    _, data_start, tensors = parse(buf)
    for t in tensors:
        if t["name"] == name:
            if t["type"] != ggml_type:
                return None
            n = 1
            for d in t["dims"]:
                n *= d
            cols = t["dims"][0] if t["dims"] else 1
            rows = n // cols if len(t["dims"]) >= 2 else 1
            base = data_start + t["offset"]
            return buf[base:base + t["nbytes"]], rows, cols
    return None
