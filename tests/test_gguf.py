"""GGUF reader (arfq_gguf_*): the library's C++ reader against the pure-Python
restatement in oracle/gguf.py and against the writer's own layout, on files
built here (the reference ships no GGUF fixtures); the GPU tests feed the
uploaded tensors to the matmul and the MoE block and check them against the
CPU oracle.  Mirrors the reference's reader tests: ggml_byte_len_matches_
block_layout, is_gguf_file_detects_magic, expert_subslice_dequant_equals_
whole_then_slice (crates/arf-core/src/model/gguf.rs:2396-2426,2578-2593,
2653-2686)."""
import struct

import numpy as np
import pytest

from conftest import rel_err
from arf_amd.synth import gguf_bytes as build
from oracle import gguf as og

TOL = 2e-3


def _write(tmp_path, name, data):
    p = tmp_path / name
    p.write_bytes(data)
    return str(p)


def _gguf(path):
    from arf_amd import Gguf
    return Gguf(path)


def _status(exc):
    return exc.value.status


def _random_kvs(rng, depth=0):
    out = []
    for i in range(int(rng.integers(0, 7))):
        vty = int(rng.choice([0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12]))
        key = f"k{depth}.{i}.é"
        if vty in (0, 7):
            v = int(rng.integers(0, 2))
        elif vty == 1:
            v = int(rng.integers(-128, 128))
        elif vty == 2:
            v = int(rng.integers(0, 65536))
        elif vty == 3:
            v = int(rng.integers(-32768, 32768))
        elif vty in (4, 10):
            v = int(rng.integers(0, 2**31))
        elif vty in (5, 11):
            v = int(rng.integers(-2**31, 2**31))
        elif vty in (6, 12):
            v = float(rng.standard_normal())
        elif vty == 8:
            v = "tok" * int(rng.integers(0, 5))
        else:  # arrays of scalars, strings or (one level of) arrays
            ety = int(rng.choice([4, 8, 9, 12]))
            n = int(rng.integers(0, 5))
            if ety == 4:
                items = [int(x) for x in rng.integers(0, 1000, n)]
            elif ety == 12:
                items = [float(x) for x in rng.standard_normal(n)]
            elif ety == 8:
                items = ["s" * int(x) for x in rng.integers(0, 4, n)]
            else:
                items = [(5, [int(x) for x in rng.integers(-9, 9, int(rng.integers(0, 4)))])
                         for _ in range(n)]
            v = (ety, items)
        out.append((key, vty, v))
    return out


_TYPES = [(8, 32, 34), (12, 256, 144), (14, 256, 210), (13, 256, 176), (0, 1, 4), (1, 1, 2),
          (2, 32, 18), (23, 256, 136)]


def _random_file(seed):
    rng = np.random.default_rng(seed)
    kvs = _random_kvs(rng)
    alignment = int(rng.choice([32, 32, 64, 256, 16, 8]))
    if alignment != 32 or rng.integers(0, 2):
        kvs.insert(int(rng.integers(0, len(kvs) + 1)), ("general.alignment", 4, alignment))
    tensors = []
    for i in range(int(rng.integers(0, 6))):
        ty, qk, bb = _TYPES[int(rng.integers(0, len(_TYPES)))]
        nd = int(rng.integers(1, 5))
        dims = [qk * int(rng.integers(1, 3))] + [int(rng.integers(1, 4)) for _ in range(nd - 1)]
        n = int(np.prod(dims))
        data = rng.integers(0, 256, n // qk * bb, dtype=np.uint8).tobytes()
        tensors.append((f"blk.{i}.ffn_down.weight", dims, ty, data))
    return build(kvs, tensors, alignment=alignment), tensors


# ---------------------------------------------------------------- CPU ----

def test_byte_len_table_matches_reference():
    # ggml_byte_len_matches_block_layout (gguf.rs:2578-2593)
    assert og.byte_len(12, 256) == 144 and og.byte_len(13, 256) == 176
    assert og.byte_len(14, 256) == 210 and og.byte_len(0, 256) == 1024 and og.byte_len(1, 256) == 512
    assert og.byte_len(12, 1_572_864) == 6144 * 144 and og.byte_len(13, 1_572_864) == 6144 * 176
    assert og.byte_len(14, 1_572_864) == 6144 * 210
    assert og.byte_len(2, 32) == 18 and og.byte_len(2, 3200) == 1800


def test_byte_len_of_the_library_matches(tmp_path):
    cases = [(12, [1_572_864]), (13, [256]), (14, [512, 3]), (0, [256]), (1, [256]), (2, [3200]),
             (8, [64, 2]), (30, [10]), (3, [32]), (20, [32]), (11, [256]), (21, [256]), (23, [256])]
    tensors = [(f"t{i}", dims, ty, b"") for i, (ty, dims) in enumerate(cases)]
    data, _ = build([], tensors)
    g = _gguf(_write(tmp_path, "len.gguf", data))
    for t, (ty, dims) in zip(g.tensors, cases):
        assert t.ggml_type == ty and list(t.dims) == dims
        assert t.nbytes == og.byte_len(ty, int(np.prod(dims)))


@pytest.mark.parametrize("seed", range(40))
def test_table_matches_oracle_and_layout(tmp_path, seed):
    (data, offs), tensors = _random_file(seed)
    _, data_start, want = og.parse(data)
    g = _gguf(_write(tmp_path, f"r{seed}.gguf", data))
    assert [t.name for t in g.tensors] == [t["name"] for t in want] == [t[0] for t in tensors]
    for got, w, (name, dims, ty, payload), off in zip(g.tensors, want, tensors, offs):
        assert got.ggml_type == w["type"] == ty
        assert list(got.dims) == w["dims"] == dims
        assert got.offset == data_start + w["offset"] == off
        assert got.nbytes == w["nbytes"] == len(payload)
        blk = g.blocks(name, ty)
        ob = og.blocks(data, name, ty)
        assert blk[0].tobytes() == ob[0] == payload
        assert blk[1:] == ob[1:]
        assert g.find(name).name == name


def test_blocks_rows_cols_and_type_mismatch(tmp_path):
    q = np.arange(3 * 2 * 144, dtype=np.uint8).tobytes()
    data, _ = build([("general.architecture", 8, "qwen3moe")],
                    [("ffn_gate_exps", [256, 2, 3], 12, q), ("v", [64], 0, bytes(256))])
    g = _gguf(_write(tmp_path, "b.gguf", data))
    b, rows, cols = g.blocks("ffn_gate_exps", 12)
    assert (rows, cols) == (6, 256) and b.tobytes() == q
    assert g.blocks("v", 0)[1:] == (1, 64)
    assert g.blocks("ffn_gate_exps", 14) is None  # stored as another type -> None
    from arf_amd.arfq import ARFQ_E_NOT_FOUND, ArfqError
    with pytest.raises(ArfqError) as e:
        g.find("missing")
    assert _status(e) == ARFQ_E_NOT_FOUND


def test_is_gguf_detects_magic(tmp_path):
    # is_gguf_file_detects_magic (gguf.rs:2396-2426)
    from arf_amd import Gguf
    assert not Gguf.is_gguf("/nonexistent/path/xyz")
    assert Gguf.is_gguf(_write(tmp_path, "good.gguf", b"GGUF\x03\x00\x00\x00"))
    assert not Gguf.is_gguf(_write(tmp_path, "bad.bin", b"XXXXdata"))
    assert not Gguf.is_gguf(_write(tmp_path, "tiny.bin", b"GG"))
    assert not Gguf.is_gguf(str(tmp_path))


def test_open_errors(tmp_path):
    from arf_amd.arfq import ARFQ_E_FORMAT, ARFQ_E_IO, ArfqError
    key = struct.pack("<Q", 1) + b"k"
    cases = {
        "magic": build([], [], magic=b"GGUG")[0],
        "version": build([], [], version=2)[0],
        "value type": build([], [], raw_kv=key + struct.pack("<I", 13))[0],
        "array element type": build([], [], raw_kv=key + struct.pack("<IIQ", 9, 13, 1) + b"\0" * 8)[0],
        "ggml type": build([], [("t", [32], 99, b"")])[0],
        "empty": b"",
    }
    for what, data in cases.items():
        with pytest.raises(ArfqError) as e:
            _gguf(_write(tmp_path, "e.gguf", data))
        assert _status(e) == ARFQ_E_FORMAT, what
        with pytest.raises(og.GgufError):
            og.parse(data)
    # an array of zero elements of an unknown type is skipped, as the reference's loop does
    ok = build([], [], raw_kv=key + struct.pack("<IIQ", 9, 13, 0))[0]
    assert _gguf(_write(tmp_path, "z.gguf", ok)).tensors == [] and og.parse(ok)[2] == []
    # stricter than the reference, which reads four bytes whatever the type and divides by them
    for what, data in {"alignment 0": build([("general.alignment", 4, 0)], [])[0],
                       "alignment type": build([("general.alignment", 10, 64)], [])[0]}.items():
        with pytest.raises(ArfqError) as e:
            _gguf(_write(tmp_path, "a.gguf", data))
        assert _status(e) == ARFQ_E_FORMAT, what
    with pytest.raises(ArfqError) as e:
        _gguf(str(tmp_path / "does-not-exist.gguf"))
    assert _status(e) == ARFQ_E_IO


def test_every_truncation_of_the_header_fails_cleanly(tmp_path):
    from arf_amd.arfq import ARFQ_E_FORMAT, ArfqError
    (data, offs), _ = _random_file(7)
    header_end = min(offs) if offs else len(data)
    (data2, offs2), _ = _random_file(3)
    for data_, end in ((data, header_end), (data2, min(offs2) if offs2 else len(data2))):
        table_end = og.parse(data_)[1]
        for cut in range(0, table_end):
            pre = data_[:cut]
            try:
                og.parse(pre)
                oracle_ok = True
            except og.GgufError:
                oracle_ok = False
            try:
                _gguf(_write(tmp_path, "t.gguf", pre))
                ok = True
            except ArfqError as e:
                assert e.status == ARFQ_E_FORMAT
                ok = False
            assert ok == oracle_ok, cut


def test_tensor_data_past_the_end(tmp_path):
    from arf_amd.arfq import ARFQ_E_FORMAT, ArfqError
    data, offs = build([], [("w", [256, 4], 12, bytes(4 * 144))])
    g = _gguf(_write(tmp_path, "cut.gguf", data[:-1]))  # the table is whole: open succeeds
    with pytest.raises(ArfqError) as e:
        g.blocks("w", 12)
    assert _status(e) == ARFQ_E_FORMAT


def test_nested_arrays_are_bounded(tmp_path):
    from arf_amd.arfq import ARFQ_E_FORMAT, ArfqError
    v = (5, [1, 2])
    for _ in range(70):
        v = (9, [v])
    data, _ = build([("deep", 9, v)], [])
    with pytest.raises(ArfqError) as e:
        _gguf(_write(tmp_path, "deep.gguf", data))
    assert _status(e) == ARFQ_E_FORMAT
    og.parse(data)  # the reference's reader accepts any depth


# ---------------------------------------------------------------- GPU ----

def _model_file(tmp_path, E=4, hidden=512, inter=256):
    from arf_amd import synth
    q4 = synth.weight("q4_k", 96, 1024, seed=1)
    q6 = synth.weight("q6_k", 40, 768, seed=2)
    q8 = synth.weight("q8_0", 72, 320, seed=3)
    q5 = synth.weight("q5_k", 56, 768, seed=8)
    iq4 = synth.weight("iq4_xs", 24, 1280, seed=9)
    qkv = synth.weight("q4_k", 48 + 2 * 16, 512, seed=4)
    gate = synth.weight("q4_k", inter, hidden, seed=5, experts=E)
    up = synth.weight("q4_k", inter, hidden, seed=6, experts=E)
    down = synth.weight("q4_k", hidden, inter, seed=7, experts=E)
    tensors = [("blk.0.ffn_up.weight", [1024, 96], 12, q4.tobytes()),
               ("blk.0.ffn_down.weight", [768, 40], 14, q6.tobytes()),
               ("output.weight", [320, 72], 8, q8.tobytes()),
               ("token_embd.weight", [768, 56], 13, q5.tobytes()),
               ("blk.2.ffn_gate.weight", [1280, 24], 23, iq4.tobytes()),
               ("blk.0.attn_qkv.weight", [512, 80], 12, qkv.tobytes()),
               ("blk.0.ffn_gate_exps.weight", [hidden, inter, E], 12, gate.tobytes()),
               ("blk.0.ffn_up_exps.weight", [hidden, inter, E], 12, up.tobytes()),
               ("blk.0.ffn_down_exps.weight", [inter, hidden, E], 12, down.tobytes()),
               ("blk.0.attn_norm.weight", [512], 0, bytes(2048))]
    data, _ = build([("general.architecture", 8, "qwen3moe"), ("general.alignment", 4, 64)],
                    tensors, alignment=64)
    return _write(tmp_path, "model.gguf", data), dict(q4=q4, q6=q6, q8=q8, q5=q5, iq4=iq4,
                                                      qkv=qkv, gate=gate, up=up, down=down)


@pytest.mark.gpu
def test_gpu_upload_matrices_and_row_slices(gpu_ctx, oracle, tmp_path):
    from arf_amd import synth
    path, raw = _model_file(tmp_path)
    g = _gguf(path)
    cases = [("blk.0.ffn_up.weight", "q4_k", raw["q4"], 96, 1024, 0, -1),
             ("blk.0.ffn_down.weight", "q6_k", raw["q6"], 40, 768, 0, -1),
             ("output.weight", "q8_0", raw["q8"], 72, 320, 0, -1),
             ("token_embd.weight", "q5_k", raw["q5"], 56, 768, 0, -1),
             ("blk.2.ffn_gate.weight", "iq4_xs", raw["iq4"], 24, 1280, 0, -1),
             # the fused q/k/v rows: q = rows 0..47, k = 48..63, v = 64..79
             ("blk.0.attn_qkv.weight", "q4_k", raw["qkv"][:48 * 2 * 144], 48, 512, 0, 48),
             ("blk.0.attn_qkv.weight", "q4_k", raw["qkv"][48 * 2 * 144:64 * 2 * 144], 16, 512, 48, 16),
             ("blk.0.attn_qkv.weight", "q4_k", raw["qkv"][64 * 2 * 144:], 16, 512, 64, -1)]
    for name, qt, blocks, n, k, row0, nrows in cases:
        print("case: gguf upload", name, row0, nrows, flush=True)
        w = gpu_ctx.upload_gguf(g, name, row0, nrows)
        assert (w.n, w.k, w.experts) == (n, k, 1)
        deq = gpu_ctx.dequant(w).numpy().reshape(-1)
        assert np.array_equal(deq.view(np.uint32), oracle.dequant(qt, blocks, n * k).view(np.uint32))
        for m in ((1, 3) if qt in ("q5_k", "iq4_xs") else (1, 5)):
            x = synth.activations(m, k, seed=m + n)
            y = gpu_ctx.empty((m, n), np.float32)
            gpu_ctx.matmul(w, gpu_ctx.to_device(x), m, y)
            assert rel_err(y.numpy(), oracle.matmul_q(qt, x, blocks, n)) <= TOL


@pytest.mark.gpu
def test_gpu_upload_shape_errors(gpu_ctx, tmp_path):
    from arf_amd.arfq import ARFQ_E_NOT_FOUND, ARFQ_E_UNSUPPORTED, ArfqError
    path, _ = _model_file(tmp_path)
    g = _gguf(path)
    for name, row0, nrows in [("blk.0.attn_qkv.weight", 70, 16), ("blk.0.attn_qkv.weight", -1, 4),
                              ("blk.0.attn_qkv.weight", 0, 0), ("blk.0.ffn_gate_exps.weight", 1, -1)]:
        with pytest.raises(ValueError):
            gpu_ctx.upload_gguf(g, name, row0, nrows)
    with pytest.raises(ArfqError) as e:
        gpu_ctx.upload_gguf(g, "blk.0.attn_norm.weight")  # F32: no matmul kernel
    assert _status(e) == ARFQ_E_UNSUPPORTED
    with pytest.raises(ArfqError) as e:
        gpu_ctx.upload_gguf(g, "nope")
    assert _status(e) == ARFQ_E_NOT_FOUND


@pytest.mark.gpu
def test_gpu_experts_from_gguf(gpu_ctx, oracle, tmp_path):
    # expert_subslice_dequant_equals_whole_then_slice (gguf.rs:2653-2686), then the MoE block
    from arf_amd import synth
    E, hidden, inter, T, top_k = 4, 512, 256, 24, 2
    path, raw = _model_file(tmp_path, E, hidden, inter)
    g = _gguf(path)
    ws = [gpu_ctx.upload_gguf(g, f"blk.0.ffn_{p}_exps.weight") for p in ("gate", "up", "down")]
    assert [(w.n, w.k, w.experts) for w in ws] == [(inter, hidden, E), (inter, hidden, E),
                                                   (hidden, inter, E)]
    whole = oracle.dequant("q4_k", raw["gate"], E * inter * hidden)
    per = inter * hidden
    x = synth.activations(3, hidden, seed=11)
    for e in range(E):
        y = gpu_ctx.empty((3, inter), np.float32)
        gpu_ctx.matmul(ws[0], gpu_ctx.to_device(x), 3, y, expert=e)
        sub = raw["gate"][e * per // 256 * 144:(e + 1) * per // 256 * 144]
        assert np.array_equal(oracle.dequant("q4_k", sub, per).view(np.uint32),
                              whole[e * per:(e + 1) * per].view(np.uint32))
        assert rel_err(y.numpy(), oracle.matmul_q("q4_k", x, sub, inter)) <= TOL
    xm = synth.activations(T, hidden, seed=12, dtype=np.float16)
    logits = synth.router_logits(T, E, seed=13)
    y = gpu_ctx.empty((T, hidden), np.float32)
    gpu_ctx.moe(ws[0], ws[1], ws[2], gpu_ctx.to_device(logits), T, top_k, True, gpu_ctx.to_device(xm), y)
    want = oracle.moe_forward(xm.astype(np.float32), raw["gate"], raw["up"], raw["down"], E, inter,
                              logits, top_k, True)
    assert rel_err(y.numpy(), want) <= TOL
