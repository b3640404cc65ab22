"""Writes tests/golden/fixtures.npz: small golden vectors for the GPU box.

Every expected output comes from the CPU oracle (oracle/arfq_oracle.c), whose
functions are pinned in tests/test_oracle.py by the reference's own known
answers, closed forms and float64 brute force.  The inputs are:

  dq_q4k_known     the known block of crates/arf-core/src/model/gguf.rs:2522-2538
                   (d=2, dmin=1, sc0=3, m0=5, q=4 -> 19.0, next weight -> -5.0)
  dq_q4k_gate_*    the bit-exact gate blocks of gguf.rs:2862-2982: the known block,
                   sign fold m=63, the two LCG cases (seeds 0x12345678 and
                   0xDEADBEEF) and the high-scale path j>=4
  dq_q6k_known     gguf.rs:2564-2575 (d=0.5, sc0=4, ql0=10 -> -44.0)
  dq_q6k_quads     one nonzero code per (half, quadrant, qh pair, scale slot)
  dq_q80_closed    q = -128..127, d in {1, 0.5, 0.001, 6e-8 (subnormal), 65504}
  mm_<fmt>_*       one small shape per format: x, weight blocks, y = oracle
                   matmul (Q4_K N=64 K=512 M=4, Q8_0 N=64 K=512 M=4,
                   Q6_K N=64 K=512 M=8, Q4_K f16 x M=80 N=64 K=512)
  route_lcg128_*   the two 128-expert top-8 cases of crates/arf-gpu/tests/
                   moe_gpu.rs:84-93 (LCG seed 99), with and without renorm
  moe_small_*      T=5, E=4, top-2, hidden=256, inter=256 Q4_K MoE block

Run from the repository root: python tests/golden/make_fixtures.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

from arf_amd import synth  # noqa: E402
from formats import (lcg_q4k_blocks, make_q6k_block, make_q80_block,  # noqa: E402
                     moe_route_lcg_logits, ref_make_q4k_block)
from oracle import oracle  # noqa: E402

OUT = os.path.join(HERE, "fixtures.npz")


def q4k_gate_blocks():
    """(name, raw, rows, cols) of the gguf.rs:2862-2982 bit-exact gate."""
    out = []
    sc = np.zeros(12, np.uint8); sc[0], sc[4] = 3, 5
    qs = np.zeros(128, np.uint8); qs[0] = 0x04
    out.append(("known", ref_make_q4k_block(2.0, 1.0, sc, qs), 1, 256))
    sc = np.zeros(12, np.uint8); sc[1], sc[5] = 10, 63
    qs = np.zeros(128, np.uint8); qs[0] = 0x70
    out.append(("signfold", ref_make_q4k_block(1.0, 0.5, sc, qs), 1, 256))
    out.append(("lcg_a", lcg_q4k_blocks(0x12345678, 3, 1.0, 64.0, 0.5, 128.0), 1, 768))
    out.append(("lcg_b", lcg_q4k_blocks(0xDEADBEEF, 2, 2.0, 128.0, 1.0, 256.0), 2, 256))
    sc = np.zeros(12, np.uint8)
    sc[0], sc[4], sc[8] = 0b1100_0101, 0b0100_0111, 0b1010_0011
    qs = np.zeros(128, np.uint8); qs[64] = 0x0F
    out.append(("highj", ref_make_q4k_block(0.25, 0.125, sc, qs), 1, 256))
    return out


def build():
    oracle.build()
    f = {}
    # ---- dequant ----
    b = np.zeros(144, np.uint8)
    b[0:2] = np.array([0x4000], np.uint16).view(np.uint8)
    b[2:4] = np.array([0x3C00], np.uint16).view(np.uint8)
    b[4], b[8], b[16] = 3, 5, 0x04
    f["dq_q4k_known_raw"] = b
    f["dq_q4k_known_y"] = oracle.dequant("q4_k", b, 256)

    for name, raw, rows, cols in q4k_gate_blocks():
        f[f"dq_q4k_gate_{name}_raw"] = raw
        f[f"dq_q4k_gate_{name}_shape"] = np.array([rows, cols], np.int64)
        f[f"dq_q4k_gate_{name}_y"] = oracle.dequant("q4_k", raw, rows * cols)

    b = np.zeros(210, np.uint8)
    b[192], b[0] = 4, 10
    b[208:210] = np.array([0x3800], np.uint16).view(np.uint8)
    f["dq_q6k_known_raw"] = b
    f["dq_q6k_known_y"] = oracle.dequant("q6_k", b, 256)

    blocks = []
    for e in range(0, 256, 5):
        for hi in range(4):
            q = [32] * 256
            q[e] = (hi << 4) | (e % 16)
            blocks.append(make_q6k_block(1.0, list(range(1, 17)), q))
    raw = np.concatenate(blocks)
    f["dq_q6k_quads_raw"] = raw
    f["dq_q6k_quads_y"] = oracle.dequant("q6_k", raw, len(blocks) * 256)

    qs = np.arange(-128, 128, dtype=np.int32)
    blocks = [make_q80_block(d, qs[i:i + 32])
              for d in (1.0, 0.5, 0.001, 6.0e-8, 65504.0) for i in range(0, 256, 32)]
    raw = np.concatenate(blocks)
    f["dq_q80_closed_raw"] = raw
    f["dq_q80_closed_y"] = oracle.dequant("q8_0", raw, len(blocks) * 32)

    # ---- matmuls ----
    for name, qtype, m, n, k, xdt in (("q4k", "q4_k", 4, 64, 512, np.float32),
                                       ("q80", "q8_0", 4, 64, 512, np.float32),
                                       ("q6k", "q6_k", 8, 64, 512, np.float32),
                                       ("q4k_f16", "q4_k", 80, 64, 512, np.float16)):
        raw = synth.weight(qtype, n, k, seed=0x601D + n + k + m)
        x = synth.activations(m, k, seed=0x601E + m).astype(xdt)
        f[f"mm_{name}_raw"] = raw
        f[f"mm_{name}_x"] = x
        f[f"mm_{name}_y"] = oracle.matmul_q(qtype, x.astype(np.float32), raw, n)

    # ---- routing ----
    state = 99
    rows = []
    for _ in range(2):
        lg, state = moe_route_lcg_logits(128, state)
        rows.append(lg)
    lg = np.stack(rows).astype(np.float32)
    f["route_lcg128_logits"] = lg
    for norm in (0, 1):
        res = [oracle.top_k_softmax(lg[t], 8, bool(norm)) for t in range(2)]
        f[f"route_lcg128_norm{norm}_ids"] = np.stack([r[0] for r in res]).astype(np.int32)
        f[f"route_lcg128_norm{norm}_w"] = np.stack([r[1] for r in res]).astype(np.float32)

    # ---- MoE block ----
    T, E, k, hidden, inter = 5, 4, 2, 256, 256
    gate = synth.weight("q4_k", inter, hidden, seed=0x601F, experts=E)
    up = synth.weight("q4_k", inter, hidden, seed=0x6020, experts=E)
    down = synth.weight("q4_k", hidden, inter, seed=0x6021, experts=E)
    x = synth.activations(T, hidden, seed=0x6022, dtype=np.float16)
    logits = synth.router_logits(T, E, seed=0x6023)
    f["moe_small_dims"] = np.array([T, E, k, hidden, inter], np.int64)
    f["moe_small_gate"] = gate
    f["moe_small_up"] = up
    f["moe_small_down"] = down
    f["moe_small_x"] = x
    f["moe_small_logits"] = logits
    f["moe_small_y"] = oracle.moe_forward(x.astype(np.float32), gate, up, down, E, inter,
                                          logits, k, True)
    return f


def main():
    f = build()
    np.savez_compressed(OUT, **f)
    print(f"wrote {OUT}: {len(f)} arrays, {os.path.getsize(OUT)} bytes")


if __name__ == "__main__":
    main()
