"""Benchmark of the GGUF quantized-matmul hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--quick]

Headline (the JSON `value`): Q4_K decode GEMV, m=1, k=5120, n=17408, f32 x times the
exact weights in f32 (the reference's arithmetic) -- one step is one GEMV launch over one
activation vector.  Weights are 8 distinct seeded
copies (8 x 50 MB, above the 256 MB MALL) used round-robin so the timed loop
streams from HBM.  Timing: HIP events recorded on the library's stream around
exactly K back-to-back launches, after one set-up launch per weight copy, a clock
settle phase (launches for SETTLE_S of wall time: the GPU's clock ramps up over the
first ~10-20 ms of sustained load, which moved C4 from 430 to 387 us), W warm-up
launches and a stream sync.
Secondary configs are measured the same way and reported under "configs".

The CPU baselines run the oracle (a C restatement of Arf's CPU matmuls) on the host
cores, partitioned as the reference does, on bounded samples of every config (the
headline's in `cpu_baseline`, the others under `configs`); they are reported baselines,
not targets.
"""
import argparse
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0         # MI355X HBM3E
SETTLE_S = 0.05               # untimed launches before each config's warm-up (clock ramp)
FP16_MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def algorithmic_bytes(qtype, m, n, k, x_bytes=4):
    from arf_amd import synth
    wb = n * (k // synth.QK[qtype]) * synth.BLOCK_BYTES[qtype]
    return wb + m * k * x_bytes + m * n * 4


def settle(ctx, launch, seconds=SETTLE_S):
    """Untimed launches (`launch(i)` issues some) until `seconds` of wall time have passed,
    so the timed region starts at the clock the GPU holds under sustained load."""
    t0, i = time.time(), 0
    while time.time() - t0 < seconds:
        for _ in range(16):  # host syncs only between batches: the GPU stays busy
            launch(i)
            i += 1
        ctx.sync()


def time_matmul(ctx, qtype, m, n, k, steps, warmup, copies, seed, x_dtype=np.float32, settle_s=SETTLE_S):
    """Average ms per launch of arfq_matmul over `steps` launches rotating `copies` weights.
    Set-up runs one untimed launch per weight copy (so no copy is first touched inside the
    timed region, whatever `warmup` is), then the `warmup` launches."""
    from arf_amd import QType, synth
    qt = QType[qtype.upper()]
    raw = synth.weight(qtype, n, k, seed=seed)
    ws = [ctx.upload(qt, raw, n, k) for _ in range(copies)]
    x = ctx.to_device(synth.activations(m, k, seed=seed + 1).astype(x_dtype))
    y = ctx.empty((m, n), np.float32)
    ctx.matmul_repeat(ws, copies, m, x, y)  # set-up: each copy once
    settle(ctx, lambda i: ctx.matmul_repeat(ws, 4 * copies, m, x, y), settle_s)
    ctx.matmul_repeat(ws, warmup, m, x, y)
    ctx.sync()
    ctx.timer_start()
    ctx.matmul_repeat(ws, steps, m, x, y)
    ms = ctx.timer_stop()
    ctx.sync()
    for w in ws:
        w.free()
    return ms / steps, ms


def time_ffn(ctx, qts, hidden, inter, m, steps, warmup, copies):
    """Average ms per arfq_ffn call (gate/up/down of qtypes qts) over `copies` weight sets."""
    from arf_amd import QType, synth
    shapes = [(inter, hidden), (inter, hidden), (hidden, inter)]
    sets = [[ctx.upload(QType[q.upper()], synth.weight(q, n, k, seed=0xA7F00010 + 3 * c + i), n, k)
             for i, (q, (n, k)) in enumerate(zip(qts, shapes))] for c in range(copies)]
    x = ctx.to_device(synth.activations(m, hidden, seed=0xA7F0000F))
    y = ctx.empty((m, hidden), np.float32)
    settle(ctx, lambda i: ctx.ffn(*sets[i % copies], x, m, y))
    for i in range(warmup):
        ctx.ffn(*sets[i % copies], x, m, y)
    ctx.sync()
    ctx.timer_start()
    for i in range(steps):
        ctx.ffn(*sets[i % copies], x, m, y)
    ms = ctx.timer_stop()
    ctx.sync()
    for ws in sets:
        for w in ws:
            w.free()
    return ms / steps


def time_moe(ctx, steps, warmup, copies, tokens=None, settle_s=SETTLE_S):
    """Average ms per arfq_moe call (C5's experts; `tokens` defaults to C5's 512) rotating
    `copies` weight sets, after `warmup` calls."""
    from arf_amd import QType, synth
    cfg = synth.CONFIGS["c5_moe"]
    E, T, k, hdim, inter = cfg["experts"], cfg["tokens"], cfg["top_k"], cfg["hidden"], cfg["inter"]
    T = tokens or T
    sets = []
    for c in range(copies):
        g = ctx.upload(QType.Q4_K, synth.weight("q4_k", inter, hdim, seed=0xA7F00005 + 3 * c, experts=E),
                       inter, hdim, E)
        u = ctx.upload(QType.Q4_K, synth.weight("q4_k", inter, hdim, seed=0xA7F00006 + 3 * c, experts=E),
                       inter, hdim, E)
        d = ctx.upload(QType.Q4_K, synth.weight("q4_k", hdim, inter, seed=0xA7F00007 + 3 * c, experts=E),
                       hdim, inter, E)
        sets.append((g, u, d))
    x = ctx.to_device(synth.activations(T, hdim, seed=0xA7F00008, dtype=np.float16))
    lg = ctx.to_device(synth.router_logits(T, E, seed=0xA7F00009))
    y = ctx.empty((T, hdim), np.float32)
    settle(ctx, lambda i: ctx.moe(*sets[i % copies], lg, T, k, True, x, y), settle_s)
    for i in range(warmup):
        g, u, d = sets[i % copies]
        ctx.moe(g, u, d, lg, T, k, True, x, y)
    ctx.sync()
    ctx.timer_start()
    for i in range(steps):
        g, u, d = sets[i % copies]
        ctx.moe(g, u, d, lg, T, k, True, x, y)
    ms = ctx.timer_stop()
    ctx.sync()
    for ws in sets:
        for w in ws:
            w.free()
    return ms / steps


def cpu_model():
    """The host CPU's model name with its family / model / stepping numbers (from
    /proc/cpuinfo, which a virtual machine may report generically) and the logical
    CPU count."""
    name = platform.processor() or platform.machine()
    fields = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if not line.strip():
                    break  # the first processor's block
                k, _, v = line.partition(":")
                fields[k.strip()] = v.strip()
    except OSError:
        pass
    if "model name" in fields:
        name = fields["model name"]
        ids = [f"{k} {fields[k]}" for k in ("cpu family", "model", "stepping") if k in fields]
        if ids:
            name += " (" + ", ".join(ids) + ")"
    return name, os.cpu_count() or 1


# threads for the reference's par_rows (std::thread::available_parallelism on the GPU box,
# capped at the 16-core share a one-GPU box gives a job)
CPU_PAR_THREADS = max(1, min(os.cpu_count() or 1, 16))


def _timed(fn, budget_s, min_reps=1):
    """Seconds per call of fn, repeated for about budget_s (at least min_reps calls)."""
    t0 = time.perf_counter()
    reps = 0
    while reps < min_reps or time.perf_counter() - t0 < budget_s:
        fn()
        reps += 1
    return (time.perf_counter() - t0) / reps, reps


def cpu_baselines(budget_s):
    """The repo's CPU path (the oracle: a C restatement of arf-ml's matmuls) on the host,
    partitioned as the reference partitions it: par_rows over M with one thread per core,
    serial when M < 2 (crates/arf-ml/src/matmul.rs:16-45), the MoE token loop serial
    (crates/arf-core/src/model/moe.rs:69).  Q4_K weights are transcoded to Q4_K_S first and
    Q6_K ones dequantized to f32 first, as the reference does at load time; neither is
    timed in the matmul figures (Q6_K's dequant is reported beside).  C4 and C5 run a
    bounded sample of rows / tokens and report the full-size rate by linear scaling."""
    from arf_amd import synth
    from oracle import oracle
    model, ncpu = cpu_model()
    out = {}
    host = f"host {model}, {ncpu} logical CPUs"

    # C2 (headline): matmul_nt_q4ks, m = 1 (serial), full size
    n, k = 17408, 5120
    raw = synth.weight("q4_k", n, k, seed=0xA7F00002)
    x = synth.activations(1, k, seed=0xA7F00003)
    q4ks = oracle.q4ks_from_ggml(raw, n, k)
    oracle.set_threads(1)
    dt, reps = _timed(lambda: oracle.matmul_q4ks(x, q4ks, n), budget_s)
    gbs = algorithmic_bytes("q4_k", 1, n, k) / dt / 1e9
    out["c2"] = {"value": round(gbs, 3), "unit": "GB/s", "cores": 1, "kind": "port",
                 "sample": f"{reps} full C2 GEMVs (m=1, k=5120, n=17408), {dt * 1e3:.1f} ms each, "
                           f"oracle matmul_nt_q4ks serial (par_rows is serial at m<2); {host}"}
    # C1: matmul_nt_q8_0, m = 1 (serial)
    raw = synth.weight("q8_0", 2048, 2048, seed=0xA7F00001)
    x = synth.activations(1, 2048, seed=0xA7F00002)
    dt, reps = _timed(lambda: oracle.matmul_q("q8_0", x, raw, 2048), budget_s / 10)
    out["c1"] = {"us_per_call": round(dt * 1e6, 1),
                 "GB/s": round(algorithmic_bytes("q8_0", 1, 2048, 2048) / dt / 1e9, 3), "cores": 1,
                 "kind": "port", "sample": f"{reps} full C1 GEMVs, oracle matmul_nt_q8_0 serial; {host}"}
    # C3: dequant_q6_k (load time) + matmul_nt at m = 1 (serial), 8, 32, 64 (par_rows)
    n, k = 5120, 17408
    raw = synth.weight("q6_k", n, k, seed=0xA7F00003)
    t0 = time.perf_counter()
    wf = oracle.dequant("q6_k", raw, n * k).reshape(n, k)
    deq = time.perf_counter() - t0
    for mm in (1, 8, 32, 64):
        x = synth.activations(mm, k, seed=0xA7F00004)
        oracle.set_threads(1 if mm < 2 else CPU_PAR_THREADS)
        dt, reps = _timed(lambda: oracle.matmul_nt(x, wf), budget_s / 20)
        cores = 1 if mm < 2 else CPU_PAR_THREADS
        out[f"c3_m{mm}"] = {"us_per_call": round(dt * 1e6, 1),
                            "GB/s": round(algorithmic_bytes("q6_k", mm, n, k) / dt / 1e9, 3),
                            "cores": cores, "kind": "port",
                            "sample": f"{reps} full C3 products at m={mm}, oracle matmul_nt on the "
                                      f"f32 dequant ({cores} thread(s)); dequant_q6_k of the weight "
                                      f"(serial, load time) took {deq * 1e3:.0f} ms; {host}"}
    # C4: matmul_nt_q4ks with par_rows over the 2048 rows: a sample of 128 rows, scaled
    n, k, M, ms_ = 17408, 5120, 2048, 128
    raw = synth.weight("q4_k", n, k, seed=0xA7F00004)
    q4ks = oracle.q4ks_from_ggml(raw, n, k)
    x = synth.activations(ms_, k, seed=0xA7F00005, dtype=np.float16).astype(np.float32)
    oracle.set_threads(CPU_PAR_THREADS)
    dt, reps = _timed(lambda: oracle.matmul_q4ks(x, q4ks, n), budget_s / 5)
    full = dt * M / ms_
    out["c4"] = {"ms_full_estimate": round(full * 1e3, 1),
                 "TFLOP/s": round(2.0 * M * n * k / full / 1e12, 5), "cores": CPU_PAR_THREADS,
                 "kind": "port",
                 "sample": f"{reps} runs of {ms_} of C4's 2048 rows ({dt * 1e3:.0f} ms each, scaled "
                           f"x{M // ms_}), oracle matmul_nt_q4ks with par_rows over "
                           f"{CPU_PAR_THREADS} threads; {host}"}
    # C5: MoeMlp::forward, serial token loop, each expert's three projections at m = 1
    cfg = synth.CONFIGS["c5_moe"]
    E, T, topk, hid, inter = cfg["experts"], cfg["tokens"], cfg["top_k"], cfg["hidden"], cfg["inter"]
    g = synth.weight("q4_k", inter, hid, seed=0xA7F00005, experts=E).reshape(E, -1)
    u = synth.weight("q4_k", inter, hid, seed=0xA7F00006, experts=E).reshape(E, -1)
    d = synth.weight("q4_k", hid, inter, seed=0xA7F00007, experts=E).reshape(E, -1)
    gs = [oracle.q4ks_from_ggml(g[e], inter, hid) for e in range(E)]
    us = [oracle.q4ks_from_ggml(u[e], inter, hid) for e in range(E)]
    ds = [oracle.q4ks_from_ggml(d[e], hid, inter) for e in range(E)]
    ts = 16
    x = synth.activations(ts, hid, seed=0xA7F00008, dtype=np.float16).astype(np.float32)
    lg = synth.router_logits(ts, E, seed=0xA7F00009)
    oracle.set_threads(1)

    def moe_sample():
        y = np.zeros((ts, hid), np.float32)
        for t in range(ts):
            ids, wts = oracle.top_k_softmax(lg[t], topk, True)
            for e, wj in zip(ids, wts):
                gg = oracle.matmul_q4ks(x[t], gs[e], inter)
                uu = oracle.matmul_q4ks(x[t], us[e], inter)
                h = (gg / (np.float32(1) + np.exp(-gg)) * uu).astype(np.float32)
                y[t] += wj * oracle.matmul_q4ks(h, ds[e], hid)[0]
        return y

    with np.errstate(over="ignore"):
        dt, reps = _timed(moe_sample, budget_s / 5)
    full = dt * T / ts
    out["c5"] = {"ms_full_estimate": round(full * 1e3, 1),
                 "TFLOP/s": round(2.0 * T * topk * 3 * inter * hid / full / 1e12, 5), "cores": 1,
                 "kind": "port",
                 "sample": f"{reps} runs of {ts} of C5's 512 tokens ({dt * 1e3:.0f} ms each, scaled "
                           f"x{T // ts}): serial token loop, top-8 routing, three matmul_nt_q4ks "
                           f"per (token, expert) at m=1; {host}"}
    oracle.set_threads(0)
    return out


def load_traffic(name, kernel):
    """HBM bytes per dispatch of the kernel whose name contains `kernel`, from a
    profiles/*_traffic.json summary of two rocprofv3 --pmc passes (FETCH_SIZE,
    WRITE_SIZE), or None."""
    p = os.path.join(ROOT, "profiles", name)
    if os.path.exists(p):
        with open(p) as f:
            for kname, v in json.load(f).get("kernels", {}).items():
                if kernel in kname:
                    return v.get("traffic_bytes_per_launch")
    return None


COPY_PROBE_BYTES = 256 << 20
COPY_PROBE_LAUNCHES = 4
TRAFFIC_PROBE_LAUNCHES = 16


def traffic_probe(ctx, copies, config="c2"):
    """Kernels for the HBM byte counters (FETCH_SIZE / WRITE_SIZE, one rocprofv3
    --pmc pass each): COPY_PROBE_LAUNCHES copies of COPY_PROBE_BYTES (the known
    size that calibrates the counters: a copy reads and writes exactly that many
    bytes), then TRAFFIC_PROBE_LAUNCHES calls of `config` (C2 by default; any
    --only name) rotating `copies` weights, as in the timed loop."""
    a = ctx.empty((COPY_PROBE_BYTES,), np.uint8)
    b = ctx.empty((COPY_PROBE_BYTES,), np.uint8)
    for _ in range(COPY_PROBE_LAUNCHES):
        ctx.copy_d2d(b, a)
    ctx.sync()
    a.free()
    b.free()
    shape = {"c1": ("q8_0", 1, 2048, 2048), "c2": ("q4_k", 1, 17408, 5120),
             "c3m1": ("q6_k", 1, 5120, 17408), "c3m8": ("q6_k", 8, 5120, 17408),
             "c3m32": ("q6_k", 32, 5120, 17408), "c3m64": ("q6_k", 64, 5120, 17408),
             "c4": ("q4_k", 2048, 17408, 5120)}
    if config == "c5":
        time_moe(ctx, TRAFFIC_PROBE_LAUNCHES, 0, copies, settle_s=0)
    else:
        qt, m, n, k = shape[config]
        time_matmul(ctx, qt, m, n, k, TRAFFIC_PROBE_LAUNCHES, 0, copies, 0xA7F00002,
                    x_dtype=np.float16 if m == 2048 else np.float32, settle_s=0)
    ctx.sync()
    log(f"[probe] {COPY_PROBE_LAUNCHES} copies of {COPY_PROBE_BYTES} B, then {config}: "
        f"{copies} set-up + {TRAFFIC_PROBE_LAUNCHES} launches over {copies} weight copies")


def gguf_reader_bench(ctx):
    """GGUF reader: open (header + key/values + tensor table) and upload (host -> device copy
    of the mapped blocks plus the device repack) of a synthetic model file."""
    import shutil
    import tempfile

    import arf_amd
    from arf_amd import synth
    c5 = synth.CONFIGS["c5_moe"]
    E, hid, inter = c5["experts"], c5["hidden"], c5["inter"]
    specs = [("blk.0.ffn_gate_exps.weight", [hid, inter, E], inter, hid, E, 1),
             ("blk.0.ffn_up_exps.weight", [hid, inter, E], inter, hid, E, 2),
             ("blk.0.ffn_down_exps.weight", [inter, hid, E], hid, inter, E, 3),
             ("blk.1.ffn_up.weight", [5120, 17408], 17408, 5120, 1, 4)]
    vocab = [f"tok{i}" for i in range(151936)]
    kvs = [("general.architecture", 8, "qwen3moe"), ("general.alignment", 4, 32),
           ("tokenizer.ggml.tokens", 9, (8, vocab)),
           ("tokenizer.ggml.token_type", 9, (5, [1] * len(vocab)))]
    tensors = []
    for name, dims, n, k, e, seed in specs:
        nbytes = e * n * (k // 256) * 144
        tensors.append((name, dims, 12, nbytes,
                        lambda f, n=n, k=k, e=e, seed=seed: synth.weight("q4_k", n, k, seed, e).tofile(f)))
    tmp = tempfile.mkdtemp(prefix="arfq_gguf_")
    try:
        path = os.path.join(tmp, "model.gguf")
        synth.gguf_write(path, kvs, tensors)
        size = os.path.getsize(path)
        opens = []
        for _ in range(5):
            t0 = time.perf_counter()
            g = arf_amd.Gguf(path)
            opens.append((time.perf_counter() - t0) * 1e3)
            g.close()
        g = arf_amd.Gguf(path)
        table_end = min(t.offset for t in g.tensors)
        ups = {}
        for rep in range(2):  # the first pass also reads the file into the page cache
            for name, *_ in specs:
                t0 = time.perf_counter()
                w = ctx.upload_gguf(g, name)
                ms = (time.perf_counter() - t0) * 1e3
                nb = g.find(name).nbytes
                ups[name] = {"bytes": nb, "ms": round(ms, 2), "GB/s": round(nb / ms / 1e6, 2)}
                w.free()
        g.close()
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    total = sum(u["bytes"] for u in ups.values())
    out = {"metric": "GGUF reader: table parse ms, upload GB/s (host page cache -> HBM)",
           "value": round(total / sum(u["ms"] for u in ups.values()) / 1e6, 2), "unit": "GB/s",
           "higher_is_better": True, "n_gpus": 1, "data": "synthetic GGUF v3 file",
           "config": {"workload": "gguf_c5_experts_c2_matrix", "file_bytes": size,
                      "header_bytes": table_end, "tensors": len(specs), "vocab_strings": len(vocab)},
           "open_ms_median": round(sorted(opens)[len(opens) // 2], 3), "upload": ups}
    log(f"[gguf] open {out['open_ms_median']} ms for a {table_end} B header; "
        f"upload {out['value']} GB/s")
    print(json.dumps(out), flush=True)


STREAM_BYTES = 512 << 20   # above the 256 MB MALL
STREAM_STAMP_WGS = 256


def stream_ceiling(ctx, c2_launches, copies):
    """The practical HBM read ceiling, measured in this run with a plain read-only
    kernel (arfq_stream_read: 16-byte loads, four in flight per lane):
      - stream_gbs: one pass over a STREAM_BYTES buffer (best of 5 timed passes);
      - stream_c2_gbs: back-to-back passes over `copies` rotating buffers of C2's
        weight bytes (50,135,040 B each), timed like the C2 loop, so the figure
        carries the same per-launch gap the GEMV pays;
      - clock_mhz: the shader clock while the big pass ran, from s_memtime against
        s_memrealtime in the first STREAM_STAMP_WGS workgroups."""
    cus, sclk_khz, wclk_khz = ctx.device_info()
    big = ctx.empty((STREAM_BYTES,), np.uint8)
    stamps = ctx.empty((STREAM_STAMP_WGS * 4,), np.uint64)
    for _ in range(3):
        ctx.stream_read(big)
    ctx.sync()
    best = None
    for _ in range(5):
        ctx.timer_start()
        ctx.stream_read(big, stamps=stamps)
        ms = ctx.timer_stop()
        best = ms if best is None else min(best, ms)
    st = stamps.numpy().reshape(-1, 4).astype(np.float64)
    dr, dc = st[:, 2] - st[:, 0], st[:, 3] - st[:, 1]
    ok = dr > 0
    clock = float(dc[ok].sum() / dr[ok].sum() * wclk_khz / 1e3) if ok.any() and wclk_khz > 0 else None
    big.free()
    stamps.free()
    c2b = 50135040
    bufs = [ctx.empty((c2b,), np.uint8) for _ in range(copies)]
    for b in bufs:
        ctx.stream_read(b)
    t0 = time.time()
    while time.time() - t0 < SETTLE_S:
        for b in bufs:
            ctx.stream_read(b)
        ctx.sync()
    ctx.timer_start()
    for i in range(c2_launches):
        ctx.stream_read(bufs[i % copies])
    ms_c2 = ctx.timer_stop() / c2_launches
    for b in bufs:
        b.free()
    out = {"stream_gbs": round(STREAM_BYTES / best / 1e6, 1),
           "stream_c2_gbs": round(c2b / ms_c2 / 1e6, 1),
           "stream_c2_us_per_launch": round(ms_c2 * 1e3, 3),
           "clock_mhz": round(clock, 0) if clock else None,
           "clock_peak_mhz": round(sclk_khz / 1e3, 0), "cus": cus}
    log(f"[bench] stream ceiling: {out}")
    return out


def only_config(ctx, args):
    """One config, timed as in the full run (args.steps launches after args.warmup)."""
    from arf_amd import synth
    import arf_amd.arfq as _arfq
    c = args.only
    if c in ("c2", "c2x16"):
        if c == "c2x16":
            ctx.set_options(_arfq.OPT_GEMV_X16)
        ms, _ = time_matmul(ctx, "q4_k", 1, 17408, 5120, args.steps, args.warmup, args.copies, 0xA7F00002)
        ctx.set_options(0)
        res = {"us_per_launch": ms * 1e3, "GB/s": algorithmic_bytes("q4_k", 1, 17408, 5120) / ms / 1e6}
    elif c == "lmhead":  # the vocab-wide Q4_K lm_head GEMV (K = 5120, N = 151936)
        ms, _ = time_matmul(ctx, "q4_k", 1, 151936, 5120, args.steps, args.warmup, 2, 0xA7F0000A)
        res = {"us_per_launch": ms * 1e3, "GB/s": algorithmic_bytes("q4_k", 1, 151936, 5120) / ms / 1e6}
    elif c == "c1n8":
        # one workgroup's worth of C1 (8 rows): the per-launch floor C1 sits on
        ms, _ = time_matmul(ctx, "q8_0", 1, 8, 2048, args.steps, args.warmup, 64, 0xA7F00001)
        res = {"us_per_launch": ms * 1e3}
    elif c == "c1":
        ms, _ = time_matmul(ctx, "q8_0", 1, 2048, 2048, args.steps, args.warmup, 64, 0xA7F00001)
        res = {"us_per_launch": ms * 1e3, "GB/s": algorithmic_bytes("q8_0", 1, 2048, 2048) / ms / 1e6}
    elif c.startswith(("q5km", "iq4m")):  # Q5_K / IQ4_XS at C2's shape, m = 1, 8, 64 or 2048
        qt, seed = ("q5_k", 0xA7F00005) if c.startswith("q5k") else ("iq4_xs", 0xA7F00006)
        mm = int(c[4:])
        xd = np.float16 if mm == 2048 else np.float32
        ms, _ = time_matmul(ctx, qt, mm, 17408, 5120, args.steps, args.warmup, 6 if mm < 2048 else 2, seed,
                            x_dtype=xd)
        res = {"us_per_launch": ms * 1e3,
               "GB/s": algorithmic_bytes(qt, mm, 17408, 5120, x_bytes=2 if mm == 2048 else 4) / ms / 1e6}
    elif c.startswith("c3"):
        if c.endswith("x16"):  # the 16-bit GEMV (m = 1) or one f16 part of x (skinny)
            ctx.set_options(_arfq.OPT_GEMV_X16)
        mm = int(c[3:].replace("x16", ""))
        ms, _ = time_matmul(ctx, "q6_k", mm, 5120, 17408, args.steps, args.warmup, 6, 0xA7F00003)
        ctx.set_options(0)
        res = {"us_per_launch": ms * 1e3, "GB/s": algorithmic_bytes("q6_k", mm, 5120, 17408) / ms / 1e6}
    elif c == "c4":
        ms, _ = time_matmul(ctx, "q4_k", 2048, 17408, 5120, args.steps, args.warmup, 2, 0xA7F00004,
                            x_dtype=np.float16)
        res = {"us_per_launch": ms * 1e3, "TFLOP/s": 2.0 * 2048 * 17408 * 5120 / ms / 1e9}
    elif c == "ffn":  # the dense Q4_K FFN of one decode step at C2's shape
        ms = time_ffn(ctx, ("q4_k", "q4_k", "q4_k"), 5120, 17408, 1, args.steps, args.warmup, 2)
        res = {"us_per_launch": ms * 1e3}
    elif c in ("moe1", "moe4", "moe16"):  # small-T MoE decode: 1, 4 or 16 tokens through C5's experts
        ms = time_moe(ctx, args.steps, args.warmup, 3, tokens=int(c[3:]))
        res = {"us_per_launch": ms * 1e3}
    else:  # c5
        ms = time_moe(ctx, args.steps, args.warmup, 3)
        res = {"us_per_launch": ms * 1e3}
    log(f"[bench] {c}: {res}")
    print(json.dumps({"only": c, "steps": args.steps, "warmup": args.warmup, **res}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--copies", type=int, default=8)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--quick", action="store_true", help="headline config only")
    ap.add_argument("--gguf-reader", action="store_true",
                    help="time the GGUF reader instead: open a synthetic model file (C5's expert "
                         "tensors, C2's matrix, a 152K-token vocabulary) and upload its tensors; "
                         "prints its own JSON line")
    ap.add_argument("--only", choices=["c1", "c2", "c2x16", "c3m1", "c3m1x16", "c3m8", "c3m32", "c3m64", "c3m64x16", "c4",
                                       "c5", "q5km1", "q5km8", "q5km64", "q5km2048", "iq4m1", "iq4m8", "iq4m64",
                                       "iq4m2048", "c1n8", "lmhead", "moe1", "moe4", "moe16", "ffn"],
                    help="time one config (for per-kernel rocprofv3 passes); prints its own JSON line")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="for rocprofv3 --pmc passes: COPY_PROBE_BYTES device copies (counter "
                         "calibration), then TRAFFIC_PROBE_LAUNCHES C2 GEMVs; prints no JSON")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked --gpus {args.gpus}); "
              "the multi-GPU sharding is design-only", file=sys.stderr)
        sys.exit(2)

    import arf_amd
    from arf_amd import synth
    ctx = arf_amd.Context(0)
    if args.traffic_probe:
        traffic_probe(ctx, args.copies, args.only or "c2")
        ctx.close()
        return
    if args.gguf_reader:
        gguf_reader_bench(ctx)
        ctx.close()
        return

    if args.only:
        only_config(ctx, args)
        ctx.close()
        return

    # ---- headline: C2 Q4_K GEMV ----
    n, k, m = 17408, 5120, 1
    log(f"[bench] C2 q4_k gemv m={m} k={k} n={n}: warmup {args.warmup}, steps {args.steps}")
    ms, total_ms = time_matmul(ctx, "q4_k", m, n, k, args.steps, args.warmup, args.copies,
                               seed=0xA7F00002)
    nbytes = algorithmic_bytes("q4_k", m, n, k)
    gbs = nbytes / (ms * 1e-3) / 1e9
    log(f"[bench] C2: {ms * 1e3:.2f} us/launch, {gbs:.1f} GB/s ({gbs / HBM_PEAK_GBS:.1%} of HBM)")
    ceiling = stream_ceiling(ctx, max(200, args.steps), args.copies)

    configs = {}
    if not args.quick:
        steps2 = max(50, args.steps // 4)
        # C2 again with ARFQ_OPT_GEMV_X16: x rounded to 16-bit fixed point per 32 elements
        # and integer v_dot8 (faster, ~1e-4 rel err): not the reference's arithmetic
        import arf_amd.arfq as _arfq
        ctx.set_options(_arfq.OPT_GEMV_X16)
        msx, _ = time_matmul(ctx, "q4_k", 1, n, k, steps2, 50, args.copies, seed=0xA7F00002)
        ctx.set_options(0)
        configs["c2_q4_k_gemv_m1_k5120_n17408_x16_option"] = {
            "us_per_launch": round(msx * 1e3, 3), "GB/s": round(nbytes / msx / 1e6, 1),
            "hbm_frac": round(nbytes / msx / 1e6 / HBM_PEAK_GBS, 4),
            "dtype": "u4xi16->i32,f32", "note": "ARFQ_OPT_GEMV_X16: x in 16-bit fixed point per "
            "32 elements (max rel err ~1e-4), integer dots; not the reference's f32 arithmetic"}
        log(f"[bench] C2 x16 option: {msx * 1e3:.2f} us/launch")
        # C1 Q8_0 GEMV
        ms1, _ = time_matmul(ctx, "q8_0", 1, 2048, 2048, steps2, 50, 64, seed=0xA7F00001)
        b1 = algorithmic_bytes("q8_0", 1, 2048, 2048)
        configs["c1_q8_0_gemv_m1_k2048_n2048"] = {
            "us_per_launch": round(ms1 * 1e3, 3), "GB/s": round(b1 / ms1 / 1e6, 1),
            "hbm_frac": round(b1 / ms1 / 1e6 / HBM_PEAK_GBS, 4), "weight_copies": 64}
        log(f"[bench] C1: {ms1 * 1e3:.2f} us/launch")
        # C3 Q6_K GEMV / skinny GEMM
        for mm in (1, 8, 32, 64):
            try:
                ms3, _ = time_matmul(ctx, "q6_k", mm, 5120, 17408, steps2, 20, 6, seed=0xA7F00003)
            except arf_amd.ArfqError as e:
                configs[f"c3_q6_k_m{mm}_k17408_n5120"] = {"error": str(e)}
                continue
            b3 = algorithmic_bytes("q6_k", mm, 5120, 17408)
            configs[f"c3_q6_k_m{mm}_k17408_n5120"] = {
                "us_per_launch": round(ms3 * 1e3, 3), "GB/s": round(b3 / ms3 / 1e6, 1),
                "hbm_frac": round(b3 / ms3 / 1e6 / HBM_PEAK_GBS, 4),
                "x": "f32" if mm == 1 else "f16 hi + mid + lo" if mm <= 8 else "f16 hi + lo"}
            log(f"[bench] C3 m={mm}: {ms3 * 1e3:.2f} us/launch")
            if mm in (32, 64):
                # the same with ARFQ_OPT_GEMV_X16: x rounded to f16 (one part), not the
                # reference's f32
                ctx.set_options(_arfq.OPT_GEMV_X16)
                msx3, _ = time_matmul(ctx, "q6_k", mm, 5120, 17408, steps2, 20, 6, seed=0xA7F00003)
                ctx.set_options(0)
                configs[f"c3_q6_k_m{mm}_k17408_n5120_x16_option"] = {
                    "us_per_launch": round(msx3 * 1e3, 3), "GB/s": round(b3 / msx3 / 1e6, 1),
                    "hbm_frac": round(b3 / msx3 / 1e6 / HBM_PEAK_GBS, 4), "x": "f16 (one part)",
                    "note": "ARFQ_OPT_GEMV_X16: x rounded to f16, not the reference's f32 arithmetic"}
                log(f"[bench] C3 m={mm} x16 option: {msx3 * 1e3:.2f} us/launch")
        # Q5_K and IQ4_XS at C2's shape: the survey's next row (no benchmark config): the
        # decode GEMV (m = 1), the skinny MFMA kernel (m = 8, 64) and, at m = 2048 (f16 x),
        # the rounded-weight prefill tile
        for qt, seed in (("q5_k", 0xA7F00005), ("iq4_xs", 0xA7F00006)):
            for mm in (1, 8, 64, 2048):
                key = f"{qt}_gemv_m1_k5120_n17408" if mm == 1 else f"{qt}_m{mm}_k5120_n17408"
                try:
                    if mm == 2048:
                        msq, _ = time_matmul(ctx, qt, mm, 17408, 5120, 10, 3, 2, seed=seed,
                                             x_dtype=np.float16)
                    else:
                        msq, _ = time_matmul(ctx, qt, mm, 17408, 5120, steps2, 50 if mm == 1 else 20,
                                             6, seed=seed)
                except arf_amd.ArfqError as e:
                    configs[key] = {"error": str(e)}
                    continue
                bq = algorithmic_bytes(qt, mm, 17408, 5120, x_bytes=2 if mm == 2048 else 4)
                configs[key] = {"us_per_launch": round(msq * 1e3, 3), "GB/s": round(bq / msq / 1e6, 1),
                                "hbm_frac": round(bq / msq / 1e6 / HBM_PEAK_GBS, 4)}
                if mm == 2048:
                    tq = 2.0 * mm * 17408 * 5120 / (msq * 1e-3) / 1e12
                    configs[key].update({"TFLOP/s": round(tq, 1), "mfma_frac": round(tq / FP16_MFMA_PEAK_TFLOPS, 4),
                                         "x": "f16", "launches": (mm + 63) // 64})
                log(f"[bench] {qt} m={mm} (C2 shape): {msq * 1e3:.2f} us/launch")
        # C4 Q4_K prefill GEMM
        try:
            ms4, _ = time_matmul(ctx, "q4_k", 2048, 17408, 5120, 30, 10, 2, seed=0xA7F00004,
                                 x_dtype=np.float16)
            fl = 2.0 * 2048 * 17408 * 5120
            tf = fl / (ms4 * 1e-3) / 1e12
            configs["c4_q4_k_gemm_m2048_k5120_n17408"] = {
                "us_per_launch": round(ms4 * 1e3, 1), "TFLOP/s": round(tf, 1),
                "mfma_frac": round(tf / FP16_MFMA_PEAK_TFLOPS, 4)}
            log(f"[bench] C4: {ms4 * 1e3:.1f} us/launch, {tf:.1f} TFLOP/s")
        except arf_amd.ArfqError as e:
            configs["c4_q4_k_gemm_m2048_k5120_n17408"] = {"error": str(e)}
        # C5 MoE block
        try:
            # steady state: the first few dozen calls after the C4 phase run ~10 % slower
            ms5 = time_moe(ctx, 60, 30, 3)
            cfg = synth.CONFIGS["c5_moe"]
            E, T, topk, hdim, inter = (cfg["experts"], cfg["tokens"], cfg["top_k"], cfg["hidden"],
                                       cfg["inter"])
            wbytes = 3 * E * inter * hdim // 256 * 144
            b5 = wbytes + T * hdim * 2 + T * E * 4 + T * hdim * 4
            fl5 = 2.0 * T * topk * 3 * inter * hdim
            configs["c5_moe_q4_k_e128_top8_t512_h2048_i768"] = {
                "us_per_launch": round(ms5 * 1e3, 1), "GB/s": round(b5 / ms5 / 1e6, 1),
                "hbm_frac": round(b5 / ms5 / 1e6 / HBM_PEAK_GBS, 4),
                "TFLOP/s": round(fl5 / (ms5 * 1e-3) / 1e12, 1), "weight_copies": 3}
            log(f"[bench] C5: {ms5 * 1e3:.1f} us/launch")
        except arf_amd.ArfqError as e:
            configs["c5_moe_q4_k_e128_top8_t512_h2048_i768"] = {"error": str(e)}
        # the survey's next rows, on the kernels above: small-T MoE decode (C5's experts at
        # T = 1, 4, 16: bytes = the distinct experts' weights the routing touches, at most
        # T * top_k) and a vocab-wide lm_head GEMV (Q6_K, N = 151936, K = 5120)
        cfg = synth.CONFIGS["c5_moe"]
        per_expert = 3 * cfg["inter"] * cfg["hidden"] // 256 * 144
        for T in (1, 4, 16):
            try:
                msT = time_moe(ctx, 200, 50, 3, tokens=T)
                ids = set()
                lg = synth.router_logits(T, cfg["experts"], seed=0xA7F00009)
                for t in range(T):
                    ids.update(np.argsort(-lg[t], kind="stable")[:cfg["top_k"]].tolist())
                bT = len(ids) * per_expert
                configs[f"moe_decode_q4_k_e128_top8_t{T}"] = {
                    "us_per_launch": round(msT * 1e3, 2), "experts_touched": len(ids),
                    "GB/s": round(bT / msT / 1e6, 1), "hbm_frac": round(bT / msT / 1e6 / HBM_PEAK_GBS, 4)}
                log(f"[bench] MoE T={T}: {msT * 1e3:.1f} us/launch ({len(ids)} experts)")
            except arf_amd.ArfqError as e:
                configs[f"moe_decode_q4_k_e128_top8_t{T}"] = {"error": str(e)}
        for qv in ("q4_k", "q6_k"):
            try:
                msv, _ = time_matmul(ctx, qv, 1, 151936, 5120, 200, 20, 2, seed=0xA7F0000A)
                bv = algorithmic_bytes(qv, 1, 151936, 5120)
                configs[f"lm_head_{qv}_gemv_m1_k5120_n151936"] = {
                    "us_per_launch": round(msv * 1e3, 2), "GB/s": round(bv / msv / 1e6, 1),
                    "hbm_frac": round(bv / msv / 1e6 / HBM_PEAK_GBS, 4)}
                log(f"[bench] lm_head {qv} m=1 n=151936: {msv * 1e3:.1f} us/launch")
            except arf_amd.ArfqError as e:
                configs[f"lm_head_{qv}_gemv_m1_k5120_n151936"] = {"error": str(e)}
        # the dense FFN (gate / up / SwiGLU / down) of one decode step at C2's shape
        for qts, tag in ((("q4_k", "q4_k", "q4_k"), "q4_k"), (("q4_k", "q4_k", "q6_k"), "q4_k_down_q6_k")):
            try:
                msf = time_ffn(ctx, qts, 5120, 17408, 1, 300, 30, 2)
                bf = sum(algorithmic_bytes(q, 1, n_, k_) for q, (n_, k_) in
                         zip(qts, [(17408, 5120), (17408, 5120), (5120, 17408)]))
                configs[f"ffn_{tag}_m1_h5120_i17408"] = {
                    "us_per_launch": round(msf * 1e3, 2), "GB/s": round(bf / msf / 1e6, 1),
                    "hbm_frac": round(bf / msf / 1e6 / HBM_PEAK_GBS, 4)}
                log(f"[bench] FFN {tag} m=1: {msf * 1e3:.1f} us/launch")
            except arf_amd.ArfqError as e:
                configs[f"ffn_{tag}_m1_h5120_i17408"] = {"error": str(e)}

    cpu = None
    if not args.no_cpu:
        log(f"[bench] cpu baselines (~{2 * args.cpu_seconds:.0f} s)")
        cpus = cpu_baselines(args.cpu_seconds)
        cpu = cpus.pop("c2")
        log(f"[bench] cpu C2: {cpu['value']} GB/s")
        keys = {"c1": "c1_q8_0_gemv_m1_k2048_n2048", "c4": "c4_q4_k_gemm_m2048_k5120_n17408",
                "c5": "c5_moe_q4_k_e128_top8_t512_h2048_i768"}
        keys.update({f"c3_m{mm}": f"c3_q6_k_m{mm}_k17408_n5120" for mm in (1, 8, 32, 64)})
        for ck, v in cpus.items():
            configs.setdefault(keys[ck], {})["cpu_baseline"] = v

    ctx.close()
    out = {
        "metric": "Q4_K GEMV weight GB/s (% of HBM peak); prefill GEMM TFLOP/s (% MFMA)",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded Q4_K superblocks per BASELINE config 2, x ~ N(0,1) f32)",
        "config": {"workload": "c2_q4_k_gemv_m1_k5120_n17408", "m": m, "k": k, "n": n,
                   "weight_copies": args.copies, "parallelism": "single-gpu",
                   "compute": "f32 x times the exact 4-bit codes (v_fma_mix_f32 on f16-subnormal "
                              "nibbles), f32 sums per 32-weight sub-block, then (d*sc)*code_sum - "
                              "(dmin*m)*x_sum in f32, as matmul_nt_q4ks"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": load_traffic("q4k_gemv_c2_traffic.json", "gemv_q4k_f32"),
                     "stream_gbs": ceiling["stream_gbs"], "stream_c2_gbs": ceiling["stream_c2_gbs"],
                     "frac_of_stream_c2": round(gbs / ceiling["stream_c2_gbs"], 4),
                     "clock_mhz": ceiling["clock_mhz"], "clock_peak_mhz": ceiling["clock_peak_mhz"],
                     "stream_note": "stream_gbs: a plain read-only kernel over 512 MB; stream_c2_gbs: the "
                                    "same kernel over C2's 50,135,040 weight bytes, rotating the same number "
                                    "of buffers back to back like the GEMV loop (launch gaps included); "
                                    "clock_mhz: shader clock during the 512 MB pass (s_memtime vs "
                                    "s_memrealtime)"},
        "cpu_baseline": cpu,
        "configs": configs,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
