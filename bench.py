"""Benchmark of the MI355X MXFP4 decode engine (one JSON line on stdout).

Workload: Llama-3-8B architecture, random-init MXFP4
weights (E2M1 + E8M0 per 32), batch 1, fp16 KV cache pre-filled to 4096
tokens, greedy decode.  A "step" is one token through all 32 layers and the
LM head.  `value` = decode tokens/s with weights and KV resident in HBM.

Extra fields: the roofline of the dominant kernel (the fused gate/up SwiGLU
GEMV), from its duration inside the decode step (every kernel of two more
steps timed by its own dispatch events, llama_engine_time_steps) and alone
(HIP events around a loop of its launches); the per-kernel table of the step;
the whole GEMV path of one token replayed alone; TinyLlama-1.1B decode tok/s
(config 3); the reference's own llama_decode harness (Llama-3.2-1B shape,
f32 scales, f32 K/V, context 512); the batched MXFP4 GEMM at M=32 and M=512
on the 8B shapes (config 5, TFLOP/s against the FP4 MFMA peak); the 8B
batched prefill; and the CPU oracle timed on the host cores (cpu_baseline,
one thread and all cores, a reported baseline only).

Profiling modes (no JSON line): `--pmc-probe decode|gemm` runs only the launch
sequence of a counter pass; `--summarize-trace DIR` and `--summarize-pmc DIR
...` turn rocprofv3 CSV output into the summaries kept under profiles/.
Regions are marked with ROCTx ranges (seen by rocprofv3 --marker-trace).
"""
import argparse
import ctypes
import csv
import glob
import json
import os
import sys
import time
from contextlib import contextmanager

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "rust-fp4-blackwell_amd"))

METRIC = "MXFP4 decode tok/s @bs1 (1.1B & 8B shapes) + GEMV HBM GB/s vs peak"
HBM_PEAK_GBS = 8000.0
SEED = 0x8B8B
KV_SEED = 0x4B56
PREFILL = 4096


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class _Roctx:
    """ROCTx ranges (rocprofv3 --marker-trace) around bench regions; no-ops
    when the library is absent."""

    def __init__(self):
        self.lib = None
        for name in ("librocprofiler-sdk-roctx.so.1", "libroctx64.so.4", "libroctx64.so"):
            for d in ("", "/opt/rocm/lib/"):
                try:
                    self.lib = ctypes.CDLL(d + name)
                    self.lib.roctxRangePushA.argtypes = [ctypes.c_char_p]
                    return
                except (OSError, AttributeError):
                    self.lib = None

    @contextmanager
    def range(self, name):
        if self.lib:
            self.lib.roctxRangePushA(name.encode())
        try:
            yield
        finally:
            if self.lib:
                self.lib.roctxRangePop()


ROCTX = _Roctx()


def gemv_bytes(n, k):
    """Algorithmic bytes of one MXFP4 GEMV: codes + E8M0 scales + x + y."""
    return n * k // 2 + n * k // 32 + 4 * k + 4 * n


def time_launches(rf, stream, fn, reps):
    e0, e1 = rf.Event(), rf.Event()
    fn()  # warm
    stream.synchronize()
    e0.record(stream)
    for _ in range(reps):
        fn()
    e1.record(stream)
    e1.synchronize()
    return e0.elapsed_ms(e1) / reps


def gemv_path(rf, eng, cfg, reps=5):
    """Every GEMV launch of one 8B token, alone, on the engine stream."""
    s = eng.stream
    qd, kvd = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim
    kmax = max(cfg.dim, cfg.ffn, qd)
    rng = np.random.default_rng(0)
    x = rf.DeviceBuffer.from_host(rng.standard_normal(kmax).astype(np.float32), s)
    y = rf.DeviceBuffer.zeroed(max(cfg.vocab, 2 * cfg.ffn), np.float32, s)
    calls, total_bytes = [], 0
    for l in range(cfg.n_layers):
        qc, qs, _, _ = eng.weight(l, 0)
        oc, os_, _, _ = eng.weight(l, 3)
        gc, gs, _, _ = eng.weight(l, 4)
        dc, ds, _, _ = eng.weight(l, 6)
        calls.append(lambda qc=qc, qs=qs: rf.mx4_gemv(s, qd + 2 * kvd, cfg.dim, qc, qs, x, y))
        calls.append(lambda oc=oc, os_=os_: rf.mx4_gemv_residual(s, cfg.dim, qd, oc, os_, x, y))
        calls.append(lambda gc=gc, gs=gs: rf.mx4_gemv_swiglu(s, cfg.ffn, cfg.dim, cfg.ffn, gc, gs, x, y))
        calls.append(lambda dc=dc, ds=ds: rf.mx4_gemv_residual(s, cfg.dim, cfg.ffn, dc, ds, x, y))
        total_bytes += gemv_bytes(qd + 2 * kvd, cfg.dim) + gemv_bytes(cfg.dim, qd) + \
            gemv_bytes(2 * cfg.ffn, cfg.dim) + gemv_bytes(cfg.dim, cfg.ffn)
    lc, ls, _, _ = eng.weight(-1, 0)
    calls.append(lambda: rf.mx4_gemv(s, cfg.vocab, cfg.dim, lc, ls, x, y))
    total_bytes += gemv_bytes(cfg.vocab, cfg.dim)
    ms = time_launches(rf, s, lambda: [c() for c in calls], reps)
    # dominant kernel: the fused gate/up SwiGLU GEMV, one launch per layer,
    # alone as the step launches it (with its fused RMSNorm, fp16 weights ~1)
    # and without the norm
    nw = rf.DeviceBuffer.from_host((1 + 0.02 * rng.standard_normal(cfg.dim)).astype(np.float16).view(np.uint16), s)
    L = rf.load()
    gate_norm = []
    for l in range(cfg.n_layers):
        gc, gs, _, _ = eng.weight(l, 4)
        gate_norm.append(lambda gc=gc, gs=gs: rf.check(L.rfp4_debug_gemv_fused(
            s.h, rf.EPI_SWIGLU, rf.SCALE_E8M0, cfg.ffn, cfg.dim, cfg.ffn, gc, gs, x.ptr, nw.ptr, rf.F32(cfg.eps),
            y.ptr, None, None)))
    ms_gate = time_launches(rf, s, lambda: [c() for c in gate_norm], reps) / cfg.n_layers
    gate = [calls[4 * l + 2] for l in range(cfg.n_layers)]
    ms_gate_plain = time_launches(rf, s, lambda: [c() for c in gate], reps) / cfg.n_layers
    gate_bytes = gemv_bytes(2 * cfg.ffn, cfg.dim) - 4 * cfg.ffn  # y holds ffn outputs, not 2*ffn
    return total_bytes, ms, gate_bytes, ms_gate, ms_gate_plain


FP4_PEAK_TFLOPS = 10100.0


def _bf16_normal(rng, rows, k):
    u = rng.standard_normal((rows, k), dtype=np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def gemm_config5(rf, eng, cfg, reps=2, m_list=(32, 512), stack=True):
    """MXFP4 GEMMs at M=32 (decode batch) and M=512 (prefill)
    on the engine's own Llama-3-8B weights, bf16 activations ~N(0,1) quantized
    per 32 along K (mx4_quantize).  Per config-5 shape, each launch uses a
    different layer's weights (no cache reuse across launches); the stack pass
    is every projection of the 32 layers plus the LM head.  reps = 0: each
    shape launched once, untimed (the counter probe)."""
    s = eng.stream
    qd, kvd = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim
    rng = np.random.default_rng(5)
    acts = {}
    for k in sorted({cfg.dim, qd, cfg.ffn}):
        a16 = rf.DeviceBuffer.from_host(_bf16_normal(rng, 512, k), s)
        ac, asc = rf.DeviceBuffer(512 * k // 2), rf.DeviceBuffer(512 * k // 32)
        ast = rf.DeviceBuffer(rf.mx4_scales_tiled_bytes(512, k))
        rf.mx4_quantize_tiled(s, 512, k, a16, True, ac, asc, ast)
        acts[k] = (a16, ac, asc, ast)
    c = rf.DeviceBuffer(512 * max(cfg.vocab, 2 * cfg.ffn) * 4)
    L = cfg.n_layers
    # weight views (codes, row-major scales, step-blocked scales) of projection p of every layer
    wv = lambda l, p: (*eng.weight(l, p)[:2], eng.weight_scales_tiled(l, p)[0])
    w = {p: [wv(l, p) for l in range(L)] for p in (0, 1, 3, 4, 6)}
    lm = wv(-1, 0)
    # config-5 shapes: (name, N, K, weight views rotating over layers)
    shapes = [
        ("4096x4096", cfg.dim, qd, w[3]),
        ("1024x4096", kvd, cfg.dim, w[1]),
        ("14336x4096", cfg.ffn, cfg.dim, w[4]),
        ("4096x14336", cfg.dim, cfg.ffn, w[6]),
        ("128256x4096", cfg.vocab, cfg.dim, [lm]),
    ]
    # the stack's q|k|v and gate|up are the stacked matrices: views of projections 0 and 4 widened
    layers = [(qd + 2 * kvd, cfg.dim, w[0]), (cfg.dim, qd, w[3]), (2 * cfg.ffn, cfg.dim, w[4]),
              (cfg.dim, cfg.ffn, w[6])]
    gemm = lambda m, n, k, a, wc, ws, wst: rf.fp4_gemm_tiled(s, m, n, k, a[1], a[2], a[3], wc, ws, wst, c)
    out = {}
    for m in m_list:
        res = {}
        for name, n, k, views in shapes:
            a = acts[k]
            nl = len(views)
            calls = [lambda wc=wc, ws=ws, wst=wst: gemm(m, n, k, a, wc, ws, wst) for wc, ws, wst in views]
            if reps == 0:
                with ROCTX.range(f"gemm_m{m}_{name}"):
                    calls[0]()
                    s.synchronize()
                res[name] = {}
                continue
            with ROCTX.range(f"gemm_m{m}_{name}"):
                ms = time_launches(rf, s, lambda: [f() for f in calls], reps) / nl
            tf = 2.0 * m * n * k / (ms * 1e-3) / 1e12
            gbs = (n * k * 17 // 32 + m * k * 17 // 32 + 4 * m * n) / (ms * 1e-3) / 1e9
            tm, tn, kz = rf.gemm_plan(m, n, k)
            res[name] = {"us": round(ms * 1e3, 2), "TFLOP_s": round(tf, 1), "frac_fp4_peak": round(tf / FP4_PEAK_TFLOPS, 4),
                         "GB_s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "tile": f"{tm}x{tn}/kz{kz}",
                         "kernel": rf.gemm_plan_kernel(m, n, k)}
        if not stack:
            out[f"m{m}"] = {"shapes": res}
            continue
        flops = 0.0
        calls, dropin = [], []
        for l in range(L):
            for n, k, views in layers:
                a = acts[k]
                wc, ws, wst = views[l]
                calls.append(lambda n=n, k=k, a=a, wc=wc, ws=ws, wst=wst: gemm(m, n, k, a, wc, ws, wst))
                dropin.append(lambda n=n, k=k, a=a, wc=wc, ws=ws: rf.fp4_gemm(s, m, n, k, a[1], a[2], wc, ws, c))
                flops += 2.0 * m * n * k
        calls.append(lambda: gemm(m, cfg.vocab, cfg.dim, acts[cfg.dim], *lm))
        dropin.append(lambda: rf.fp4_gemm(s, m, cfg.vocab, cfg.dim, acts[cfg.dim][1], acts[cfg.dim][2], lm[0], lm[1], c))
        flops += 2.0 * m * cfg.vocab * cfg.dim
        ms = time_launches(rf, s, lambda: [f() for f in calls], reps)
        tf = flops / (ms * 1e-3) / 1e12
        # the drop-in fp4_gemm (row-major scales only: the tiled kernels' step-blocked copies made per call)
        ms_dropin = time_launches(rf, s, lambda: [f() for f in dropin], reps) if m > 32 else ms
        qms = time_launches(rf, s, lambda: rf.mx4_quantize(s, m, cfg.dim, acts[cfg.dim][0], True, acts[cfg.dim][1],
                                                           acts[cfg.dim][2]), 20)
        out[f"m{m}"] = {"stack_us": round(ms * 1e3, 1), "stack_TFLOP": round(flops / 1e12, 4),
                        "stack_TFLOP_s": round(tf, 1), "stack_frac_fp4_peak": round(tf / FP4_PEAK_TFLOPS, 4),
                        "stack_us_dropin_fp4_gemm": round(ms_dropin * 1e3, 1),
                        "quantize_us_k4096": round(qms * 1e3, 2), "shapes": res}
        log(f"gemm M={m}: stack {ms * 1e3:.0f} us, {tf:.0f} TFLOP/s ({100 * tf / FP4_PEAK_TFLOPS:.1f}% of FP4 peak); "
            + ", ".join(f"{k} {v['us']}us {v['TFLOP_s']}TF" for k, v in res.items()))
    for a16, ac, asc, ast in acts.values():
        a16.free(), ac.free(), asc.free(), ast.free()
    c.free()
    out["workload"] = ("Llama-3-8B projections as MXFP4 GEMMs, bf16 activations ~N(0,1) quantized to MXFP4 per 32 "
                       "along K; stack = 32 layers x (qkv, o, gate+up, down) + LM head; fp4_gemm_tiled with the "
                       "engine's step-blocked weight scales (stack_us_dropin_fp4_gemm: fp4_gemm, which makes them "
                       "per call)")
    out["peak_TFLOP_s"] = FP4_PEAK_TFLOPS
    return out


COPY_FLOATS = 64 << 20  # calibration copy: 256 MiB read + 256 MiB written per launch


def _copy_calibration(rf, s):
    src = rf.DeviceBuffer.zeroed(COPY_FLOATS, np.float32, s)
    dst = rf.DeviceBuffer.zeroed(COPY_FLOATS, np.float32, s)
    for _ in range(4):
        rf.copy_into(s, COPY_FLOATS, 0, src, dst)
    s.synchronize()
    src.free(), dst.free()


def pmc_probe(rf, which):
    """Fixed launch sequences for the counter passes (rocprofv3 --pmc, one
    counter set per run), each followed by a plain f32 copy of COPY_FLOATS
    floats four times, whose known bytes scale FETCH_SIZE / WRITE_SIZE.
    decode: two decode steps of the 8B model at context 4096, launched one
    kernel at a time (every kernel of the step); gemm: each config-5 MXFP4
    GEMM shape once at M = 512."""
    cfg = rf.model_config("llama3-8b", max_seq=PREFILL + 16)
    eng = rf.Engine(cfg, SEED)
    s = eng.stream
    if which == "decode":
        eng.prefill_kv(KV_SEED, PREFILL)
        eng.use_graph(False)
        eng.begin([1], PREFILL, 4)
        eng.run_steps(2)
        s.synchronize()
        done = {"decode_steps": 2, "context": PREFILL}
    else:
        res = gemm_config5(rf, eng, cfg, reps=0, m_list=(512,), stack=False)
        done = {"gemm_shapes": list(res["m512"]["shapes"])}
    _copy_calibration(rf, s)
    eng.close()
    print(json.dumps({"pmc_probe": which, **done, "copy_launches": 4, "copy_read_bytes": 4 * COPY_FLOATS,
                      "copy_write_bytes": 4 * COPY_FLOATS}), flush=True)


def trace_tiny_eager(rf, steps=64):
    """The TinyLlama-1.1B decode launched kernel by kernel (no step graph) for
    a rocprofv3 kernel trace: a 16-token prompt then `steps` greedy steps in
    the ROCTx range tinyllama_decode_eager.  (Tracing the graph replays of
    this model aborted inside the runtime's graph launch under the profiler;
    the untraced graph replays of the same path pass.)"""
    cfg = rf.model_config("tinyllama-1.1b", max_seq=16 + steps + 8)
    eng = rf.Engine(cfg, SEED)
    eng.use_graph(False)
    prompt = np.random.default_rng(16).integers(0, cfg.vocab, 16).astype(np.uint32)
    eng.begin(prompt, 0, 16 + steps + 1)
    eng.run_steps(15)
    eng.stream.synchronize()
    with ROCTX.range("tinyllama_decode_eager"):
        eng.run_steps(steps)
        eng.stream.synchronize()
    ids = eng.read_ids(16 + steps)
    eng.close()
    print(json.dumps({"trace_probe": "tinyllama_decode_eager", "steps": steps, "last_token": int(ids[-1])}), flush=True)


TRAFFIC_JSON = os.path.join(ROOT, "profiles", "decode_llama3-8b_traffic.json")


def load_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed counter summary
    (two --pmc passes over `--pmc-probe decode`, scaled by the copy), or None."""
    if not os.path.exists(TRAFFIC_JSON):
        return None
    with open(TRAFFIC_JSON) as f:
        k = json.load(f).get("kernels", {}).get(kernel)
    return k.get("traffic_bytes") if k else None


# ---------------------------------------------------------------- profile summaries
def _rows(path):
    with open(path, newline="") as f:
        return list(csv.DictReader(f))


def _find(dirs, suffix):
    out = []
    for d in dirs:
        out += sorted(glob.glob(os.path.join(d, "**", "*" + suffix), recursive=True))
    return out


def summarize_trace(dirs):
    """Per-kernel duration statistics of rocprofv3 --kernel-trace CSV output,
    one table per ROCTx range of this script (--marker-trace), or one table
    over every dispatch if no marker file is present."""
    kern = []
    for p in _find(dirs, "kernel_trace.csv"):
        for r in _rows(p):
            kern.append((r["Kernel_Name"], int(r["Start_Timestamp"]), int(r["End_Timestamp"])))
    if not kern:
        sys.exit("no *kernel_trace.csv under " + " ".join(dirs))
    ranges = []
    for p in _find(dirs, "marker_api_trace.csv"):
        for r in _rows(p):
            name = next((r[c] for c in ("Message", "Function", "Name", "Operation") if r.get(c)), None)
            if name and r.get("Start_Timestamp") and r.get("End_Timestamp"):
                ranges.append((name, int(r["Start_Timestamp"]), int(r["End_Timestamp"])))
    if not ranges:
        ranges = [("all dispatches", min(k[1] for k in kern), max(k[2] for k in kern))]
    lines = []
    for name, t0, t1 in sorted(ranges, key=lambda x: x[1]):
        sel = [k for k in kern if t0 <= k[1] <= t1]
        if not sel:
            continue
        stats = {}
        for kn, a, b in sel:
            stats.setdefault(kn, []).append((b - a) / 1e3)
        total = sum(sum(v) for v in stats.values())
        lines.append(f"range {name}: {len(sel)} dispatches, {total / 1e3:.3f} ms of kernel time, "
                     f"{(t1 - t0) / 1e6:.3f} ms wall")
        lines.append(f"{'kernel':48s} {'calls':>6s} {'avg_us':>8s} {'min_us':>8s} {'max_us':>8s} {'total_ms':>9s} {'pct':>6s}")
        for kn, v in sorted(stats.items(), key=lambda kv: -sum(kv[1])):
            lines.append(f"{kn:48s} {len(v):6d} {np.mean(v):8.2f} {min(v):8.2f} {max(v):8.2f} {sum(v) / 1e3:9.3f} "
                         f"{100 * sum(v) / total:6.2f}")
        lines.append("")
    print("\n".join(lines))


def summarize_pmc(dirs):
    """Per-kernel averages of rocprofv3 --pmc counter passes (one directory
    per pass).  FETCH_SIZE and WRITE_SIZE (KiB) are scaled by what they read
    for the calibration copy (rfp4_copy_into_f32: 4*COPY_FLOATS bytes read and
    written per launch); writes profiles/decode_llama3-8b_traffic.json-style
    JSON to stdout after the table when both counters are present."""
    vals = {}
    for p in _find(dirs, "counter_collection.csv"):
        for r in _rows(p):
            key = (r["Kernel_Name"], r["Counter_Name"])
            vals.setdefault(key, {})[(p, r["Dispatch_Id"])] = float(r["Counter_Value"])
    if not vals:
        sys.exit("no *counter_collection.csv under " + " ".join(dirs))
    avg = {k: (float(np.mean(list(v.values()))), len(v)) for k, v in vals.items()}
    counters = sorted({c for _, c in avg})
    kernels = sorted({k for k, _ in avg})
    scale = {}
    for c in ("FETCH_SIZE", "WRITE_SIZE"):
        cal = avg.get(("rfp4_copy_into_f32", c))
        if cal and cal[0] > 0:
            scale[c] = 4.0 * COPY_FLOATS / (cal[0] * 1024.0)
    print(f"{'kernel':48s} {'calls':>6s} " + " ".join(f"{c:>22s}" for c in counters))
    for k in kernels:
        n = max(avg[(k, c)][1] for c in counters if (k, c) in avg)
        print(f"{k:48s} {n:6d} " + " ".join(f"{avg[(k, c)][0]:22.1f}" if (k, c) in avg else f"{'-':>22s}"
                                             for c in counters))
    if scale:
        print("\nscale (true bytes / counter bytes, from the copy): " +
              ", ".join(f"{c} {v:.3f}" for c, v in scale.items()))
    if len(scale) == 2:
        out = {"scale": scale, "kernels": {}}
        for k in kernels:
            if (k, "FETCH_SIZE") in avg and (k, "WRITE_SIZE") in avg:
                fb = avg[(k, "FETCH_SIZE")][0] * 1024.0 * scale["FETCH_SIZE"]
                wb = avg[(k, "WRITE_SIZE")][0] * 1024.0 * scale["WRITE_SIZE"]
                out["kernels"][k] = {"fetch_bytes": round(fb), "write_bytes": round(wb), "traffic_bytes": round(fb + wb)}
        print(json.dumps(out))


def decode_run(rf, preset, max_seq, prefill, prompt, warmup, steps):
    cfg = rf.model_config(preset, max_seq=max_seq)
    eng = rf.Engine(cfg, SEED)
    if prefill:
        eng.prefill_kv(KV_SEED, prefill)
    n_prompt = len(prompt)
    eng.begin(prompt, prefill, n_prompt + warmup + steps + TIMED_STEPS + 1)
    eng.run_steps(n_prompt - 1 + warmup)
    eng.stream.synchronize()
    e0, e1 = rf.Event(), rf.Event()
    t0 = time.perf_counter()
    with ROCTX.range(f"{preset}_decode_timed"):
        e0.record(eng.stream)
        eng.run_steps(steps)
        e1.record(eng.stream)
        e1.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_ms(e1)
    ids = eng.read_ids(n_prompt + warmup + steps)
    assert np.all(ids < cfg.vocab)
    return eng, cfg, ms, wall, ids


TIMED_STEPS = 2  # steps whose kernels are timed one by one after the timed region


def persistent_run(rf, eng, steps=32, warmup=2):
    """The same 8B decode with every layer of a step in one cooperative launch
    (llama_engine_use_persistent; off by default): the KV cache refilled to
    PREFILL, `steps` steps timed with stream events, tokens compared with the
    graph step's run from the same state."""
    if not eng.persistent_available:
        return None
    out = {}
    for mode in (True, False):
        eng.use_persistent(mode)
        eng.prefill_kv(KV_SEED, PREFILL)
        eng.begin([1], PREFILL, 1 + warmup + steps + 1)
        eng.run_steps(warmup)
        e0, e1 = rf.Event(), rf.Event()
        e0.record(eng.stream)
        eng.run_steps(steps)
        e1.record(eng.stream)
        e1.synchronize()
        out[mode] = (e0.elapsed_ms(e1), eng.read_ids(1 + warmup + steps))
    eng.use_persistent(False)
    ms = out[True][0]
    return {"tok_s": round(steps / (ms / 1e3), 1), "ms_per_token": round(ms / steps, 4),
            "graph_tok_s_same_run": round(steps / (out[False][0] / 1e3), 1),
            "tokens_identical_to_graph": bool(np.array_equal(out[True][1], out[False][1])),
            "workload": f"Llama-3-8B decode at ctx {PREFILL}, {steps} steps, all layers of a step in one cooperative "
                        "launch (grid barriers between stages), opt-in"}


def step_kernels(eng, preset):
    """Every kernel of TIMED_STEPS more decode steps, each timed by its own
    dispatch events (llama_engine_time_steps): {name: [calls per step, avg us]}."""
    with ROCTX.range(f"{preset}_step_kernels"):
        rec = eng.time_steps(TIMED_STEPS)
    out = {}
    for name, us in rec:
        out.setdefault(name, []).append(us)
    return {k: [len(v) / TIMED_STEPS, round(float(np.mean(v)), 3)] for k, v in out.items()}



def prefill_run(rf, eng, cfg, n=512, reps=3):
    """Batched prefill of n random tokens at position 0 through the MXFP4 GEMM
    (llama_engine_prefill): every projection an M=n GEMM, causal attention
    rows, then the last row's LM head.  GPU time from stream events."""
    prompt = np.random.default_rng(512).integers(0, cfg.vocab, n).astype(np.uint32)
    tok = eng.prefill(prompt, 0)  # warm: workspace allocation, code objects
    e0, e1 = rf.Event(), rf.Event()
    best = None
    for _ in range(reps):
        e0.record(eng.stream)
        t = eng.prefill(prompt, 0)
        e1.record(eng.stream)
        e1.synchronize()
        ms = e0.elapsed_ms(e1)
        best = ms if best is None else min(best, ms)
        assert t == tok
    qd, kvd = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim
    per_layer = (qd + 2 * kvd) * cfg.dim + cfg.dim * qd + 2 * cfg.ffn * cfg.dim + cfg.dim * cfg.ffn
    flops = 2.0 * n * per_layer * cfg.n_layers
    return {"tokens": n, "ms": round(best, 3), "tok_s": round(n / (best / 1e3), 1),
            "projection_TFLOP": round(flops / 1e12, 3), "TFLOP_s": round(flops / (best / 1e3) / 1e12, 1),
            "frac_fp4_peak": round(flops / (best / 1e3) / 1e12 / FP4_PEAK_TFLOPS, 4),
            "workload": f"Llama-3-8B arch, {n} random tokens at position 0 through llama_engine_prefill "
                        "(MXFP4 activations per 32), best of %d" % reps}


def cpu_model():
    """The host CPU's model name (what lscpu prints as "Model name")."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(threads, steps, steps_one):
    """The oracle decode loop (oracle/, C, f32, k-order) on the host cores:
    config-4 model, context pre-filled to 4096; `steps` decode steps timed on
    `threads` threads, then `steps_one` more on one thread (the reference's
    CPU loops are serial).  Row-partitioned threads: same tokens either way."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle

    pyoracle.set_threads(threads)
    cfg = dict(dim=4096, n_layers=32, n_heads=32, n_kv_heads=8, head_dim=128, ffn=14336, vocab=128256,
               theta=500000.0, eps=1e-5, max_seq=PREFILL + steps + steps_one + 2)
    t0 = time.perf_counter()
    m = pyoracle.Model(cfg, SEED)
    m.prefill_kv(KV_SEED, PREFILL)
    t_setup = time.perf_counter() - t0
    tok = 1
    t0 = time.perf_counter()
    for i in range(steps):
        tok = m.step(tok, PREFILL + i)
    dt = time.perf_counter() - t0
    pyoracle.set_threads(1)
    t0 = time.perf_counter()
    for i in range(steps_one):
        tok = m.step(tok, PREFILL + steps + i)
    dt1 = time.perf_counter() - t0
    m.close()
    return steps / dt, dt, steps_one / dt1, dt1, t_setup


def _timed(fn, min_s=0.25, max_reps=64):
    """Seconds per call of fn: repeated until min_s has passed (at least once)."""
    fn()
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        dt = time.perf_counter() - t0
        if dt >= min_s or n >= max_reps:
            return dt / n


def cpu_legs(threads, tiny_steps=256, tiny_steps_one=4, tiny_gpu_ids=None):
    """The rest of the CPU baseline, on the same host cores:
    - GEMV (the reference's k-order loop, fp4_gemv/src/main.rs:130-143, E8M0
      scales) at config 1 and the Llama-3-8B per-layer shapes: GB/s of the
      algorithmic bytes, on `threads` threads and on one;
    - the batched GEMM's closed form (trackb/fp4_scale_test.cu:37 over M x N x K,
      float64 accumulation: the oracle's checker) at M = 32, GFLOP/s;
    - TinyLlama-1.1B decode (config 3): the bench's 16-token prompt fed token by
      token, then `tiny_steps` greedy steps timed on `threads` threads and
      `tiny_steps_one` more on one (llama_run/src/main.rs:492-536); the tokens
      are compared with the GPU run's when given."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle

    out = {}
    rng = np.random.default_rng(0xC0)
    gemv = {}
    for name, n, k in (("config1_2048x2048", 2048, 2048), ("8b_qkv_6144x4096", 6144, 4096),
                       ("8b_o_4096x4096", 4096, 4096), ("8b_gate_up_28672x4096", 28672, 4096),
                       ("8b_down_4096x14336", 4096, 14336)):
        codes = rng.integers(0, 256, n * k // 2, dtype=np.uint8)
        scales = rng.integers(121, 130, n * k // 32, dtype=np.uint8)  # 2^-6 .. 2^2, config 1's range
        x = rng.standard_normal(k).astype(np.float32)
        row = {"bytes": gemv_bytes(n, k)}
        for th, key in ((threads, "all"), (1, "one_thread")):
            pyoracle.set_threads(th)
            sec = _timed(lambda: pyoracle.gemv_e8m0(n, k, codes, scales, x), min_s=0.2)
            row[key] = {"ms": round(sec * 1e3, 3), "GB_s": round(gemv_bytes(n, k) / sec / 1e9, 2)}
        gemv[name] = row
    out["gemv"] = gemv
    m, n, k = 32, 4096, 4096
    ac = rng.integers(0, 256, m * k // 2, dtype=np.uint8)
    asc = rng.integers(121, 130, m * k // 32, dtype=np.uint8)
    wc = rng.integers(0, 256, n * k // 2, dtype=np.uint8)
    wsc = rng.integers(121, 130, n * k // 32, dtype=np.uint8)
    pyoracle.set_threads(threads)
    sec = _timed(lambda: pyoracle.gemm_mx_f64(m, n, k, ac, asc, wc, wsc), min_s=0.5, max_reps=4)
    out["gemm_m32"] = {"shape": f"{m}x{n}x{k}", "ms": round(sec * 1e3, 2), "GFLOP_s": round(2.0 * m * n * k / sec / 1e9, 2),
                       "cores": threads, "accumulate": "f64 (the closed form of trackb/fp4_scale_test.cu:37)"}
    cfg = dict(dim=2048, n_layers=22, n_heads=32, n_kv_heads=4, head_dim=64, ffn=5632, vocab=32000, theta=10000.0,
               eps=1e-5, max_seq=16 + tiny_steps + tiny_steps_one + 2)
    prompt = np.random.default_rng(16).integers(0, 32000, 16).astype(np.uint32)
    mdl = pyoracle.Model(cfg, SEED)
    tok = 0
    for i, t in enumerate(prompt):
        tok = mdl.step(int(t), i)
    ids = [tok]
    t0 = time.perf_counter()
    for i in range(tiny_steps - 1):
        ids.append(mdl.step(ids[-1], 16 + i))
    dt = time.perf_counter() - t0
    pyoracle.set_threads(1)
    t0 = time.perf_counter()
    for i in range(tiny_steps_one):
        ids.append(mdl.step(ids[-1], 16 + tiny_steps - 1 + i))
    dt1 = time.perf_counter() - t0
    mdl.close()
    out["tinyllama"] = {"tok_s": round((tiny_steps - 1) / dt, 3), "cores": threads,
                        "one_thread": {"tok_s": round(tiny_steps_one / dt1, 3), "steps": tiny_steps_one},
                        "steps": tiny_steps,
                        "tokens_identical_to_gpu": (bool(np.array_equal(np.array(ids[:tiny_steps], np.uint32),
                                                                        tiny_gpu_ids[:tiny_steps]))
                                                    if tiny_gpu_ids is not None else None)}
    return out


# llama_decode/src/main.rs:289-298,357-360: the reference's random-weight
# decode harness, 221.6 tok/s on an RTX 5070 Ti (main.tex:208)
HARNESS_P, HARNESS_WARM, HARNESS_GEN = 512, 4, 32
HARNESS_PUBLISHED = 221.6


def harness_run(rf):
    """llama_decode replayed on the engine: Llama-3.2-1B shape, mk_fp4 weights
    from 0xdeadbeef with f32 scales, f32 K/V at 0.01 to P = 512, WARM steps
    untimed then GEN timed, no embedding (x carries over)."""
    cfg = rf.model_config(max_seq=HARNESS_P + HARNESS_WARM + HARNESS_GEN + 8, dim=2048, n_layers=16, n_heads=32,
                          n_kv_heads=8, head_dim=64, ffn=8192, vocab=128256, theta=500000.0, eps=1e-5,
                          scale_format=rf.SCALE_F32, kv_format=rf.KV_F32)
    eng = rf.Engine(cfg, 0xDEADBEEF)
    eng.begin_harness(HARNESS_P, 1 + HARNESS_WARM + HARNESS_GEN)
    eng.run_steps(HARNESS_WARM)
    eng.stream.synchronize()
    e0, e1 = rf.Event(), rf.Event()
    with ROCTX.range("harness_timed"):
        e0.record(eng.stream)
        eng.run_steps(HARNESS_GEN)
        e1.record(eng.stream)
        e1.synchronize()
    ms = e0.elapsed_ms(e1)
    ids = eng.read_ids(1 + HARNESS_WARM + HARNESS_GEN)[1:]
    finite = bool(np.all(np.isfinite(eng.logits())))
    eng.close()
    tok_s = HARNESS_GEN / (ms / 1e3)
    return {"tok_s": round(tok_s, 1), "ms_per_token": round(ms / HARNESS_GEN, 4), "logits_finite": finite,
            "last_token": int(ids[-1]), "reference_tok_s": HARNESS_PUBLISHED,
            "reference_hw": "RTX 5070 Ti, 896 GB/s GDDR7 (main.tex:208; context, not a target)",
            "workload": "llama_decode harness: Llama-3.2-1B shape, mk_fp4 weights (seed 0xdeadbeef) with f32 "
                        "scales, f32 K/V pre-filled with 0.01 to 512, 4 warm + 32 timed steps, no embedding"}


def gemv_step_table(cfg, kern):
    """The step's GEMV kernels with their algorithmic bytes and in-step GB/s."""
    qd, kvd = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim
    shapes = {"qkv": (qd + 2 * kvd, cfg.dim, 0), "o": (cfg.dim, qd, 0), "gate_up": (2 * cfg.ffn, cfg.dim, -4 * cfg.ffn),
              "down": (cfg.dim, cfg.ffn, 0), "lm_head": (cfg.vocab, cfg.dim, 0)}
    names = [k for k in kern if k.startswith("rfp4_gemv_")]
    # launch order within a layer: qkv (store), o (resid), gate/up (swiglu), down (resid); the LM head (argmax)
    role = {}
    for k in names:
        if "_swiglu_" in k:
            role["gate_up"] = k
        elif "_argmax_" in k:
            role["lm_head"] = k
        elif "_store_" in k:
            role["qkv"] = k
    resid = [k for k in names if "_resid_" in k]
    if len(resid) == 1:
        role["o"] = role["down"] = resid[0]
    else:
        for k in resid:  # same epilogue: o has K = n_heads*head_dim (fewer slices) than down (K = ffn)
            role["down" if int(k.split("_s")[-1].split("_")[0]) * 2048 >= cfg.ffn else "o"] = k
    out, tot_b, tot_us = {}, 0, 0.0
    for r, (n, k, adj) in shapes.items():
        if r not in role:
            continue
        calls, us = kern[role[r]]
        if role.get("o") == role.get("down") and r in ("o", "down"):
            us = None  # one kernel name for both: no per-role split
        b = gemv_bytes(n, k) + adj
        out[r] = {"kernel": role[r], "bytes": b, "us": us,
                  "GB_s": round(b / us / 1e3, 1) if us else None, "frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4) if us else None}
    per_tok_us = sum(kern[k][0] * kern[k][1] for k in names)
    # roles with a GEMV launch of their own (the q|k|v GEMV may be fused with
    # the attention into one launch, rfp4_qkva_*: not a GEMV-only time)
    per_tok_b = cfg.n_layers * sum(gemv_bytes(n, k) + adj for r, (n, k, adj) in shapes.items()
                                   if r != "lm_head" and r in role) + gemv_bytes(cfg.vocab, cfg.dim)
    return out, {"bytes_per_token": per_tok_b, "us_per_token": round(per_tok_us, 2),
                 "GB_s": round(per_tok_b / per_tok_us / 1e3, 1), "frac": round(per_tok_b / per_tok_us / 1e3 / HBM_PEAK_GBS, 4)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=4)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--cpu-steps", type=int, default=8, help="decode steps of the CPU oracle on all threads")
    ap.add_argument("--cpu-steps-one", type=int, default=4, help="decode steps of the CPU oracle on one thread")
    ap.add_argument("--no-persistent", action="store_true",
                    help="skip the opt-in persistent step (its cooperative launch; taken out of profiler runs)")
    ap.add_argument("--no-tiny", action="store_true", help="skip the TinyLlama-1.1B line")
    ap.add_argument("--no-harness", action="store_true", help="skip the llama_decode harness line")
    ap.add_argument("--no-gemm", action="store_true", help="skip the config-5 batched GEMM figures")
    ap.add_argument("--no-prefill", action="store_true", help="skip the batched prefill figure")
    ap.add_argument("--prefill-tokens", type=int, default=512, help="prompt length of the batched prefill figure")
    ap.add_argument("--pmc-probe", choices=["decode", "gemm"], help="only the launch sequence of a counter pass")
    ap.add_argument("--trace-tiny-eager", action="store_true",
                    help="only the TinyLlama decode launched kernel by kernel (for a kernel trace)")
    ap.add_argument("--summarize-trace", nargs="+", metavar="DIR", help="summarise rocprofv3 kernel traces")
    ap.add_argument("--summarize-pmc", nargs="+", metavar="DIR", help="summarise rocprofv3 counter passes")
    args = ap.parse_args()
    if args.summarize_trace:
        summarize_trace(args.summarize_trace)
        return
    if args.summarize_pmc:
        summarize_pmc(args.summarize_pmc)
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path "
              "(the decode step would shard tensor-parallel: q|k|v and gate|up by output rows, o and down by "
              "input columns with one small all-reduce each, attention by KV head). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import rfp4 as rf

    rf.init(0)
    if args.pmc_probe:
        pmc_probe(rf, args.pmc_probe)
        return
    if args.trace_tiny_eager:
        trace_tiny_eager(rf)
        return
    # ---- config 4: Llama-3-8B decode at batch 1, ctx 4096
    max_seq = PREFILL + args.warmup + max(args.steps, 40) + TIMED_STEPS + 8  # (the persistent line takes 34 steps)
    eng, cfg, ms, wall, ids = decode_run(rf, "llama3-8b", max_seq, PREFILL, [1], args.warmup, args.steps)
    tok_s = args.steps / (ms / 1e3)
    ms_step = ms / args.steps
    weight_bytes = eng.weight_bytes()
    log(f"llama3-8b: {ms_step * 1e3:.1f} us/token, {tok_s:.1f} tok/s (wall {args.steps / wall:.1f}); "
        f"weights {weight_bytes / 1e9:.3f} GB -> {weight_bytes / ms_step / 1e6:.0f} GB/s effective")
    kern = step_kernels(eng, "llama3-8b")
    gemv_roles, gemv_in_step = gemv_step_table(cfg, kern)
    # attention (+ its merge kernel) per layer; where the engine fuses the
    # q|k|v GEMV and the attention into one launch (rfp4_qkva_*), that launch
    fused = any(k.startswith("rfp4_qkva_") for k in kern)
    attn_us = sum(v[0] * v[1] for k, v in kern.items() if k.startswith("rfp4_attn_")) / cfg.n_layers
    qkva_us = sum(v[0] * v[1] for k, v in kern.items()
                  if k.startswith("rfp4_qkva_") or (fused and k.startswith("rfp4_attn_merge"))) / cfg.n_layers
    log("in-step kernels (us): " + ", ".join(f"{k} {v[1]}" for k, v in sorted(kern.items(), key=lambda kv: -kv[1][0] * kv[1][1])))
    if fused:
        log(f"q|k|v GEMV + attention (one launch) per layer {qkva_us:.2f} us; GEMV path in the step {gemv_in_step['GB_s']} GB/s")
    else:
        log(f"attention + merge per layer {attn_us:.2f} us; GEMV path in the step {gemv_in_step['GB_s']} GB/s")

    with ROCTX.range("gemv_path_isolated"):
        path_bytes, path_ms, gate_bytes, gate_ms, gate_plain_ms = gemv_path(rf, eng, cfg)
    gate_gbs = gate_bytes / gate_ms / 1e6
    path_gbs = path_bytes / path_ms / 1e6
    gate_kernel = gemv_roles["gate_up"]["kernel"]
    gate_in_us = kern[gate_kernel][1]
    gate_in_gbs = gate_bytes / gate_in_us / 1e3
    log(f"GEMV path alone: {path_bytes / 1e9:.3f} GB in {path_ms * 1e3:.1f} us -> {path_gbs:.0f} GB/s; "
        f"gate/up GEMV {gate_in_us:.2f} us in the step ({gate_in_gbs:.0f} GB/s), {gate_ms * 1e3:.2f} us alone "
        f"({gate_gbs:.0f} GB/s), {gate_plain_ms * 1e3:.2f} us alone without its fused norm")
    persistent = None if args.no_persistent else persistent_run(rf, eng)
    if persistent:
        log(f"persistent decode (opt-in): {persistent['tok_s']} tok/s vs graph {persistent['graph_tok_s_same_run']} "
            f"tok/s, tokens identical: {persistent['tokens_identical_to_graph']}")
    gemm = None if args.no_gemm else gemm_config5(rf, eng, cfg)
    prefill = None
    if not args.no_prefill:
        with ROCTX.range("prefill"):
            prefill = prefill_run(rf, eng, cfg, n=args.prefill_tokens)
        log(f"prefill {prefill['tokens']}: {prefill['ms']} ms, {prefill['tok_s']} tok/s, {prefill['TFLOP_s']} TFLOP/s")
    eng.close()

    tiny, tiny_ids = None, None
    if not args.no_tiny:
        r = np.random.default_rng(16).integers(0, 32000, 16).astype(np.uint32)
        teng, tcfg, tms, twall, tids = decode_run(rf, "tinyllama-1.1b", 16 + 256 + TIMED_STEPS + 8, 0, r, 0, 256)
        tkern = step_kernels(teng, "tinyllama-1.1b")
        tiny_ids = tids[16:16 + 256]
        tiny = {"tok_s": round(256 / (tms / 1e3), 1), "ms_per_token": round(tms / 256, 4),
                "step_kernels_us": {k: v[1] for k, v in tkern.items()},
                "workload": "TinyLlama-1.1B arch, 16-token prompt, 256 greedy steps"}
        log(f"tinyllama: {tiny['tok_s']} tok/s")
        teng.close()

    harness = None
    if not args.no_harness:
        harness = harness_run(rf)
        log(f"llama_decode harness: {harness['tok_s']} tok/s (reference {HARNESS_PUBLISHED} on an RTX 5070 Ti)")

    cpu = None
    if not args.no_cpu:
        threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or min(16, os.cpu_count() or 1)
        tok_all, t_all, tok_one, t_one, t_setup = cpu_baseline(threads, args.cpu_steps, args.cpu_steps_one)
        cpu = {"value": round(tok_all, 4), "unit": "tok/s", "cores": threads, "kind": "port",
               "single_thread": {"value": round(tok_one, 4), "unit": "tok/s", "cores": 1, "steps": args.cpu_steps_one,
                                 "seconds": round(t_one, 2)},
               "nproc": os.cpu_count(), "cpu_model": cpu_model(),
               "sample": f"oracle/ C decode loop, Llama-3-8B config 4 at ctx {PREFILL}: {args.cpu_steps} steps on "
                         f"{threads} threads ({t_all:.1f} s), then {args.cpu_steps_one} on 1 thread ({t_one:.1f} s); "
                         f"setup {t_setup:.1f} s untimed"}
        log(f"cpu oracle: {tok_all:.3f} tok/s on {threads} threads, {tok_one:.3f} tok/s on 1 ({cpu_model()}, nproc "
            f"{os.cpu_count()})")
        legs = cpu_legs(threads, tiny_gpu_ids=tiny_ids)
        cpu.update(legs)
        log("cpu oracle GEMV GB/s (all / 1 thread): " + ", ".join(
            f"{k} {v['all']['GB_s']}/{v['one_thread']['GB_s']}" for k, v in legs["gemv"].items()) +
            f"; GEMM M=32 {legs['gemm_m32']['GFLOP_s']} GFLOP/s; TinyLlama {legs['tinyllama']['tok_s']} tok/s "
            f"({legs['tinyllama']['one_thread']['tok_s']} on 1), tokens = GPU: {legs['tinyllama']['tokens_identical_to_gpu']}")

    out = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "Llama-3-8B arch decode, batch 1, fp16 KV pre-filled to 4096, greedy (BASELINE config 4)",
            "weights": "MXFP4 E2M1 + E8M0/32, random init",
            "global_batch": 1,
            "seq_len": PREFILL,
            "parallelism": "none (1 GPU)",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": f"fused gate/up SwiGLU GEMV ({gate_kernel}) inside the decode step",
            "achieved": round(gate_in_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gate_in_gbs / HBM_PEAK_GBS, 4),
            "traffic": load_traffic(gate_kernel),
            "bytes_per_launch": gate_bytes,
            "us_per_launch": round(gate_in_us, 3),
            "isolated": {"us_per_launch": round(gate_ms * 1e3, 3), "achieved": round(gate_gbs, 1),
                         "frac": round(gate_gbs / HBM_PEAK_GBS, 4),
                         "what": "the same launch (fused RMSNorm + SwiGLU) alone over the 32 layers' weights",
                         "without_norm_us_per_launch": round(gate_plain_ms * 1e3, 3)},
        },
        "step_kernels_us": {k: v[1] for k, v in kern.items()},
        "attention_us_per_layer": None if fused else round(attn_us, 3),
        "qkv_attention_fused_us_per_layer": round(qkva_us, 3) if fused else None,
        "gemv_in_step": dict(gemv_in_step, roles=gemv_roles),
        "gemv_path": {
            "bytes_per_token": path_bytes,
            "us_per_token": round(path_ms * 1e3, 2),
            "GB_s": round(path_gbs, 1),
            "frac": round(path_gbs / HBM_PEAK_GBS, 4),
        },
        "persistent_decode": persistent,
        "tinyllama": tiny,
        "llama_decode_harness": harness,
        "gemm_config5": gemm,
        "prefill": prefill,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
