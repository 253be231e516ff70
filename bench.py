"""Benchmark of the MI355X MXFP4 decode engine (one JSON line on stdout).

Workload: Llama-3-8B architecture, random-init MXFP4
weights (E2M1 + E8M0 per 32), batch 1, fp16 KV cache pre-filled to 4096
tokens, greedy decode.  A "step" is one token through all 32 layers and the
LM head.  `value` = decode tokens/s with weights and KV resident in HBM.

Extra fields: the roofline of the dominant kernel (the fused gate/up SwiGLU
GEMV) timed with HIP events on the engine's stream, the whole GEMV path of
one token replayed alone, TinyLlama-1.1B decode tok/s (config 3), the
batched MXFP4 GEMM at M=32 and M=512 on the 8B shapes (config 5, TFLOP/s
against the FP4 MFMA peak), and the CPU oracle timed on the host cores
(cpu_baseline, a reported baseline only).  `--pmc-probe` runs only the
launch sequence used for the HBM-traffic counter runs.
"""
import argparse
import json
import os
import sys
import time

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
    # dominant kernel: the fused gate/up SwiGLU GEMV, one launch per layer
    gate = [calls[4 * l + 2] for l in range(cfg.n_layers)]
    ms_gate = time_launches(rf, s, lambda: [c() for c in gate], reps) / cfg.n_layers
    gate_bytes = gemv_bytes(2 * cfg.ffn, cfg.dim) - 4 * cfg.ffn  # y holds ffn outputs, not 2*ffn
    return total_bytes, ms, gate_bytes, ms_gate


FP4_PEAK_TFLOPS = 10100.0


def _bf16_normal(rng, rows, k):
    u = rng.standard_normal((rows, k), dtype=np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def gemm_config5(rf, eng, cfg, reps=2):
    """MXFP4 GEMMs at M=32 (decode batch) and M=512 (prefill)
    on the engine's own Llama-3-8B weights, bf16 activations ~N(0,1) quantized
    per 32 along K (mx4_quantize).  Per config-5 shape, each launch uses a
    different layer's weights (no cache reuse across launches); the stack pass
    is every projection of the 32 layers plus the LM head."""
    s = eng.stream
    qd, kvd = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim
    rng = np.random.default_rng(5)
    acts = {}
    for k in sorted({cfg.dim, qd, cfg.ffn}):
        a16 = rf.DeviceBuffer.from_host(_bf16_normal(rng, 512, k), s)
        ac, asc = rf.DeviceBuffer(512 * k // 2), rf.DeviceBuffer(512 * k // 32)
        rf.mx4_quantize(s, 512, k, a16, True, ac, asc)
        acts[k] = (a16, ac, asc)
    c = rf.DeviceBuffer(512 * max(cfg.vocab, 2 * cfg.ffn) * 4)
    L = cfg.n_layers
    w = {p: [eng.weight(l, p)[:2] for l in range(L)] for p in (0, 3, 4, 6)}
    lm = eng.weight(-1, 0)[:2]
    # config-5 shapes: (name, N, K, weight views rotating over layers)
    shapes = [
        ("4096x4096", cfg.dim, qd, w[3]),
        ("1024x4096", kvd, cfg.dim, [(wc + qd * cfg.dim // 2, ws + qd * cfg.dim // 32) for wc, ws in w[0]]),
        ("14336x4096", cfg.ffn, cfg.dim, w[4]),
        ("4096x14336", cfg.dim, cfg.ffn, w[6]),
        ("128256x4096", cfg.vocab, cfg.dim, [lm]),
    ]
    stack = [(qd + 2 * kvd, cfg.dim, w[0]), (cfg.dim, qd, w[3]), (2 * cfg.ffn, cfg.dim, w[4]),
             (cfg.dim, cfg.ffn, w[6])]
    out = {}
    for m in (32, 512):
        res = {}
        for name, n, k, views in shapes:
            _, ac, asc = acts[k]
            nl = len(views)
            calls = [lambda wc=wc, ws=ws: rf.fp4_gemm(s, m, n, k, ac, asc, wc, ws, c) for wc, ws in views]
            ms = time_launches(rf, s, lambda: [f() for f in calls], reps) / nl
            tf = 2.0 * m * n * k / (ms * 1e-3) / 1e12
            gbs = (n * k * 17 // 32 + m * k * 17 // 32 + 4 * m * n) / (ms * 1e-3) / 1e9
            tm, tn, kz = rf.gemm_plan(m, n, k)
            res[name] = {"us": round(ms * 1e3, 2), "TFLOP_s": round(tf, 1), "frac_fp4_peak": round(tf / FP4_PEAK_TFLOPS, 4),
                         "GB_s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "tile": f"{tm}x{tn}/kz{kz}"}
        flops = 0.0
        calls = []
        for l in range(L):
            for n, k, views in stack:
                _, ac, asc = acts[k]
                wc, ws = views[l]
                calls.append(lambda n=n, k=k, ac=ac, asc=asc, wc=wc, ws=ws: rf.fp4_gemm(s, m, n, k, ac, asc, wc, ws, c))
                flops += 2.0 * m * n * k
        calls.append(lambda: rf.fp4_gemm(s, m, cfg.vocab, cfg.dim, acts[cfg.dim][1], acts[cfg.dim][2], lm[0], lm[1], c))
        flops += 2.0 * m * cfg.vocab * cfg.dim
        ms = time_launches(rf, s, lambda: [f() for f in calls], reps)
        tf = flops / (ms * 1e-3) / 1e12
        qms = time_launches(rf, s, lambda: rf.mx4_quantize(s, m, cfg.dim, acts[cfg.dim][0], True, acts[cfg.dim][1],
                                                           acts[cfg.dim][2]), 20)
        out[f"m{m}"] = {"stack_us": round(ms * 1e3, 1), "stack_TFLOP": round(flops / 1e12, 4),
                        "stack_TFLOP_s": round(tf, 1), "stack_frac_fp4_peak": round(tf / FP4_PEAK_TFLOPS, 4),
                        "quantize_us_k4096": round(qms * 1e3, 2), "shapes": res}
        log(f"gemm M={m}: stack {ms * 1e3:.0f} us, {tf:.0f} TFLOP/s ({100 * tf / FP4_PEAK_TFLOPS:.1f}% of FP4 peak); "
            + ", ".join(f"{k} {v['us']}us {v['TFLOP_s']}TF" for k, v in res.items()))
    for a16, ac, asc in acts.values():
        a16.free(), ac.free(), asc.free()
    c.free()
    out["workload"] = ("Llama-3-8B projections as MXFP4 GEMMs, bf16 activations ~N(0,1) quantized to MXFP4 per 32 "
                       "along K; stack = 32 layers x (qkv, o, gate+up, down) + LM head")
    out["peak_TFLOP_s"] = FP4_PEAK_TFLOPS
    return out


def pmc_probe(rf):
    """Fixed launch sequence for the HBM-traffic counter runs (rocprofv3
    --pmc FETCH_SIZE, then WRITE_SIZE): the gate/up SwiGLU GEMV of all 32
    layers of the 8B model, then a plain f32 copy of 64 Mi floats (256 MiB
    read + 256 MiB written) used to scale the counters."""
    cfg = rf.model_config("llama3-8b", max_seq=64)
    eng = rf.Engine(cfg, SEED)
    s = eng.stream
    x = rf.DeviceBuffer.from_host(np.random.default_rng(0).standard_normal(cfg.ffn).astype(np.float32), s)
    y = rf.DeviceBuffer.zeroed(cfg.ffn, np.float32, s)
    for l in range(cfg.n_layers):
        gc, gs, _, _ = eng.weight(l, 4)
        rf.mx4_gemv_swiglu(s, cfg.ffn, cfg.dim, cfg.ffn, gc, gs, x, y)
    s.synchronize()
    n = 64 << 20
    src = rf.DeviceBuffer.zeroed(n, np.float32, s)
    dst = rf.DeviceBuffer.zeroed(n, np.float32, s)
    for _ in range(4):
        rf.copy_into(s, n, 0, src, dst)
    s.synchronize()
    eng.close()
    print(json.dumps({"pmc_probe": "done", "gemv_launches": cfg.n_layers, "gemv_bytes": gemv_bytes(2 * cfg.ffn, cfg.dim)
                      - 4 * cfg.ffn, "copy_launches": 4, "copy_read_bytes": 4 * n, "copy_write_bytes": 4 * n}),
          flush=True)


def load_traffic():
    """HBM bytes per launch of the gate/up GEMV from the committed counter
    summary (profiles/gemv_swiglu_llama3-8b_traffic.json), or None."""
    p = os.path.join(ROOT, "profiles", "gemv_swiglu_llama3-8b_traffic.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        return json.load(f).get("traffic_bytes_per_launch")


def decode_run(rf, preset, max_seq, prefill, prompt, warmup, steps):
    cfg = rf.model_config(preset, max_seq=max_seq)
    eng = rf.Engine(cfg, SEED)
    if prefill:
        eng.prefill_kv(KV_SEED, prefill)
    n_prompt = len(prompt)
    eng.begin(prompt, prefill, n_prompt + warmup + steps)
    eng.run_steps(n_prompt - 1 + warmup)
    eng.stream.synchronize()
    e0, e1 = rf.Event(), rf.Event()
    t0 = time.perf_counter()
    e0.record(eng.stream)
    eng.run_steps(steps)
    e1.record(eng.stream)
    e1.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_ms(e1)
    ids = eng.read_ids(n_prompt + warmup + steps)
    assert np.all(ids < cfg.vocab)
    return eng, cfg, ms, wall, ids


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


def cpu_baseline(threads, steps=2):
    """The oracle decode loop (oracle/, C, f32, k-order) on the host cores:
    config-4 model, context pre-filled to 4096, `steps` decode steps timed."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle

    pyoracle.set_threads(threads)
    cfg = dict(dim=4096, n_layers=32, n_heads=32, n_kv_heads=8, head_dim=128, ffn=14336, vocab=128256,
               theta=500000.0, eps=1e-5, max_seq=PREFILL + steps + 2)
    t0 = time.perf_counter()
    m = pyoracle.Model(cfg, SEED)
    m.prefill_kv(KV_SEED, PREFILL)
    t_setup = time.perf_counter() - t0
    tok = 1
    t0 = time.perf_counter()
    for i in range(steps):
        tok = m.step(tok, PREFILL + i)
    dt = time.perf_counter() - t0
    m.close()
    return steps / dt, t_setup, dt


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=4)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--cpu-steps", type=int, default=20)
    ap.add_argument("--no-tiny", action="store_true", help="skip the TinyLlama-1.1B line")
    ap.add_argument("--no-gemm", action="store_true", help="skip the config-5 batched GEMM figures")
    ap.add_argument("--no-prefill", action="store_true", help="skip the batched prefill figure")
    ap.add_argument("--prefill-tokens", type=int, default=512, help="prompt length of the batched prefill figure")
    ap.add_argument("--pmc-probe", action="store_true", help="only the launch sequence of the counter runs")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path "
              "(the decode step would shard tensor-parallel: q|k|v and gate|up by output rows, o and down by "
              "input columns with one small all-reduce each, attention by KV head). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import rfp4 as rf

    rf.init(0)
    if args.pmc_probe:
        pmc_probe(rf)
        return
    # ---- config 4: Llama-3-8B decode at batch 1, ctx 4096
    max_seq = PREFILL + args.warmup + args.steps + 8
    eng, cfg, ms, wall, ids = decode_run(rf, "llama3-8b", max_seq, PREFILL, [1], args.warmup, args.steps)
    tok_s = args.steps / (ms / 1e3)
    ms_step = ms / args.steps
    weight_bytes = eng.weight_bytes()
    log(f"llama3-8b: {ms_step * 1e3:.1f} us/token, {tok_s:.1f} tok/s (wall {args.steps / wall:.1f}); "
        f"weights {weight_bytes / 1e9:.3f} GB -> {weight_bytes / ms_step / 1e6:.0f} GB/s effective")

    path_bytes, path_ms, gate_bytes, gate_ms = gemv_path(rf, eng, cfg)
    gate_gbs = gate_bytes / gate_ms / 1e6
    path_gbs = path_bytes / path_ms / 1e6
    log(f"GEMV path: {path_bytes / 1e9:.3f} GB in {path_ms * 1e3:.1f} us -> {path_gbs:.0f} GB/s; "
        f"gate/up GEMV {gate_ms * 1e3:.2f} us -> {gate_gbs:.0f} GB/s")
    gemm = None if args.no_gemm else gemm_config5(rf, eng, cfg)
    prefill = None if args.no_prefill else prefill_run(rf, eng, cfg, n=args.prefill_tokens)
    if prefill:
        log(f"prefill {prefill['tokens']}: {prefill['ms']} ms, {prefill['tok_s']} tok/s, {prefill['TFLOP_s']} TFLOP/s")
    eng.close()

    tiny = None
    if not args.no_tiny:
        r = np.random.default_rng(16).integers(0, 32000, 16).astype(np.uint32)
        teng, tcfg, tms, twall, tids = decode_run(rf, "tinyllama-1.1b", 16 + 256 + 8, 0, r, 0, 256)
        tiny = {"tok_s": round(256 / (tms / 1e3), 1), "ms_per_token": round(tms / 256, 4),
                "workload": "TinyLlama-1.1B arch, 16-token prompt, 256 greedy steps"}
        log(f"tinyllama: {tiny['tok_s']} tok/s")
        teng.close()

    cpu = None
    if not args.no_cpu:
        threads = min(16, os.cpu_count() or 1)
        cpu_tok_s, t_setup, t_run = cpu_baseline(threads, args.cpu_steps)
        cpu = {"value": round(cpu_tok_s, 4), "unit": "tok/s", "cores": threads, "kind": "port",
               "sample": f"oracle/ C decode loop, Llama-3-8B config 4 at ctx {PREFILL}, {args.cpu_steps} steps "
                         f"timed ({t_run:.1f} s; setup {t_setup:.1f} s untimed)"}
        log(f"cpu oracle: {cpu_tok_s:.3f} tok/s on {threads} threads")

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
            "kernel": "fused gate/up SwiGLU GEMV (rfp4_gemv_e8m0_swiglu)",
            "achieved": round(gate_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gate_gbs / HBM_PEAK_GBS, 4),
            "traffic": load_traffic(),
            "bytes_per_launch": gate_bytes,
            "us_per_launch": round(gate_ms * 1e3, 3),
        },
        "gemv_path": {
            "bytes_per_token": path_bytes,
            "us_per_token": round(path_ms * 1e3, 2),
            "GB_s": round(path_gbs, 1),
            "frac": round(path_gbs / HBM_PEAK_GBS, 4),
        },
        "tinyllama": tiny,
        "gemm_config5": gemm,
        "prefill": prefill,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
