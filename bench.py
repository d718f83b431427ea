"""Benchmark of the MI355X verify path.

Default (the metric of BASELINE.json): speculative decoding on a random-init
Qwen3-4B-shaped int4 g64 model, batch 16, k = 4, greedy, draft = the target's
first 4 layers, 128-token uniform-random prompts (seed 0).  A step is one
speculative round over the whole batch (4 batched draft forwards, one
80-row verify forward, acceptance, commit).  value = accepted tokens/s =
committed tokens (A+1 per sequence per round) / wall time of the timed rounds,
with inputs resident on the GPU.

Also reported: the verify-step HBM GB/s, a roofline object for the int4 GEMM
kernel (the dominant kernel; HIP events on the engine's stream, in separate
profiled rounds after the timed ones), and the CPU baseline — the oracle
restatement of the reference's path (oracle/libvxo.so) timed on the host for
one round of the same workload with a 4-token prompt.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
  python bench.py --mode qmm   # config 1: isolated verify GEMMs, cache-rotated
  python bench.py --mode continuous   # config 4: scheduler, Qwen3-8B shape
  python bench.py --mode tree   # config 3: tree verification at context 2048
  python bench.py --mode config0   # config 0 end to end, GPU and CPU oracle
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
PEAK_MFMA_F16_TFLOPS = 2500.0  # dense f16/bf16 MFMA, MI355X
METRIC = "accepted tok/s, Qwen3-4B-shape int4 k=4 batch 16; verify-step HBM GB/s"
# HBM bytes per verify GEMM op measured with rocprofv3 --pmc FETCH_SIZE /
# WRITE_SIZE over this bench, scaled by a calibration copy (see the file)
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_verify_gemm_qwen3_4b_b16_k4.json")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def host_cpu():
    """Host cores this process may run on, and the CPU model."""
    cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return cores, model


def snapshot_kv(engine_obj, states, target_pages, draft_pages):
    """Host copies of the KV pages the states hold after the GPU prefill:
    {(which, layer, kv): (block table, f16 pages [n, h_kv, ps, d])}."""
    import ctypes as C

    from velox_amd._lib import lib

    rt = C.CDLL("libamdhip64.so.7")
    rt.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    snap = []
    for which, pg in ((0, target_pages), (1, draft_pages)):
        shape = (pg.num_pages, pg.num_kv_heads, pg.page_size, pg.head_dim)
        tables = []
        for s in states:
            n = lib.vx_spec_state_pages(engine_obj._h, s.id, which, None, 0)
            buf = (C.c_uint32 * n)()
            lib.vx_spec_state_pages(engine_obj._h, s.id, which, buf, n)
            tables.append(np.array(buf[:n], np.uint32))
        used = np.unique(np.concatenate(tables))
        for layer in range(pg.num_layers):
            for kv in (0, 1):
                pool = np.empty(shape, np.float16)
                assert rt.hipMemcpy(pool.ctypes.data, pg.layer_pool_ptr(layer, kv), pool.nbytes, 2) == 0
                snap.append((which, layer, kv, tables, {int(u): pool[u].copy() for u in used}))
    return snap


def cpu_baseline(cfg, weights, prompts, k, kv_snapshot, rounds=2):
    """The oracle (the reference's algorithm restated in C: qmm_4bit_cpu loop
    order, OpenMP over output features) running the same spec rounds on the
    host: full Qwen3-4B-shape target, 4-layer draft, batch 16, k = 4, greedy,
    the same 128-token prompts.  The oracle's states take the KV pages of the
    GPU prefill (copied, not timed: a 16 x 127-row prefill through 36 layers
    is far beyond a bounded CPU sample); one warm-up round, then `rounds`
    timed full rounds at the GPU run's context."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import vxo

    from velox_amd import synth

    cores, model = host_cpu()
    os.environ.setdefault("OMP_NUM_THREADS", str(cores))
    wt = synth.as_model_dtype(weights, "bf16")
    ocfg = dict(cfg, dtype=vxo.BF16)
    B, L, HK, D = len(prompts), cfg["layers"], cfg["n_kv_heads"], cfg["head_dim"]
    t = vxo.Model(ocfg, wt, threads=cores)
    d = vxo.Model(ocfg, wt, n_layers=4, threads=cores)
    del wt
    npg = B * ((len(prompts[0]) + (rounds + 2) * (k + 1) + 15) // 16 + 1)
    tp, dp = vxo.Pages(L, HK, D, 16, npg), vxo.Pages(4, HK, D, 16, npg)
    e = vxo.SpecEngine(t, tp, d, dp)
    st = e.adopt(prompts)
    for which, layer, kv, tables, pages in kv_snapshot:
        pool = (tp if which == 0 else dp).pool(layer, kv)
        for b in range(B):
            ob = st[b].target_blocks if which == 0 else st[b].draft_blocks
            for i, gpage in enumerate(tables[b]):
                pool[ob[i]] = pages[int(gpage)].astype(np.float32)
    log(f"[cpu] oracle states adopted with the GPU prefill's KV; warm-up round ({cores} threads)")
    e.step(st, k)
    t0 = time.perf_counter()
    committed = 0
    for _ in range(rounds):
        out = e.step(st, k)
        committed += int(sum(len(c) for c in out["committed"]))
    dt = time.perf_counter() - t0
    log(f"[cpu] {rounds} full rounds in {dt:.2f}s, {committed} tokens")
    return {"value": committed / dt, "unit": "accepted tok/s", "cores": cores, "kind": "port",
            "sample": (f"oracle spec loop (oracle/vxo.c restating spec.rs / qwen3.rs / metal_kernels.rs CPU refs, "
                       f"OpenMP {cores} threads on {model}, nproc {os.cpu_count()}): {rounds} timed full rounds "
                       f"(36-layer target, 4-layer draft, batch {B}, k={k}, greedy, 128-token prompts) after one "
                       f"warm-up round, from states holding the GPU prefill's KV pages; {dt:.2f} s, "
                       f"{committed} tokens")}


def traffic_per_op():
    """HBM bytes per verify GEMM op from the committed rocprofv3 --pmc summary, or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f)["bytes_per_op"]
    except (OSError, KeyError, ValueError):
        return None


def run_spec(args):
    import torch

    from velox_amd import engine, synth

    torch.cuda.set_device(0)
    if args.calib_copy:
        # one device copy of known size: the counter calibration of the --pmc runs
        nb = args.calib_copy << 20
        src = torch.ones(nb, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] calibration copy of {nb} bytes done")
        del src, dst
    B, k = args.batch, args.k
    cfg = synth.qwen3_config("qwen3-4b", max_pos=8192)
    t0 = time.time()
    w = synth.host_weights(cfg, seed=0)
    log(f"[bench] synthetic Qwen3-4B weights generated in {time.time() - t0:.1f}s")
    target = engine.PagedQwen3(cfg, w)
    draft = engine.PagedQwen3(cfg, w, n_layers=4)
    log(f"[bench] models on device ({time.time() - t0:.1f}s)")
    rounds = args.warmup + args.steps + 2 * args.profile_steps
    max_len = args.prompt + (rounds + 1) * (k + 1) + 16
    pages_per_seq = (max_len + 15) // 16 + 1
    HK, D = cfg["n_kv_heads"], cfg["head_dim"]
    tp = engine.PagedKvCache(cfg["layers"], HK, D, 16, B * pages_per_seq + 8)
    dp = engine.PagedKvCache(4, HK, D, 16, B * pages_per_seq + 8)
    e = engine.SpecEngine(target, tp, draft, dp)
    prompts = [synth.prompt(0, args.prompt, cfg["vocab"], stream=b) for b in range(B)]
    t1 = time.time()
    states = e.prefill_batch(prompts)
    torch.cuda.synchronize()
    log(f"[bench] prefill {B}x{args.prompt} in {time.time() - t1:.1f}s")
    kv_snapshot = None if args.no_cpu_baseline else snapshot_kv(e, states, tp, dp)
    for i in range(args.warmup):
        e.step_batch(states, k)
    torch.cuda.synchronize()
    log(f"[bench] warmup {args.warmup} rounds done")
    committed = 0
    accepted = 0
    torch.cuda.synchronize()
    ts = time.perf_counter()
    for i in range(args.steps):
        outs = e.step_batch(states, k)
        committed += sum(len(o.committed_tokens) for o in outs)
        accepted += sum(o.accepted for o in outs)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - ts
    log(f"[bench] timed {args.steps} rounds: {elapsed * 1e3:.1f} ms, {committed} tokens")
    # outside the timed region: the last round's decisions, re-derived from
    # its own verify logits (argmax_slice: first index of the maximum)
    cand, vlog = e.last_trace(B, k)
    decisions_ok = True
    for b in range(B):
        am = vlog[b].argmax(axis=1)
        a = 0
        while a < k and cand[b, a] == am[a]:
            a += 1
        want = list(cand[b, :a]) + [am[a]]
        decisions_ok &= outs[b].accepted == a and list(outs[b].committed_tokens) == [int(x) for x in want]
    log(f"[bench] last round's accept decisions re-derived from its logits: {'ok' if decisions_ok else 'MISMATCH'}")
    # undisturbed phase times (events at the draft / verify / accept boundaries only)
    e.set_profiling(True, phases_only=True)
    phases = []
    for i in range(args.profile_steps):
        e.step_batch(states, k)
        phases.append(e.last_profile())
    e.set_profiling(False)
    # profiled rounds (HIP events on the engine stream around every kernel)
    e.set_profiling(True)
    profs = []
    for i in range(args.profile_steps):
        e.step_batch(states, k)
        profs.append(e.last_profile())
    e.set_profiling(False)
    ctx = states[0].kv_len
    if profs:
        agg = {key: float(np.mean([p[key] for p in profs])) for key in profs[0]}
        log("[bench] profile " + json.dumps({kk: round(v, 4) for kk, v in agg.items()}))
        qmm_gbs = agg["verify_qmm_bytes"] / (agg["verify_qmm_ms"] * 1e-3) / 1e9
        verify_bytes = agg["verify_qmm_bytes"] + agg["verify_attention_bytes"]
    else:  # no profiled rounds (e.g. under a profiler): no live kernel figures
        agg, qmm_gbs, verify_bytes = None, None, None
    phase_ms = None if not phases else {
        kk: float(np.mean([p[kk] for p in phases])) for kk in ("draft_ms", "verify_ms", "accept_ms")}
    # the measured device copy rate, reported next to the published peak
    copy_gbs = device_copy_gbs() if profs else None
    # the same GEMM ops against the dense f16 MFMA peak: algorithmic flops
    # (2 M N K over the verify rows M = B (k+1), no padding) per round
    H, F, V, L = cfg["hidden"], cfg["inter"], cfg["vocab"], cfg["layers"]
    QW, KW = cfg["n_heads"] * cfg["head_dim"], cfg["n_kv_heads"] * cfg["head_dim"]
    verify_flops = 2.0 * B * (k + 1) * (L * (H * (QW + 2 * KW) + QW * H + H * 2 * F + F * H) + H * V)
    qmm_tflops = None if agg is None else verify_flops / (agg["verify_qmm_ms"] * 1e-3) / 1e12
    res = {
        "metric": METRIC,
        "value": committed / elapsed,
        "unit": "accepted tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": elapsed * 1e3 / args.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 weights, bf16 activations (f16 carriers), f32 accumulate",
        "data": "synthetic (random-init Qwen3-4B shape, seeded Philox streams)",
        "config": {"workload": "spec-decode greedy, Qwen3-4B shape int4 g64, draft = first 4 layers",
                   "global_batch": B, "k": k, "prompt_len": args.prompt, "context_at_end": ctx,
                   "seq_len": ctx, "parallelism": "single GPU"},
        "acceptance_rate": accepted / (args.steps * B * k),
        # the verify phase of undisturbed rounds (events at its boundaries
        # only) over the algorithmic bytes of its GEMMs and attention
        "verify_step": None if (agg is None or not phases) else {
            "ms": phase_ms["verify_ms"], "algorithmic_bytes": verify_bytes,
            "hbm_gbs": verify_bytes / (phase_ms["verify_ms"] * 1e-3) / 1e9,
            "draft_ms": phase_ms["draft_ms"], "accept_ms": phase_ms["accept_ms"]},
        "roofline": {"bound": "hbm",
                     "kernel": "qmm_f16_k2_kernel: the verify step's int4 GEMMs (36 layers "
                               "x qkv, o, gate|up with its SwiGLU finish, down; plus the LM head), average per op",
                     "achieved": qmm_gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": None if qmm_gbs is None else qmm_gbs / PEAK_HBM_GBS,
                     "device_copy_gbs": copy_gbs,
                     "mfma_tflops": qmm_tflops, "mfma_peak_tflops": PEAK_MFMA_F16_TFLOPS,
                     "mfma_frac": None if qmm_tflops is None else qmm_tflops / PEAK_MFMA_F16_TFLOPS,
                     "traffic": traffic_per_op(),
                     "launches_per_step": None if agg is None else agg["verify_qmm_launches"],
                     "avg_launch_us": None if agg is None else
                     agg["verify_qmm_ms"] * 1e3 / max(1, agg["verify_qmm_launches"]),
                     "algorithmic_bytes_per_launch": None if agg is None else
                     agg["verify_qmm_bytes"] / max(1, agg["verify_qmm_launches"])},
        "ms_per_round": elapsed * 1e3 / args.steps,
        "decisions_check": "ok" if decisions_ok else "mismatch",
        # phase times of undisturbed rounds (they sum to about ms_per_step;
        # the commit's host work is the remainder)
        "kernel_breakdown_ms": phase_ms,
        # per-class sums from the per-kernel event rounds: each event pair also
        # brackets its kernel's dispatch gap, so these run above the phases
        "kernel_class_ms_event_bracketed": None if agg is None else {
            kk: v for kk, v in agg.items() if kk.endswith("_ms") and kk not in ("draft_ms", "verify_ms", "accept_ms")},
    }
    if not args.no_cpu_baseline:
        t2 = time.time()
        res["cpu_baseline"] = cpu_baseline(cfg, w, prompts, k, kv_snapshot)
        log(f"[bench] cpu baseline in {time.time() - t2:.1f}s")
    else:
        res["cpu_baseline"] = None
    print(json.dumps(res), flush=True)


def device_copy_gbs(mb=1024, iters=10):
    """Measured device bandwidth next to the published 8 TB/s: a torch device
    copy of `mb` MiB (read + write), back to back, HIP events."""
    import torch

    src = torch.ones(mb << 20, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(iters):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    gbs = 2 * (mb << 20) * iters / (e0.elapsed_time(e1) * 1e-3) / 1e9
    del src, dst
    torch.cuda.empty_cache()
    return gbs


def graph_us_per_launch(launches, out, reps=5):
    """Capture `launches` (closures over preallocated buffers, an explicit
    workspace and the current stream) in one HIP graph and time its replays
    with HIP events: microseconds per launch, without host launch overhead.
    The replayed output must equal the eager result of the last launch."""
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for fn in launches:
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    eager = out.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for fn in launches:
            fn()
    ts = []
    for _ in range(reps):
        out.zero_()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        if not torch.equal(out, eager):
            raise RuntimeError("graph replay differs from the eager result")
        ts.append(e0.elapsed_time(e1) * 1e3 / len(launches))
    del g
    return sorted(ts)[len(ts) // 2]


def run_qmm(args):
    """Config 1: each verify GEMM shape at M = 5 and 80, f16 X ~N(0,1), through
    the MLX-layout entry (vx_qmm_4bit_ex, the qmm_4bit kernel into a
    preallocated output) and the engine's packed path (vx_qmm_4bit_packed).
    More than 640 MB of distinct weight copies are rotated so no launch finds
    its weights warm in the 256 MB Infinity Cache; the launches are captured in
    a HIP graph and replayed, so the time per launch excludes host overhead
    (it includes the dispatch gap between consecutive kernels)."""
    import torch

    from velox_amd import _lib, ops, synth

    torch.cuda.set_device(0)
    copy_gbs = device_copy_gbs()
    log(f"[qmm] device copy {copy_gbs:.0f} GB/s (read + write)")
    shapes = [("qkv_literal", 4608, 2560), ("qkv", 6144, 2560), ("o", 2560, 4096), ("gate_up", 19456, 2560),
              ("gate", 9728, 2560), ("down", 2560, 9728), ("lm_head", 151936, 2560)]
    ws = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
    out = []
    for name, n, kk in shapes:
        lin = synth.qlinear(1, f"bench.{name}", n, kk, 64)
        wbytes = 0.5625 * n * kk
        copies = max(2, int(np.ceil(640e6 / wbytes)))
        W = torch.from_numpy(lin["qweight"].view(np.int32)).cuda()
        S = torch.from_numpy(lin["scales"]).cuda()
        Bs = torch.from_numpy(lin["biases"]).cuda()
        mlx = [(W.clone(), S.clone(), Bs.clone()) for _ in range(copies)]
        packed = [ops.qmm_pack_4bit(*mlx[i]) for i in range(copies)] if n % 32 == 0 else None
        del W, S, Bs
        for m in (5, 80):
            x = torch.randn((m, kk), dtype=torch.float16, device="cuda")
            y = torch.empty((m, n), dtype=torch.float16, device="cuda")
            it = max(4 * copies, 40)
            paths = {"mlx": [(lambda i=i: ops.qmm_4bit_ex(x, *mlx[i % copies], y, round_dtype=_lib.F16,
                                                          workspace=ws)) for i in range(it)]}
            if packed is not None:
                paths["packed"] = [(lambda i=i: ops.qmm_4bit_packed(x, packed[i % copies], n, y,
                                                                    round_dtype=_lib.F16, workspace=ws))
                                   for i in range(it)]
            for path, launches in paths.items():
                us = graph_us_per_launch(launches, y)
                byt = wbytes + 2 * m * kk + 2 * m * n
                gbs = byt / (us * 1e-6) / 1e9
                out.append({"shape": name, "n": n, "k": kk, "m": m, "path": path, "us_per_launch": us,
                            "algorithmic_bytes": byt, "gbs": gbs, "frac": gbs / PEAK_HBM_GBS,
                            "frac_of_copy": gbs / copy_gbs})
                log(f"[qmm] {name:12s} m={m:3d} {path:6s} {us:8.2f} us  {gbs:7.0f} GB/s "
                    f"({100 * gbs / PEAK_HBM_GBS:.1f}% of 8 TB/s, {100 * gbs / copy_gbs:.1f}% of copy)")
        del mlx, packed
        torch.cuda.empty_cache()
    print(json.dumps({"mode": "qmm", "device_copy_gbs": copy_gbs, "peak_gbs": PEAK_HBM_GBS, "results": out}),
          flush=True)


def run_config0(args):
    """Config 0, the reference's CPU-runnable case, end to end: greedy spec
    decode on a random-init Qwen3-0.6B-shaped int4 g64 model (seed 0), batch 1,
    draft = the target's first 4 layers, a 128-token uniform-random prompt,
    k = 4, 64 generated tokens.  The GPU engine and the CPU oracle (the
    reference's spec loop restated, OpenMP) run the identical workload; each
    reports generated tokens / wall time of its rounds (prefill excluded), and
    the two token streams are compared.  The GPU figure is the second of two
    runs (the first warms the allocator and code objects)."""
    import torch

    from velox_amd import engine, synth

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import vxo

    torch.cuda.set_device(0)
    k, n_new, plen = 4, 64, 128
    cfg = synth.qwen3_config("qwen3-0.6b", max_pos=4096)
    w = synth.host_weights(cfg, seed=0)
    prompt = synth.prompt(0, plen, cfg["vocab"])
    L, HK, D = cfg["layers"], cfg["n_kv_heads"], cfg["head_dim"]
    pages = (plen + n_new + 2 * (k + 1) + 15) // 16 + 4
    target = engine.PagedQwen3(cfg, w)
    draft = engine.PagedQwen3(cfg, w, n_layers=4)

    def gpu_run():
        e = engine.SpecEngine(target, engine.PagedKvCache(L, HK, D, 16, pages), draft,
                              engine.PagedKvCache(4, HK, D, 16, pages))
        st = e.prefill_batch([prompt])
        torch.cuda.synchronize()
        toks, acc, rounds = [], 0, 0
        t0 = time.perf_counter()
        while len(toks) < n_new:
            out = e.step_batch(st, k)[0]
            toks += out.committed_tokens
            acc += out.accepted
            rounds += 1
        torch.cuda.synchronize()
        return toks, acc, rounds, time.perf_counter() - t0

    gpu_run()
    g_toks, g_acc, g_rounds, g_s = gpu_run()
    log(f"[config0] gpu: {len(g_toks)} tokens in {g_rounds} rounds, {g_s * 1e3:.1f} ms")
    threads = min(16, os.cpu_count() or 1)
    wt = synth.as_model_dtype(w, "bf16")
    ocfg = dict(cfg, dtype=vxo.BF16)
    oe = vxo.SpecEngine(vxo.Model(ocfg, wt, threads=threads), vxo.Pages(L, HK, D, 16, pages),
                        vxo.Model(ocfg, wt, n_layers=4, threads=threads), vxo.Pages(4, HK, D, 16, pages))
    t0 = time.perf_counter()
    ost = oe.prefill([prompt])
    log(f"[config0] cpu prefill {time.perf_counter() - t0:.1f}s")
    c_toks, c_acc, c_rounds = [], 0, 0
    t0 = time.perf_counter()
    while len(c_toks) < n_new:
        out = oe.step(ost, k)
        c_toks += [int(t) for t in out["committed"][0]]
        c_acc += int(out["accepted"][0])
        c_rounds += 1
    c_s = time.perf_counter() - t0
    log(f"[config0] cpu: {len(c_toks)} tokens in {c_rounds} rounds, {c_s:.1f} s")
    same = 0
    while same < min(n_new, len(g_toks), len(c_toks)) and g_toks[same] == c_toks[same]:
        same += 1
    res = {"mode": "config0", "metric": "accepted tok/s, Qwen3-0.6B-shape int4 k=4 batch 1 (config 0)",
           "workload": "greedy spec decode, Qwen3-0.6B shape int4 g64 seed 0, draft = first 4 layers, "
                       "128-token prompt, k=4, 64 new tokens, batch 1",
           "gpu": {"value": len(g_toks) / g_s, "unit": "accepted tok/s", "tokens": len(g_toks),
                   "rounds": g_rounds, "seconds": g_s, "acceptance_rate": g_acc / (g_rounds * k)},
           "cpu_baseline": {"value": len(c_toks) / c_s, "unit": "accepted tok/s", "tokens": len(c_toks),
                            "rounds": c_rounds, "seconds": c_s, "acceptance_rate": c_acc / (c_rounds * k),
                            "cores": threads, "kind": "port",
                            "sample": "the full config-0 workload on the oracle (oracle/vxo.c, OpenMP)"},
           "streams": {"tokens_compared": n_new, "identical_leading_tokens": same}}
    print(json.dumps(res), flush=True)


def run_continuous(args):
    """Config 4: continuous-batching speculative decoding on a random-init
    Qwen3-8B-shaped int4 g64 model: 32 requests, prompt lengths U[256, 4096]
    whose first 512 tokens are shared within groups of 8, k = 6 from the
    target's first 2 layers, temperature 0.7 (Philox streams per request,
    seed 4), 256 new tokens each, 16-token pages, through the scheduler
    (vx_sched_*) with its prefix cache.  value = generated tokens / wall time
    from the first submit to the last finished request (prefill included);
    also the decode-only rate over the steps that ran no prefill."""
    import torch

    from velox_amd import engine, synth
    from velox_amd.scheduler import BatchScheduler, SchedulerConfig

    torch.cuda.set_device(0)
    n_req, k, new_tokens, group, shared_len = 32, 6, 256, 8, 512
    cfg = synth.qwen3_config("qwen3-8b", max_pos=8192)
    t0 = time.time()
    w = synth.host_weights(cfg, seed=4)
    log(f"[cont] synthetic Qwen3-8B weights generated in {time.time() - t0:.1f}s")
    target = engine.PagedQwen3(cfg, w)
    draft = engine.PagedQwen3(cfg, w, n_layers=2)
    del w
    log(f"[cont] models on device ({time.time() - t0:.1f}s)")
    rng = np.random.Generator(np.random.Philox(key=[4, 0x636F6E74]))
    lens = rng.integers(256, 4097, size=n_req)
    V = cfg["vocab"]
    shared = [synth.prompt(4, shared_len, V, stream=1000 + g) for g in range(n_req // group)]
    # a prompt shorter than the shared prefix is a prefix of it
    prompts = [np.concatenate([shared[i // group][:int(lens[i])],
                               synth.prompt(4, max(0, int(lens[i]) - shared_len), V, stream=i)])
               for i in range(n_req)]
    ps = 16
    pages = sum(-(-(int(n) + new_tokens + k + 1) // ps) for n in lens) + 64
    HK, D = cfg["n_kv_heads"], cfg["head_dim"]
    tp = engine.PagedKvCache(cfg["layers"], HK, D, ps, pages)
    dp = engine.PagedKvCache(2, HK, D, ps, pages)
    e = engine.SpecEngine(target, tp, draft, dp, temperature=0.7, sample_seed=4)
    scfg = SchedulerConfig(max_running_requests=n_req, max_batch_tokens=args.batch_tokens,
                           prefix_cache_capacity=1024, draft_k=k)
    # warm-up: grow every device buffer to the sizes the run needs, on unrelated prompts
    s = BatchScheduler(e, (), scfg)
    for i in range(n_req):
        s.submit(synth.prompt(5, args.batch_tokens // n_req + 2, V, stream=i), 8, temperature=0.7)
    s.run()
    s.close()
    torch.cuda.synchronize()
    log(f"[cont] warm-up done ({time.time() - t0:.1f}s); {pages} pages per pool")
    s = BatchScheduler(e, (), scfg)
    torch.cuda.synchronize()
    ts = time.perf_counter()
    ids = [s.submit(p, new_tokens, temperature=0.7) for p in prompts]
    dec_s, dec_tok, steps, last_log = 0.0, 0, 0, ts
    while s.num_waiting() + s.num_running():
        before = s.stats()
        a = time.perf_counter()
        s.step()
        b = time.perf_counter()
        after = s.stats()
        steps += 1
        if after["prefill_tokens"] == before["prefill_tokens"]:
            dec_s += b - a
            dec_tok += after["tokens_generated"] - before["tokens_generated"]
        if b - last_log > 20:
            log(f"[cont] step {steps}: {after['tokens_generated']} tokens, {s.num_running()} running, "
                f"{s.num_waiting()} waiting")
            last_log = b
    torch.cuda.synchronize()
    wall = time.perf_counter() - ts
    st = s.stats()
    gen = sum(len(s.poll(r).tokens) for r in ids)
    assert gen == n_req * new_tokens, f"generated {gen} tokens, expected {n_req * new_tokens}"
    res = {
        "mode": "continuous", "metric": "generated tok/s, config 4 (Qwen3-8B shape int4, 32 requests, k=6, T=0.7)",
        "value": gen / wall, "unit": "generated tok/s", "wall_s": wall, "steps": steps,
        "decode_tok_s": dec_tok / dec_s if dec_s else None, "decode_s": dec_s,
        "prefill_tokens": st["prefill_tokens"], "prefix_tokens_skipped": st["prefix_tokens_skipped"],
        "prefix_cache_hits": st["prefix_cache_hits"], "rounds": st["rounds"],
        "acceptance_rate": st["draft_tokens_accepted"] / max(1, st["draft_tokens_proposed"]),
        "config": {"workload": "continuous-batching spec decode", "model": "Qwen3-8B shape int4 g64",
                   "requests": n_req, "prompt_len": "U[256, 4096]", "shared_prefix": f"{shared_len} per {group}",
                   "k": k, "draft_layers": 2, "temperature": 0.7, "new_tokens": new_tokens,
                   "max_batch_tokens": args.batch_tokens},
        "data": "synthetic (random-init weights, Philox prompts)",
    }
    s.close()
    print(json.dumps(res), flush=True)


def run_tree(args):
    """Config 3: tree verification on a random-init Qwen3-4B-shaped int4 g64
    model (seed 3).  16 sequences with 2048-token contexts in paged f16 KV
    (16-token pages, block tables in shuffled pool order); each step verifies
    a 16-node draft tree with branching 4-2-2 under the last context token
    (17 rows per sequence, ancestor-only attention), selects the longest
    accepted path greedily (vx_accept_tree) and moves that path's K/V rows
    to consecutive positions (vx_kv_compact_path).  The tree's tokens are
    synthetic.  Reported: ms per verify step over the whole batch, from the
    host call of the forward to the end of the compaction."""
    import torch

    from velox_amd import engine, ops, synth

    torch.cuda.set_device(0)
    B, ctx, ps = 16, 2048, 16
    par = [-1, 0, 0, 0, 0] + [p for p in range(1, 5) for _ in range(2)] + [p for p in (5, 6) for _ in range(2)]
    R = len(par)
    cfg = synth.qwen3_config("qwen3-4b", max_pos=8192)
    t0 = time.time()
    w = synth.host_weights(cfg, seed=3)
    target = engine.PagedQwen3(cfg, w)
    del w
    log(f"[tree] model on device ({time.time() - t0:.1f}s)")
    V, HK, D = cfg["vocab"], cfg["n_kv_heads"], cfg["head_dim"]
    need = -(-(ctx - 1 + R) // ps)
    pool = engine.PagedKvCache(cfg["layers"], HK, D, ps, B * need + 16)
    rng = np.random.Generator(np.random.Philox(key=[3, 0x74726565]))
    # allocate every page, then hand them out in shuffled order
    allp = np.array(pool.alloc(B * need), np.uint32)
    bts = allp[rng.permutation(allp.size)].reshape(B, need)
    prompts = [synth.prompt(3, ctx, V, stream=b) for b in range(B)]
    t1 = time.time()
    for b0 in range(0, B, 4):  # prefill positions 0..ctx-2 four sequences at a time
        ids = np.concatenate([prompts[b][:ctx - 1] for b in range(b0, b0 + 4)])
        target.forward(pool, ids, [(ctx - 1, 0, bts[b]) for b in range(b0, b0 + 4)])
    torch.cuda.synchronize()
    log(f"[tree] prefill {B}x{ctx - 1} in {time.time() - t1:.1f}s")
    nodes = rng.integers(0, V, size=(B, R)).astype(np.uint32)
    nodes[:, 0] = [prompts[b][ctx - 1] for b in range(B)]
    ids = nodes.reshape(-1)
    seqs = [(R, ctx - 1, bts[b]) for b in range(B)]
    node_dev = torch.from_numpy(nodes.view(np.int32)).cuda()
    bt_dev = torch.from_numpy(bts.view(np.int32)).cuda()
    kvo_dev = torch.full((B,), ctx - 1, dtype=torch.int32, device="cuda")

    def step():
        logits = target.forward_all(pool, ids, seqs, tree_parents=par)
        acc, path, _ = ops.accept_tree(logits.view(B, R, V), par, node_dev)
        ops.kv_compact_path(pool, bt_dev, kvo_dev, acc, path)
        return acc

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # each step ends on the host (the accepted counts), so steps time one by
    # one; the first few after the prefill run slower and vary by box, so the
    # value is the median step
    times, accepted = [], 0
    for _ in range(args.steps):
        ts = time.perf_counter()
        accepted += int(step().sum().item()) + B
        times.append((time.perf_counter() - ts) * 1e3)
    ms = float(np.median(times))
    res = {"mode": "tree", "metric": "tree-verify step latency, config 3 (Qwen3-4B shape int4, 16 seqs x ctx 2048, "
                                      "4-2-2 tree)", "value": ms, "unit": "ms per step (median)", "higher_is_better": False,
           "mean_ms": float(np.mean(times)), "min_ms": float(np.min(times)),
           "rows_per_s": B * R / (ms * 1e-3), "committed_tokens_per_step": accepted / args.steps,
           "steps": args.steps, "warmup": args.warmup,
           "config": {"workload": "tree verification + greedy path accept + KV compaction", "batch": B,
                      "context": ctx, "tree_nodes": R - 1, "branching": "4-2-2", "page_size": ps,
                      "block_tables": "shuffled"},
           "data": "synthetic (random-init weights, Philox prompts and tree tokens)"}
    print(json.dumps(res), flush=True)


def run_gemm(args):
    """One verify GEMM shape launched back to back on the engine's packed path
    (cache-rotated weight copies), for counter runs under rocprofv3 --pmc:
    e.g. --mode gemm --shape gate_up --m 80."""
    import torch

    from velox_amd import _lib, ops, synth

    torch.cuda.set_device(0)
    shapes = {"qkv": (6144, 2560), "o": (2560, 4096), "gate_up": (19456, 2560), "down": (2560, 9728),
              "lm_head": (151936, 2560)}
    n, kk = shapes[args.shape]
    lin = synth.qlinear(1, f"bench.{args.shape}", n, kk, 64)
    W = torch.from_numpy(lin["qweight"].view(np.int32)).cuda()
    S = torch.from_numpy(lin["scales"]).cuda()
    Bs = torch.from_numpy(lin["biases"]).cuda()
    copies = max(2, int(np.ceil(640e6 / (0.5625 * n * kk))))
    packed = [ops.qmm_pack_4bit(W, S, Bs) for _ in range(copies)]
    epi = _lib.EPI_SWIGLU if args.shape == "gate_up" else _lib.EPI_STORE
    x = torch.randn((args.m, kk), dtype=torch.float16, device="cuda")
    y = torch.empty((args.m, n // 2 if epi == _lib.EPI_SWIGLU else n), dtype=torch.float16, device="cuda")
    ws = torch.zeros(256 << 20, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(args.iters):
        ops.qmm_4bit_packed(x, packed[i % copies], n, y, epilogue=epi, workspace=ws)
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / args.iters
    byt = 0.5625 * n * kk + 2 * args.m * kk + 2 * y.numel()
    print(json.dumps({"mode": "gemm", "shape": args.shape, "n": n, "k": kk, "m": args.m, "iters": args.iters,
                      "us_per_launch": us, "algorithmic_bytes": byt, "gbs": byt / (us * 1e-6) / 1e9}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=12)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--profile-steps", type=int, default=2)
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--k", type=int, default=4)
    ap.add_argument("--prompt", type=int, default=128)
    ap.add_argument("--mode", choices=["spec", "qmm", "continuous", "tree", "config0", "gemm"], default="spec")
    ap.add_argument("--shape", choices=["qkv", "o", "gate_up", "down", "lm_head"], default="gate_up",
                    help="gemm mode: the verify GEMM shape")
    ap.add_argument("--m", type=int, default=80, help="gemm mode: rows")
    ap.add_argument("--iters", type=int, default=200, help="gemm mode: launches")
    ap.add_argument("--batch-tokens", type=int, default=8192, help="continuous mode: max_batch_tokens")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calib-copy", type=int, default=0, metavar="MB",
                    help="first do one device copy of MB MiB (counter calibration for rocprofv3 --pmc)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); the verify path "
              "shards data-parallel over sequences with no cross-GPU exchange.", file=sys.stderr)
        sys.exit(2)
    if args.mode == "gemm":
        return run_gemm(args)
    if args.mode == "qmm":
        run_qmm(args)
    elif args.mode == "continuous":
        run_continuous(args)
    elif args.mode == "tree":
        run_tree(args)
    elif args.mode == "config0":
        run_config0(args)
    else:
        run_spec(args)


if __name__ == "__main__":
    main()
