#!/usr/bin/env python
"""Throughput of the feed-forward reconstruction forward on one MI355X.

A step is one forward of the configuration's network over its batch of views (seeded
synthetic weights and images, inputs resident in HBM before the timed region, outputs left
in HBM). The default workload is BASELINE config 4: MapAnything (ViT-L/14 encoder, 24-block
768-wide alternating-attention transformer, DPT + pose + scale heads), 6 views at 518x392,
bf16. Prints one JSON line; details go to stderr.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--config C1..C5]
"""
import argparse
import dataclasses
import json
import os
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "splatting-rs_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

PEAK_TFLOPS = {"bf16": 2500.0, "f16": 2500.0, "f32": 157.3}   # dense MFMA, MI355X
PEAK_HBM_GBS = 8000.0
MFMA_KERNELS = ("gemm", "conv_igemm", "attention")
COPY_CAL_BYTES = 256 << 20
# HBM bytes per launch of a kernel class, from FETCH_SIZE / WRITE_SIZE counter runs of this
# script (each scaled by the same counter on the --copy-calibration kernel); written next to
# the rocprofv3 summaries it comes from.
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")


def measured_traffic(cfg_key, kernel):
    try:
        with open(TRAFFIC_FILE) as f:
            rec = json.load(f).get(cfg_key, {}).get(kernel)
    except (OSError, ValueError):
        return None
    return rec["bytes_per_launch"] if rec else None


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def build_model(ctx, cfg, seed, tmpdir):
    from splathip import specs, synth
    t = time.time()
    if cfg.model == "da3":
        spec = specs.DA3_VARIANTS[cfg.spec]
        w = synth.generate(synth.da3_shapes(spec), seed=seed)
    else:
        spec = specs.MA_SPECS[cfg.spec]
        w = synth.generate(synth.ma_shapes(spec), seed=seed)
    path = os.path.join(tmpdir, f"{cfg.key}.safetensors")
    synth.save(path, w)
    log(f"weights: {sum(v.size for v in w.values()) / 1e6:.1f} M params, generated+saved in {time.time() - t:.1f} s")
    t = time.time()
    if cfg.model == "da3":
        ctx.load_da3(path, cfg.spec, cfg.dtype, specs.REF_SADDLE)
    else:
        ctx.load_mapanything(path, spec, cfg.dtype)
    log(f"loaded in {time.time() - t:.1f} s")
    os.unlink(path)
    return spec, w


def make_step(ctx, cfg, spec, images_dev, torch):
    V, H, W = cfg.views, cfg.height, cfg.width
    R, Cc = H // 14, W // 14
    dev = "cuda"
    if cfg.model == "da3":
        outs = {
            "depth": torch.empty(V, H, W, device=dev),
            "depth_conf": torch.empty(V, H, W, device=dev),
            "ray_logits": torch.empty(V, 7, 8 * R, 8 * Cc, device=dev),
            "pose_encoding": torch.empty(V, 9, device=dev),
            "camera_tokens": torch.empty(V, 2 * spec.dim, device=dev),
        }
        ref = torch.zeros(1, dtype=torch.int32, device=dev)
        ptrs = {k: v.data_ptr() for k, v in outs.items()}

        def step():
            ctx.da3_forward_raw_device(images_dev.data_ptr(), V, H, W, ptrs, ref.data_ptr())
        return step, outs
    if cfg.encoder_only:
        tok = torch.empty(V, 1 + R * Cc, spec.enc_dim, device=dev)

        def step():
            ctx.ma_encode_device(images_dev.data_ptr(), V, H, W, tok.data_ptr())
        return step, {"tokens": tok}
    outs = {
        "raw": torch.empty(V, 6, H, W, device=dev),
        "quaternion": torch.empty(V, 4, device=dev),
        "translation": torch.empty(V, 3, device=dev),
        "scale": torch.empty(1, device=dev),
        "points": torch.empty(V, H, W, 3, device=dev),
        "conf": torch.empty(V, H, W, device=dev),
        "mask": torch.empty(V, H, W, dtype=torch.uint8, device=dev),
    }
    ptrs = {k: v.data_ptr() for k, v in outs.items()}

    def step():
        ctx.ma_forward_device(images_dev.data_ptr(), V, H, W, ptrs)
    return step, outs


def host_cpu():
    """What the host offers this process: nproc, the CPUs it may run on, the CPU model, and
    the thread count the job is given (OMP_NUM_THREADS: this pool gives a one-GPU job 16)."""
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), "")
    except OSError:
        pass
    nproc = os.cpu_count() or 1
    affinity = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else nproc
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or min(16, affinity)
    return {"nproc": nproc, "affinity_cpus": affinity, "job_threads": max(1, min(share, affinity)), "cpu_model": model}


def _oracle_forward(cfg, spec, p, images):
    from oracle import da3 as OD
    from oracle import mapanything as OM
    if cfg.model == "da3":
        OD.forward_raw(p, spec, images)
    else:
        OM.forward(p, spec, images, encoder_only=cfg.encoder_only)


def cpu_baseline(cfg, spec, weights, seed, threads, host):
    """The CPU oracle (torch fp32, a restatement of the reference, not candle) timed on a
    bounded sample of the workload: the full forward up to 6 views, else the same
    architecture on 6 of the views (the encoder-only config stays encoder-only)."""
    import torch
    from splathip import synth
    torch.set_num_threads(threads)
    views = min(cfg.views, 6)
    images = synth.config_images(cfg, seed)[:views]
    p = {k: torch.from_numpy(v) for k, v in weights.items()}
    t = time.perf_counter()
    _oracle_forward(cfg, spec, p, images)
    dt = time.perf_counter() - t
    return {"value": views / dt, "unit": "views/s", "cores": threads, "kind": "port",
            "sample": f"{views}-view forward of the {cfg.key} architecture at {cfg.height}x{cfg.width}, fp32 "
                      f"torch-CPU restatement of the reference (not candle), {dt:.1f} s on {threads} threads",
            "nproc": host["nproc"], "affinity_cpus": host["affinity_cpus"], "cpu_model": host["cpu_model"]}


def cpu_one_thread_c2(seed):
    """BASELINE config 2 (DA3-Small, 6 views 378x504) on one thread, fp32 restatement: the
    counterpart of the reference's own single-thread number (23.5 s for the same network and
    views on an M5 core, wasm32; instantsplat-rs/web/README.md:35-38)."""
    import torch
    from splathip import specs, synth
    cfg = specs.CONFIGS["C2"]
    spec = specs.DA3_VARIANTS[cfg.spec]
    w = synth.generate(synth.da3_shapes(spec), seed=seed)
    p = {k: torch.from_numpy(v) for k, v in w.items()}
    images = synth.config_images(cfg, seed + 1)
    prev = torch.get_num_threads()
    torch.set_num_threads(1)
    try:
        t = time.perf_counter()
        _oracle_forward(cfg, spec, p, images)
        dt = time.perf_counter() - t
    finally:
        torch.set_num_threads(prev)
    return {"seconds": dt, "views_per_s": cfg.views / dt, "threads": 1, "kind": "port",
            "sample": "C2: DA3-Small, 6 views 378x504, full forward, fp32 torch-CPU restatement (not candle)"}


def time_config(ctx, key, seed, steps, warmup, tmp, torch, loaded=None):
    """GPU ms/forward of another configuration (graph replay, inputs resident in HBM), for the
    extra keys of the line. `loaded`: the (model, spec, dtype) the context holds, reused when the
    configuration runs the same network (its weights come from the same seed)."""
    import splathip
    from splathip import specs, synth
    cfg = specs.CONFIGS[key]
    if loaded == (cfg.model, cfg.spec, cfg.dtype):
        spec = specs.DA3_VARIANTS[cfg.spec] if cfg.model == "da3" else specs.MA_SPECS[cfg.spec]
    else:
        spec, _ = build_model(ctx, cfg, seed, tmp)
    images = torch.from_numpy(synth.config_images(cfg, seed + 1)).cuda()
    step, _ = make_step(ctx, cfg, spec, images, torch)
    stream = torch.cuda.ExternalStream(ctx.stream)
    torch.cuda.synchronize()
    for _ in range(max(1, warmup)):
        step()
    ctx.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        step()
    e1.record(stream)
    ctx.synchronize()
    ms = e0.elapsed_time(e1) / steps
    log(f"{key}: {ms:.3f} ms/forward (events, {steps} forwards)")
    return {"ms_per_forward": ms, "views_per_s": cfg.views / (ms * 1e-3), "dtype": cfg.dtype, "steps": steps,
            "workload": f"{key}: {cfg.description}"}


def time_host_io(ctx, cfg, seed, reps):
    """ms per forward through the host-pointer entry point (images copied in, outputs copied
    out over PCIe, synchronous), the reference's calling convention."""
    from splathip import synth
    images = synth.config_images(cfg, seed + 1)
    fwd = (lambda: ctx.da3_forward_raw(images)) if cfg.model == "da3" else \
          (lambda: ctx.ma_encode(images)) if cfg.encoder_only else (lambda: ctx.ma_forward(images))
    fwd()
    t = time.perf_counter()
    for _ in range(reps):
        fwd()
    return 1e3 * (time.perf_counter() - t) / reps


# (M, N, K, epilogue): the transformer layers' GEMMs of the benchmark configurations. "ln": a
# folded-LayerNorm consumer (qkv, or fc1 with GELU), "res": a residual producer with row
# statistics and a bf16 copy (proj, fc2). M = 6222 (C4: 6 views of 1037 encoder tokens), 6223 (C4
# info-sharing, 6 x 1037 + 1), 5838 (C2: 6 x 973).
GEMM_SHAPES = [(6222, 3072, 1024, "ln"), (6222, 1024, 1024, "res"), (6222, 4096, 1024, "ln-gelu"),
               (6222, 1024, 4096, "res"), (6223, 2304, 768, "ln"), (6223, 768, 768, "res"),
               (6223, 3072, 768, "ln-gelu"), (6223, 768, 3072, "res"), (5838, 1152, 384, "ln"),
               (5838, 384, 384, "res"), (5838, 1536, 384, "ln-gelu"), (5838, 384, 1536, "res"),
               (8192, 8192, 8192, "plain")]


def gemm_vs_hipblaslt(torch, splathip):
    """The library's bf16 GEMM (splat_kernel_gemm, bias epilogue; splat_kernel_gemm_ln, the fused
    epilogue the forward uses) against torch.addmm on the same operands (rocBLAS/hipBLASLt), each
    timed with events around 50 back-to-back launches (10 for 8192^3) after 5 warm-up ones."""
    ctx = splathip.Context(0)
    ours = torch.cuda.ExternalStream(ctx.stream)
    dt, tdt = splathip.BF16, torch.bfloat16

    def timed(fn, stream, reps):
        for _ in range(5):
            fn()
        torch.cuda.synchronize()
        ctx.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        ctx.synchronize()
        return e0.elapsed_time(e1) / reps * 1e3

    g = torch.Generator(device="cuda").manual_seed(0)
    for (M, N, K, epi) in GEMM_SHAPES:
        reps = 10 if M == 8192 else 50
        A = torch.randn(M, K, device="cuda", generator=g).to(tdt)
        W = (torch.randn(N, K, device="cuda", generator=g) * 0.05).to(tdt)
        b = torch.randn(N, device="cuda", generator=g)
        out = torch.empty(M, N, device="cuda", dtype=tdt)
        bt = b.to(tdt)
        torch.cuda.synchronize()
        t_plain = timed(lambda: ctx.kernel_gemm(dt, A.data_ptr(), M, K, W.data_ptr(), N, K, b.data_ptr(), 0,
                                                out.data_ptr(), False), ours, reps)
        t_lib = timed(lambda: torch.addmm(bt, A, W.t(), out=out), torch.cuda.current_stream(), reps)
        t_fused = None
        if epi.startswith("ln"):
            c1 = torch.randn(N, device="cuda", generator=g)
            st = torch.rand(M, K // 64, 2, device="cuda", generator=g) + 1
            act = 2 if epi == "ln-gelu" else 0
            torch.cuda.synchronize()
            t_fused = timed(lambda: ctx.kernel_gemm_ln(dt, A.data_ptr(), M, K, W.data_ptr(), N, K, b.data_ptr(), act,
                                                       out.data_ptr(), False, ln_in=st.data_ptr(), c1=c1.data_ptr(),
                                                       eps=1e-6, group=64), ours, reps)
        elif epi == "res":
            gm = torch.rand(N, device="cuda", generator=g)
            r = torch.randn(M, N, device="cuda", generator=g)
            o32 = torch.empty(M, N, device="cuda")
            stats = torch.empty(M, N // 64, 2, device="cuda")
            cp = torch.empty(M, N, device="cuda", dtype=tdt)
            torch.cuda.synchronize()
            t_fused = timed(lambda: ctx.kernel_gemm_ln(dt, A.data_ptr(), M, K, W.data_ptr(), N, K, b.data_ptr(), 0,
                                                       o32.data_ptr(), True, gamma=gm.data_ptr(), res=r.data_ptr(),
                                                       ln_out=stats.data_ptr(), copy=cp.data_ptr(), group=64),
                            ours, reps)
        fl = 2.0 * M * N * K
        line = {"shape": [M, N, K], "epilogue": epi, "ours_plain_us": round(t_plain, 2),
                "hipblaslt_us": round(t_lib, 2), "ours_plain_tflops": round(fl / t_plain / 1e6, 1),
                "hipblaslt_tflops": round(fl / t_lib / 1e6, 1)}
        if t_fused is not None:
            line["ours_fused_us"] = round(t_fused, 2)
        print(json.dumps(line), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="C4", choices=["C1", "C2", "C3", "C4", "C5"])
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--dtype", choices=["bf16", "f16", "f32"], default=None,
                    help="model dtype (default: the configuration's, bf16 for the benchmark line)")
    ap.add_argument("--no-graphs", action="store_true", help="eager launches instead of HIP graph replay")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the extra keys (other configurations' GPU times, host-I/O time, 1-thread C2 CPU time)")
    ap.add_argument("--profile-out", default="", help="write the per-kernel-class profile as JSON here")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run a plain 256 MiB -> 256 MiB streaming kernel (torch.neg on fp32), the "
                         "reference that scales FETCH_SIZE / WRITE_SIZE counter runs to bytes")
    ap.add_argument("--gemm-vs-hipblaslt", action="store_true",
                    help="instead of the forward: time the library's GEMM on the network's layer shapes (plain "
                         "bias epilogue, then the forward's fused epilogue) next to torch.matmul on the same "
                         "shapes (hipBLASLt), one JSON line per shape")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (the network would "
              "shard by views with one K/V exchange per global block). Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    import splathip
    from splathip import specs, synth

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.gemm_vs_hipblaslt:
        gemm_vs_hipblaslt(torch, splathip)
        return
    if args.copy_calibration:
        src = torch.ones(COPY_CAL_BYTES // 4, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst
    cfg = specs.CONFIGS[args.config]
    if args.dtype and args.dtype != cfg.dtype:
        cfg = dataclasses.replace(cfg, dtype=args.dtype,
                                  description=cfg.description.replace(f", {cfg.dtype}", f", {args.dtype}"))
    host = host_cpu()
    ctx = splathip.Context(0)
    with tempfile.TemporaryDirectory(dir="/tmp") as tmp:
        spec, weights = build_model(ctx, cfg, args.seed, tmp)
    images = torch.from_numpy(synth.config_images(cfg, args.seed + 1)).cuda()
    ctx.set_graphs(not args.no_graphs)
    step, outs = make_step(ctx, cfg, spec, images, torch)
    stream = torch.cuda.ExternalStream(ctx.stream)
    torch.cuda.synchronize()  # images were written on torch's stream; the library uses its own

    for _ in range(max(1, args.warmup)):
        step()
    ctx.synchronize()
    torch.cuda.synchronize()

    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    wall0 = time.perf_counter()
    e0.record(stream)
    for _ in range(args.steps):
        step()
    e1.record(stream)
    ctx.synchronize()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms = e0.elapsed_time(e1) / args.steps
    log(f"{cfg.key}: {ms:.3f} ms/forward (events), wall {1e3 * wall / args.steps:.3f} ms/step")
    # after the timed region: forwards timed one by one (an event pair around each) for the
    # median and the 90th percentile
    pairs = []
    for _ in range(min(args.steps, 50)):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        step()
        b.record(stream)
        pairs.append((a, b))
    ctx.synchronize()
    each = sorted(a.elapsed_time(b) for a, b in pairs)
    ms_median, ms_p90 = each[len(each) // 2], each[min(len(each) - 1, (9 * len(each)) // 10)]
    log(f"{cfg.key}: median {ms_median:.3f} ms, p90 {ms_p90:.3f} ms over {len(each)} single forwards")

    # one profiled forward: per-kernel-class durations from HIP events on the library stream
    ctx.profile_begin()
    step()
    stats = ctx.profile_end()
    for s in stats:
        log(f"  {s['name']:16s} launches {s['launches']:5d}  {s['ms']:8.3f} ms  "
            f"{s['flops'] / max(s['ms'], 1e-9) / 1e9:8.1f} TFLOP/s  {s['bytes'] / max(s['ms'], 1e-9) / 1e6:8.1f} GB/s")
    if args.profile_out:
        with open(args.profile_out, "w") as f:
            json.dump({"config": cfg.key, "ms_per_forward": ms, "kernels": stats}, f, indent=1)
    dom = stats[0]
    if dom["name"] in MFMA_KERNELS:
        achieved = dom["flops"] / (dom["ms"] * 1e-3) / 1e12
        roof = {"bound": "mfma", "achieved": achieved, "peak": PEAK_TFLOPS[cfg.dtype], "unit": "TFLOP/s"}
    else:
        achieved = dom["bytes"] / (dom["ms"] * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s"}
    roof["frac"] = roof["achieved"] / roof["peak"]
    roof["traffic"] = measured_traffic(cfg.key, dom["name"])
    roof["kernel"] = dom["name"]
    roof["launches_per_forward"] = dom["launches"]
    roof["avg_launch_us"] = 1e3 * dom["ms"] / dom["launches"]
    mfma_flops = sum(s["flops"] for s in stats if s["name"] in MFMA_KERNELS)
    mfma_ms = sum(s["ms"] for s in stats if s["name"] in MFMA_KERNELS)

    extra = {}
    if not args.no_extra:
        extra["host_io_ms_per_forward"] = time_host_io(ctx, cfg, args.seed, max(3, args.steps // 4))
        log(f"{cfg.key} through host buffers (PCIe in and out): {extra['host_io_ms_per_forward']:.3f} ms/forward")
        # every other BASELINE configuration, the MapAnything ones first while the ViT-L model
        # is loaded; C5's 24-view forwards (~60 ms) get a tenth of the steps
        others = {}
        loaded = (cfg.model, cfg.spec, cfg.dtype)
        with tempfile.TemporaryDirectory(dir="/tmp") as tmp:
            for key in ("C3", "C5", "C1", "C2"):
                if key == cfg.key:
                    continue
                k = specs.CONFIGS[key]
                n = max(10, args.steps // 10) if k.views > 6 else args.steps
                others[key] = time_config(ctx, key, args.seed, n, args.warmup, tmp, torch, loaded)
                loaded = (k.model, k.spec, k.dtype)
        extra["other_configs"] = others

    cpu = None
    if not args.no_cpu_baseline:
        log(f"timing the CPU baseline ({host['job_threads']} threads of {host['nproc']}, {host['cpu_model']}) ...")
        cpu = cpu_baseline(cfg, spec, weights, args.seed + 1, host["job_threads"], host)
        log(f"cpu baseline: {cpu}")
        if not args.no_extra:
            log("timing C2 on one CPU thread ...")
            extra["cpu_c2_one_thread"] = cpu_one_thread_c2(args.seed)
            log(f"cpu C2 one thread: {extra['cpu_c2_one_thread']}")

    V = cfg.views
    R, Cc = cfg.height // 14, cfg.width // 14
    tokens = V * (R * Cc + 1) + (1 if cfg.model == "ma" and not cfg.encoder_only else 0)
    line = {
        "metric": "views/sec",
        "value": V / (ms * 1e-3),
        "unit": "views/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg.dtype,
        "data": "synthetic: seeded N(0,0.02) weights (LayerScale 1e-5), seeded "
                + ("uniform" if cfg.images == "uniform" else "procedural") + " images",
        "config": {"workload": f"{cfg.key}: {cfg.description}", "views": V, "height": cfg.height,
                   "width": cfg.width, "global_tokens": tokens, "graphs": not args.no_graphs,
                   "parallelism": "none (1 GPU)"},
        "ms_per_forward": ms,
        "ms_per_forward_median": ms_median,
        "ms_per_forward_p90": ms_p90,
        "forward_tflop": mfma_flops / 1e12,
        "mfma_util_forward": mfma_flops / (ms * 1e-3) / 1e12 / PEAK_TFLOPS[cfg.dtype],
        "mfma_util_mfma_kernels": (mfma_flops / (mfma_ms * 1e-3) / 1e12 / PEAK_TFLOPS[cfg.dtype]) if mfma_ms else None,
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    line.update(extra)
    print(json.dumps(line), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
