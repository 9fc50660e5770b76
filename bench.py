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
import json
import os
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "splatting-rs_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

PEAK_TFLOPS = {"bf16": 2500.0, "f32": 157.3}   # dense MFMA, MI355X
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


def cpu_baseline(cfg, spec, weights, seed):
    """The CPU oracle (torch fp32, a restatement of the reference, not candle) timed on a
    bounded sample of the workload: the full forward up to 6 views, else the same
    architecture on 6 of the views (the encoder-only config stays encoder-only)."""
    import torch
    from splathip import synth
    from oracle import da3 as OD
    from oracle import mapanything as OM
    threads = max(1, min(16, os.cpu_count() or 1))
    torch.set_num_threads(threads)
    views = min(cfg.views, 6)
    images = synth.config_images(cfg, seed)[:views]
    p = {k: torch.from_numpy(v) for k, v in weights.items()}
    t = time.perf_counter()
    if cfg.model == "da3":
        OD.forward_raw(p, spec, images)
    else:
        OM.forward(p, spec, images, encoder_only=cfg.encoder_only)
    dt = time.perf_counter() - t
    return {"value": views / dt, "unit": "views/s", "cores": threads, "kind": "port",
            "sample": f"{views}-view forward of the {cfg.key} architecture at {cfg.height}x{cfg.width}, fp32 "
                      f"torch-CPU restatement of the reference (not candle), {dt:.1f} s"}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="C4", choices=["C1", "C2", "C3", "C4", "C5"])
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-graphs", action="store_true", help="eager launches instead of HIP graph replay")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--profile-out", default="", help="write the per-kernel-class profile as JSON here")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run a plain 256 MiB -> 256 MiB streaming kernel (torch.neg on fp32), the "
                         "reference that scales FETCH_SIZE / WRITE_SIZE counter runs to bytes")
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
    if args.copy_calibration:
        src = torch.ones(COPY_CAL_BYTES // 4, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst
    cfg = specs.CONFIGS[args.config]
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

    cpu = None
    if not args.no_cpu_baseline:
        log("timing the CPU baseline ...")
        cpu = cpu_baseline(cfg, spec, weights, args.seed + 1)
        log(f"cpu baseline: {cpu}")

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
        "forward_tflop": mfma_flops / 1e12,
        "mfma_util_forward": mfma_flops / (ms * 1e-3) / 1e12 / PEAK_TFLOPS[cfg.dtype],
        "mfma_util_mfma_kernels": (mfma_flops / (mfma_ms * 1e-3) / 1e12 / PEAK_TFLOPS[cfg.dtype]) if mfma_ms else None,
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
