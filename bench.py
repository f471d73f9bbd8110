"""Benchmark: the codec decoder stack on one MI355X.

One step = one decode of 48 lanes x 250 latent frames (1024-d, f16) through the qwen3tts-shaped
waveform stack (head conv 1024->1536 k7; 4 upsampling blocks, rates 8/5/4/3, channels
1536->768->384->192->96, 3 residual units each; SnakeBeta; conv 96->1 k7; tanh) to
48 x 120000 samples at 24 kHz = 240 s of audio. Inputs and random-init weights are resident
in HBM before the timed region; the value is audio-seconds per wall-second.

Prints one JSON line. `roofline` is the dominant kernel (largest summed launch time in a
decode), timed per launch with HIP events on the decode's stream; `cpu_baseline` times the
oracle's f32 restatement of the reference's CPU route on a bounded sample of lanes.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "dream-tts_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "codec audio-sec/sec at 48 lanes; fused-op HBM GB/s as % of peak"
PEAK_TFLOPS_F16 = 2500.0  # MI355X dense f16 MFMA
PEAK_HBM_GBS = 8000.0     # MI355X HBM3E
SAMPLE_RATE = 24000


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def dominant(stages_runs):
    """Per kernel: summed algorithmic flops/bytes of one decode's launches and their summed ms
    (mean over the profile runs); returns the kernel with the largest time."""
    by = {}
    for s in stages_runs[0]:
        e = by.setdefault(s["kernel"], dict(flops=0.0, bytes=0.0, ms=0.0, launches=0))
        e["flops"] += s["flops"]
        e["bytes"] += s["bytes"]
        e["launches"] += 1
    for run in stages_runs:
        for s in run:
            by[s["kernel"]]["ms"] += s["ms"] / len(stages_runs)
    name = max(by, key=lambda k: by[k]["ms"])
    return name, by[name], by


def cpu_baseline(geo, weights, latent_np, budget_s=12.0, max_lanes=48):
    import oracle  # noqa: F401  (the oracle is the timed CPU baseline, never the product)
    from oracle import codec as ocodec

    prep = ocodec.prepare(geo, weights)
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    frames = latent_np.shape[1]
    ocodec.decode_f32_reference(geo, prep, latent_np[0, : max(2, frames // 50)])  # warm-up, untimed
    t0 = time.perf_counter()
    done = 0
    while done < max_lanes:
        ocodec.decode_f32_reference(geo, prep, latent_np[done])
        done += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    wall = time.perf_counter() - t0
    audio_s = done * frames * geo.hop / SAMPLE_RATE
    return dict(value=round(audio_s / wall, 3), unit="audio-s/s", cores=threads, kind="port",
                sample=f"{done} lane(s) x {frames} frames of the same workload through the oracle's "
                       f"f32 restatement of the reference CPU route (SnakeBeta passes; pad+cat+GEMM+bias "
                       f"per conv; polyphase transposed convs), {wall:.1f} s on {threads} threads")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--lanes", type=int, default=48)
    ap.add_argument("--frames", type=int, default=250)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--profile-runs", type=int, default=3)
    ap.add_argument("--stages-out", default=None, help="write the per-launch profile as JSON here")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also run a plain 1 GiB copy kernel 3 times (calibrates HBM byte counters)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(lanes are data-parallel; see DESIGN.md for how the path shards)", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from dtts import codec, synth

    dev = torch.device("cuda:0")
    geo = codec.CONFIG5
    t0 = time.perf_counter()
    w = codec.random_weights(geo, seed=0)
    latent_np = synth.normal(0, "latent", (args.lanes, args.frames, geo.latent_dim))
    model = codec.Codec(geo, w, dev)
    latent = torch.from_numpy(synth.f16_bits(latent_np).view(np.int16)).view(torch.float16).to(dev)
    audio = torch.empty((args.lanes, args.frames * geo.hop), dtype=torch.float16, device=dev)
    model.workspace(args.lanes, args.frames)
    torch.cuda.synchronize()
    log(f"setup {time.perf_counter() - t0:.1f} s; weights {model.weight_bytes() / 1e6:.1f} MB on device")

    for _ in range(args.warmup):
        model.decode(latent, out=audio)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        model.decode(latent, out=audio)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = wall * 1e3 / args.steps
    audio_s = args.lanes * args.frames * geo.hop / SAMPLE_RATE
    value = audio_s / (ms / 1e3)
    if not torch.isfinite(audio.float()).all():
        raise SystemExit("bench: non-finite audio")
    log(f"decode: {ms:.3f} ms/step -> {value:.1f} audio-s/s")

    runs = [model.profile(latent, out=audio) for _ in range(args.profile_runs)]
    kname, dom, by = dominant(runs)
    per_launch_ms = dom["ms"] / dom["launches"]
    intensity = dom["flops"] / max(dom["bytes"], 1.0)
    if intensity > PEAK_TFLOPS_F16 * 1e12 / (PEAK_HBM_GBS * 1e9):
        achieved = dom["flops"] / dom["launches"] / (per_launch_ms / 1e3) / 1e12
        roof = dict(bound="mfma", achieved=round(achieved, 2), peak=PEAK_TFLOPS_F16, unit="TFLOP/s")
    else:
        achieved = dom["bytes"] / dom["launches"] / (per_launch_ms / 1e3) / 1e9
        roof = dict(bound="hbm", achieved=round(achieved, 1), peak=PEAK_HBM_GBS, unit="GB/s")
    roof["frac"] = round(roof["achieved"] / roof["peak"], 4)
    roof["traffic"] = None
    roof["kernel"] = kname
    roof["launches_per_step"] = dom["launches"]
    roof["ms_per_launch"] = round(per_launch_ms, 4)
    total_prof = sum(s["ms"] for s in runs[-1])
    log(f"profile: {total_prof:.3f} ms summed over {len(runs[-1])} launches")
    for k, e in sorted(by.items(), key=lambda kv: -kv[1]["ms"]):
        log(f"  {e['ms']:8.3f} ms  {e['launches']:2d}x  {e['flops'] / e['ms'] / 1e9:8.1f} TFLOP/s  "
            f"{e['bytes'] / e['ms'] / 1e6:7.0f} GB/s  {k}")
    for s in runs[-1]:
        log(f"    {s['name']:22s} L={s['len']:6d} {s['cin']:5d}->{s['cout']:5d} k{s['k']} d{s['dilation']}  "
            f"{s['ms']:7.3f} ms  {s['flops'] / s['ms'] / 1e9:7.1f} TFLOP/s  {s['bytes'] / s['ms'] / 1e6:6.0f} GB/s")
    if args.stages_out:
        with open(args.stages_out, "w") as f:
            json.dump(dict(ms_per_step=ms, stages=runs[-1]), f, indent=1)

    if args.copy_probe:
        src = torch.ones(1 << 29, dtype=torch.float16, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.mul(src, 1.0, out=dst)  # an elementwise kernel (a same-dtype copy_ may go to DMA)
        torch.cuda.synchronize()
        log(f"copy probe: 3 x {src.numel() * 2} bytes read and written by a mul kernel")
        del src, dst

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(geo, w, latent_np)
        log(f"cpu baseline: {cpu}")

    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "audio-s/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "config5: codec decoder stack, f16 storage / f32 accumulation, "
                               "random-init weights (Kaiming-normal gain 1)",
                   "lanes": args.lanes, "frames": args.frames, "latent_dim": geo.latent_dim,
                   "channels": list(geo.channels), "rates": list(geo.rates),
                   "audio_s_per_step": audio_s, "parallelism": "single GPU"},
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
