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
import re
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


def cpu_model():
    """The host CPU as /proc/cpuinfo names it, with its family and model numbers (which identify the
    generation where a VM shortens the name) and the logical CPUs the system reports."""
    fields = {}
    try:
        for line in open("/proc/cpuinfo"):
            key, _, val = line.partition(":")
            key = key.strip()
            if key in ("model name", "cpu family", "model") and key not in fields:
                fields[key] = val.strip()
            if len(fields) == 3:
                break
    except OSError:
        return None
    if "model name" not in fields:
        return None
    return (f"{fields['model name']} (family {fields.get('cpu family', '?')}, model {fields.get('model', '?')}, "
            f"{os.cpu_count()} logical CPUs)")


def kernel_rooflines(by):
    """Every kernel of one decode at its own roofline: MFMA-bound when its algorithmic intensity
    (FLOP per byte, each input, output and weight once) is above the ridge, HBM-bound below."""
    ridge = PEAK_TFLOPS_F16 * 1e12 / (PEAK_HBM_GBS * 1e9)
    out = []
    for name, e in sorted(by.items(), key=lambda kv: -kv[1]["ms"]):
        per = e["ms"] / e["launches"]
        if e["flops"] / max(e["bytes"], 1.0) > ridge:
            ach, peak, unit, bound = e["flops"] / e["launches"] / (per / 1e3) / 1e12, PEAK_TFLOPS_F16, "TFLOP/s", "mfma"
        else:
            ach, peak, unit, bound = e["bytes"] / e["launches"] / (per / 1e3) / 1e9, PEAK_HBM_GBS, "GB/s", "hbm"
        out.append({"kernel": name, "launches": e["launches"], "ms_per_launch": round(per, 4),
                    "share": None, "bound": bound, "achieved": round(ach, 1), "peak": peak, "unit": unit,
                    "frac": round(ach / peak, 4)})
    total = sum(e["ms"] for e in by.values())
    for o, (name, e) in zip(out, sorted(by.items(), key=lambda kv: -kv[1]["ms"])):
        o["share"] = round(e["ms"] / total, 4)
    return out


def cpu_baseline(geo, weights, latent_np, budget_s=12.0, max_lanes=48):
    import oracle  # noqa: F401  (the oracle is the timed CPU baseline, never the product)
    from oracle import codec as ocodec

    prep = ocodec.prepare(geo, weights)
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    frames = latent_np.shape[1]
    ocodec.decode_f32_reference(geo, prep, latent_np[0, : max(2, frames // 50)])  # warm-up, untimed
    t0 = time.perf_counter()
    lane_s = []
    while len(lane_s) < max_lanes:
        t1 = time.perf_counter()
        ocodec.decode_f32_reference(geo, prep, latent_np[len(lane_s)])
        lane_s.append(time.perf_counter() - t1)
        if time.perf_counter() - t0 >= budget_s:
            break
    wall = time.perf_counter() - t0
    done = len(lane_s)
    audio_s = done * frames * geo.hop / SAMPLE_RATE
    med = sorted(lane_s)[done // 2]
    return dict(value=round(audio_s / wall, 3), unit="audio-s/s", cores=threads, kind="port", cpu_model=cpu_model(),
                sample=f"{done} lane(s) x {frames} frames of the same workload through the oracle's "
                       f"f32 restatement of the reference CPU route (SnakeBeta passes; pad+cat+GEMM+bias "
                       f"per conv; polyphase transposed convs), {wall:.1f} s on {threads} threads; per lane "
                       f"median {med:.2f} s, range {min(lane_s):.2f}-{max(lane_s):.2f} s")


# ---------------------------------------------------------------- configs 1-4 (per-op lines)

PEAK_TFLOPS_F32 = 157.3   # MI355X dense fp32 matrix


def _time(fn, reps=20, warm=3):
    """Mean ms per call between HIP events on torch's current stream (where libdtts launches)."""
    import torch

    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def _graph_time(fn, reps=20, inner=1):
    """Mean ms per call of `fn`, captured `inner` times back to back in one HIP graph and
    replayed (the host launch cost leaves; what remains is the kernels' own time on the GPU)."""
    import torch

    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(inner):
            fn()
    g.replay()
    torch.cuda.synchronize()
    return _time(g.replay, reps=reps, warm=2) / inner


def _line(workload, metric, value, unit, ops_, extra=None):
    d = {"metric": metric, "value": round(value, 3), "unit": unit, "n_gpus": 1, "higher_is_better": True,
         "dtype": None, "data": "synthetic", "config": {"workload": workload}, "ops": ops_}
    if extra:
        d.update(extra)
    return d


def workload_cfg1(dev, args):
    """Config 1: one residual unit [1, 512, 4800] f32, channel-major (f32 matrix cores)."""
    import numpy as np
    import torch

    from dtts import nlc, synth
    import oracle

    c, length = 512, 4800
    x = torch.from_numpy(synth.normal(0, "cfg1.x", (1, c, length))).to(dev)
    a1 = synth.uniform(0, "cfg1.alpha1", (c,), 0.5, 1.5)
    a2 = synth.uniform(0, "cfg1.alpha2", (c,), 0.5, 1.5)
    f = lambda v: torch.from_numpy(np.ascontiguousarray(v, np.float32)).to(dev)
    w1_oik = synth.kaiming_normal(0, "cfg1.w1", (c, c, 7), c * 7)
    w2_oik = synth.kaiming_normal(0, "cfg1.w2", (c, c, 1), c)
    w1, w2 = f(nlc.tap_major_weight(w1_oik)), f(nlc.tap_major_weight(w2_oik))  # the product's host layout
    b1, b2 = f(synth.normal(0, "cfg1.b1", (c,), 0, 0.01)), f(synth.normal(0, "cfg1.b2", (c,), 0, 0.01))
    s1, s2 = (f(a1), f(1.0 / a1)), (f(a2), f(1.0 / a2))
    h = torch.empty_like(x)
    y = torch.empty_like(x)
    k7 = lambda: nlc.conv1d_ncl_f32(x, w1, b1, k=7, dilation=3, pad_left=9, snake_in=s1, snake_out=s2, out=h)
    k1 = lambda: nlc.conv1d_ncl_f32(h, w2, b2, k=1, residual=x, out=y)
    t7, t1 = _time(k7), _time(k1)
    f7, f1 = 2.0 * c * c * 7 * length, 2.0 * c * c * length
    by = 4.0 * c * length
    ops_ = {"conv7_snake2": {"ms": t7, "tflops": f7 / t7 / 1e9, "frac_f32_peak": f7 / t7 / 1e9 / PEAK_TFLOPS_F32},
            "conv1_residual": {"ms": t1, "tflops": f1 / t1 / 1e9, "gbs": 3 * by / t1 / 1e6}}
    # CPU: the reference route on the oracle (snake pass, im2col + GEMM + bias, snake, GEMM, + x)
    xn = synth.normal(0, "cfg1.x", (1, c, length))
    w1n, w2n = oracle.tap_major_weight_f32(w1_oik), oracle.tap_major_weight_f32(w2_oik)
    t0 = time.perf_counter()
    sn = oracle.snake_ncl_f32(xn, a1, (1.0 / a1).astype(np.float32))
    hn = oracle.conv1d_ncl_gemm_f32(sn, w1n, b1.cpu().numpy(), 7, 3, 9)
    hn = oracle.snake_ncl_f32(hn, a2, (1.0 / a2).astype(np.float32))
    _ = oracle.conv1d_ncl_gemm_f32(hn, w2n, b2.cpu().numpy(), 1, 1, 0) + xn
    cpu_ms = (time.perf_counter() - t0) * 1e3
    return _line("config1: residual unit [1,512,4800] f32 NCL", "residual-unit ms (f32)", t7 + t1, "ms", ops_,
                 {"higher_is_better": False, "dtype": "f32",
                  "cpu_baseline": {"value": round(cpu_ms, 2), "unit": "ms", "kind": "port",
                                   "cores": int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1)),
                                   "sample": "the whole unit through the oracle's im2col + GEMM route"}})


def workload_cfg2(dev, args):
    """Config 2: talker per-step norm/position ops at 48 lanes, f16 (latency-bound)."""
    import numpy as np
    import torch

    from dtts import ops, synth

    b, heads, n_kv, hd, cap = 48, 16, 8, 128, 2048
    f16 = lambda v: torch.from_numpy(synth.f16_bits(v).view(np.int16)).view(torch.float16).to(dev)
    hsd = f16(synth.normal(0, "cfg2.h", (b, 1, 1024)))
    gam = f16(synth.uniform(0, "cfg2.gamma", (1024,), 0.9, 1.1))
    q = f16(synth.normal(0, "cfg2.q", (b, heads, hd)))
    k = f16(synth.normal(0, "cfg2.k", (b, n_kv, hd)))
    v = f16(synth.normal(0, "cfg2.v", (b, n_kv, hd)))
    qkv = f16(synth.normal(0, "cfg2.qkv", (b, (heads + 2 * n_kv) * hd)))
    norms = torch.from_numpy(synth.uniform(0, "cfg2.norms", (2, hd), 0.5, 1.5)).to(dev)
    c, s = ops.rope_table_f32(cap, hd, 1e6)
    c, s = torch.from_numpy(c).to(dev), torch.from_numpy(s).to(dev)
    pos = synth.randint(0, "cfg2.pos", (b,), 0, cap - 1).astype(np.int32)
    kc = torch.zeros((b, n_kv, cap, hd), dtype=torch.float16, device=dev)
    vc = torch.zeros_like(kc)
    yq, yk, yh = torch.empty_like(q), torch.empty_like(k), torch.empty_like(hsd)
    qa = torch.from_numpy(synth.normal(0, "cfg2.qa", (b, n_kv, heads // n_kv, hd), 0, 0.1)).to(dev)
    ya = torch.empty_like(qa)
    kc.copy_(torch.from_numpy(synth.normal(0, "cfg2.kc", (b, n_kv, cap, hd))).half())
    vc.copy_(torch.from_numpy(synth.normal(0, "cfg2.vc", (b, n_kv, cap, hd))).half())
    span = pos.astype(np.int32) + 1
    wsa = torch.empty(ops.decode_attention_workspace_bytes(b, n_kv, heads // n_kv, hd, int(span.max())),
                      dtype=torch.uint8, device=dev)
    fns = {
        "rms_norm_f16": (lambda: ops.rms_norm(hsd, gam, 1e-6, out=yh), 2 * 2 * b * 1024 + 2048),
        "rope_q_f16": (lambda: ops.rope(q, c, s, pos, out=yq), 2 * 2 * q.numel() + 8 * b * hd // 2),
        "rope_k_f16": (lambda: ops.rope(k, c, s, pos, out=yk), 2 * 2 * k.numel() + 8 * b * hd // 2),
        "kv_append_f16": (lambda: ops.kv_append(k, v, pos, kc, vc), 2 * 2 * (k.numel() + v.numel())),
        "qk_norm_rope_kv_append_f16": (lambda: ops.qk_norm_rope_kv_append(qkv, norms, c, s, pos, kc, vc, heads, 1e-6),
                                       2 * qkv.numel() + 2 * b * heads * hd + 2 * 2 * b * n_kv * hd),
        # each lane attends to its positions 0..pos (the cache read once per kv head)
        "decode_attention_f16": (lambda: ops.decode_attention(qa, kc, vc, span, out=ya, workspace=wsa),
                                 int(2 * 2 * n_kv * hd * span.sum()) + 2 * 4 * qa.numel()),
    }
    res = {}
    for name, (fn, nbytes) in fns.items():
        t = _graph_time(fn, reps=20, inner=100)
        res[name] = {"us": t * 1e3, "gbs": nbytes / t / 1e6, "bytes": nbytes}
    total = sum(r["us"] for r in res.values())
    # The attention above replays one cache, whose 198 MB read fits the 256 MB MALL: part of it can
    # come from there. Three copies read in turn (594 MB between reuses) give the HBM-bound rate
    # the talker step sees (28 layers' caches per step); reported beside the line, not in its sum.
    sets = [(kc, vc)] + [(kc.clone(), vc.clone()) for _ in range(2)]
    rot = lambda: [ops.decode_attention(qa, a, b_, span, out=ya, workspace=wsa) for a, b_ in sets]
    t = _graph_time(rot, reps=10, inner=20) / len(sets)
    nb = fns["decode_attention_f16"][1]
    res["decode_attention_f16_past_mall"] = {"us": t * 1e3, "gbs": nb / t / 1e6, "bytes": nb,
                                             "note": "three caches read in turn; not in the line's sum"}
    del sets
    return _line("config2: talker step norm/RoPE/KV append and decode attention over the cache, 48 lanes f16 "
                 "(graph-replayed; all but attention launch-latency bound)",
                 "per-step op time (us)", total, "us", res, {"higher_is_better": False, "dtype": "f16"})


def workload_cfg3(dev, args):
    """Config 3: Qwen3-talker-layer f16 projections at M=48, 28 distinct layers rotated."""
    import torch

    layers, m = 28, 48
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    w_qkv = [torch.randn((4096, 1024), device=dev, generator=gen).mul_(0.02).half() for _ in range(layers)]
    w_gu = [torch.randn((6144, 1024), device=dev, generator=gen).mul_(0.02).half() for _ in range(layers)]
    w_dn = [torch.randn((1024, 3072), device=dev, generator=gen).mul_(0.02).half() for _ in range(layers)]
    x = torch.randn((m, 1024), device=dev, generator=gen).half()
    hh = torch.randn((m, 3072), device=dev, generator=gen).half()
    from dtts import ops

    ws = torch.empty(max(ops.gemm_workspace_bytes(m, 1024, 4096), ops.gemm_workspace_bytes(m, 1024, 3072, True),
                         ops.gemm_workspace_bytes(m, 3072, 1024), 1), dtype=torch.uint8, device=dev)
    y_qkv = torch.empty((m, 4096), dtype=torch.float32, device=dev)
    y_gu = torch.empty((m, 3072), dtype=torch.float32, device=dev)
    y_dn = torch.empty((m, 1024), dtype=torch.float32, device=dev)
    runs = {
        "qkv_48x1024x4096": (lambda: [ops.matmul_nt(x, w, ws, y_qkv) for w in w_qkv], 1024 * 4096),
        "gateup_silu_48x1024x6144": (lambda: [ops.gateup_silu(x, w, ws, y_gu) for w in w_gu], 1024 * 6144),
        "down_48x3072x1024": (lambda: [ops.matmul_nt(hh, w, ws, y_dn) for w in w_dn], 3072 * 1024),
    }
    res, tot_ms, tot_bytes = {}, 0.0, 0.0
    for name, (fn, kn) in runs.items():
        t = _graph_time(fn, reps=10) / layers
        by = 2.0 * kn + 2.0 * m * (kn // (6144 if "gateup" in name else (4096 if "qkv" in name else 1024)))
        fl = 2.0 * m * kn
        res[name] = {"us_per_layer": t * 1e3, "gbs": 2.0 * kn / t / 1e6, "tflops": fl / t / 1e9}
        tot_ms += t
        tot_bytes += 2.0 * kn
    return _line("config3: f16 decode projections M=48, 28 layers rotated (763 MB of weights), graph-replayed",
                 "weight-streaming GB/s", tot_bytes / tot_ms / 1e6, "GB/s", res,
                 {"dtype": "f16", "frac_hbm_peak": round(tot_bytes / tot_ms / 1e6 / PEAK_HBM_GBS, 4),
                  "us_per_layer": round(tot_ms * 1e3, 2)})


def workload_cfg4(dev, args):
    """Config 4: Q8_0 GEMV/GEMM at M in {1, 8, 48}, K=1024 N=6144 and K=3072 N=1024."""
    import numpy as np
    import torch

    from dtts import ops, synth

    res = {}
    for (k, n) in ((1024, 6144), (3072, 1024)):
        w = synth.normal(0, f"cfg4.w{k}", (n, k), 0, 0.02)
        blocks = torch.from_numpy(ops.q8_0_quantize(w)).to(dev)
        copies = max(1, int(300e6 // blocks.numel()))  # rotate > the 256 MB MALL
        sets = [blocks.clone() for _ in range(copies)]
        packed = [ops.q8_0_repack(b, k) for b in sets[:copies]]
        for m in (1, 8, 48):
            x = torch.from_numpy(synth.f16_bits(synth.normal(0, f"cfg4.x{m}", (m, k))).view(np.int16)).view(torch.float16).to(dev)
            ws = torch.empty(max(ops.q8_0_workspace_bytes(m, k, n), 16), dtype=torch.uint8, device=dev)
            for mode in ("w8a16", "w8a8"):
                # the workspace-free kernel, the A-sharing one with k ranges (dtts_gemm_q8_0_ws) and
                # the same on the load-time repacked layout (dtts_gemm_q8_0_packed)
                variants = (("", lambda: [ops.q8_0_matmul(x, b, mode) for b in sets]),
                            ("_ws", lambda: [ops.q8_0_matmul(x, b, mode, workspace=ws) for b in sets]),
                            ("_packed", lambda: [ops.q8_0_matmul_packed(x, pb, n, mode, workspace=ws) for pb in packed]))
                for tag, fn in variants:
                    t = _graph_time(fn, reps=5) / copies
                    wb = 34.0 * n * k / 32
                    res[f"k{k}_n{n}_m{m}_{mode}{tag}"] = {"us": t * 1e3,
                                                          "gbs": (wb + 2.0 * m * k + 4.0 * m * n) / t / 1e6,
                                                          "tops": 2.0 * m * n * k / t / 1e9}
            # Proj::forward's own interface: f32 activations (the _f32 entry points), W8A8
            # quantizing them directly and W8A32 at f32 precision
            x32 = torch.from_numpy(synth.normal(0, f"cfg4.x32.{m}", (m, k)).astype(np.float32)).to(dev)
            for mode in ("w8a8", "w8a32"):
                variants = (("_f32", lambda: [ops.q8_0_matmul(x32, b, mode) for b in sets]),
                            ("_ws_f32", lambda: [ops.q8_0_matmul(x32, b, mode, workspace=ws) for b in sets]),
                            ("_packed_f32", lambda: [ops.q8_0_matmul_packed(x32, pb, n, mode, workspace=ws)
                                                     for pb in packed]))
                for tag, fn in variants:
                    t = _graph_time(fn, reps=5) / copies
                    wb = 34.0 * n * k / 32
                    res[f"k{k}_n{n}_m{m}_{mode}{tag}"] = {"us": t * 1e3,
                                                          "gbs": (wb + 4.0 * m * k + 4.0 * m * n) / t / 1e6,
                                                          "tops": 2.0 * m * n * k / t / 1e9}
        del sets, packed
    best = max(r["gbs"] for r in res.values())
    return _line("config4: Q8_0 projections (GGML blocks), weights rotated past the MALL, graph-replayed",
                 "best weight-streaming GB/s", best, "GB/s", res, {"dtype": "int8/f16"})


def workload_stack(dev, args):
    """Row f-2: one decode step of the talker (28 layers) and of the code predictor (5 layers) at 48
    lanes, each lane at its own position, f16 weights and caches, eager and graph-replayed."""
    import numpy as np
    import torch

    from dtts import stack, synth

    lanes = 48
    res = {}
    best = None
    for name, geo, cap in (("talker", stack.TALKER, 2048), ("predictor", stack.PREDICTOR, 17)):
        from dataclasses import replace

        geo = replace(geo, capacity=cap)
        layers, fn = stack.random_device_weights(geo, dev, seed=0)
        st = stack.Stack(geo, layers, fn, dev)
        state = st.new_state(lanes, cap)
        gen = torch.Generator(device=dev)
        gen.manual_seed(1)
        for t in state.k + state.v:
            t.copy_(torch.randn(t.shape, generator=gen, device=dev))
        x = torch.randn((lanes, geo.dim), generator=gen, device=dev)
        out = torch.empty_like(x)
        pos = synth.randint(0, f"stack.{name}.pos", (lanes,), 0, cap - 1).astype(np.int32)
        ws = st.workspace(lanes, cap)
        t_eager = _time(lambda: st.decode(x, state, pos, out=out, workspace=ws), reps=10)
        t_graph = _time(lambda: st.decode(x, state, pos, out=out, graph=True, workspace=ws), reps=20)
        if not torch.isfinite(out).all():
            raise SystemExit(f"bench: non-finite {name} output")
        wbytes = geo.layers * geo.weight_bytes_per_layer()
        kv = geo.layers * 2 * 2 * geo.n_kv * geo.head_dim * int((pos.astype(np.int64) + 1).sum())
        res[name] = {"layers": geo.layers, "cap": cap, "ms_graph": round(t_graph, 4), "ms_eager": round(t_eager, 4),
                     "tokens_per_s": round(lanes / (t_graph / 1e3), 1), "weight_bytes": wbytes, "kv_bytes": kv,
                     "gbs": round((wbytes + kv) / t_graph / 1e6, 1),
                     "us_per_layer": round(t_graph * 1e3 / geo.layers, 2)}
        # the prefill branch: the predictor's per-frame [hidden, code0] (48 lanes x 2), the
        # talker's prompt (8 lanes x 256 positions, as prefill_batch groups lanes)
        pl, pt = (48, 2) if name == "predictor" else (8, 256)
        pstate = st.new_state(pl, cap)
        px = torch.randn((pl, pt, geo.dim), generator=gen, device=dev)
        pout = torch.empty_like(px)
        pws = torch.empty(st.prefill_workspace_bytes(pl, pt), dtype=torch.uint8, device=dev)
        t_pre = _time(lambda: st.prefill(px, pstate, 0, out=pout, workspace=pws), reps=10)
        if not torch.isfinite(pout).all():
            raise SystemExit(f"bench: non-finite {name} prefill output")
        res[name]["prefill"] = {"lanes": pl, "t": pt, "ms": round(t_pre, 4),
                                "positions_per_s": round(pl * pt / (t_pre / 1e3), 1)}
        if best is None:
            best = res[name]
        del st, state, layers, pstate
        torch.cuda.empty_cache()
        if name != "talker":
            continue
        # the talker at Stack::load's other weight kinds (f32 caches): decode steps, graph-replayed
        for kind in ("f32", "q8_0", "q8_0_a32"):
            layers, fn = stack.random_device_weights(geo, dev, seed=0, weight=kind)
            st = stack.Stack(geo, layers, fn, dev, weight=kind)
            state = st.new_state(lanes, cap)
            for t in state.k + state.v:
                t.copy_(torch.randn(t.shape, generator=gen, device=dev))
            ws = st.workspace(lanes, cap)
            t_graph = _time(lambda: st.decode(x, state, pos, out=out, graph=True, workspace=ws), reps=20)
            if not torch.isfinite(out).all():
                raise SystemExit(f"bench: non-finite talker output ({kind})")
            wk = sum(v.numel() * v.element_size() for L in layers for key, v in L.items()
                     if key in ("wqkv", "wo", "w_gateup", "wdown"))
            kvk = kv * 2  # f32 caches
            res[f"talker_{kind}"] = {"ms_graph": round(t_graph, 4), "tokens_per_s": round(lanes / (t_graph / 1e3), 1),
                                     "weight_bytes": wk, "kv_bytes": kvk, "gbs": round((wk + kvk) / t_graph / 1e6, 1),
                                     "us_per_layer": round(t_graph * 1e3 / geo.layers, 2)}
            del st, state, layers
            torch.cuda.empty_cache()
    return _line("row f-2: decoder-stack decode step, 48 lanes at per-lane positions (talker 28 layers, cap 2048; "
                 "code predictor 5 layers), f16 weights and KV cache, one HIP graph per step; the talker also "
                 "with f32 and Q8_0 layers (f32 caches)",
                 "talker decode tokens/s at 48 lanes", best["tokens_per_s"], "tokens/s", res,
                 {"dtype": "f16 weights / f32 activations",
                  "frac_hbm_peak": round(best["gbs"] / PEAK_HBM_GBS, 4)})


def workload_front(dev, args):
    """Row f-3: the codec's front half (split RVQ, pre_conv, 8-layer windowed transformer, two
    TransConv + ConvNeXt stages) over 48 lanes x 325 code frames (one Codec::decode window each),
    and Codec::decode of one 3000-frame document (10 windows as lanes) through the front half and
    the waveform stack to f32 audio."""
    import numpy as np
    import torch

    from dtts import codec, codec_front, synth

    geo = codec_front.CODEC
    hw = codec_front.random_weights(geo, 0)
    front = codec_front.CodecFront(geo, hw, dev)
    lanes, frames = 48, codec_front.CHUNK_FRAMES + codec_front.CHUNK_LEFT_CONTEXT
    codes = synth.randint(0, "front.codes", (lanes, frames, geo.n_books), 0, geo.book_size - 1).astype(np.int32)
    latent = torch.empty((lanes, frames * geo.upsample, geo.latent_dim), dtype=torch.float16, device=dev)
    front.workspace(lanes, frames)
    t_front = _time(lambda: front.decode(codes, out=latent), reps=10)
    if not torch.isfinite(latent.float()).all():
        raise SystemExit("bench: non-finite latent")
    wave = codec.Codec(codec.CONFIG5, codec.random_weights(codec.CONFIG5, seed=0), dev)
    spf = geo.upsample * codec.CONFIG5.hop
    n_doc = 3000
    doc = synth.randint(0, "front.doc", (n_doc, geo.n_books), 0, geo.book_size - 1).astype(np.int32)
    audio = torch.empty(n_doc * spf, dtype=torch.float32, device=dev)
    t_doc = _time(lambda: codec_front.decode_document(front, wave, doc, out=audio), reps=3, warm=1)
    if not torch.isfinite(audio).all():
        raise SystemExit("bench: non-finite document audio")
    fl = geo.flops_per_frame() * lanes * frames
    windows = -(-n_doc // codec_front.CHUNK_FRAMES)
    doc_fl = windows * frames * (geo.flops_per_frame() + geo.upsample * codec.CONFIG5.flops_per_frame())
    res = {"front": {"lanes": lanes, "frames": frames, "ms": round(t_front, 4),
                     "code_frames_per_s": round(lanes * frames / (t_front / 1e3), 1),
                     "tflops": round(fl / (t_front / 1e3) / 1e12, 2)},
           "document": {"frames": n_doc, "windows": windows, "ms": round(t_doc, 3),
                        "audio_s": n_doc * spf / SAMPLE_RATE,
                        "audio_s_per_s": round(n_doc * spf / SAMPLE_RATE / (t_doc / 1e3), 1),
                        "tflops": round(doc_fl / (t_doc / 1e3) / 1e12, 2),
                        "note": "timed from host codes to device audio; includes the host-side "
                                "window assembly and the codes' upload"}}
    del front, wave
    torch.cuda.empty_cache()
    return _line("row f-3: codec front half, 48 lanes x 325 code frames (codes -> latent), and Codec::decode "
                 "of a 3000-frame document (chunk 300, left context 25; codes -> f32 audio)",
                 "front-half code frames/s at 48 lanes", res["front"]["code_frames_per_s"], "frames/s", res,
                 {"dtype": "f16 storage / f32 accumulation",
                  "frac_mfma_peak": round(res["front"]["tflops"] / PEAK_TFLOPS_F16, 4)})


def workload_cfg5f32(dev, args):
    """Config 5's geometry at the reference's own precision (WAV_DTYPE = F32): 48 lanes x 250 frames
    through dtts_codec_decode_f32, whose convs run f32-accurate on the f16 matrix cores (split
    operands: three f16 products per f32 term, conv_split.hip). An extra line; the f16 decode stays
    the headline. A split kernel's roofline is its issued matrix work (3x the algorithmic FLOPs)
    against the f16 peak; `achieved` stays the algorithmic f32 rate."""
    import numpy as np
    import torch

    from dtts import codec, synth

    geo = codec.CONFIG5
    lanes, frames = args.lanes, args.frames
    model = codec.Codec(geo, codec.random_weights(geo, seed=0), dev, dtype="f32")
    latent = torch.from_numpy(synth.normal(0, "latent", (lanes, frames, geo.latent_dim))).to(dev)
    audio = torch.empty((lanes, frames * geo.hop), dtype=torch.float32, device=dev)
    model.workspace(lanes, frames)
    t = _time(lambda: model.decode(latent, out=audio), reps=5, warm=1)
    if not torch.isfinite(audio).all():
        raise SystemExit("bench: non-finite f32 audio")
    stages = model.profile(latent, out=audio)
    by = {}
    for st in stages:
        e = by.setdefault(st["kernel"], dict(flops=0.0, bytes=0.0, ms=0.0, launches=0))
        e["flops"] += st["flops"]
        e["bytes"] += st["bytes"]
        e["ms"] += st["ms"]
        e["launches"] += 1
    kern = []
    for name, e in sorted(by.items(), key=lambda kv: -kv[1]["ms"]):
        per = e["ms"] / e["launches"]
        split = name.startswith("conv_split_mfma")
        mpeak, issue = (PEAK_TFLOPS_F16, 3.0) if split else (PEAK_TFLOPS_F32, 1.0)
        mfma = issue * e["flops"] / max(e["bytes"], 1.0) > mpeak * 1e12 / (PEAK_HBM_GBS * 1e9)
        ach = (e["flops"] if mfma else e["bytes"]) / e["launches"] / (per / 1e3) / (1e12 if mfma else 1e9)
        peak = mpeak if mfma else PEAK_HBM_GBS
        row = {"kernel": name, "launches": e["launches"], "ms_per_launch": round(per, 4),
               "bound": "mfma" if mfma else "hbm", "achieved": round(ach, 1), "peak": peak,
               "unit": "TFLOP/s" if mfma else "GB/s", "frac": round((issue if mfma else 1.0) * ach / peak, 4)}
        if split and mfma:
            row["issued_tflops"] = round(issue * ach, 1)
        kern.append(row)
    audio_s = lanes * frames * geo.hop / SAMPLE_RATE
    flops = lanes * frames * geo.flops_per_frame()
    del model
    torch.cuda.empty_cache()
    return _line("config5 geometry at f32 (the reference's WAV_DTYPE): codec decoder stack, 48 lanes x 250 frames, "
                 "f32-accurate convs on the f16 matrix cores (activations as f16 hi/lo pairs, three products "
                 "per term), full-precision SnakeBeta",
                 "codec audio-sec/sec at 48 lanes (f32)", audio_s / (t / 1e3), "audio-s/s",
                 {"ms_per_step": round(t, 3), "tflops": round(flops / (t / 1e3) / 1e12, 2),
                  "frac_f32_matrix_peak": round(flops / (t / 1e3) / 1e12 / PEAK_TFLOPS_F32, 4), "kernels": kern},
                 {"dtype": "f32"})


# ---------------------------------------------------------------- rocprofv3 counter digest

COPY_PROBE_BYTES = 1 << 30  # --copy-probe: a mul kernel reading and writing 1 GiB
# The runs a --pmc-summary digest comes from (from the repository root on the GPU box, after
# `cd /tmp && export TMPDIR=/tmp`; paths relative to the repository), recorded in the digest.
PMC_COMMANDS = [
    "rocprofv3 --pmc FETCH_SIZE --output-format csv -d gpurun_out/prof_fetch -o fetch -- python3 bench.py "
    "--no-cpu-baseline --steps 1 --warmup 0 --profile-runs 1 --copy-probe --stages-out gpurun_out/stages.json",
    "rocprofv3 --pmc WRITE_SIZE --output-format csv -d gpurun_out/prof_write -o write -- python3 bench.py "
    "--no-cpu-baseline --steps 1 --warmup 0 --profile-runs 1 --copy-probe",
    "python3 bench.py --pmc-summary gpurun_out/prof_fetch/fetch_counter_collection.csv "
    "gpurun_out/prof_write/write_counter_collection.csv gpurun_out/stages.json",
]


def pmc_summary(fetch_csv, write_csv, stages_json):
    """Per-kernel HBM traffic of one decode from two rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE,
    KiB per dispatch), each scaled by what its counter reads for the copy probe, next to the
    algorithmic bytes of the same launches (dtts_codec_profile's accounting)."""
    import csv

    def rows(path, counter):
        return [r for r in csv.DictReader(open(path)) if r["Counter_Name"] == counter]

    def calib(rs):
        probe = [float(r["Counter_Value"]) * 1024 for r in rs
                 if "elementwise" in r["Kernel_Name"] and float(r["Counter_Value"]) * 1024 > COPY_PROBE_BYTES / 4]
        if not probe:
            raise SystemExit("pmc-summary: no copy-probe dispatch in " + fetch_csv)
        return COPY_PROBE_BYTES / (sum(probe) / len(probe))

    fr, wr = rows(fetch_csv, "FETCH_SIZE"), rows(write_csv, "WRITE_SIZE")
    cf, cw = calib(fr), calib(wr)
    stages = json.load(open(stages_json))["stages"]
    dtts = lambda rs: [r for r in rs if "dtts::" in r["Kernel_Name"]]
    fd, wd = dtts(fr), dtts(wr)
    n = len(stages)
    if len(fd) < n or len(wd) < n:
        raise SystemExit("pmc-summary: fewer dtts dispatches than stages")
    # the last n dispatches are the profile run's: one plan over all lanes on one stream, in stage
    # order (the timed decode before it interleaves its two half-batch plans)
    out = {"commands": PMC_COMMANDS, "fetch_scale": cf, "write_scale": cw, "kernels": {}, "stages": []}
    for st, f, w in zip(stages, fd[-n:], wd[-n:]):
        rd, wb = float(f["Counter_Value"]) * 1024 * cf, float(w["Counter_Value"]) * 1024 * cw
        out["stages"].append({"name": st["name"], "kernel": st["kernel"], "fetch_bytes": rd, "write_bytes": wb,
                              "alg_bytes": st["bytes"]})
        k = out["kernels"].setdefault(st["kernel"], {"launches": 0, "fetch_bytes": 0.0, "write_bytes": 0.0,
                                                     "alg_bytes": 0.0})
        k["launches"] += 1
        k["fetch_bytes"] += rd
        k["write_bytes"] += wb
        k["alg_bytes"] += st["bytes"]
    for k in out["kernels"].values():
        k["traffic_per_launch"] = (k["fetch_bytes"] + k["write_bytes"]) / k["launches"]
        k["alg_per_launch"] = k["alg_bytes"] / k["launches"]
        k["ratio"] = k["traffic_per_launch"] / k["alg_per_launch"]
    return out


def pmc_counters(stages_json, csv_paths):
    """Per-kernel SQ/GRBM counters of one decode from rocprofv3 --pmc runs (one CSV per pass; the
    last dtts dispatches of each are the profile run's, in stage order, as for pmc_summary): the mean
    per launch of every counter, plus VALU instructions per MFMA instruction, the share of LDS
    instruction cycles lost to bank conflicts and the MFMA-busy fraction of the SIMDs."""
    import csv

    stages = json.load(open(stages_json))["stages"]
    n = len(stages)
    per_stage = [dict() for _ in range(n)]
    for path in csv_paths:
        disp = {}
        for r in csv.DictReader(open(path)):
            if "dtts::" not in r["Kernel_Name"]:
                continue
            disp.setdefault(int(r["Dispatch_Id"]), {})[r["Counter_Name"]] = float(r["Counter_Value"])
        order = sorted(disp)
        if len(order) < n:
            raise SystemExit(f"pmc-counters: {len(order)} dtts dispatches in {path} < {n} stages")
        for i, d in enumerate(order[-n:]):
            per_stage[i].update(disp[d])
    out = {"source": [os.path.basename(p) for p in csv_paths], "kernels": {}}
    for st, c in zip(stages, per_stage):
        k = out["kernels"].setdefault(st["kernel"], {"launches": 0, "ms": 0.0, "flops": 0.0, "counters": {}})
        k["launches"] += 1
        k["ms"] += st["ms"]
        k["flops"] += st["flops"]
        for name, v in c.items():
            k["counters"][name] = k["counters"].get(name, 0.0) + v
    for k in out["kernels"].values():
        c = {name: v / k["launches"] for name, v in k["counters"].items()}
        k["counters"] = c
        if c.get("SQ_INSTS_MFMA"):
            k["valu_per_mfma"] = round(c.get("SQ_INSTS_VALU", 0.0) / c["SQ_INSTS_MFMA"], 3)
        if c.get("SQ_ACTIVE_INST_LDS"):
            k["lds_bank_conflict_per_lds_cycle"] = round(c.get("SQ_LDS_BANK_CONFLICT", 0.0) / c["SQ_ACTIVE_INST_LDS"], 4)
        if c.get("SQ_BUSY_CU_CYCLES") and "SQ_VALU_MFMA_BUSY_CYCLES" in c:
            # per-SIMD MFMA-busy cycles over the CUs' busy cycles (both summed over the chip; four
            # SIMDs per CU). GRBM_GUI_ACTIVE reads as the sum over the 8 XCDs, so it is not used.
            k["mfma_busy_frac"] = round(c["SQ_VALU_MFMA_BUSY_CYCLES"] / (4.0 * c["SQ_BUSY_CU_CYCLES"]), 4)
        if c.get("SQ_BUSY_CU_CYCLES") and "SQ_INSTS_VALU" in c:
            # wave64 VALU instructions take 4 issue cycles on a SIMD
            k["valu_issue_frac"] = round(4.0 * c["SQ_INSTS_VALU"] / (4.0 * c["SQ_BUSY_CU_CYCLES"]), 4)
        if c.get("SQ_BUSY_CU_CYCLES") and "SQ_LDS_IDX_ACTIVE" in c:
            k["lds_active_frac"] = round(c["SQ_LDS_IDX_ACTIVE"] / c["SQ_BUSY_CU_CYCLES"], 4)
        k["tflops"] = round(k["flops"] / k["ms"] / 1e9, 1)
    return out


def pmc_clock(csv_paths):
    """Per-kernel clock and matrix-core figures from rocprofv3 --pmc GRBM_GUI_ACTIVE SQ_BUSY_CU_CYCLES
    SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_MFMA --kernel-trace runs (every kernel with MFMA work, dtts's and
    the vendor library's alike). Per dispatch: duration from its timestamps; the CU clock as
    SQ_BUSY_CU_CYCLES / 256 CUs / duration (cycles the CUs were busy, so a lower bound of the shader
    clock); the MFMA-busy share of the SIMDs; the matrix work done, 1024 FLOP per SIMD MFMA-busy
    cycle (a 32x32x16 f16 MFMA is 32 busy cycles, a 16x16x32 one 16); and the peak that clock
    allows, 256 CUs x 4 SIMDs x 1024 FLOP per cycle."""
    import csv

    disp = {}
    for path in csv_paths:
        for r in csv.DictReader(open(path)):
            d = disp.setdefault((path, int(r["Dispatch_Id"])), {"name": r["Kernel_Name"],
                                                                 "ns": int(r["End_Timestamp"]) - int(r["Start_Timestamp"])})
            d[r["Counter_Name"]] = float(r["Counter_Value"])
    out = {}
    for d in disp.values():
        if not d.get("SQ_INSTS_MFMA") or d["ns"] <= 0:
            continue
        name = d["name"].replace("void ", "").replace("dtts::", "").replace("(anonymous namespace)::", "")
        if "Cijk" in name:  # the vendor library's: its macro tile and stream-K flag name it
            mt = re.search(r"MT\d+x\d+x\d+", name)
            name = ("Custom_" if name.startswith("Custom") else "") + "Cijk " + (mt.group(0) if mt else name[:40]) + \
                (" SK" if "_SK" in name else "")
        else:
            name = name.split("(")[0]
        k = out.setdefault(name, {"dispatches": 0, "us": 0.0, "cu_clock_ghz": 0.0, "mfma_busy": 0.0, "tflops": 0.0,
                                  "clock_peak_tflops": 0.0})
        f_cu = d["SQ_BUSY_CU_CYCLES"] / 256.0 / d["ns"]  # cycles per ns = GHz
        k["dispatches"] += 1
        k["us"] += d["ns"] / 1e3
        k["cu_clock_ghz"] += f_cu
        k["mfma_busy"] += d["SQ_VALU_MFMA_BUSY_CYCLES"] / (4.0 * d["SQ_BUSY_CU_CYCLES"])
        k["tflops"] += d["SQ_VALU_MFMA_BUSY_CYCLES"] * 1024.0 / d["ns"] / 1e3
        k["clock_peak_tflops"] += f_cu * 256 * 4 * 1024 / 1e3
    for k in out.values():
        n = k["dispatches"]
        for f in ("us", "cu_clock_ghz", "mfma_busy", "tflops", "clock_peak_tflops"):
            k[f] = round(k[f] / n, 3)
        k["frac_of_nameplate"] = round(k["tflops"] / PEAK_TFLOPS_F16, 4)
    return out


def vendor_gemm(stages, lanes, dev, reps=10):
    """The vendor library's f16 GEMM (torch.matmul -> hipBLASLt) on each conv stage's im2col'd shape:
    M = lanes x positions, K = taps x cin, N = cout; a fused residual unit as its two GEMMs (K = 7C
    and C). The GEMM alone, no im2col pass, no epilogue, f16 out -- a bound for a library route."""
    import torch

    shapes, cache, out = [], {}, []
    for s in stages:
        m = lanes * s["len"]
        if s["kernel"].startswith("ru_nlc"):
            g = [(m, s["k"] * s["cin"], s["cout"]), (m, s["cout"], s["cout"])]
        elif s["cout"] == 1 or not s["kernel"].startswith("conv_nlc_f16_mfma"):
            continue
        else:
            g = [(m, s["k"] * s["cin"], s["cout"])]
        shapes.append((s, g))
    for s, g in shapes:
        total = 0.0
        for (m, k, n) in g:
            if (m, k, n) not in cache:
                a = torch.randn(m, k, device=dev, dtype=torch.float16)
                b = torch.randn(n, k, device=dev, dtype=torch.float16).t()
                for _ in range(3):
                    c = torch.matmul(a, b)
                ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
                ev[0].record()
                for _ in range(reps):
                    c = torch.matmul(a, b)
                ev[1].record()
                torch.cuda.synchronize()
                cache[(m, k, n)] = ev[0].elapsed_time(ev[1]) / reps
                del a, b, c
                torch.cuda.empty_cache()
            total += cache[(m, k, n)]
        out.append({"stage": s["name"], "kernel": s["kernel"], "dtts_ms": round(s["ms"], 4), "gemms": g,
                    "vendor_gemm_ms": round(total, 4), "dtts_over_vendor": round(s["ms"] / total, 3),
                    "flops": s["flops"]})
        log(f"    {s['name']:22s} dtts {s['ms']:7.3f} ms   vendor GEMM {total:7.3f} ms   ratio {s['ms'] / total:5.2f}")
    # a reference point for the library itself: a square GEMM, its best case
    a = torch.randn(8192, 8192, device=dev, dtype=torch.float16)
    b = torch.randn(8192, 8192, device=dev, dtype=torch.float16).t()
    for _ in range(3):
        c = torch.matmul(a, b)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    ev[0].record()
    for _ in range(reps):
        c = torch.matmul(a, b)
    ev[1].record()
    torch.cuda.synchronize()
    ms = ev[0].elapsed_time(ev[1]) / reps
    out.append({"stage": "square 8192 (reference)", "kernel": None, "dtts_ms": None, "gemms": [(8192, 8192, 8192)],
                "vendor_gemm_ms": round(ms, 4), "dtts_over_vendor": None, "flops": 2.0 * 8192 ** 3})
    log(f"    square 8192^3 vendor GEMM {ms:7.3f} ms = {2.0 * 8192 ** 3 / ms / 1e9:.0f} TFLOP/s")
    del a, b, c
    return out


def achievable_peaks(dev, reps=20):
    """What the box delivers, next to the spec-sheet peaks the rooflines use: HBM from a copy kernel
    over 2 GiB (read + write counted; far past the 256 MB MALL), f16 and f32 matrix throughput from
    the vendor library's square GEMMs (torch.matmul), each timed with HIP events after warm-up."""
    import torch

    def timed(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    out = {}
    src = torch.ones(1 << 30, dtype=torch.float16, device=dev)
    dst = torch.empty_like(src)
    ms = timed(lambda: torch.mul(src, 1.0, out=dst))
    out["hbm_copy"] = {"gbs": round(2 * src.numel() * 2 / ms / 1e6, 1), "bytes_per_pass": 2 * src.numel() * 2,
                       "frac_of_peak": round(2 * src.numel() * 2 / ms / 1e6 / PEAK_HBM_GBS, 4)}
    del src, dst
    for name, dt, n, peak in (("gemm_f16", torch.float16, 8192, PEAK_TFLOPS_F16),
                              ("gemm_f32", torch.float32, 8192, PEAK_TFLOPS_F32)):
        a = torch.randn(n, n, device=dev, dtype=dt)
        b = torch.randn(n, n, device=dev, dtype=dt)
        ms = timed(lambda: torch.matmul(a, b))
        tf = 2.0 * n ** 3 / ms / 1e9
        out[name] = {"shape": [n, n, n], "tflops": round(tf, 1), "frac_of_peak": round(tf / peak, 4)}
        del a, b
    torch.cuda.empty_cache()
    return out


WORKLOADS = {"cfg1": workload_cfg1, "cfg2": workload_cfg2, "cfg3": workload_cfg3, "cfg4": workload_cfg4,
             "stack": workload_stack, "front": workload_front, "cfg5f32": workload_cfg5f32}


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
    ap.add_argument("--pmc-summary", nargs=3, metavar=("FETCH_CSV", "WRITE_CSV", "STAGES_JSON"),
                    help="digest rocprofv3 FETCH_SIZE / WRITE_SIZE runs into per-kernel traffic (no GPU)")
    ap.add_argument("--pmc-counters", nargs="+", metavar="STAGES_JSON CSV",
                    help="digest rocprofv3 --pmc runs of SQ/GRBM counters into per-kernel figures (no GPU)")
    ap.add_argument("--traffic-json", default=os.path.join(ROOT, "profiles", "codec_config5_pmc.json"),
                    help="per-kernel traffic from --pmc-summary, reported in roofline.traffic")
    ap.add_argument("--workload", default="cfg5",
                    choices=["cfg1", "cfg2", "cfg3", "cfg4", "stack", "front", "cfg5f32", "cfg5", "all"],
                    help="cfg5 (default) is the headline codec line; cfg1-4 time the other rows' ops; stack "
                         "times the decoder-stack decode step; front the codec front half and document decode")
    ap.add_argument("--pmc-clock", nargs="+", metavar="CSV",
                    help="digest rocprofv3 --pmc GRBM_GUI_ACTIVE SQ_BUSY_CU_CYCLES SQ_VALU_MFMA_BUSY_CYCLES "
                         "SQ_INSTS_MFMA --kernel-trace runs into per-kernel clock and MFMA figures (no GPU)")
    ap.add_argument("--vendor-gemm", default=None, metavar="JSON",
                    help="after the profile run, time the vendor f16 GEMM on every conv stage's im2col'd "
                         "shape and write the comparison here")
    ap.add_argument("--peaks", action="store_true",
                    help="measure the box's achievable HBM copy bandwidth and f16/f32 GEMM throughput, then exit")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also run a plain 1 GiB copy kernel 3 times (calibrates HBM byte counters)")
    args = ap.parse_args()

    if args.pmc_summary:
        print(json.dumps(pmc_summary(*args.pmc_summary), indent=1))
        return
    if args.pmc_counters:
        print(json.dumps(pmc_counters(args.pmc_counters[0], args.pmc_counters[1:]), indent=1))
        return
    if args.pmc_clock:
        print(json.dumps(pmc_clock(args.pmc_clock), indent=1))
        return

    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(lanes are data-parallel: N GPUs would each take lanes / N with the weights replicated)",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from dtts import codec, synth

    dev = torch.device("cuda:0")
    if args.peaks:
        print(json.dumps({"achievable_peaks": achievable_peaks(dev),
                          "spec": {"hbm_gbs": PEAK_HBM_GBS, "f16_tflops": PEAK_TFLOPS_F16,
                                   "f32_matrix_tflops": PEAK_TFLOPS_F32}}))
        return
    if args.workload != "cfg5":
        for w in (["cfg1", "cfg2", "cfg3", "cfg4", "stack", "front", "cfg5f32"] if args.workload == "all"
                  else [args.workload]):
            print(json.dumps(WORKLOADS[w](dev, args)), flush=True)
        if args.workload != "all":
            return
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
    # per-step HIP events on the decode's stream, recorded between steps (no host wait inside)
    events = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    t0 = time.perf_counter()
    events[0].record()
    for i in range(args.steps):
        model.decode(latent, out=audio)
        events[i + 1].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = wall * 1e3 / args.steps
    step_ms = sorted(events[i].elapsed_time(events[i + 1]) for i in range(args.steps))
    steps_stat = {"median_ms": round(step_ms[len(step_ms) // 2], 4), "min_ms": round(step_ms[0], 4),
                  "max_ms": round(step_ms[-1], 4), "first_ms": round(events[0].elapsed_time(events[1]), 4),
                  "last_ms": round(events[-2].elapsed_time(events[-1]), 4)}
    audio_s = args.lanes * args.frames * geo.hop / SAMPLE_RATE
    value = audio_s / (ms / 1e3)
    if not torch.isfinite(audio.float()).all():
        raise SystemExit("bench: non-finite audio")
    log(f"decode: {ms:.3f} ms/step -> {value:.1f} audio-s/s")

    # one profile run first, untimed, as the decode's own warm-up steps: the switch from the
    # two-stream decode to the one-plan profile makes the first run's launches slower
    warm = model.profile(latent, out=audio)
    runs = [model.profile(latent, out=audio) for _ in range(args.profile_runs)]
    kname, dom, by = dominant(runs)
    wk = [s["ms"] for s in warm if s["kernel"] == kname]
    log(f"profile warm-up run: {kname} {sum(wk) / max(len(wk), 1):.4f} ms per launch (not used); "
        f"measured runs: {[round(sum(s['ms'] for s in r if s['kernel'] == kname) / dom['launches'], 4) for r in runs]}")
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
    if os.path.exists(args.traffic_json):
        tk = json.load(open(args.traffic_json))["kernels"].get(kname)
        if tk:  # measured offline with rocprofv3 --pmc on this kernel (see --pmc-summary)
            roof["traffic"] = round(tk["traffic_per_launch"])
            roof["traffic_over_algorithmic"] = round(tk["ratio"], 3)
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

    if args.vendor_gemm:
        log("vendor GEMM on the stages' im2col'd shapes:")
        with open(args.vendor_gemm, "w") as f:
            json.dump({"lanes": args.lanes, "frames": args.frames,
                       "stages": vendor_gemm(runs[-1], args.lanes, dev)}, f, indent=1)

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
        "step_ms": steps_stat,
        "roofline": roof,
        "kernels": kernel_rooflines(by),
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
