#!/usr/bin/env python3
"""Benchmark of the MI355X ternary linear path (one JSON line on stdout).

Headline workload (value): decode ternary GEMV at LLaMA-7B FFN shapes. One
step = one decode pass of B tokens through the three FFN projections
(W_gate, W_up [11008,4096] on x, W_down [4096,11008] on its own [B,11008]
input), bf16 activations, fp32 accumulation, bf16 outputs: gate and up as
one frx_ternary_linear_group launch (they share x, as the model's decode
step issues them), down as frx_ternary_linear; the step as three launches
is reported beside it. Weights, scales and activations are resident in
HBM before timing; the weights rotate over enough distinct copies (>= 0.5 GB)
that the 256 MB Infinity Cache cannot serve them (one copy per timed step).
value = algorithmic bytes
per step (packed weights + scales + x + y) / time per step, the K timed steps
replayed from one HIP graph.

roofline: the dominant kernel, the gate/up group launch (two thirds of the
step): its algorithmic bytes / its average launch time over back-to-back
launches (HIP events on the launch stream around the sequence).
cpu_baseline: the reference's CPU decode path (ternary_matmul_packed_parallel,
src/model/ternary.rs:471-529, restated in C by the oracle) on the same three
matrices at B=1, timed on this host's cores; its breakdown adds the branchy
i8 loop and the CPU 2:4 matmul (one thread each) and the single 2048x2048
linear, each with median, p10 and p90.

Per-launch GPU times carry the median, p10 and p90 over the individual
replays (decode) or launches (prefill, 2:4, MoE; 200 back-to-back).

extra: the decode FFN of the same layer through frx_ternary_ffn (the
default, one-launch and two-launch executions), the same decode step and
decode FFN at B = 4 and 16 (default run), the B=1 GEMV at growing weight sizes (up to
the stacked LLaMA-70B gate/up, 117 MB), prefill GEMM (X[2048,4096] x
W[N,4096], N in {4096, 11008}), 2:4 sparse GEMM and the MoE expert layer, as
TFLOP/s and fraction of the dense bf16 MFMA peak; the 2:4 decode GEMV (one
token through the same 2:4 weights, metadata rotated over cold copies) and
the MoE layer at one token (weights rotated over cold expert sets).
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

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA, TFLOP/s


def gemv_bytes(n: int, k: int, b: int, xb: int = 2, yb: int = 2) -> int:
    return n * k // 4 + 4 * n + xb * b * k + yb * b * n


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--batch", type=int, default=1, help="decode tokens per step (1, 4 or 16)")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--profile-target", choices=["prefill", "sparse24", "moe"], default=None,
                    help="run only this workload's kernels (for rocprofv3 counter passes)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: the ternary linear path runs on exactly one GPU here; --gpus {args.gpus} "
              "is not supported (sharding across GPUs is a design, not run).", file=sys.stderr)
        sys.exit(2)

    import torch
    import ferrisres_amd as frx
    from ferrisres_amd import synth

    assert torch.cuda.is_available(), "bench.py needs a gfx950 GPU"
    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream(device=dev)
    ctx = frx.Context(0)
    ctx.set_stream(stream)
    if args.profile_target:
        res = run_extra(torch, frx, synth, ctx, stream, dev, only=args.profile_target, iters=args.steps)
        print(json.dumps({"profile_target": args.profile_target, "extra": res}), flush=True)
        return
    B = args.batch
    H, I = 4096, 11008

    # ---- inputs (resident before timing) -------------------------------------
    log("bench: generating weights")
    t_g = synth.ternary_uniform("bench/decode", "w_gate", I, H)
    t_u = synth.ternary_uniform("bench/decode", "w_up", I, H)
    t_d = synth.ternary_uniform("bench/decode", "w_down", H, I)
    w_g = torch.from_numpy(synth.pack_rows_u32(t_g).view(np.int32)).to(dev)
    w_u = torch.from_numpy(synth.pack_rows_u32(t_u).view(np.int32)).to(dev)
    w_d = torch.from_numpy(synth.pack_rows_u32(t_d).view(np.int32)).to(dev)
    s_g = torch.from_numpy(synth.row_scales("bench/decode", "s_gate", I, samples=256)).to(dev)
    s_u = torch.from_numpy(synth.row_scales("bench/decode", "s_up", I, samples=256)).to(dev)
    s_d = torch.from_numpy(synth.row_scales("bench/decode", "s_down", H, samples=256)).to(dev)
    step_weight_bytes = (w_g.numel() + w_u.numel() + w_d.numel()) * 4
    copies = max(2, int(np.ceil(512e6 / step_weight_bytes)) + 1)
    # The timed graph gives every step a copy of its own (steps + 3 copies at
    # least): each copy it reads was last read a whole replay (>= 0.5 GB)
    # earlier, so no timed step is served by the 256 MB Infinity Cache.
    # The per-launch timings rotate over all of them too: >= 56 copies keep
    # even the one-matrix rotations (56 x 11.3 MB) above twice the cache.
    step_copies = max(copies, args.steps + 3, 56)
    W = [(w_g.clone(), w_u.clone(), w_d.clone()) for _ in range(step_copies)]
    del w_g, w_u, w_d
    _, xb = synth.activations("bench/decode", "x", B, H)
    _, hb = synth.activations("bench/decode", "h", B, I)
    x = torch.from_numpy(xb.view(np.int16)).to(dev).view(torch.bfloat16)
    xd = torch.from_numpy(hb.view(np.int16)).to(dev).view(torch.bfloat16)  # down-projection input
    g = torch.empty((B, I), dtype=torch.bfloat16, device=dev)
    u = torch.empty((B, I), dtype=torch.bfloat16, device=dev)
    y = torch.empty((B, H), dtype=torch.bfloat16, device=dev)
    h = torch.empty((B, I), dtype=torch.float32, device=dev)  # fused FFN: gated product
    torch.cuda.synchronize()

    b_gu = gemv_bytes(I, H, B)
    b_dn = gemv_bytes(H, I, B)
    # gate and up share x: one same-x group launch reads it once
    b_grp = 2 * (I * H // 4 + 4 * I) + 2 * B * H + 2 * 2 * B * I
    step_bytes = b_grp + b_dn

    def step(i):
        """One decode step: the three LLaMA-7B FFN projections as GEMVs,
        gate and up (same x) as one frx_ternary_linear_group launch, down as
        frx_ternary_linear on its own input."""
        wg, wu, wd = W[i % step_copies]
        ctx.ternary_linear_group(x, [wg, wu], [s_g, s_u], [g, u])
        ctx.ternary_linear(wd, s_d, xd, y)

    def step3(i):
        """The same step as three frx_ternary_linear launches."""
        wg, wu, wd = W[i % step_copies]
        ctx.ternary_linear(wg, s_g, x, g)
        ctx.ternary_linear(wu, s_u, x, u)
        ctx.ternary_linear(wd, s_d, xd, y)

    log(f"bench: warmup {args.warmup} steps ({step_copies} weight copies, "
        f"{step_copies * step_weight_bytes / 1e6:.0f} MB)")
    with torch.cuda.stream(stream):
        for i in range(args.warmup):
            step(i)
            wg, wu, wd = W[i % copies]
            ctx.ternary_ffn(x, wg, s_g, wu, s_u, wd, s_d, y)  # allocates the FFN workspace
    torch.cuda.synchronize()

    # The decode loop is launch-bound, so the timed K steps run as one
    # captured HIP graph (weights rotating over the copies step by step);
    # eager launches are the fallback where capture is unavailable.
    def capture(fn):
        try:
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr, stream=stream):
                fn()
            torch.cuda.synchronize()
            return gr
        except Exception as e:  # noqa: BLE001 - reported in the JSON line
            log(f"bench: graph capture unavailable ({e}); timing eager launches")
            torch.cuda.synchronize()
            return None

    def timed(fn):
        """Seconds for fn() run from a captured graph (or eagerly). The graph
        is replayed once untimed first, so the timed replay does not include
        its one-time upload."""
        gr = capture(fn)
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            (gr.replay() if gr is not None else fn())
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        with torch.cuda.stream(stream):
            (gr.replay() if gr is not None else fn())
        torch.cuda.synchronize()
        return time.perf_counter() - t0, gr is not None

    # timed region (value): exactly args.steps steps
    elapsed, graphed = timed(lambda: [step(i) for i in range(args.steps)])
    timing = "hip_graph" if graphed else "eager"
    ms_per_step = elapsed / args.steps * 1e3
    value = step_bytes / (elapsed / args.steps) / 1e9
    log(f"bench: decode GEMV B={B}: {ms_per_step * 1e3:.1f} us/step, {value:.1f} GB/s ({timing})")
    el3, _ = timed(lambda: [step3(i) for i in range(args.steps)])
    step3_res = {"us_per_step": round(el3 / args.steps * 1e6, 2),
                 "gb_s": round((2 * b_gu + b_dn) / (el3 / args.steps) / 1e9, 1),
                 "hbm_fraction": round((2 * b_gu + b_dn) / (el3 / args.steps) / 1e9 / HBM_PEAK_GBS, 4)}
    log(f"bench: decode GEMV B={B} as three launches: {step3_res['us_per_step']} us/step, {step3_res['gb_s']} GB/s")

    # Per-launch kernel time: back-to-back launches of one kernel (weights
    # rotating over the copies), HIP events on the launch stream around the
    # whole sequence, divided by the number of launches.
    def per_launch(fn_one, per_copy, reps, stats=None):
        """Average seconds per launch; with `stats` (a dict) also the median,
        p10 and p90 of the per-launch time over the individual replays."""
        def seq():
            for i in range(step_copies):
                fn_one(i)
        gr = capture(seq) if graphed else None
        with torch.cuda.stream(stream):
            (gr.replay() if gr is not None else seq())
        torch.cuda.synchronize()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
        with torch.cuda.stream(stream):
            ev[0].record(stream)
            for r in range(reps):
                (gr.replay() if gr is not None else seq())
                ev[r + 1].record(stream)
        torch.cuda.synchronize()
        per = step_copies * per_copy
        if stats is not None:
            samples = np.array([ev[r].elapsed_time(ev[r + 1]) * 1e3 / per for r in range(reps)])
            stats.update({"median_us": round(float(np.median(samples)), 3),
                          "p10_us": round(float(np.percentile(samples, 10)), 3),
                          "p90_us": round(float(np.percentile(samples, 90)), 3),
                          "samples": reps, "launches_per_sample": per})
        return ev[0].elapsed_time(ev[reps]) * 1e-3 / (reps * per)

    reps = max(3, args.steps // step_copies)
    dist_reps = max(reps, 30)  # enough replays for the percentiles (>= 200 launches per shape)
    dist = {"group_2x11008x4096": {}, "11008x4096": {}, "4096x11008": {}}
    t_grp = per_launch(lambda i: ctx.ternary_linear_group(x, [W[i][0], W[i][1]], [s_g, s_u], [g, u]), 1,
                       dist_reps, dist["group_2x11008x4096"])
    t_gu = per_launch(lambda i: (ctx.ternary_linear(W[i][0], s_g, x, g), ctx.ternary_linear(W[i][1], s_u, x, u)),
                      2, dist_reps, dist["11008x4096"])
    t_dn = per_launch(lambda i: ctx.ternary_linear(W[i][2], s_d, xd, y), 1, dist_reps, dist["4096x11008"])
    # the dominant kernel: the gate/up group launch (two thirds of the step)
    achieved = b_grp / t_grp / 1e9
    roofline = {
        "kernel": ("frx::gemv_bal_kernel same-x group (gate + up, 22016 rows, B=1, bf16 in, bf16 out)" if B == 1
                   else "gate and up as separate launches (the group is one launch at B=1 only): "
                        + ("frx::gemv_rows4_kernel" if 2 <= B <= 4 else "frx::gemv_xs_kernel")),
        "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
        "algorithmic_bytes_per_launch": b_grp,
        "avg_us": {"group_2x11008x4096": round(t_grp * 1e6, 3), "11008x4096": round(t_gu * 1e6, 3),
                   "4096x11008": round(t_dn * 1e6, 3)},
        "step_launches_weighted": {"achieved": round((b_grp + b_dn) / (t_grp + t_dn) / 1e9, 1),
                                   "frac": round((b_grp + b_dn) / (t_grp + t_dn) / 1e9 / HBM_PEAK_GBS, 4)},
        "launch_time_distribution": dist,
        "bytes_per_launch": {"group_2x11008x4096": b_grp, "11008x4096": b_gu, "4096x11008": b_dn},
        "timing": timing,
    }
    traffic_file = os.path.join(ROOT, "profiles", "gemv_traffic.json")
    ffn_traffic = None
    if os.path.exists(traffic_file):
        try:
            tr = json.load(open(traffic_file)).get("by_batch", {}).get(str(B))
            if tr:
                by = tr["bytes_per_launch"]
                roofline["traffic"] = by.get("group_2x11008x4096")
                roofline["traffic_by_shape"] = {k: by[k] for k in ("group_2x11008x4096", "11008x4096", "4096x11008")
                                                if k in by}
                ffn_traffic = {k: by[k] for k in ("ffn_glu_planes_11008x4096", "ffn_down_planes_4096x11008",
                                                  "glu_f32h_11008x4096", "down_f32x_4096x11008", "ffn1_llama7b")
                               if k in by}
        except (OSError, ValueError, KeyError):
            pass

    # The decode FFN of the same layer through frx_ternary_ffn, in each of
    # its modes: the default (B <= 2: gate/up/SiLU rows into bf16 hi/lo planes
    # of h, then the down rows over both planes; B = 3: one launch with a
    # grid barrier; B >= 4: two launches), the one-launch kernel (B <= 3) and
    # the two-launch execution. The frx_ternary_glu entry (fp32 h) and the
    # fp32-input down GEMV are timed on their own as well.
    b_glu = 2 * (I * H // 4 + 4 * I) + 2 * B * H + 4 * B * I
    b_down32 = H * I // 4 + 4 * H + 4 * B * I + 2 * B * H
    b_ffn = 2 * (I * H // 4 + 4 * I) + (H * I // 4 + 4 * H) + 2 * B * H + 2 * B * H

    def ffn_step(i):
        wg, wu, wd = W[i % step_copies]
        ctx.ternary_ffn(x, wg, s_g, wu, s_u, wd, s_d, y)
    fused = {"algorithmic_bytes_per_step": b_ffn}
    modes = [(frx.FFN_AUTO, "default"), (frx.FFN_TWO_LAUNCH, "two_launch")]
    if B <= 3:
        modes.append((frx.FFN_ONE_LAUNCH, "one_launch"))
    for mode, key in modes:
        ctx.set_ffn_mode(mode)
        with torch.cuda.stream(stream):  # first call per mode outside capture (it may allocate)
            ffn_step(0)
        torch.cuda.synchronize()
        el_f, _ = timed(lambda: [ffn_step(i) for i in range(args.steps)])
        ctx.synchronize()
        fused[key] = {"us_per_step": round(el_f / args.steps * 1e6, 2),
                      "gb_s": round(b_ffn / (el_f / args.steps) / 1e9, 1),
                      "hbm_fraction": round(b_ffn / (el_f / args.steps) / 1e9 / HBM_PEAK_GBS, 4)}
    ctx.set_ffn_mode(frx.FFN_AUTO)
    fused["default"]["launches_per_step"] = 1 if B == 3 else 2
    fused["default"]["kernels"] = (
        "gemv_bal_kernel gate/up/SiLU -> h planes, gemv_bal_kernel down over both planes" if B == 1 else
        "gemv_rows4_kernel gate/up/SiLU -> h planes, gemv_rows4_kernel down over both planes" if B == 2 else
        "ffn1_kernel" if B == 3 else "GLU + down GEMV (planes at B >= 4)")
    fused["two_launch"]["launches_per_step"] = 2
    if "one_launch" in fused:
        fused["one_launch"].update({"launches_per_step": 1, "kernels": "ffn1_kernel"})
        if ffn_traffic and "ffn1_llama7b" in ffn_traffic:
            fused["one_launch"]["traffic"] = ffn_traffic["ffn1_llama7b"]
    t_glu = per_launch(lambda i: ctx.ternary_glu(x, W[i][0], s_g, W[i][1], s_u, h), 1, reps)
    t_d32 = per_launch(lambda i: ctx.ternary_linear(W[i][2], s_d, h, y), 1, reps)
    fused["glu_entry_and_f32_down"] = {
        "gate_up_silu_avg_us": round(t_glu * 1e6, 3), "gate_up_silu_gb_s": round(b_glu / t_glu / 1e9, 1),
        "down_f32_in_avg_us": round(t_d32 * 1e6, 3), "down_f32_in_gb_s": round(b_down32 / t_d32 / 1e9, 1),
        "algorithmic_bytes": {"glu_11008x4096": b_glu, "down_f32_4096x11008": b_down32},
        "traffic": ffn_traffic}
    log(f"bench: decode FFN: default {fused['default']['us_per_step']} us/step "
        f"({fused['default']['launches_per_step']} launches), two-launch {fused['two_launch']['us_per_step']} us"
        + (f", one-launch {fused['one_launch']['us_per_step']} us" if "one_launch" in fused else "")
        + f"; frx_ternary_glu {t_glu * 1e6:.2f} us, fp32-input down {t_d32 * 1e6:.2f} us")

    extra = {"decode_ffn_fused_llama7b": fused, "decode_step_three_launches": step3_res}
    if B == 1 and not args.no_extra:
        # The decode configuration's other batch sizes: the same three
        # projections, weights rotating, timed the same way (B = 4: the
        # four-segment rows kernel; B = 16: the tall and direct kernels).
        batches = {}
        for bx in (4, 16):
            _, xbx = synth.activations("bench/decode", "x", bx, H)
            _, hbx = synth.activations("bench/decode", "h", bx, I)
            xx = torch.from_numpy(xbx.view(np.int16)).to(dev).view(torch.bfloat16)
            xdx = torch.from_numpy(hbx.view(np.int16)).to(dev).view(torch.bfloat16)
            gx = torch.empty((bx, I), dtype=torch.bfloat16, device=dev)
            ux = torch.empty((bx, I), dtype=torch.bfloat16, device=dev)
            yx = torch.empty((bx, H), dtype=torch.bfloat16, device=dev)

            def stepx(i, xx=xx, xdx=xdx, gx=gx, ux=ux, yx=yx):
                wg, wu, wd = W[i % step_copies]
                ctx.ternary_linear(wg, s_g, xx, gx)
                ctx.ternary_linear(wu, s_u, xx, ux)
                ctx.ternary_linear(wd, s_d, xdx, yx)
            with torch.cuda.stream(stream):
                for i in range(2):
                    stepx(i)
            torch.cuda.synchronize()
            el_x, _ = timed(lambda: [stepx(i) for i in range(args.steps)])
            bytes_x = 2 * gemv_bytes(I, H, bx) + gemv_bytes(H, I, bx)
            dist_x = {"11008x4096": {}, "4096x11008": {}}
            tgu_x = per_launch(lambda i: (ctx.ternary_linear(W[i][0], s_g, xx, gx),
                                          ctx.ternary_linear(W[i][1], s_u, xx, ux)), 2, dist_reps,
                               dist_x["11008x4096"])
            tdn_x = per_launch(lambda i: ctx.ternary_linear(W[i][2], s_d, xdx, yx), 1, dist_reps,
                               dist_x["4096x11008"])
            yfx = torch.empty((bx, H), dtype=torch.bfloat16, device=dev)

            def ffnx(i, xx=xx, yfx=yfx):
                wg, wu, wd = W[i % step_copies]
                ctx.ternary_ffn(xx, wg, s_g, wu, s_u, wd, s_d, yfx)
            with torch.cuda.stream(stream):  # first call outside capture (workspace)
                ffnx(0)
            torch.cuda.synchronize()
            el_fx, _ = timed(lambda: [ffnx(i) for i in range(args.steps)])
            b_ffn_x = 2 * (I * H // 4 + 4 * I) + (H * I // 4 + 4 * H) + 2 * bx * H + 2 * bx * H
            batches[f"B{bx}"] = {
                "decode_ffn_us_per_step": round(el_fx / args.steps * 1e6, 2),
                "decode_ffn_gb_s": round(b_ffn_x / (el_fx / args.steps) / 1e9, 1),
                "us_per_step": round(el_x / args.steps * 1e6, 2),
                "gb_s": round(bytes_x / (el_x / args.steps) / 1e9, 1),
                "hbm_fraction": round(bytes_x / (el_x / args.steps) / 1e9 / HBM_PEAK_GBS, 4),
                "avg_us": {"11008x4096": round(tgu_x * 1e6, 3), "4096x11008": round(tdn_x * 1e6, 3)},
                "launch_time_distribution": dist_x,
                "kernel": "frx::gemv_rows4_kernel" if bx <= 4 else "frx::gemv_kernel (staged)" if bx < 8
                else "frx::gemv_xs_kernel",
            }
            log(f"bench: decode GEMV B={bx}: {batches[f'B{bx}']['us_per_step']} us/step, "
                f"{batches[f'B{bx}']['gb_s']} GB/s; frx_ternary_ffn {batches[f'B{bx}']['decode_ffn_us_per_step']} us")
        extra["decode_gemv_llama7b_batches"] = batches
        # The literal drop-in: TernaryMatMulOp::dispatch and
        # gpu_ternary_matmul_vram hand over f32 activations and take f32
        # outputs. Per-launch times at the decode shapes, f32 in / f32 out.
        f32res = {}
        for bx in (1, 4, 16):
            xf32 = torch.randn((bx, H), dtype=torch.float32, device=dev)
            hf32 = torch.randn((bx, I), dtype=torch.float32, device=dev)
            yg = torch.empty((bx, I), dtype=torch.float32, device=dev)
            yd = torch.empty((bx, H), dtype=torch.float32, device=dev)
            with torch.cuda.stream(stream):
                ctx.ternary_linear(W[0][0], s_g, xf32, yg)
                ctx.ternary_linear(W[0][2], s_d, hf32, yd)
            torch.cuda.synchronize()
            t1 = per_launch(lambda i, xf32=xf32, yg=yg: ctx.ternary_linear(W[i][0], s_g, xf32, yg), 1, reps)
            t2 = per_launch(lambda i, hf32=hf32, yd=yd: ctx.ternary_linear(W[i][2], s_d, hf32, yd), 1, reps)
            f32res[f"B{bx}"] = {
                "avg_us": {"11008x4096": round(t1 * 1e6, 3), "4096x11008": round(t2 * 1e6, 3)},
                "gb_s": {"11008x4096": round(gemv_bytes(I, H, bx, 4, 4) / t1 / 1e9, 1),
                         "4096x11008": round(gemv_bytes(H, I, bx, 4, 4) / t2 / 1e9, 1)}}
            log(f"bench: f32 in/out B={bx}: {t1 * 1e6:.2f} / {t2 * 1e6:.2f} us per launch")
        extra["decode_gemv_f32_in_out"] = f32res
    if B == 1 and not args.no_extra:
        extra["decode_gemv_b1_by_weight_size"] = gemv_size_sweep(torch, ctx, stream, dev)
        extra["decode_gemv_b1_qkv_3x4096x4096"] = qkv_group(torch, ctx, stream, dev)
    if not args.no_extra:
        extra.update(run_extra(torch, frx, synth, ctx, stream, dev))

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(t_g, t_d, B, args.cpu_seconds)

    out = {
        "metric": "ternary GEMV GB/s (% HBM peak) + GEMM TFLOP/s (% MFMA peak), 1 MI355X",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "decode_gemv_llama7b_ffn_shapes",
            "batch_tokens": B,
            "projections": ["gate 11008x4096", "up 11008x4096", "down 4096x11008"],
            "x_dtype": "bf16", "y_dtype": "bf16", "accumulate": "fp32",
            "weight_copies": step_copies,
            "hbm_fraction": round(value / HBM_PEAK_GBS, 4),
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(out), flush=True)


def _time_kernel(torch, stream, fn, iters, warm=3, stats=None):
    """Average seconds per launch over `iters` back-to-back launches (HIP
    events on the launch stream); with `stats` also the median, p10 and p90
    of the individual launch times."""
    with torch.cuda.stream(stream):
        for _ in range(warm):
            fn()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(iters + 1)]
    with torch.cuda.stream(stream):
        ev[0].record(stream)
        for i in range(iters):
            fn()
            ev[i + 1].record(stream)
    torch.cuda.synchronize()
    if stats is not None:
        samples = np.array([ev[i].elapsed_time(ev[i + 1]) * 1e3 for i in range(iters)])
        stats.update({"median_us": round(float(np.median(samples)), 2),
                      "p10_us": round(float(np.percentile(samples, 10)), 2),
                      "p90_us": round(float(np.percentile(samples, 90)), 2), "launches": iters})
    return ev[0].elapsed_time(ev[iters]) * 1e-3 / iters


def _time_graph(torch, stream, fns, reps, stats=None):
    """Average seconds per launch of a short kernel: the launches `fns`
    captured back to back in one HIP graph (eager launches from Python would
    time the host), replayed `reps` times between HIP events; with `stats`
    also the median, p10 and p90 of the per-launch time over the replays."""
    def seq():
        for fn in fns:
            fn()
    with torch.cuda.stream(stream):
        seq()
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=stream):
        seq()
    with torch.cuda.stream(stream):
        gr.replay()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
    with torch.cuda.stream(stream):
        ev[0].record(stream)
        for r in range(reps):
            gr.replay()
            ev[r + 1].record(stream)
    torch.cuda.synchronize()
    n = len(fns)
    if stats is not None:
        samples = np.array([ev[r].elapsed_time(ev[r + 1]) * 1e3 / n for r in range(reps)])
        stats.update({"median_us": round(float(np.median(samples)), 2),
                      "p10_us": round(float(np.percentile(samples, 10)), 2),
                      "p90_us": round(float(np.percentile(samples, 90)), 2), "launches": reps * n})
    return ev[0].elapsed_time(ev[reps]) * 1e-3 / (reps * n)


def run_extra(torch, frx, synth, ctx, stream, dev, only=None, iters=200):
    res = {}
    M, K = 2048, 4096
    _, xb = synth.activations("bench/prefill", "x", M, K)
    X = torch.from_numpy(xb.view(np.int16)).to(dev).view(torch.bfloat16)
    for N in (4096, 11008):
        t = synth.ternary_uniform("bench/prefill", f"w{N}", N, K)
        w = torch.from_numpy(synth.pack_rows_u32(t).view(np.int32)).to(dev)
        s = torch.from_numpy(synth.row_scales("bench/prefill", f"s{N}", N, samples=256)).to(dev)
        Y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        if only in (None, "prefill"):
            st = {}
            dt = _time_kernel(torch, stream, lambda: ctx.ternary_linear(w, s, X, Y), iters, stats=st)
            tf = 2.0 * M * N * K / dt / 1e12
            res[f"prefill_gemm_{M}x{K}x{N}"] = {"us": round(dt * 1e6, 2), "tflops": round(tf, 1),
                                                "frac_bf16_peak": round(tf / BF16_PEAK_TFLOPS, 4), **st}
            log(f"bench: prefill N={N}: {dt * 1e6:.1f} us, {tf:.1f} TFLOP/s")
        if only in (None, "sparse24"):
            t24 = synth.sparse24_uniform("bench/sp24", f"w{N}", N, K)
            meta = torch.from_numpy(frx.pack_sparse24_gpu(t24).view(np.int32)).to(dev)
            st = {}
            dt = _time_kernel(torch, stream, lambda: ctx.sparse24_ternary_linear(meta, s, X, Y), iters, stats=st)
            tf = 2.0 * M * N * K / dt / 1e12
            res[f"sparse24_gemm_{M}x{K}x{N}"] = {"us": round(dt * 1e6, 2), "tflops_dense_equiv": round(tf, 1),
                                                 "frac_bf16_peak": round(tf / BF16_PEAK_TFLOPS, 4), **st}
            log(f"bench: 2:4 N={N}: {dt * 1e6:.1f} us, {tf:.1f} TFLOP/s dense-equivalent")
            # the same weights prepared once (frx_sparse24_prepare at upload):
            # the GEMM alone, and the preparing pass alone
            prep = torch.empty((N, K // 16), dtype=torch.int32, device=dev)
            st = {}
            dtp = _time_kernel(torch, stream, lambda: ctx.sparse24_prepare(meta, K, prep), iters, stats=st)
            res[f"sparse24_prepare_{N}x{K}"] = {"us": round(dtp * 1e6, 2), **st}
            st = {}
            dt = _time_kernel(torch, stream, lambda: ctx.sparse24_prepared_linear(prep, s, X, Y), iters, stats=st)
            tf = 2.0 * M * N * K / dt / 1e12
            res[f"sparse24_prepared_gemm_{M}x{K}x{N}"] = {
                "us": round(dt * 1e6, 2), "tflops_dense_equiv": round(tf, 1),
                "frac_bf16_peak": round(tf / BF16_PEAK_TFLOPS, 4), **st}
            log(f"bench: 2:4 prepared N={N}: {dt * 1e6:.1f} us (prepare {dtp * 1e6:.1f} us)")
            # one token through the 5-bit layout (the table GEMV), rotating over
            # enough copies of the metadata that every launch reads it from HBM
            mb = meta.numel() * 4
            ncp = (320 << 20) // mb + 1
            metas = [meta] + [meta.clone() for _ in range(ncp - 1)]
            x1 = X[:1]
            y1 = torch.empty((1, N), dtype=torch.bfloat16, device=dev)
            st = {}
            dt = _time_graph(torch, stream, [lambda c=c: ctx.sparse24_ternary_linear(metas[c], s, x1, y1)
                                             for c in range(ncp)], max(3, iters // ncp + 1), stats=st)
            res[f"sparse24_decode_gemv_1x{K}x{N}"] = {
                "us": round(dt * 1e6, 2), "metadata_gb_s": round(mb / dt / 1e9, 1), "metadata_bytes": mb,
                "copies": ncp, **st}
            log(f"bench: 2:4 decode GEMV N={N}, one token: {dt * 1e6:.2f} us")
            del meta, prep, metas
        del w, Y
    if only is None:
        res["gemm_ceilings"] = gemm_ceilings(torch, stream, dev, X)
    if only not in (None, "moe"):
        return res
    # MoE expert layer
    T, Hm, Im, E, k = 512, 2048, 5632, 16, 2
    _, xb = synth.activations("bench/moe", "x", T, Hm)
    _, rb = synth.activations("bench/moe", "router", E, Hm, std=0.02)
    xm = torch.from_numpy(xb.view(np.int16)).to(dev).view(torch.bfloat16)
    rm = torch.from_numpy(rb.view(np.int16)).to(dev).view(torch.bfloat16)
    tg = synth.ternary_uniform("bench/moe", "w", Im, Hm)
    td = synth.ternary_uniform("bench/moe", "wd", Hm, Im)
    pg = torch.from_numpy(synth.pack_rows_u32(tg).view(np.int32)).to(dev)
    pd = torch.from_numpy(synth.pack_rows_u32(td).view(np.int32)).to(dev)
    sg = torch.from_numpy(synth.row_scales("bench/moe", "s", Im, samples=256)).to(dev)
    sd = torch.from_numpy(synth.row_scales("bench/moe", "sd", Hm, samples=256)).to(dev)
    wg = [pg.clone() for _ in range(E)]
    wu = [pg.clone() for _ in range(E)]
    wd = [pd.clone() for _ in range(E)]
    ym = torch.empty((T, Hm), dtype=torch.bfloat16, device=dev)
    fn = lambda: ctx.moe_ternary_ffn(xm, rm, wg, [sg] * E, wu, [sg] * E, wd, [sd] * E, ym, top_k=k)  # noqa: E731
    st = {}
    dt = _time_kernel(torch, stream, fn, iters, stats=st)
    fl = T * k * 3 * 2.0 * Im * Hm
    tf = fl / dt / 1e12
    res["moe_512tok_h2048_i5632_e16_top2"] = {"us": round(dt * 1e6, 2), "tflops": round(tf, 1),
                                              "frac_bf16_peak": round(tf / BF16_PEAK_TFLOPS, 4), **st}
    log(f"bench: MoE: {dt * 1e6:.1f} us, {tf:.1f} TFLOP/s")
    # one token (the decode path: routing, a GEMV per routed row, combine),
    # graph replays over NS sets of the 16 experts so that the two routed
    # experts' weights (17 MB a call) come from HBM, not the 256 MB Infinity
    # Cache
    NS = 24
    del wg, wu, wd
    allg = torch.empty((NS * E,) + tuple(pg.shape), dtype=pg.dtype, device=dev)
    allu = torch.empty_like(allg)
    alld = torch.empty((NS * E,) + tuple(pd.shape), dtype=pd.dtype, device=dev)
    allg.copy_(pg.expand_as(allg))
    allu.copy_(pg.expand_as(allu))
    alld.copy_(pd.expand_as(alld))
    x1 = xm[:1]
    y1 = torch.empty((1, Hm), dtype=torch.bfloat16, device=dev)
    fns = [lambda c=c: ctx.moe_ternary_ffn(x1, rm, [allg[c * E + e] for e in range(E)], [sg] * E,
                                           [allu[c * E + e] for e in range(E)], [sg] * E,
                                           [alld[c * E + e] for e in range(E)], [sd] * E, y1, top_k=k)
           for c in range(NS)]
    st = {}
    dt = _time_graph(torch, stream, fns, 10, stats=st)
    res["moe_1tok_h2048_i5632_e16_top2"] = {"us": round(dt * 1e6, 2), "weight_sets": NS, **st}
    log(f"bench: MoE one token: {dt * 1e6:.2f} us")
    del allg, allu, alld
    return res


def gemm_ceilings(torch, stream, dev, X, iters=100):
    """What the matrix pipe and the vendor GEMM reach on this box, beside the
    ternary GEMMs: (i) frxb_mfma (libfrx_bench.so), back-to-back 16x16x32
    bf16 MFMAs on register operands with no memory traffic, 4 and 8 waves
    per compute unit; (ii) torch.matmul in bf16 (hipBLASLt) on the prefill
    shapes X[2048,4096] x W[4096,N] with W dense bf16 (N in {4096, 11008}),
    the same flops as the ternary prefill GEMM."""
    out = {}
    bl = _bench_lib()
    sink = torch.empty(bl.frxb_read_grid(), dtype=torch.float32, device=dev)
    cus = bl.frxb_read_grid() // 2
    mi = 20000
    for wpc in (4, 8):
        def run(wpc=wpc):
            rc = bl.frxb_mfma(mi, wpc, sink.data_ptr(), stream.cuda_stream)
            assert rc == 0, rc
        dt = _time_kernel(torch, stream, run, 10)
        fl = cus * wpc * mi * 8 * 16384.0
        out[f"mfma_loop_{wpc}_waves_per_cu"] = {"tflops": round(fl / dt / 1e12, 1),
                                                "frac_bf16_peak": round(fl / dt / 1e12 / BF16_PEAK_TFLOPS, 4),
                                                "us": round(dt * 1e6, 1)}
        log(f"bench: MFMA loop ({wpc} waves/CU): {fl / dt / 1e12:.0f} TFLOP/s")
    M, K = X.shape
    for N in (4096, 11008):
        Wt = torch.randn((K, N), device=dev).to(torch.bfloat16).contiguous()
        Y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        st = {}
        dt = _time_kernel(torch, stream, lambda: torch.matmul(X, Wt, out=Y), iters, stats=st)
        tf = 2.0 * M * N * K / dt / 1e12
        out[f"torch_matmul_bf16_{M}x{K}x{N}"] = {"us": round(dt * 1e6, 2), "tflops": round(tf, 1),
                                                  "frac_bf16_peak": round(tf / BF16_PEAK_TFLOPS, 4), **st}
        log(f"bench: torch.matmul bf16 N={N}: {dt * 1e6:.1f} us, {tf:.1f} TFLOP/s")
        del Wt, Y
    return out


def _graph_time(torch, stream, calls, reps):
    """Seconds per call: `calls` (a list of launch closures) captured in one
    HIP graph, replayed once untimed, then `reps` times between HIP events on
    the launch stream; also the median, p10 and p90 per call over replays."""
    with torch.cuda.stream(stream):
        for c in calls:
            c()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for c in calls:
            c()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        g.replay()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
    with torch.cuda.stream(stream):
        ev[0].record(stream)
        for r in range(reps):
            g.replay()
            ev[r + 1].record(stream)
    torch.cuda.synchronize()
    per = np.array([ev[r].elapsed_time(ev[r + 1]) * 1e-3 / len(calls) for r in range(reps)])
    total = ev[0].elapsed_time(ev[reps]) * 1e-3 / (reps * len(calls))
    return total, {"median_us": round(float(np.median(per)) * 1e6, 3),
                   "p10_us": round(float(np.percentile(per, 10)) * 1e6, 3),
                   "p90_us": round(float(np.percentile(per, 90)) * 1e6, 3),
                   "launches": reps * len(calls)}


def _bench_lib():
    """libfrx_bench.so (bench-only helpers: the streaming read ceiling)."""
    import ctypes
    h = ctypes.CDLL(os.path.join(ROOT, "ferrisres_amd", "libfrx_bench.so"))
    h.frxb_read.restype = ctypes.c_int
    h.frxb_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p]
    h.frxb_read_grid.restype = ctypes.c_int
    h.frxb_mfma.restype = ctypes.c_int
    h.frxb_mfma.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    return h


def gemv_size_sweep(torch, ctx, stream, dev, reps=40):
    """The B=1 decode GEMV (bf16 x, bf16 y) at growing weight sizes: the
    LLaMA-7B projection, the LLaMA-70B gate/up projection [28672, 8192] and
    both of them stacked [57344, 8192]. Each launch pays a fixed start-up
    (dispatch and the first HBM round trip); larger matrices spread it over
    more bytes, so the rate approaches what the kernel streams at. Weights
    are uniform ternary codes made on the device, rotating over copies that
    total >= 0.5 GB. Beside each GEMV, with the same rotation and timing:
    a plain streaming read of the same packed words (libfrx_bench.so
    frxb_read: 16-byte loads, two workgroups per CU, no decode), the ceiling
    a launch of that many bytes reaches, and torch's device copy of them
    (read + write). All three are timed as HIP-graph replays of one launch
    per weight copy."""
    res = {}
    bl = _bench_lib()
    sink = torch.empty(bl.frxb_read_grid(), dtype=torch.int32, device=dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(20240607)
    shifts = (2 * torch.arange(16, device=dev, dtype=torch.int64))
    for n, k in ((11008, 4096), (28672, 8192), (57344, 8192)):
        codes = torch.randint(0, 3, (n, k // 16, 16), generator=gen, device=dev, dtype=torch.int64)
        w0 = (codes << shifts).sum(dim=2).to(torch.int64)
        w0 = torch.where(w0 >= 2 ** 31, w0 - 2 ** 32, w0).to(torch.int32)
        del codes
        s = torch.full((n,), 0.0159, dtype=torch.float32, device=dev)
        x = torch.randn((1, k), generator=gen, device=dev).to(torch.bfloat16)
        y = torch.empty((1, n), dtype=torch.bfloat16, device=dev)
        nbytes = gemv_bytes(n, k, 1)
        wbytes = n * k // 4
        copies = max(3, int(np.ceil(512e6 / wbytes)) + 1)
        ws = [w0] + [w0.clone() for _ in range(copies - 1)]
        gemv_calls = [(lambda w=w: ctx.ternary_linear(w, s, x, y)) for w in ws]
        dt, st = _graph_time(torch, stream, gemv_calls, reps)

        def rd(w):
            rc = bl.frxb_read(w.data_ptr(), wbytes, sink.data_ptr(), stream.cuda_stream)
            assert rc == 0, rc
        dr, str_ = _graph_time(torch, stream, [(lambda w=w: rd(w)) for w in ws], reps)
        dst = torch.empty_like(w0)
        dc, _ = _graph_time(torch, stream, [(lambda w=w: dst.copy_(w)) for w in ws], reps)
        res[f"{n}x{k}"] = {"us": round(dt * 1e6, 3), "gb_s": round(nbytes / dt / 1e9, 1),
                           "hbm_fraction": round(nbytes / dt / 1e9 / HBM_PEAK_GBS, 4),
                           "algorithmic_bytes": nbytes, "weight_copies": copies, **st,
                           "read_ceiling_us": round(dr * 1e6, 3),
                           "read_ceiling_gb_s": round(wbytes / dr / 1e9, 1),
                           "read_ceiling_median_us": str_["median_us"],
                           "gemv_over_read_ceiling": round(dt / dr, 3),
                           "torch_copy_us": round(dc * 1e6, 3),
                           "torch_copy_gb_s_read_plus_write": round(2 * wbytes / dc / 1e9, 1)}
        log(f"bench: GEMV B=1 {n}x{k}: {dt * 1e6:.2f} us, {nbytes / dt / 1e9:.1f} GB/s; "
            f"read ceiling {dr * 1e6:.2f} us ({wbytes / dr / 1e9:.1f} GB/s); "
            f"torch copy {dc * 1e6:.2f} us")
        del dst
        del ws, w0, gemv_calls
        torch.cuda.synchronize()
    return res


def qkv_group(torch, ctx, stream, dev, reps=40):
    """The decode step's Q, K and V projections of one token (three
    [4096, 4096] ternary matrices against the same bf16 x, bf16 outputs),
    as three frx_ternary_linear launches and as one frx_ternary_linear_group
    launch, timed as HIP-graph replays over weight copies totalling >= 0.5 GB.
    Algorithmic bytes: 3 (N K / 4 + 4 N + 2 N) for the weights, scales and
    outputs, plus 2 K for x, which the group reads once and the separate
    launches three times."""
    n = k = 4096
    gen = torch.Generator(device=dev)
    gen.manual_seed(20240611)
    shifts = (2 * torch.arange(16, device=dev, dtype=torch.int64))
    base = []
    for _ in range(3):
        codes = torch.randint(0, 3, (n, k // 16, 16), generator=gen, device=dev, dtype=torch.int64)
        w = (codes << shifts).sum(dim=2)
        base.append(torch.where(w >= 2 ** 31, w - 2 ** 32, w).to(torch.int32))
    del codes
    copies = int(np.ceil(512e6 / (3 * n * k // 4))) + 1
    ws = [[b.clone() for b in base] for _ in range(copies)]
    s = [torch.full((n,), 0.0159, dtype=torch.float32, device=dev) for _ in range(3)]
    x = torch.randn((1, k), generator=gen, device=dev).to(torch.bfloat16)
    ys = [torch.empty((1, n), dtype=torch.bfloat16, device=dev) for _ in range(3)]
    nbytes = 3 * (n * k // 4 + 4 * n + 2 * n) + 2 * k
    sep = [(lambda w=w: [ctx.ternary_linear(w[j], s[j], x, ys[j]) for j in range(3)]) for w in ws]
    grp = [(lambda w=w: ctx.ternary_linear_group(x, w, s, ys)) for w in ws]
    t_sep, st_sep = _graph_time(torch, stream, sep, reps)
    t_grp, st_grp = _graph_time(torch, stream, grp, reps)
    log(f"bench: Q/K/V 3x4096x4096 B=1: three launches {t_sep * 1e6:.2f} us, "
        f"one group launch {t_grp * 1e6:.2f} us ({nbytes / t_grp / 1e9:.1f} GB/s)")
    res = {"algorithmic_bytes": nbytes, "weight_copies": copies,
           "group_launch": {"us": round(t_grp * 1e6, 3), "gb_s": round(nbytes / t_grp / 1e9, 1),
                            "hbm_fraction": round(nbytes / t_grp / 1e9 / HBM_PEAK_GBS, 4), **st_grp},
           "three_launches": {"us": round(t_sep * 1e6, 3), "gb_s": round(nbytes / t_sep / 1e9, 1),
                              "hbm_fraction": round(nbytes / t_sep / 1e9 / HBM_PEAK_GBS, 4), **st_sep}}
    del ws, base
    torch.cuda.synchronize()
    return res


def _cpu_time(fn, seconds, max_reps=200):
    """Median, p10 and p90 wall seconds of fn() over enough calls to fill
    about `seconds` (at least 3)."""
    t0 = time.perf_counter()
    fn()  # warm-up call, also the calibration
    t1 = time.perf_counter() - t0
    reps = max(3, min(max_reps, int(seconds / max(t1, 1e-6))))
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    ts = np.array(ts)
    return float(np.median(ts)), float(np.percentile(ts, 10)), float(np.percentile(ts, 90)), reps


def _cpu_entry(kernel, shapes, t, byts, flops, threads):
    med, p10, p90, reps = t
    return {"kernel": kernel, "shapes": shapes, "threads": threads, "reps": reps,
            "ms": round(med * 1e3, 3), "p10_ms": round(p10 * 1e3, 3), "p90_ms": round(p90 * 1e3, 3),
            "gb_s": round(byts / med / 1e9, 2), "gflop_s": round(flops / med / 1e9, 2)}


def cpu_baseline(t_gu, t_dn, B, seconds):
    """The reference's CPU linear paths restated in C by the oracle, on this
    host's cores (capped at 16, the CPU share of one GPU):

    value: ternary_matmul_packed_parallel (src/model/ternary.rs:471-529, u8
    packed, row batches over a thread pool) on the decode step's three
    matrices at B=1, in GB/s over the same algorithmic bytes as the GPU
    metric (f32 x and y on the CPU).

    breakdown: at the single-linear configuration (x[1,2048] f32,
    W[2048,2048]) and at the decode shapes, (i) the branchy i8 loop of
    benches/ternary_bench.rs:87-106 on one thread, (ii) the packed parallel
    path, (iii) the CPU 2:4 matmul SparseTernaryMatrix::matmul_decode
    (src/model/sparse_ternary.rs:255-320) on one thread; ms are medians over
    the reps, GB/s over the bytes each kernel reads (i8, u8 packed or
    pattern+sign bytes, plus f32 x and y), GFLOP/s as 2*N*K."""
    import oracle
    threads = max(1, min(16, os.cpu_count() or 1))
    n_gu, k_gu = t_gu.shape
    n_dn, k_dn = t_dn.shape
    p_gu = oracle.pack_ternary(t_gu)
    p_dn = oracle.pack_ternary(t_dn)
    x = np.linspace(-1, 1, k_gu, dtype=np.float32)
    h = np.linspace(-1, 1, k_dn, dtype=np.float32)
    # one calibration call, then reps so the sample takes ~half of `seconds`
    t1, _ = oracle.time_packed_parallel(p_gu, 0.01, x, n_gu, k_gu, threads, 1)
    t2, _ = oracle.time_packed_parallel(p_dn, 0.01, h, n_dn, k_dn, threads, 1)
    reps = max(3, int(0.5 * seconds / max(1e-6, 2 * t1 + t2)))
    q1 = np.zeros(2)
    q2 = np.zeros(2)
    t1, _ = oracle.time_packed_parallel(p_gu, 0.01, x, n_gu, k_gu, threads, reps, q1)
    t2, _ = oracle.time_packed_parallel(p_dn, 0.01, h, n_dn, k_dn, threads, reps, q2)
    step_t = 2 * t1 + t2
    # same algorithmic byte count as the GPU metric at B=1 (f32 x/y on CPU)
    byts = 2 * gemv_bytes(n_gu, k_gu, 1, 4, 4) + gemv_bytes(n_dn, k_dn, 1, 4, 4)

    from ferrisres_amd import synth
    budget = 0.5 * seconds / 4  # the rest of the sample over the four single-thread entries
    breakdown = []
    # single linear x[1,2048] f32 ~N(0,1), W[2048,2048] U{-1,0,+1}
    n1 = k1 = 2048
    w1 = synth.ternary_uniform("cpu/linear", "w", n1, k1)
    x1, _ = synth.activations("cpu/linear", "x", 1, k1, bf16=False)
    x1 = np.ascontiguousarray(x1.reshape(-1), dtype=np.float32)
    sc1 = float(synth.row_scales("cpu/linear", "s", 1)[0])
    fl1 = 2.0 * n1 * k1
    breakdown.append(_cpu_entry(
        "ternary_bench i8 (benches/ternary_bench.rs:87-106)", "1x2048x2048",
        _cpu_time(lambda: oracle.bench_ternary_matmul(x1, w1, sc1, 1, n1, k1), budget),
        n1 * k1 + 4 * k1 + 4 * n1, fl1, 1))
    p1 = oracle.pack_ternary(w1)
    q = np.zeros(2)
    t_p1, _ = oracle.time_packed_parallel(p1, sc1, x1, n1, k1, threads, 200, q)
    breakdown.append(_cpu_entry(
        "ternary_matmul_packed_parallel (ternary.rs:471-529)", "1x2048x2048",
        (t_p1, q[0], q[1], 200), gemv_bytes(n1, k1, 1, 4, 4) - 4 * n1, fl1, threads))
    s1 = synth.sparse24_uniform("cpu/linear", "w24", n1, k1)
    pt1, sg1 = oracle.sparse24_cpu_from_ternary(s1, n1, k1)
    breakdown.append(_cpu_entry(
        "SparseTernaryMatrix::matmul_decode (sparse_ternary.rs:255-320)", "1x2048x2048",
        _cpu_time(lambda: oracle.sparse24_cpu_matmul_decode(pt1, sg1, sc1, n1, k1, x1), budget),
        pt1.nbytes + sg1.nbytes + 4 * k1 + 4 * n1, fl1, 1))
    # decode shapes: one token through gate/up [11008,4096] and down [4096,11008]
    fl_step = 2.0 * (2 * n_gu * k_gu + n_dn * k_dn)
    breakdown.append(_cpu_entry(
        "ternary_bench i8 (benches/ternary_bench.rs:87-106)", "decode step 2x(11008x4096)+4096x11008",
        _cpu_time(lambda: (oracle.bench_ternary_matmul(x, t_gu, 0.01, 1, n_gu, k_gu),
                           oracle.bench_ternary_matmul(x, t_gu, 0.01, 1, n_gu, k_gu),
                           oracle.bench_ternary_matmul(h, t_dn, 0.01, 1, n_dn, k_dn)), budget, max_reps=20),
        2 * (n_gu * k_gu + 4 * k_gu + 4 * n_gu) + n_dn * k_dn + 4 * k_dn + 4 * n_dn, fl_step, 1))
    # p10/p90 of the step: the per-matrix percentiles added up (2 x gate/up + down)
    breakdown.append(_cpu_entry(
        "ternary_matmul_packed_parallel (ternary.rs:471-529)", "decode step 2x(11008x4096)+4096x11008",
        (step_t, 2 * q1[0] + q2[0], 2 * q1[1] + q2[1], reps), byts - 4 * (2 * n_gu + n_dn), fl_step, threads))
    s_gu = synth.sparse24_uniform("cpu/decode", "w24_gu", n_gu, k_gu)
    s_dn = synth.sparse24_uniform("cpu/decode", "w24_dn", n_dn, k_dn)
    pg, sgg = oracle.sparse24_cpu_from_ternary(s_gu, n_gu, k_gu)
    pd, sgd = oracle.sparse24_cpu_from_ternary(s_dn, n_dn, k_dn)
    breakdown.append(_cpu_entry(
        "SparseTernaryMatrix::matmul_decode (sparse_ternary.rs:255-320)", "decode step 2x(11008x4096)+4096x11008",
        _cpu_time(lambda: (oracle.sparse24_cpu_matmul_decode(pg, sgg, 0.01, n_gu, k_gu, x),
                           oracle.sparse24_cpu_matmul_decode(pg, sgg, 0.01, n_gu, k_gu, x),
                           oracle.sparse24_cpu_matmul_decode(pd, sgd, 0.01, n_dn, k_dn, h)), budget, max_reps=20),
        2 * (pg.nbytes + sgg.nbytes + 4 * k_gu + 4 * n_gu) + pd.nbytes + sgd.nbytes + 4 * k_dn + 4 * n_dn,
        fl_step, 1))
    try:
        avail = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        avail = os.cpu_count() or 1
    return {"value": round(byts / step_t / 1e9, 2), "unit": "GB/s", "cores": threads, "kind": "port",
            "host_cores": {"os_cpu_count": os.cpu_count(), "affinity": avail, "threads_used": threads,
                           "note": "threads capped at 16, the host share of one GPU on this machine"},
            "sample": f"ternary_matmul_packed_parallel (ternary.rs:471-529) restated in C, u8 layout, f32 x, "
                      f"1 token through 11008x4096 x2 + 4096x11008, median of {reps} reps each "
                      f"({step_t * 1e3:.2f} ms/step on {threads} threads)",
            "breakdown": breakdown}


if __name__ == "__main__":
    main()
