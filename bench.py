"""Benchmark of the SeedVR2 DiT window-attention hot path on one MI355X.

Workload (one step = one DiT block's hot path at the SeedVR2-3B 720p video
shape, 21 frames at 1280x720 -> 6x45x80 = 21,600 video tokens + 64 text
tokens, hidden 2560, 20 heads x 128, bf16 with fp32 accumulation):

  SharedLinear QKV   2560 -> 7680        (both streams, one grouped launch) and
  AdaptiveWindowAttention, regular 3-D windows (27 windows of 780/810 tokens),
                     in one call (s2_awa_qkv_forward: the window gather, RMSNorm
                     and RoPE run in the projection's epilogue)
  SharedLinear out   2560 -> 2560
  SharedLinear MLP   2560 -> 10240, GELU
  SharedLinear MLP   10240 -> 2560

Algorithmic work per step: 4*H*d*sum_w (n_w+64)^2 attention FLOPs (206.45 G)
plus 2*M*K*N per GEMM with M = 21,664 (3,407.45 G): 3.614 TFLOP.  Inputs and
weights are resident in HBM before the timed region (seeded N(0,1)
activations, N(0,0.02) weights).  The shifted-window block (64 ragged
windows) is timed too and reported beside the headline, as is the same block
with the projection and the attention as two calls (s2_shared_linear_forward
writing the QKV blob, then s2_awa_forward), and so is the
SeedVR2-7B-shaped stack of 32 blocks (hidden 3072, 24 heads x 128, MLP
3072 -> 12288 -> 3072, regular windows in even and shifted windows in odd
blocks, 64 text tokens projected 5120 -> 3072 once) under "stack_7b".  The
frontend/tail kernels (patchify, unpatchify, CFG, Euler update) at the 720p
latent are timed under "sampler_tail", the VAE decoder's DecomposedConv3D
layers under "vae_conv3d" and its VAEChunkedMHA under "vae_mha".

Prints one JSON line.  `--gpus` above 1 is refused: this build measures one GPU.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0     # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0         # MI355X HBM3E

VIDEO_SHAPE = (6, 45, 80)
TEXT_TOKENS = 64
HIDDEN, HEADS, HEAD_DIM, PAIRS = 2560, 20, 128, 21
MLP = 10240
TARGET = (4, 3, 3)


def attention_flops(shifted):
    from seedvr2_ncnn_amd import capi
    wins, _, _ = capi.plan_windows([VIDEO_SHAPE], TARGET, shifted)
    return sum(4 * HEADS * HEAD_DIM * (w[8] + TEXT_TOKENS) ** 2 for w in wins)


def prologue_bytes(shifted, hidden=HIDDEN):
    """Algorithmic HBM bytes of the attention prologue: read the bf16 q, k, v
    of every video and text token once and write the windowed bf16 Q, K and
    V^T of every token once (a window's video rows to its segment, a sample's
    text rows to its one staging copy).  The window index math reads no
    tables; the same for both window modes."""
    lv = VIDEO_SHAPE[0] * VIDEO_SHAPE[1] * VIDEO_SHAPE[2]
    return 2 * (lv + TEXT_TOKENS) * 3 * hidden * 2


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "shared_linear_mlp_up_720p_video_traffic.md")


def measured_traffic():
    """HBM bytes per launch of the MLP-up GEMM from the committed rocprofv3
    PMC summary (FETCH_SIZE + WRITE_SIZE, copy-calibrated), or None."""
    try:
        with open(TRAFFIC_PROFILE) as f:
            for line in f:
                if line.startswith("TRAFFIC_BYTES_PER_LAUNCH"):
                    return int(line.split("=")[1].strip())
    except OSError:
        pass
    return None


def host_cpu():
    """CPU model, logical CPUs of the host and CPUs this process may run on."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    logical = os.cpu_count() or 1
    try:
        allowed = len(os.sched_getaffinity(0))
    except AttributeError:
        allowed = logical
    return model, logical, allowed


def job_cpu_threads():
    """Threads of the multi-threaded CPU legs: the CPUs this process may run
    on, at most 16, which is one GPU's share of the host's cores on a shared
    8-GPU machine."""
    return max(1, min(16, host_cpu()[2]))


def _torch_gemm_seconds(rows, k, n, act, threads, g):
    """fp32 torch.matmul on the CPU (oneDNN/MKL-backed) of `rows` x k by
    k x n plus bias and, for act == 1, erf-GELU: the optimised-library
    stand-in for ncnn's Gemm."""
    import torch
    torch.set_num_threads(threads)
    x = torch.from_numpy(g.standard_normal((rows, k), dtype="float32"))
    w = torch.from_numpy(0.02 * g.standard_normal((n, k), dtype="float32"))
    b = torch.from_numpy(0.02 * g.standard_normal(n, dtype="float32"))
    y = torch.addmm(b, x, w.t())   # warm-up (page-in, thread pool)
    best = float("inf")
    for _ in range(2):
        t0 = time.perf_counter()
        y = torch.addmm(b, x, w.t())
        if act == 1:
            y = torch.nn.functional.gelu(y)
        best = min(best, time.perf_counter() - t0)
    return best


def cpu_baseline(threads):
    """The reference's CPU path restated and timed on this host's cores.

    Attention: the oracle's optimised build (oracle/liboracle_fast.so, the
    reference CPU forward of adaptive_window_attention.cpp:764-978 restated in
    C: serial window loop, fp32 SDPA per head) over all 27 windows with
    `threads` OpenMP threads, and over windows 0 and 1 on one thread (the
    reference build's NCNN_OPENMP OFF), scaled by FLOPs to all 27.
    GEMMs: fp32 torch.matmul (addmm) as the optimised-library stand-in for
    ncnn's Gemm, on the first rows of each of the four GEMMs (2048 rows with
    `threads` threads, 256 rows on one), scaled to all 21,664 rows.
    About 15-30 s of CPU work."""
    import numpy as np
    import torch
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from common import make_awa_inputs, oracle_awa
    from seedvr2_ncnn_amd import capi

    t_start = time.time()
    shapes, tl = [VIDEO_SHAPE], [TEXT_TOKENS]
    case = make_awa_inputs(7, shapes, tl, HEADS, HEAD_DIM, PAIRS, bf16=True)
    wins, _, _ = capi.plan_windows([VIDEO_SHAPE], TARGET, 0)
    win_flops = [4 * HEADS * HEAD_DIM * (w[8] + TEXT_TOKENS) ** 2 for w in wins]
    t0 = time.perf_counter()
    oracle_awa(case, HEADS, HEAD_DIM, TARGET, 0, 1e-5, PAIRS, shapes, tl, threads=threads, fast=True)
    attn_mt = time.perf_counter() - t0
    subset = [0, 1]
    t0 = time.perf_counter()
    oracle_awa(case, HEADS, HEAD_DIM, TARGET, 0, 1e-5, PAIRS, shapes, tl, threads=1, fast=True,
               window_subset=subset)
    attn_1 = (time.perf_counter() - t0) * sum(win_flops) / sum(win_flops[i] for i in subset)
    del case
    m = VIDEO_SHAPE[0] * VIDEO_SHAPE[1] * VIDEO_SHAPE[2] + TEXT_TOKENS
    shapes_g = ((HIDDEN, 3 * HIDDEN, 0), (HIDDEN, HIDDEN, 0), (HIDDEN, MLP, 1), (MLP, HIDDEN, 0))
    g = np.random.default_rng(3)
    prev = torch.get_num_threads()
    gemm_mt = sum(_torch_gemm_seconds(2048, k, n, a, threads, g) * m / 2048 for k, n, a in shapes_g)
    gemm_1 = sum(_torch_gemm_seconds(256, k, n, a, 1, g) * m / 256 for k, n, a in shapes_g)
    torch.set_num_threads(prev)
    total = sum(win_flops) + 2 * m * (HIDDEN * 3 * HIDDEN + HIDDEN * HIDDEN + 2 * HIDDEN * MLP)
    block_mt, block_1 = attn_mt + gemm_mt, attn_1 + gemm_1
    model, logical, allowed = host_cpu()
    return {
        "value": round(total / block_mt / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"attention: oracle/liboracle_fast.so (the reference CPU forward restated in C, "
                   f"fp32, OpenMP over heads) on all 27 windows ({sum(win_flops) / 1e9:.1f} GFLOP, "
                   f"{attn_mt:.2f} s on {threads} threads); GEMMs: fp32 torch.addmm on the CPU as "
                   f"the optimised-library stand-in for ncnn Gemm, first 2048 of 21664 rows of "
                   f"QKV/out/MLP-up+GELU/MLP-down scaled to all rows ({gemm_mt:.2f} s): "
                   f"{block_mt:.1f} s per block; sampled in {time.time() - t_start:.1f} s"),
        "ms_per_block": round(block_mt * 1e3, 1),
        "one_thread": {
            "value": round(total / block_1 / 1e12, 6), "unit": "TFLOP/s", "cores": 1,
            "ms_per_block": round(block_1 * 1e3, 1),
            "sample": (f"attention windows 0-1 of 27 on one thread scaled by FLOPs "
                       f"({attn_1:.1f} s per layer); GEMMs on the first 256 rows scaled "
                       f"({gemm_1:.1f} s per block); the reference build runs ncnn with "
                       f"NCNN_OPENMP OFF"),
        },
        "cpu_model": model,
        "host_logical_cpus": logical,
        "cpus_allowed": allowed,
        "threads_note": "multi-threaded legs use the CPUs this process may run on, at most 16 "
                        "(one GPU's share of a shared 8-GPU host)",
    }


def awa_configs(threads, reps=20):
    """The single-layer attention configurations, each on the GPU (kernel
    time of one s2_awa_forward, HIP events on the launching stream, inputs
    resident) and on the CPU (the oracle's optimised build on one thread and
    on `threads` threads), with the parity of the GPU output against the
    oracle's test build on the same inputs, computed outside the timed
    region:
      cfg1  grid 1x32x32, 8 heads x 64, target (1,8,8), unshifted, fp32 in/out
      cfg2  grid 1x64x64, 20 heads x 128, target (4,3,3), regular and shifted, bf16 in
      cfg3  grid 6x45x80, 20 heads x 128, target (4,3,3), regular and shifted, bf16 in
            (parity only: its time is the headline's attention)."""
    import numpy as np
    import torch
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from common import MAX_ABS_TOL, COSINE_TOL, make_awa_inputs, metrics, oracle_awa
    from seedvr2_ncnn_amd import capi
    dev = torch.device("cuda:0")
    cases = [("cfg1", (1, 32, 32), 8, 64, 10, (1, 8, 8), 0, False),
             ("cfg2_regular", (1, 64, 64), 20, 128, 21, (4, 3, 3), 0, True),
             ("cfg2_shifted", (1, 64, 64), 20, 128, 21, (4, 3, 3), 1, True),
             ("cfg3_regular", VIDEO_SHAPE, 20, 128, 21, (4, 3, 3), 0, True),
             ("cfg3_shifted", VIDEO_SHAPE, 20, 128, 21, (4, 3, 3), 1, True)]
    out = {}
    for name, grid, heads, d, pairs, target, shifted, bf16 in cases:
        shapes, tl = [grid], [TEXT_TOKENS]
        inner = heads * d
        case = make_awa_inputs(101, shapes, tl, heads, d, pairs, bf16=bf16)
        dt = torch.bfloat16 if bf16 else torch.float32
        v = torch.from_numpy(case["video"]).to(dev).to(dt)
        t = torch.from_numpy(case["text"]).to(dev).to(dt)
        norms = torch.from_numpy(case["norms"]).to(dev)
        freqs = torch.from_numpy(case["freqs"]).to(dev)
        cfg = capi.awa_config(heads, d, target, shifted, 1e-5, pairs)
        rec = {"grid": list(grid), "heads": heads, "head_dim": d, "target": list(target),
               "shifted": shifted, "dtype": "bf16" if bf16 else "fp32", "text_tokens": TEXT_TOKENS}
        with capi.AwaPlan(cfg, shapes, tl) as plan:
            ws = torch.empty(plan.info.workspace_bytes, dtype=torch.uint8, device=dev)
            ov = torch.empty(plan.info.video_tokens, inner, dtype=torch.float32, device=dev)
            ot = torch.empty(plan.info.text_tokens, inner, dtype=torch.float32, device=dev)

            def fwd():
                capi.awa_forward(plan, norms, freqs, v[:, :inner], v[:, inner:2 * inner],
                                 v[:, 2 * inner:], t[:, :inner], t[:, inner:2 * inner],
                                 t[:, 2 * inner:], workspace=ws, out_video=ov, out_text=ot)
            fwd()
            torch.cuda.synchronize()
            got_v, got_t = ov.cpu().numpy(), ot.cpu().numpy()
            if not name.startswith("cfg3"):
                for _ in range(3):
                    fwd()
                start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                start.record()
                for _ in range(reps):
                    fwd()
                end.record()
                torch.cuda.synchronize()
                gpu_ms = start.elapsed_time(end) / reps
                wins, _ = plan.windows()
                flops = sum(4 * heads * d * (w[8] + TEXT_TOKENS) ** 2 for w in wins)
                rec.update(gpu_ms=round(gpu_ms, 4), gflop=round(flops / 1e9, 3),
                           gpu_tflops=round(flops / (gpu_ms * 1e-3) / 1e12, 1))
        ref_v, ref_t = oracle_awa(case, heads, d, target, shifted, 1e-5, pairs, shapes, tl,
                                  threads=threads)
        ma_v, cs_v = metrics(got_v, ref_v)
        ma_t, cs_t = metrics(got_t, ref_t)
        rec["parity"] = {"video_max_abs": ma_v, "video_cosine": cs_v, "text_max_abs": ma_t,
                         "text_cosine": cs_t, "tol_max_abs": MAX_ABS_TOL, "tol_cosine": COSINE_TOL,
                         "pass": bool(max(ma_v, ma_t) <= MAX_ABS_TOL and min(cs_v, cs_t) >= COSINE_TOL)}
        if not name.startswith("cfg3"):
            cpu = {}
            for th in (1, threads):
                t0 = time.perf_counter()
                oracle_awa(case, heads, d, target, shifted, 1e-5, pairs, shapes, tl, threads=th,
                           fast=True)
                cpu[th] = (time.perf_counter() - t0) * 1e3
            rec["cpu_ms_one_thread"] = round(cpu[1], 2)
            rec[f"cpu_ms_{threads}_threads"] = round(cpu[threads], 2)
        out[name] = rec
        del v, t
    return out


def gemm_parity(x_v, x_t, weights, rows=256):
    """Parity of the four block GEMMs (cfg4 shapes) on the first `rows`
    video rows and all text rows: the GPU's fp32-output SharedLinear on the
    same bf16 inputs against the oracle's fp32 X W^T + b, outside the timed
    region."""
    import numpy as np
    import torch
    import oracle
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from common import MAX_ABS_TOL, COSINE_TOL, metrics
    from seedvr2_ncnn_amd import capi
    out = {}
    threads = job_cpu_threads()
    for name, (w, bias, act) in weights.items():
        k = w.shape[1]
        xv = x_v[:, :k] if x_v.shape[1] >= k else None
        if xv is None:
            g = torch.Generator(device=x_v.device).manual_seed(5)
            xv = torch.randn(x_v.shape[0], k, generator=g, device=x_v.device).to(torch.bfloat16)
            xt = torch.randn(x_t.shape[0], k, generator=g, device=x_v.device).to(torch.bfloat16)
        else:
            xt = x_t[:, :k]
        xv, xt = xv.contiguous(), xt.contiguous()
        yv, yt = capi.shared_linear(xv, xt, w, bias, act, out_dtype=torch.float32)
        torch.cuda.synchronize()
        xs = torch.cat([xv[:rows], xt]).float().cpu().numpy()
        ref = oracle.linear(xs, w.float().cpu().numpy(), bias.cpu().numpy(), act, threads=threads)
        got = torch.cat([yv[:rows], yt]).cpu().numpy()
        ma, cs = metrics(got, ref)
        out[name] = {"rows_checked": int(xs.shape[0]), "max_abs": ma, "cosine": cs,
                     "tol_max_abs": MAX_ABS_TOL, "tol_cosine": COSINE_TOL,
                     "pass": bool(ma <= MAX_ABS_TOL and cs >= COSINE_TOL)}
    return out


LATENT_SHAPE = (6, 90, 160)    # 720p latent: 21 frames -> 6, 720/8, 1280/8


def sampler_tail(reps=50):
    """The frontend and tail kernels around the block stack at the 720p
    latent (6x90x160 = 86,400 tokens, 21,600 patches), each timed over
    `reps` back-to-back launches with HIP events on the launching stream.
    Algorithmic bytes: every input element read once, every output element
    written once (fp32); the Euler update reads and writes the 16 latent
    planes.  Also times the oracle's serial CPU restatement of one denoise
    step's tail (unpatchify twice, CFG with rescale, Euler) on one core."""
    import numpy as np
    import torch
    import oracle
    from seedvr2_ncnn_amd import capi

    t, h, w = LATENT_SHAPE
    tokens, patches = t * h * w, t * h * w // 4
    stride = tokens
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(99)

    def randn(*shape):
        return torch.randn(*shape, generator=gen, device=dev, dtype=torch.float32)

    lat, cond = randn(16, stride), randn(16, stride)
    video, pos, neg = randn(tokens, 33), randn(patches, 64), randn(patches, 64)
    pp, pn = torch.empty(tokens, 16, device=dev), torch.empty(tokens, 16, device=dev)
    out132 = torch.empty(patches, 132, device=dev)
    cfg_out = torch.empty(tokens, 16, device=dev)
    f4 = 4
    pl = tokens * 16 * f4          # one prediction / one set of 16 planes
    cases = {
        "latent_patches": (lambda: capi.latent_patches(lat, cond, t, h, w, stride, patches=out132),
                           2 * pl + patches * 132 * f4),
        "patchify": (lambda: capi.patchify_video(video, [LATENT_SHAPE], patches=out132),
                     2 * tokens * 33 * f4),
        "unpatchify": (lambda: capi.unpatchify_prediction(pos, [LATENT_SHAPE], prediction=pp), 2 * pl),
        "apply_cfg_rescale": (lambda: capi.apply_cfg(pp, pn, 6.5, 0.7, output=cfg_out), 3 * pl),
        "euler_step": (lambda: capi.euler_step(lat, stride, cfg_out, 0.0), 3 * pl),
        "denoise_update_cfg_rescale": (
            lambda: capi.denoise_update(pos, neg, t, h, w, 6.5, 0.7, 0.0, lat, stride), 4 * pl),
    }
    capi.unpatchify_prediction(neg, [LATENT_SHAPE], prediction=pn)
    out = {}
    for name, (fn, nbytes) in cases.items():
        for _ in range(5):
            fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            fn()
        b.record()
        torch.cuda.synchronize()
        ms = a.elapsed_time(b) / reps
        out[name] = {"us": round(ms * 1e3, 2), "algorithmic_bytes": nbytes,
                     "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                     "frac_hbm_peak": round(nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}
    unfused = sum(out[k]["us"] for k in ("unpatchify", "apply_cfg_rescale", "euler_step")) + out["unpatchify"]["us"]
    out["step_tail_unfused_us"] = round(unfused, 2)
    out["step_tail_fused_us"] = out["denoise_update_cfg_rescale"]["us"]

    g = np.random.default_rng(5)
    h_pos = g.standard_normal((patches, 64), dtype=np.float32)
    h_neg = g.standard_normal((patches, 64), dtype=np.float32)
    h_lat = g.standard_normal((16, stride), dtype=np.float32)
    t0 = time.perf_counter()
    _, a = oracle.unpatchify_prediction(h_pos, [LATENT_SHAPE])
    _, b = oracle.unpatchify_prediction(h_neg, [LATENT_SHAPE])
    guided = oracle.apply_cfg(a.ravel(), b.ravel(), 6.5, 0.7).reshape(a.shape)
    oracle.euler_step(h_lat, guided, -0.02)
    out["cpu_step_tail_ms"] = round((time.perf_counter() - t0) * 1e3, 2)
    out["workload"] = (f"720p latent {t}x{h}x{w} = {tokens} tokens, {patches} patches; "
                       "fp32; CFG scale 6.5, rescale 0.7")
    del lat, cond, video, pos, neg, pp, pn, out132, cfg_out
    torch.cuda.empty_cache()
    return out


# VAE decoder DecomposedConv3D layers (3x3x3, pad 1, causal 2-frame memory)
# at 720p: one temporal slice of 4 output frames at each resolution level
# (one frame at the two lowest), and the encoder's RGB input layer over 4
# full-resolution frames
VAE_CONV_LAYERS = [
    ("full_res_128", 128, 128, 4, 720, 1280),
    ("half_res_256", 256, 256, 4, 360, 640),
    ("quarter_res_512", 512, 512, 1, 180, 320),
    ("rgb_out_128_to_3", 128, 3, 4, 720, 1280),
    ("rgb_in_3_to_128", 3, 128, 4, 720, 1280),
    ("latent_res_512", 512, 512, 1, 90, 160),
]


def vae_conv3d(reps=5, cpu_threads=16, cpu=True):
    """DecomposedConv3D at the VAE decoder's layer shapes.  Each forward
    continues a 2-frame temporal memory (the decoder's slices after the first,
    seedvr2_vae.cpp:424-447), so every output frame is a full 3x3x3 window:
    algorithmic FLOPs 2 * out_pixels * cout * cin * 27.  Timed end to end
    (staging + implicit GEMM) with HIP events over `reps` forwards, bf16
    device blobs, and fp32 blobs for the full-resolution layer.  The CPU
    baseline is the oracle's fp64-accumulating restatement (liboracle_fast)
    on a band of 64 output rows of one output frame of the full-resolution
    layer, scaled to the whole slice."""
    import numpy as np
    import torch
    from seedvr2_ncnn_amd import capi

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(7)
    out = {}
    for name, cin, cout, frames, h, w in VAE_CONV_LAYERS:
        cfg = capi.conv3d_config(num_output=cout, num_input=cin, kernel_t=3, kernel_h=3,
                                 kernel_w=3, pad_h=1, pad_w=1, head_frames=2, bias_term=1)
        wts = torch.randn(3, cout, cin, 3, 3, generator=gen, device=dev) / (cin * 27) ** 0.5
        conv = capi.Conv3d(cfg, wts, torch.randn(cout, generator=gen, device=dev) * 0.1)
        flops = 2.0 * frames * h * w * cout * cin * 27
        dtypes = (torch.bfloat16, torch.float32) if name == "full_res_128" else (torch.bfloat16,)
        for dt in dtypes:
            x = torch.randn(cin, frames * h * w, generator=gen, device=dev).to(dt)
            conv.forward(x, frames, h, w, keep_memory=True)
            for _ in range(2):
                conv.forward(x, frames, h, w, use_memory=True, keep_memory=True)
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(reps):
                y, _ = conv.forward(x, frames, h, w, use_memory=True, keep_memory=True)
            b.record()
            torch.cuda.synchronize()
            ms = a.elapsed_time(b) / reps
            key = f"{name}_{'bf16' if dt == torch.bfloat16 else 'fp32'}"
            out[key] = {"shape": f"{cin}->{cout} 3x3x3, {frames} frames {h}x{w} + 2 cached",
                        "ms": round(ms, 3), "tflop": round(flops / 1e12, 3),
                        "tflops": round(flops / (ms * 1e-3) / 1e12, 1),
                        "frac_bf16_peak": round(flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)}
            if cout <= 3:
                # bound by its input: the narrow kernel reads each input row
                # once (and the rows above and below a band of rows once
                # more), writes the output and passes two frames of partial
                # sums from forward to forward
                esz = 2 if dt == torch.bfloat16 else 4
                nbytes = (cin * frames * h * w * esz + cout * frames * h * w * esz +
                          2 * 2 * cout * h * w * 4)
                out[key].update({
                    "bound": "hbm", "algorithmic_bytes": int(nbytes),
                    "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                    "frac_hbm_peak": round(nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                    "bytes_note": "input frames once, output, memory partial sums read and "
                                  "written; a layer that cached its last two 128-channel input "
                                  "frames instead would also read those (1.42 GB per 4-frame "
                                  "bf16 slice in all)"})
            elif cin <= 8:
                # bound by its output: the RGB-input kernel writes cout
                # channel planes per frame from a few input channels (the
                # staged 8-channel pixels and the memory frames are read
                # once more than the input planes, and counted here)
                esz = 2 if dt == torch.bfloat16 else 4
                nbytes = (cin * frames * h * w * esz + cout * frames * h * w * esz +
                          (frames + 2) * h * w * 16)
                out[key].update({
                    "bound": "hbm", "algorithmic_bytes": int(nbytes),
                    "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                    "frac_hbm_peak": round(nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                    "bytes_note": "input planes and output planes once, the 8-channel staged "
                                  "pixels (input and 2 memory frames) once"})
            del x, y
        del conv, wts
        torch.cuda.empty_cache()
    if cpu:
        import oracle
        rows = 64
        g = np.random.default_rng(1)
        cfg_o = oracle.conv3d_config(num_output=128, num_input=128, kernel_t=3, kernel_h=3,
                                     kernel_w=3, pad_h=1, pad_w=0, head_frames=2, bias_term=1)
        # 1 output frame of a band of `rows` output rows (rows + 2 input rows,
        # the left/right padding applied by hand), 3 input frames via the memory
        x = g.standard_normal((128, 1, rows + 2, 1282), dtype=np.float32)
        x[:, :, :, 0] = x[:, :, :, -1] = 0
        mem = g.standard_normal((128, 2, rows + 2, 1282), dtype=np.float32)
        wt = (g.standard_normal((3, 128, 128, 3, 3), dtype=np.float32) / 60).astype(np.float32)
        cfg_o.pad_h = 0
        t0 = time.perf_counter()
        code, _, _ = oracle.decomposed_conv3d(cfg_o, x, wt, np.zeros(128, np.float32), memory=mem,
                                              threads=cpu_threads, fast=True)
        dt = time.perf_counter() - t0
        band = 2.0 * rows * 1280 * 128 * 128 * 27
        full = 2.0 * 4 * 720 * 1280 * 128 * 128 * 27
        out["cpu_baseline_full_res_128"] = {
            "value": round(band / dt / 1e12, 6), "unit": "TFLOP/s", "cores": cpu_threads,
            "kind": "port", "ms_per_slice": round(dt * full / band * 1e3, 1),
            "sample": f"oracle (liboracle_fast) on 1 output frame x {rows} rows x 1280 of the "
                      f"128->128 layer ({band / 1e9:.1f} GFLOP, {dt:.1f} s), scaled to 4x720x1280"}
    return out


def vae_mha(reps=5, cpu_threads=16, cpu=True):
    """VAEChunkedMHA at one 720p latent frame: 90 x 160 = 14,400 tokens of
    width 512, one head.  Algorithmic FLOPs: the q, k, v and out
    projections 4 * 2 * seq * 512^2 plus the two attention products
    2 * 2 * seq^2 * 512.  Timed end to end with HIP events over `reps`
    forwards (bf16 device blobs).  The CPU baseline is the oracle (fp64,
    liboracle_fast): its k/v projections, then 64 query rows, scaled to all
    rows."""
    import numpy as np
    import torch
    from seedvr2_ncnn_amd import capi

    seq, e = 14400, 512
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(11)
    w = [torch.randn(e, e, generator=gen, device=dev) / e ** 0.5 for _ in range(4)]
    b = [torch.randn(e, generator=gen, device=dev) * 0.1 for _ in range(4)]
    mha = capi.Mha(1, w[0], b[0], w[1], b[1], w[2], b[2], w[3], b[3])
    x = torch.randn(seq, e, generator=gen, device=dev).to(torch.bfloat16)
    for _ in range(2):
        mha.forward(x)
    torch.cuda.synchronize()
    a, z = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        y = mha.forward(x)
    z.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(z) / reps
    flops = 4 * 2.0 * seq * e * e + 2 * 2.0 * seq * seq * e
    out = {"shape": f"{seq} tokens x {e}, 1 head (one 90x160 latent frame)", "ms": round(ms, 3),
           "gflop": round(flops / 1e9, 1), "tflops": round(flops / (ms * 1e-3) / 1e12, 1),
           "frac_bf16_peak": round(flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)}
    del mha, x, y
    torch.cuda.empty_cache()
    if cpu:
        import oracle
        g = np.random.default_rng(2)
        xs = g.standard_normal((seq, e), dtype=np.float32)
        ws = [g.standard_normal((e, e), dtype=np.float32) / 23 for _ in range(4)]
        bs = [np.zeros(e, np.float32) for _ in range(4)]
        args = (ws[0], bs[0], ws[1], bs[1], ws[2], bs[2], ws[3], bs[3])
        t0 = time.perf_counter()
        oracle.mha(xs, 1, *args, rows=np.zeros(0, np.int32), threads=cpu_threads, fast=True)
        t_kv = time.perf_counter() - t0
        rows = np.linspace(0, seq - 1, 64).astype(np.int32)
        t0 = time.perf_counter()
        oracle.mha(xs, 1, *args, rows=rows, threads=cpu_threads, fast=True)
        t_rows = time.perf_counter() - t0 - t_kv
        full = t_kv + t_rows * seq / len(rows)
        out["cpu_baseline"] = {
            "value": round(flops / full / 1e12, 6), "unit": "TFLOP/s", "cores": cpu_threads,
            "kind": "port", "ms": round(full * 1e3, 1),
            "sample": f"oracle (liboracle_fast): k/v projections ({t_kv:.1f} s) and 64 of "
                      f"{seq} query rows ({t_rows:.1f} s), scaled to all rows"}
    return out


STACK_HIDDEN, STACK_HEADS, STACK_MLP, STACK_BLOCKS, STACK_TEXT_WIDTH = 3072, 24, 12288, 32, 5120


def stack_7b(steps, warmup):
    """SeedVR2-7B-shaped 32-block stack of the hot path at the 720p video
    grid: per block QKV -> window attention (regular windows in even blocks,
    shifted in odd ones) -> out -> MLP up GELU -> down, each block's output
    feeding the next; the 64 text tokens are projected 5120 -> 3072 once per
    stack.  Every block has its own random-init bf16 weights (7.2 GB).  Also
    timed: the same stack with every block's norm and AdaSingle modulation."""
    import torch
    from seedvr2_ncnn_amd import capi
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(7)
    bf = torch.bfloat16
    D, H, F = STACK_HIDDEN, STACK_HEADS, STACK_MLP
    lv = VIDEO_SHAPE[0] * VIDEO_SHAPE[1] * VIDEO_SHAPE[2]
    lt = TEXT_TOKENS

    def randn(*shape, std=1.0):
        return (torch.randn(*shape, generator=gen, device=dev, dtype=torch.float32) * std).to(bf)

    def bias(n):
        return torch.randn(n, generator=gen, device=dev) * 0.02

    blocks = [dict(qkv=randn(3 * D, D, std=0.02), bqkv=bias(3 * D), o=randn(D, D, std=0.02),
                   bo=bias(D), up=randn(F, D, std=0.02), bup=bias(F), dn=randn(D, F, std=0.02),
                   bdn=bias(D), norms=(1.0 + 0.02 * torch.randn(4, HEAD_DIM, generator=gen,
                                                                device=dev)).contiguous())
              for _ in range(STACK_BLOCKS)]
    w_text, b_text = randn(D, STACK_TEXT_WIDTH, std=0.02), bias(D)
    freqs = (10000.0 ** (-torch.arange(PAIRS, device=dev, dtype=torch.float64) / PAIRS)).float()
    x_v0, text_in = randn(lv, D), randn(lt, STACK_TEXT_WIDTH)
    x_v, x_t = torch.empty(lv, D, dtype=bf, device=dev), torch.empty(lt, D, dtype=bf, device=dev)
    a_v, a_t = torch.empty_like(x_v), torch.empty_like(x_t)
    o_v, o_t = torch.empty_like(x_v), torch.empty_like(x_t)
    h_v = torch.empty(lv, F, dtype=bf, device=dev)
    h_t = torch.empty(lt, F, dtype=bf, device=dev)
    plans = {s: capi.AwaPlan(capi.awa_config(H, HEAD_DIM, TARGET, s, 1e-5, PAIRS), [VIDEO_SHAPE], [lt])
             for s in (0, 1)}
    for p in plans.values():
        p.cache_rope(freqs)   # the layer keeps its frequencies' cos/sin table with the plan
    ws = torch.empty(max(p.info.workspace_bytes for p in plans.values()), dtype=torch.uint8, device=dev)

    def forward():
        x_v.copy_(x_v0)
        capi.shared_linear(text_in, None, w_text, b_text, capi.ACT_NONE, y_video=x_t)
        for i, blk in enumerate(blocks):
            capi.awa_qkv_forward(plans[i % 2], x_v, x_t, blk["qkv"], blk["bqkv"], blk["norms"],
                                 freqs, workspace=ws, out_video=a_v, out_text=a_t)
            capi.shared_linear(a_v, a_t, blk["o"], blk["bo"], capi.ACT_NONE, y_video=o_v, y_text=o_t)
            capi.shared_linear(o_v, o_t, blk["up"], blk["bup"], capi.ACT_GELU, y_video=h_v, y_text=h_t)
            capi.shared_linear(h_v, h_t, blk["dn"], blk["bdn"], capi.ACT_NONE, y_video=x_v, y_text=x_t)

    # The whole stack with each block's norm and AdaSingle modulation on an
    # fp32 residual stream: block i's MLP gate and residual sum share one
    # s2_dit_ada_out_in pass with block i + 1's attention norm and modulation.
    res_v = torch.empty(lv, D, device=dev)
    res_t = torch.empty(lt, D, device=dev)
    hin_v, hin_t = torch.empty_like(x_v), torch.empty_like(x_t)
    mods = [{k: torch.randn(1, D, generator=gen, device=dev) * 0.1 + (1.0 if k.endswith("scale") else 0.0)
             for k in ("a_shift", "a_scale", "a_gate", "m_shift", "m_scale", "m_gate")}
            for _ in range(STACK_BLOCKS)]
    vr, tr = [lv], [lt]

    def forward_full():
        res_v.copy_(x_v0)
        capi.shared_linear(text_in, None, w_text, b_text, capi.ACT_NONE, y_video=x_t)
        res_t.copy_(x_t)
        capi.ada_in(res_v, res_t, vr, tr, mods[0]["a_shift"], mods[0]["a_scale"],
                    out_video=hin_v, out_text=hin_t)
        for i, blk in enumerate(blocks):
            md = mods[i]
            capi.awa_qkv_forward(plans[i % 2], hin_v, hin_t, blk["qkv"], blk["bqkv"],
                                 blk["norms"], freqs, workspace=ws, out_video=a_v, out_text=a_t)
            capi.shared_linear(a_v, a_t, blk["o"], blk["bo"], capi.ACT_NONE, y_video=o_v, y_text=o_t)
            capi.ada_out_in(res_v, res_t, o_v, o_t, vr, tr, md["a_gate"], md["m_shift"],
                            md["m_scale"], h_video=hin_v, h_text=hin_t)
            capi.shared_linear(hin_v, hin_t, blk["up"], blk["bup"], capi.ACT_GELU, y_video=h_v,
                               y_text=h_t)
            capi.shared_linear(h_v, h_t, blk["dn"], blk["bdn"], capi.ACT_NONE, y_video=o_v,
                               y_text=o_t)
            if i + 1 < len(blocks):
                nx = mods[i + 1]
                capi.ada_out_in(res_v, res_t, o_v, o_t, vr, tr, md["m_gate"], nx["a_shift"],
                                nx["a_scale"], h_video=hin_v, h_text=hin_t)
            else:
                capi.ada_out(res_v, res_t, o_v, o_t, vr, tr, md["m_gate"])

    # The same with the gated residual sums in the epilogues of the out and
    # MLP-down projections (s2_shared_linear_residual, in place) and the two
    # norms per block as s2_dit_ada_in passes: bit for bit the stack above.
    def forward_fused():
        res_v.copy_(x_v0)
        capi.shared_linear(text_in, None, w_text, b_text, capi.ACT_NONE, y_video=x_t)
        res_t.copy_(x_t)
        for i, blk in enumerate(blocks):
            md = mods[i]
            capi.ada_in(res_v, res_t, vr, tr, md["a_shift"], md["a_scale"], out_video=hin_v,
                        out_text=hin_t)
            capi.awa_qkv_forward(plans[i % 2], hin_v, hin_t, blk["qkv"], blk["bqkv"],
                                 blk["norms"], freqs, workspace=ws, out_video=a_v, out_text=a_t)
            capi.shared_linear_residual(a_v, a_t, blk["o"], blk["bo"], vr, tr, res_v, res_t,
                                        md["a_gate"])
            capi.ada_in(res_v, res_t, vr, tr, md["m_shift"], md["m_scale"], out_video=hin_v,
                        out_text=hin_t)
            capi.shared_linear(hin_v, hin_t, blk["up"], blk["bup"], capi.ACT_GELU, y_video=h_v,
                               y_text=h_t)
            capi.shared_linear_residual(h_v, h_t, blk["dn"], blk["bdn"], vr, tr, res_v, res_t,
                                        md["m_gate"])

    def timed(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(steps):
            fn()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / steps

    ms = timed(forward)
    finite = bool(torch.isfinite(x_v.float()).all().item())
    ms_full = timed(forward_full)
    full_out = res_v.clone()
    ms_fused = timed(forward_fused)
    finite = finite and bool(torch.isfinite(res_v).all().item())
    same = bool(torch.equal(full_out, res_v))
    del full_out

    m = lv + lt
    gemm = 2 * m * D * (3 * D + D + 2 * F)
    attn = {s: sum(4 * H * HEAD_DIM * (w[8] + lt) ** 2 for w in capi.plan_windows([VIDEO_SHAPE], TARGET, s)[0])
            for s in (0, 1)}
    flops = (2 * lt * STACK_TEXT_WIDTH * D
             + sum(gemm + attn[i % 2] for i in range(STACK_BLOCKS)))
    for p in plans.values():
        p.close()
    del blocks
    torch.cuda.empty_cache()
    tf = flops / (ms * 1e-3) / 1e12
    return {"workload": f"SeedVR2-7B-shaped {STACK_BLOCKS}-block stack at 6x45x80 + {lt} text tokens: "
                        f"hidden {D}, {H}x{HEAD_DIM} heads, MLP {D}->{F} GELU ->{D}, even blocks "
                        f"regular / odd blocks shifted windows, text {STACK_TEXT_WIDTH}->{D} once",
            "steps": steps, "warmup": warmup, "ms_per_stack": round(ms, 3),
            "ms_per_block": round(ms / STACK_BLOCKS, 4), "stack_tflop": round(flops / 1e12, 3),
            "tflops": round(tf, 1), "pct_bf16_peak": round(100 * tf / PEAK_BF16_TFLOPS, 2),
            "ms_per_stack_with_modulation": round(min(ms_fused, ms_full), 3),
            "ms_per_stack_with_modulation_residual_in_gemm_epilogue": round(ms_fused, 3),
            "ms_per_stack_with_modulation_separate_residual": round(ms_full, 3),
            "fused_equals_separate_bit_for_bit": same,
            "modulation_note": "fp32 residual stream; each block's norm + AdaSingle modulation "
                               "and gated residual sums: the residual sums in the out and "
                               "MLP-down GEMM epilogues (s2_shared_linear_residual) and two "
                               "s2_dit_ada_in passes per block; separately: s2_dit_ada_in once, "
                               "s2_dit_ada_out_in twice per block, s2_dit_ada_out after the last",
            "output_finite": finite}


V3_MLP = 3456   # SwiGLU gate/up width of v3 manifests (seedvr2_pipeline.cpp:434-438)


def v3_block(steps, warmup):
    """The v3 DiT block shape at 720p (hidden 2560, 20x128 heads): separate
    q, k and v projections 2560 -> 2560 feeding the attention's split form,
    out 2560 -> 2560, the SwiGLU gate/up projection 2560 -> 2 x 3456 with
    silu(gate) * up in the GEMM's epilogue, down 3456 -> 2560.  Also timed:
    the same block with q/k/v as one fused projection (s2_awa_qkv_forward on
    the concatenated weights)."""
    import torch
    from seedvr2_ncnn_amd import capi
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(11)
    bf = torch.bfloat16
    D, F = HIDDEN, V3_MLP
    lv = VIDEO_SHAPE[0] * VIDEO_SHAPE[1] * VIDEO_SHAPE[2]
    lt = TEXT_TOKENS
    m = lv + lt

    def randn(*shape, std=1.0):
        return (torch.randn(*shape, generator=gen, device=dev) * std).to(bf)

    def bias(n):
        return torch.randn(n, generator=gen, device=dev) * 0.02

    x_v, x_t = randn(lv, D), randn(lt, D)
    wq, wk, wv, wo = (randn(D, D, std=0.02) for _ in range(4))
    bq, bk, bv, bo = (bias(D) for _ in range(4))
    w_gu, b_gu = capi.swiglu_pack_weight(randn(F, D, std=0.02), randn(F, D, std=0.02), bias(F), bias(F))
    w_dn, b_dn = randn(D, F, std=0.02), bias(D)
    w_qkv, b_qkv = torch.cat([wq, wk, wv]).contiguous(), torch.cat([bq, bk, bv])
    norms = (1.0 + 0.02 * torch.randn(4, HEAD_DIM, generator=gen, device=dev)).contiguous()
    freqs = (10000.0 ** (-torch.arange(PAIRS, device=dev, dtype=torch.float64) / PAIRS)).float()
    plan = capi.AwaPlan(capi.awa_config(HEADS, HEAD_DIM, TARGET, 0, 1e-5, PAIRS), [VIDEO_SHAPE], [lt])
    plan.cache_rope(freqs)
    ws = torch.empty(plan.info.workspace_bytes, dtype=torch.uint8, device=dev)
    q = [(torch.empty(lv, D, dtype=bf, device=dev), torch.empty(lt, D, dtype=bf, device=dev))
         for _ in range(3)]
    a_v, a_t = torch.empty(lv, D, dtype=bf, device=dev), torch.empty(lt, D, dtype=bf, device=dev)
    o_v, o_t = torch.empty_like(a_v), torch.empty_like(a_t)
    h_v, h_t = torch.empty(lv, F, dtype=bf, device=dev), torch.empty(lt, F, dtype=bf, device=dev)
    y_v, y_t = torch.empty_like(a_v), torch.empty_like(a_t)
    names = ["q", "k", "v", "attention", "out", "swiglu_gate_up", "down"]

    def step(fused, ev=None):
        def mark(i):
            if ev is not None:
                ev[i].record()
        mark(0)
        if fused:
            capi.awa_qkv_forward(plan, x_v, x_t, w_qkv, b_qkv, norms, freqs, workspace=ws,
                                 out_video=a_v, out_text=a_t)
            for i in range(1, 4):
                mark(i)
        else:
            for i, (w, b_) in enumerate(((wq, bq), (wk, bk), (wv, bv))):
                capi.shared_linear(x_v, x_t, w, b_, capi.ACT_NONE, y_video=q[i][0], y_text=q[i][1])
                mark(i + 1)
            capi.awa_forward(plan, norms, freqs, q[0][0], q[1][0], q[2][0], q[0][1], q[1][1],
                             q[2][1], workspace=ws, out_video=a_v, out_text=a_t)
        mark(4)
        capi.shared_linear(a_v, a_t, wo, bo, capi.ACT_NONE, y_video=o_v, y_text=o_t)
        mark(5)
        capi.shared_linear(o_v, o_t, w_gu, b_gu, capi.ACT_SWIGLU, y_video=h_v, y_text=h_t)
        mark(6)
        capi.shared_linear(h_v, h_t, w_dn, b_dn, capi.ACT_NONE, y_video=y_v, y_text=y_t)
        mark(7)

    flops = {"q": 2 * m * D * D, "k": 2 * m * D * D, "v": 2 * m * D * D,
             "attention": attention_flops(0), "out": 2 * m * D * D,
             "swiglu_gate_up": 2 * m * D * 2 * F, "down": 2 * m * F * D}
    total = sum(flops.values())
    out = {"workload": f"v3 block shape at 6x45x80 + {lt} text tokens: q/k/v {D}->{D} each, "
                       f"window attention (split form, regular windows), out {D}->{D}, SwiGLU "
                       f"{D}->2x{F} (silu(gate)*up fused), down {F}->{D}",
           "block_tflop": round(total / 1e12, 4)}
    for fused in (False, True):
        for _ in range(warmup):
            step(fused)
        torch.cuda.synchronize()
        evs = [[torch.cuda.Event(enable_timing=True) for _ in range(8)] for _ in range(steps)]
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for i in range(steps):
            step(fused, evs[i])
        end.record()
        torch.cuda.synchronize()
        ms = start.elapsed_time(end) / steps
        per = {n: sum(e[j].elapsed_time(e[j + 1]) for e in evs) / steps for j, n in enumerate(names)}
        rec = {"ms_per_block": round(ms, 4), "tflops": round(total / (ms * 1e-3) / 1e12, 1),
               "pct_bf16_peak": round(100 * total / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 2)}
        if fused:
            qa = sum(per[n] for n in ("q", "k", "v", "attention"))
            rec["qkv_attention_ms"] = round(qa, 4)
        else:
            rec["kernels"] = {n: {"ms": round(per[n], 4),
                                  "tflops": round(flops[n] / (per[n] * 1e-3) / 1e12, 1)}
                              for n in names}
        out["fused_qkv" if fused else "separate_qkv"] = rec
    plan.close()
    del ws, q, a_v, a_t, o_v, o_t, h_v, h_t, y_v, y_t
    torch.cuda.empty_cache()
    out["graph"] = v3_graph(steps, warmup, flops)
    return out


def _v3_graph_text():
    """The v3 block at 720p as an ncnn .param (one block, regular windows):
    DiTAdaIn -> q / k / v SharedLinear -> AdaptiveWindowAttention (8-input
    form) -> out SharedLinear -> DiTAdaOutIn -> gate / up SharedLinear ->
    Swish, BinaryOp mul per stream -> down SharedLinear -> DiTAdaOut, Splits
    where a blob has several readers, as an ncnn export writes them."""
    D, F = HIDDEN, V3_MLP
    layers = [("Input", f"in{i}", [], [f"in{i}"], "") for i in range(10)]
    layers += [
        ("DiTAdaIn", "ada_in", ["in0", "in1", "in4", "in5"], ["h_v", "h_t"], f"0={D} 1=1.000000e-05 2=0"),
        ("SharedLinear", "q", ["h_v", "h_t"], ["q_v", "q_t"], f"0={D} 1={D} 2=1"),
        ("SharedLinear", "k", ["h_v", "h_t"], ["k_v", "k_t"], f"0={D} 1={D} 2=1"),
        ("SharedLinear", "v", ["h_v", "h_t"], ["v_v", "v_t"], f"0={D} 1={D} 2=1"),
        ("AdaptiveWindowAttention", "attn", ["q_v", "k_v", "v_v", "q_t", "k_t", "v_t", "in2", "in3"],
         ["a_v", "a_t"], f"0={HEADS} 1={HEAD_DIM} 2={TARGET[0]} 3={TARGET[1]} 4={TARGET[2]} 5=0 "
                         f"6=1.000000e-05 7={PAIRS} 8=0 9=0 10=0"),
        ("SharedLinear", "out", ["a_v", "a_t"], ["o_v", "o_t"], f"0={D} 1={D} 2=1"),
        ("DiTAdaOutIn", "ada_out_in", ["in0", "in1", "o_v", "o_t", "in6", "in7", "in8"],
         ["r_v", "r_t", "m_v", "m_t"], f"0={D} 1=1.000000e-05 2=0"),
        ("SharedLinear", "gate", ["m_v", "m_t"], ["g_v", "g_t"], f"0={F} 1={D} 2=1"),
        ("SharedLinear", "up", ["m_v", "m_t"], ["u_v", "u_t"], f"0={F} 1={D} 2=1"),
        ("Swish", "silu_v", ["g_v"], ["sg_v"], ""), ("Swish", "silu_t", ["g_t"], ["sg_t"], ""),
        ("BinaryOp", "glu_v", ["sg_v", "u_v"], ["gu_v"], "0=2"),
        ("BinaryOp", "glu_t", ["sg_t", "u_t"], ["gu_t"], "0=2"),
        ("SharedLinear", "down", ["gu_v", "gu_t"], ["y_v", "y_t"], f"0={D} 1={F} 2=1"),
        ("DiTAdaOut", "ada_out", ["r_v", "r_t", "y_v", "y_t", "in9"], ["out0", "out1"], f"0={D} 2=0"),
    ]
    uses = {}
    for _, _, bottoms, _, _ in layers:
        for b_ in bottoms:
            uses[b_] = uses.get(b_, 0) + 1
    taken, lines, blobs = {}, [], set()
    for type_, name, bottoms, tops, params in layers:
        nb = []
        for b_ in bottoms:
            if uses[b_] > 1:
                nb.append(f"{b_}_s{taken.get(b_, 0)}")
                taken[b_] = taken.get(b_, 0) + 1
            else:
                nb.append(b_)
        lines.append(f"{type_} {name} {len(nb)} {len(tops)} " + " ".join(nb + tops) + (" " + params if params else ""))
        blobs.update(tops)
        for t in tops:
            if uses.get(t, 0) > 1:
                st = [f"{t}_s{i}" for i in range(uses[t])]
                lines.append(f"Split split_{t} 1 {len(st)} {t} " + " ".join(st))
                blobs.update(st)
    return "7767517\n" + f"{len(lines)} {len(blobs)}\n" + "\n".join(lines) + "\n"


def v3_graph(steps, warmup, flops):
    """The v3 block of v3_block as a graph: the .param above and a raw-fp32
    .bin of seeded weights, loaded by seedvr2::DiTBlockGraph (the ncnn Net /
    Extractor with its graph folds: q / k / v stacked into the attention's
    fused QKV projection, gate / up / Swish / mul into the SwiGLU epilogue)
    and run on device blobs (bf16 video and text rows, fp32 modulation
    vectors, the shape blobs on the host), through the C wrapper the graph
    tests use (tests/harness/liblayer_harness.so).  Each run ends with its
    outputs copied out and the stream synchronised, so the time includes the
    executor's host work; the norm / modulation passes (DiTAdaIn,
    DiTAdaOutIn, DiTAdaOut) run too, and are not in the FLOPs."""
    import ctypes
    import numpy as np
    import torch
    path = os.path.join(ROOT, "tests", "harness", "liblayer_harness.so")
    if not os.path.exists(path):
        return {"skipped": "tests/harness/liblayer_harness.so is not built"}
    L = ctypes.CDLL(path)
    P, vp, ci = ctypes.POINTER, ctypes.c_void_p, ctypes.c_int

    class HBlob(ctypes.Structure):
        _fields_ = [("dims", ci), ("w", ci), ("h", ci), ("elemsize", ci), ("device", ci), ("data", vp)]
    L.h_graph_create.argtypes = [ctypes.c_char_p, vp, ctypes.c_long, ci, ci, P(vp)]
    L.h_graph_fused_swiglu.argtypes = [vp]
    L.h_graph_fused_qkv.argtypes = [vp]
    L.h_graph_destroy.argtypes = [vp]
    L.h_graph_run.argtypes = [vp, P(ci), P(ci), ci, P(HBlob), P(HBlob), ci, P(ctypes.c_char_p)]
    D, F = HIDDEN, V3_MLP
    g = np.random.default_rng(31)
    parts = []

    def lin(n, k):
        parts.append((0.02 * g.standard_normal((n, k), dtype=np.float32)))
        parts.append((0.02 * g.standard_normal(n, dtype=np.float32)))
    for _ in range(3):
        lin(D, D)
    parts.append((1.0 + 0.02 * g.standard_normal(4 * HEAD_DIM, dtype=np.float32)))
    parts.append((10000.0 ** (-np.arange(PAIRS, dtype=np.float64) / PAIRS)).astype(np.float32))
    lin(D, D)
    lin(F, D)
    lin(F, D)
    lin(D, F)
    model = b"".join(np.ascontiguousarray(p_, dtype="<f4").tobytes() for p_ in parts)
    del parts
    nbytes = len(model)
    buf = ctypes.create_string_buffer(model, nbytes)
    del model
    h = ctypes.c_void_p()
    text = _v3_graph_text()
    ret = L.h_graph_create(text.encode(), buf, nbytes, 0, 3, ctypes.byref(h))
    del buf
    if ret != 0:
        return {"skipped": f"graph load returned {ret}"}
    try:
        dev = torch.device("cuda:0")
        gen = torch.Generator(device=dev).manual_seed(12)
        lv = VIDEO_SHAPE[0] * VIDEO_SHAPE[1] * VIDEO_SHAPE[2]
        lt = TEXT_TOKENS
        x_v = torch.randn(lv, D, generator=gen, device=dev).to(torch.bfloat16)
        x_t = torch.randn(lt, D, generator=gen, device=dev).to(torch.bfloat16)
        mods = [torch.randn(1, D, generator=gen, device=dev) * 0.1 + (1.0 if k in (1, 4) else 0.0)
                for k in range(6)]
        shape = np.asarray([VIDEO_SHAPE], np.float32)
        tlen = np.asarray([[lt]], np.float32)
        ins = (HBlob * 10)()
        ins[0] = HBlob(2, D, lv, 2, 1, x_v.data_ptr())
        ins[1] = HBlob(2, D, lt, 2, 1, x_t.data_ptr())
        ins[2] = HBlob(2, 3, 1, 4, 0, shape.ctypes.data)
        ins[3] = HBlob(2, 1, 1, 4, 0, tlen.ctypes.data)
        for i, m_ in enumerate(mods):
            ins[4 + i] = HBlob(2, D, 1, 4, 1, m_.data_ptr())
        o_v = torch.empty(lv, D, dtype=torch.bfloat16, device=dev)
        o_t = torch.empty(lt, D, dtype=torch.bfloat16, device=dev)
        outs = (HBlob * 2)()
        outs[0] = HBlob(2, D, lv, 2, 1, o_v.data_ptr())
        outs[1] = HBlob(2, D, lt, 2, 1, o_t.data_ptr())
        sh = np.asarray(VIDEO_SHAPE, np.int32)
        tl = np.asarray([lt], np.int32)
        names = (ctypes.c_char_p * 1)()
        ip = ctypes.POINTER(ctypes.c_int)

        def run():
            r = L.h_graph_run(h, sh.ctypes.data_as(ip), tl.ctypes.data_as(ip), 1, ins, outs, 0, names)
            if r != 0:
                raise RuntimeError(f"graph run returned {r}")
        torch.cuda.synchronize()
        for _ in range(max(2, warmup)):
            run()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            run()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / steps
        total = sum(flops.values())
        rec = {"ms_per_block": round(ms, 4), "tflops_hot_path": round(total / (ms * 1e-3) / 1e12, 1),
               "fused_swiglu": L.h_graph_fused_swiglu(h), "fused_qkv": L.h_graph_fused_qkv(h),
               "output_finite": bool(torch.isfinite(o_v.float()).all().item()),
               "note": "wall time per graph run (host executor + device work + output copy "
                       "and stream sync); includes the block's norm / modulation passes"}
        return rec
    finally:
        L.h_graph_destroy(h)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-parity", action="store_true",
                    help="skip the single-layer configurations (cfg1-cfg3 timings and parity) "
                         "and the GEMM parity records")
    ap.add_argument("--block-only", action="store_true",
                    help="time only the DiT block (no stack, sampler tail, VAE, parity or CPU "
                         "baseline): the run that rocprofv3 counter passes profile")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--no-stack", action="store_true", help="skip the 32-block 7B-shaped stack")
    ap.add_argument("--no-v3", action="store_true",
                    help="skip the v3-shaped block (split q/k/v, SwiGLU 3456)")
    ap.add_argument("--stack-steps", type=int, default=3)
    ap.add_argument("--no-tail", action="store_true",
                    help="skip the frontend/tail kernels at the 720p latent")
    ap.add_argument("--no-vae", action="store_true",
                    help="skip the VAE DecomposedConv3D and VAEChunkedMHA layers")
    ap.add_argument("--vae-only", action="store_true",
                    help="time only the VAE DecomposedConv3D and VAEChunkedMHA layers "
                         "(one JSON object)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run one 1 GiB device copy (a plain copy kernel of known size) so "
                         "that PMC byte counters can be calibrated in the same profiler run")
    args = ap.parse_args()
    if args.block_only:
        args.no_stack = args.no_tail = args.no_vae = args.no_parity = args.no_cpu_baseline = True
        args.no_v3 = True
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported by this build "
              "(the multi-GPU sharding is a design, not a measured path)", file=sys.stderr)
        sys.exit(2)

    import torch
    from seedvr2_ncnn_amd import capi

    assert torch.cuda.is_available() and capi.device_count() >= 1, "needs a gfx950 GPU"
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.copy_calibration:
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if args.vae_only:
        threads = args.cpu_threads or job_cpu_threads()
        print(json.dumps({"vae_conv3d": vae_conv3d(cpu_threads=threads,
                                                   cpu=not args.no_cpu_baseline),
                          "vae_mha": vae_mha(cpu_threads=threads, cpu=not args.no_cpu_baseline)}),
              flush=True)
        return
    gen = torch.Generator(device=dev).manual_seed(20240601)
    bf = torch.bfloat16
    lv = VIDEO_SHAPE[0] * VIDEO_SHAPE[1] * VIDEO_SHAPE[2]
    lt = TEXT_TOKENS

    def randn(*shape, std=1.0):
        return (torch.randn(*shape, generator=gen, device=dev, dtype=torch.float32) * std).to(bf)

    x_v, x_t = randn(lv, HIDDEN), randn(lt, HIDDEN)
    w_qkv, w_o = randn(3 * HIDDEN, HIDDEN, std=0.02), randn(HIDDEN, HIDDEN, std=0.02)
    w_up, w_dn = randn(MLP, HIDDEN, std=0.02), randn(HIDDEN, MLP, std=0.02)
    b = {n: (torch.randn(n, generator=gen, device=dev) * 0.02) for n in (3 * HIDDEN, HIDDEN, MLP)}
    norms = (1.0 + 0.02 * torch.randn(4, HEAD_DIM, generator=gen, device=dev)).contiguous()
    freqs = (10000.0 ** (-torch.arange(PAIRS, device=dev, dtype=torch.float64) / PAIRS)).float()

    qkv_v = torch.empty(lv, 3 * HIDDEN, dtype=bf, device=dev)
    qkv_t = torch.empty(lt, 3 * HIDDEN, dtype=bf, device=dev)
    a_v = torch.empty(lv, HIDDEN, dtype=bf, device=dev)
    a_t = torch.empty(lt, HIDDEN, dtype=bf, device=dev)
    o_v, o_t = torch.empty_like(a_v), torch.empty_like(a_t)
    h_v = torch.empty(lv, MLP, dtype=bf, device=dev)
    h_t = torch.empty(lt, MLP, dtype=bf, device=dev)
    y_v, y_t = torch.empty_like(a_v), torch.empty_like(a_t)

    plans = {s: capi.AwaPlan(capi.awa_config(HEADS, HEAD_DIM, TARGET, s, 1e-5, PAIRS),
                             [VIDEO_SHAPE], [lt]) for s in (0, 1)}
    # the RoPE cos/sin table depends only on the plan and the frequency
    # weights: the plan keeps it, as the layer does (s2_awa_plan_cache_rope)
    for p in plans.values():
        p.cache_rope(freqs)
    ws = torch.empty(max(p.info.workspace_bytes for p in plans.values()), dtype=torch.uint8, device=dev)

    ops = ["qkv", "attention", "out", "mlp_up", "mlp_down"]
    fused_ops = ["qkv_attention", "out", "mlp_up", "mlp_down"]

    def step(shifted, ev=None, fused=True):
        def mark(i):
            if ev is not None:
                ev[i].record()
        mark(0)
        if fused:
            # QKV projection with the attention prologue in its epilogue,
            # then the attention (s2_awa_qkv_forward)
            capi.awa_qkv_forward(plans[shifted], x_v, x_t, w_qkv, b[3 * HIDDEN], norms, freqs,
                                 workspace=ws, out_video=a_v, out_text=a_t)
        else:
            capi.shared_linear(x_v, x_t, w_qkv, b[3 * HIDDEN], capi.ACT_NONE, y_video=qkv_v,
                               y_text=qkv_t)
            mark(1)
            capi.awa_forward(plans[shifted], norms, freqs,
                             qkv_v[:, :HIDDEN], qkv_v[:, HIDDEN:2 * HIDDEN], qkv_v[:, 2 * HIDDEN:],
                             qkv_t[:, :HIDDEN], qkv_t[:, HIDDEN:2 * HIDDEN], qkv_t[:, 2 * HIDDEN:],
                             workspace=ws, out_video=a_v, out_text=a_t)
        o = 1 if fused else 2
        mark(o)
        capi.shared_linear(a_v, a_t, w_o, b[HIDDEN], capi.ACT_NONE, y_video=o_v, y_text=o_t)
        mark(o + 1)
        capi.shared_linear(o_v, o_t, w_up, b[MLP], capi.ACT_GELU, y_video=h_v, y_text=h_t)
        mark(o + 2)
        capi.shared_linear(h_v, h_t, w_dn, b[HIDDEN], capi.ACT_NONE, y_video=y_v, y_text=y_t)
        mark(o + 3)

    def run(shifted, steps, warmup, fused=True):
        names = fused_ops if fused else ops
        for _ in range(warmup):
            step(shifted, fused=fused)
        torch.cuda.synchronize()
        evs = [[torch.cuda.Event(enable_timing=True) for _ in range(len(names) + 1)]
               for _ in range(steps)]
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        start.record()
        for i in range(steps):
            step(shifted, evs[i], fused=fused)
        end.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        total_ms = start.elapsed_time(end)
        per_op = {op: sum(e[j].elapsed_time(e[j + 1]) for e in evs) / steps for j, op in enumerate(names)}
        return total_ms / steps, per_op, wall

    def full_block(steps, warmup):
        """The whole block around the hot path (regular windows) on an fp32
        residual stream: the norm and AdaSingle modulation before the
        attention (s2_dit_ada_in, bf16 out), the fused QKV + attention, the
        out projection with the attention's gate and residual sum in its
        epilogue (s2_shared_linear_residual, in place), the MLP's norm and
        modulation (s2_dit_ada_in), the MLP up projection with GELU and the
        down projection with the MLP's gate and residual sum in its epilogue.
        The same block with the projections writing bf16 blobs and separate
        gate / residual passes (s2_dit_ada_out_in, s2_dit_ada_out), the chain
        the fused form replaces bit for bit, is timed beside it.  Algorithmic
        bytes per value of the modulation passes: 6 (fp32 in, bf16 out), 12
        (fp32 residual and bf16 branch in, fp32 residual and bf16 out) and 10
        (fp32 residual and bf16 branch in, fp32 out)."""
        res0_v = torch.randn(lv, HIDDEN, generator=gen, device=dev)
        res0_t = torch.randn(lt, HIDDEN, generator=gen, device=dev)
        res_v, res_t = res0_v.clone(), res0_t.clone()
        mods = {k: torch.randn(1, HIDDEN, generator=gen, device=dev) * 0.1 + (1.0 if k.endswith("scale") else 0.0)
                for k in ("attn_shift", "attn_scale", "attn_gate", "mlp_shift", "mlp_scale", "mlp_gate")}
        hin_v = torch.empty(lv, HIDDEN, dtype=bf, device=dev)
        hin_t = torch.empty(lt, HIDDEN, dtype=bf, device=dev)
        vr, tr = [lv], [lt]
        fused_names = ["attn_norm_modulate", "qkv_attention", "out_gate_residual",
                       "mlp_norm_modulate", "mlp_up", "mlp_down_gate_residual"]
        split_names = ["attn_norm_modulate", "qkv_attention", "out",
                       "attn_gate_residual_mlp_norm_modulate", "mlp_up", "mlp_down",
                       "mlp_gate_residual"]

        def fstep(ev=None):
            def mark(i):
                if ev is not None:
                    ev[i].record()
            mark(0)
            capi.ada_in(res_v, res_t, vr, tr, mods["attn_shift"], mods["attn_scale"],
                        out_video=hin_v, out_text=hin_t)
            mark(1)
            capi.awa_qkv_forward(plans[0], hin_v, hin_t, w_qkv, b[3 * HIDDEN], norms, freqs,
                                 workspace=ws, out_video=a_v, out_text=a_t)
            mark(2)
            capi.shared_linear_residual(a_v, a_t, w_o, b[HIDDEN], vr, tr, res_v, res_t,
                                        mods["attn_gate"])
            mark(3)
            capi.ada_in(res_v, res_t, vr, tr, mods["mlp_shift"], mods["mlp_scale"],
                        out_video=hin_v, out_text=hin_t)
            mark(4)
            capi.shared_linear(hin_v, hin_t, w_up, b[MLP], capi.ACT_GELU, y_video=h_v, y_text=h_t)
            mark(5)
            capi.shared_linear_residual(h_v, h_t, w_dn, b[HIDDEN], vr, tr, res_v, res_t,
                                        mods["mlp_gate"])
            mark(6)

        def sstep(ev=None):
            def mark(i):
                if ev is not None:
                    ev[i].record()
            mark(0)
            capi.ada_in(res_v, res_t, vr, tr, mods["attn_shift"], mods["attn_scale"],
                        out_video=hin_v, out_text=hin_t)
            mark(1)
            capi.awa_qkv_forward(plans[0], hin_v, hin_t, w_qkv, b[3 * HIDDEN], norms, freqs,
                                 workspace=ws, out_video=a_v, out_text=a_t)
            mark(2)
            capi.shared_linear(a_v, a_t, w_o, b[HIDDEN], capi.ACT_NONE, y_video=o_v, y_text=o_t)
            mark(3)
            capi.ada_out_in(res_v, res_t, o_v, o_t, vr, tr, mods["attn_gate"], mods["mlp_shift"],
                            mods["mlp_scale"], h_video=hin_v, h_text=hin_t)
            mark(4)
            capi.shared_linear(hin_v, hin_t, w_up, b[MLP], capi.ACT_GELU, y_video=h_v, y_text=h_t)
            mark(5)
            capi.shared_linear(h_v, h_t, w_dn, b[HIDDEN], capi.ACT_NONE, y_video=y_v, y_text=y_t)
            mark(6)
            capi.ada_out(res_v, res_t, y_v, y_t, vr, tr, mods["mlp_gate"])
            mark(7)

        def timed(fn, names):
            for _ in range(warmup):
                fn()
            torch.cuda.synchronize()
            evs = [[torch.cuda.Event(enable_timing=True) for _ in range(len(names) + 1)]
                   for _ in range(steps)]
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            for i in range(steps):
                fn(evs[i])
            end.record()
            torch.cuda.synchronize()
            assert bool(torch.isfinite(res_v).all())
            per = {op: sum(e[j].elapsed_time(e[j + 1]) for e in evs) / steps
                   for j, op in enumerate(names)}
            return start.elapsed_time(end) / steps, per

        # one block from the same residual both ways: bit for bit
        fstep()
        fused_out = res_v.clone()
        res_v.copy_(res0_v)
        res_t.copy_(res0_t)
        sstep()
        torch.cuda.synchronize()
        same = bool(torch.equal(fused_out, res_v))
        ms_f, per_f = timed(fstep, fused_names)
        ms_s, per_s = timed(sstep, split_names)
        m_rows = lv + lt

        def hbm(per, op, bytes_per_value):
            nbytes = bytes_per_value * m_rows * HIDDEN
            return {"ms": round(per[op], 4), "algorithmic_bytes": int(nbytes),
                    "gbs": round(nbytes / (per[op] * 1e-3) / 1e9, 1),
                    "frac_hbm_peak": round(nbytes / (per[op] * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}
        m = lv + lt
        fused = {
            "ms": round(ms_f, 4),
            "ops_ms": {op: round(v, 4) for op, v in per_f.items()},
            "out_gate_residual": op_record(per_f["out_gate_residual"], 2 * m * HIDDEN * HIDDEN),
            "mlp_down_gate_residual": op_record(per_f["mlp_down_gate_residual"], 2 * m * MLP * HIDDEN),
            "norm_modulate": hbm(per_f, "attn_norm_modulate", 6.0),
        }
        separate = {
            "ms": round(ms_s, 4),
            "ops_ms": {op: round(v, 4) for op, v in per_s.items()},
            "norm_modulate": hbm(per_s, "attn_norm_modulate", 6.0),
            "gate_residual_norm_modulate": hbm(per_s, "attn_gate_residual_mlp_norm_modulate", 12.0),
            "gate_residual": hbm(per_s, "mlp_gate_residual", 10.0),
        }
        best = "residual_in_gemm_epilogue" if ms_f <= ms_s else "separate_residual_passes"
        return {
            "ms": round(min(ms_f, ms_s), 4),
            "chain": best,
            "residual_in_gemm_epilogue": fused,
            "separate_residual_passes": separate,
            "fused_equals_separate_bit_for_bit": same,
            "note": "fp32 residual stream; per-sample modulation vectors; regular windows",
        }

    m = lv + lt
    gemm = {"qkv": 2 * m * HIDDEN * 3 * HIDDEN, "out": 2 * m * HIDDEN * HIDDEN,
            "mlp_up": 2 * m * HIDDEN * MLP, "mlp_down": 2 * m * MLP * HIDDEN}
    results, separate = {}, {}
    for shifted in (0, 1):
        attn = attention_flops(shifted)
        ms, per_op, wall = run(shifted, args.steps, args.warmup)
        flops = dict(gemm, attention=attn)
        results[shifted] = (ms, per_op, flops, wall)
        ms_u, per_op_u, _ = run(shifted, args.steps, args.warmup, fused=False)
        separate[shifted] = (ms_u, per_op_u, flops)

    # per-kernel times of the attention forward from events the library
    # records around its four stages (separate runs: the timed loops above
    # record none)
    def stage_times(shifted, fused):
        capi.awa_stage_timing(True)
        acc = {}
        reps = max(3, args.steps // 2)
        for _ in range(reps):
            step(shifted, fused=fused)
            for key, v in capi.awa_stage_times().items():
                acc[key] = acc.get(key, 0.0) + v / reps
        capi.awa_stage_timing(False)
        return acc

    stages = {}
    for shifted in (0, 1):
        mode = "shifted" if shifted else "regular"
        af = attention_flops(shifted)
        acc = stage_times(shifted, False)
        pb = prologue_bytes(shifted)
        stages[mode] = {
            "rope_table_ms": round(acc["rope_table"], 4),
            "prologue_ms": round(acc["prologue"], 4),
            "prologue_algorithmic_bytes": pb,
            "prologue_gbs": round(pb / (acc["prologue"] * 1e-3) / 1e9, 1),
            "prologue_frac_hbm_peak": round(pb / (acc["prologue"] * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
            "attention_kernel_ms": round(acc["attention"], 4),
            "attention_kernel_tflops": round(af / (acc["attention"] * 1e-3) / 1e12, 1),
            "attention_kernel_frac_bf16_peak": round(af / (acc["attention"] * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
            "text_pool_ms": round(acc["text_pool"], 4),
        }
        accf = stage_times(shifted, True)
        qf = gemm["qkv"]
        stages[mode + "_fused"] = {
            "rope_table_ms": round(accf["rope_table"], 4),
            "qkv_projection_ms": round(accf["prologue"], 4),
            "qkv_prologue_tflops": round(qf / (accf["prologue"] * 1e-3) / 1e12, 1),
            "attention_kernel_ms": round(accf["attention"], 4),
            "text_pool_ms": round(accf["text_pool"], 4),
        }

    ms, per_op, flops, wall = results[0]
    block_flops = sum(flops.values())
    value = block_flops / (ms * 1e-3) / 1e12

    def op_record(t_ms, gf):
        return {"ms": round(t_ms, 4), "gflop": round(gf / 1e9, 3),
                "tflops": round(gf / (t_ms * 1e-3) / 1e12, 1),
                "frac_bf16_peak": round(gf / (t_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)}
    kernels = {"qkv_attention": op_record(per_op["qkv_attention"], flops["qkv"] + flops["attention"])}
    kernels.update({op: op_record(per_op[op], flops[op]) for op in ("out", "mlp_up", "mlp_down")})
    ms_u, per_op_u, flops_u = separate[0]
    separate_rec = {"ms_per_block": round(ms_u, 4),
                    "ms_per_block_shifted": round(separate[1][0], 4),
                    "kernels": {op: op_record(per_op_u[op], flops_u[op]) for op in ops},
                    "note": "the QKV GEMM writing a bf16 QKV blob, then s2_awa_forward (window "
                            "gather prologue, attention, text pool); the headline runs "
                            "s2_awa_qkv_forward, whose outputs are bit-identical"}
    up_ms = per_op["mlp_up"]
    up_tf = flops["mlp_up"] / (up_ms * 1e-3) / 1e12
    ms_s, per_op_s, flops_s, _ = results[1]
    line = {
        "metric": "window-attn+SharedLinear TFLOP/s & % bf16 MFMA peak; ms/DiT block @720p video",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) activations, N(0,0.02) weights, random init)",
        "config": {
            "workload": "SeedVR2-3B DiT block hot path at 720p video: 21 frames 1280x720 -> "
                        "6x45x80 = 21600 video + 64 text tokens, hidden 2560, 20x128 heads, "
                        "regular 3-D windows (target 4,3,3); QKV 2560->7680 with the window "
                        "gather, RMSNorm and RoPE in its epilogue, window attention, "
                        "out 2560->2560, MLP 2560->10240 GELU ->2560",
            "video_tokens": lv, "text_tokens": lt, "hidden": HIDDEN, "heads": HEADS,
            "head_dim": HEAD_DIM, "block_tflop": round(block_flops / 1e12, 4),
        },
        "pct_bf16_peak": round(100 * value / PEAK_BF16_TFLOPS, 2),
        "ms_per_block": round(ms, 4),
        "ms_per_block_shifted": round(ms_s, 4),
        "tflops_shifted": round(sum(flops_s.values()) / (ms_s * 1e-3) / 1e12, 2),
        "qkv_attention_shifted": op_record(per_op_s["qkv_attention"],
                                           flops_s["qkv"] + flops_s["attention"]),
        "kernels": kernels,
        "separate_qkv_and_attention": separate_rec,
        "attention_stages": dict(stages, rope_table_note=(
            "the plans keep the RoPE cos/sin table (s2_awa_plan_cache_rope, as the layer does), "
            "so rope_table_ms is the empty stage between two events")),
        "roofline": {
            "kernel": "s2::shared_linear_256_kernel<1, 1, 0> (MLP up 2560->10240 + GELU, bf16 out, M=21664)",
            "bound": "mfma",
            "achieved": round(up_tf, 1),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(up_tf / PEAK_BF16_TFLOPS, 4),
            "traffic": measured_traffic(),
            "traffic_source": "profiles/shared_linear_mlp_up_720p_video_traffic.md (two rocprofv3 "
                              "--pmc passes, FETCH_SIZE and WRITE_SIZE, copy-calibrated); read "
                              "from that file, not measured in this run",
        },
        "wall_s_timed_region": round(wall, 3),
    }
    line["full_block"] = full_block(args.steps, args.warmup)
    if not args.no_parity:
        line["parity_gemm_cfg4"] = gemm_parity(
            x_v, x_t, {"qkv": (w_qkv, b[3 * HIDDEN], capi.ACT_NONE), "out": (w_o, b[HIDDEN], capi.ACT_NONE),
                       "mlp_up": (w_up, b[MLP], capi.ACT_GELU), "mlp_down": (w_dn, b[HIDDEN], capi.ACT_NONE)})
    for p in plans.values():
        p.close()
    del x_v, x_t, w_qkv, w_o, w_up, w_dn, qkv_v, qkv_t, a_v, a_t, o_v, o_t, h_v, h_t, y_v, y_t, ws
    torch.cuda.empty_cache()
    if not args.no_parity:
        line["attention_configs"] = awa_configs(args.cpu_threads or job_cpu_threads())
    if not args.no_stack:
        line["stack_7b"] = stack_7b(args.stack_steps, 1)
    if not args.no_v3:
        line["v3_block"] = v3_block(max(5, args.steps // 2), 2)
    if not args.no_tail:
        line["sampler_tail"] = sampler_tail()
    if not args.no_vae:
        threads = args.cpu_threads or job_cpu_threads()
        line["vae_conv3d"] = vae_conv3d(cpu_threads=threads, cpu=not args.no_cpu_baseline)
        line["vae_mha"] = vae_mha(cpu_threads=threads, cpu=not args.no_cpu_baseline)
    if not args.no_cpu_baseline:
        threads = args.cpu_threads or job_cpu_threads()
        line["cpu_baseline"] = cpu_baseline(threads)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
