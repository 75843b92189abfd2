"""Benchmark: seconds per denoise step of the Qwen-Image-shaped dual-stream MMDiT at 1024x1024 on one MI355X.

Workload (a step): 60 dual-stream blocks, hidden 3072, 24 heads x 128, FFN 12288 (GELU-tanh), shift/scale/gate
adaLN; 4096 image tokens (a 64 x 64 grid of 2x2-patched 16-channel latents) + 256 text tokens of width 3584 projected
to 3072; classifier-free guidance as a batch of 2 (positive and negative prompt), then the guidance combine and the
Euler update. bf16 weights (random-init N(0, 0.02), 40.8 GB) and activations, fp32 accumulation and residual stream.
Synthetic inputs: prompts and latents N(0, 1), resident on the device when the timed region starts.

Prints one JSON line. `roofline` is the dominant kernel (the launch shape with the most time a step: the grouped
FFN-down GEMM): its algorithmic FLOPs per launch divided by its average launch duration, from HIP events recorded
around each launch on the engine's stream in a separate timed pass of the same steps; `gemm_class` is the same over
every GEMM launch, `attention_gemm_mfma_frac` over every GEMM and attention launch (their FLOPs over the union of
their launch intervals). `cpu_baseline` is the oracle (CPU restatement of the same step) on a bounded sample of one
block, timed on this host's cores and scaled by FLOPs to a whole step.
"""
import argparse
import json
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path[:0] = [str(ROOT / "mako-image_amd"), str(ROOT / "oracle")]

METRIC = "s/denoise-step Qwen-Image MMDiT 1024² bf16; attention+GEMM % of MFMA peak"
PEAK_BF16 = 2.5e15  # MI355X dense bf16 MFMA, published
CFG = dict(blocks=60, dim=3072, heads=24, head_dim=128, ffn=12288, text_dim=3584)
# (latent grid side, text tokens, weight dtype) of each workload; the default is the metric's (1024x1024, bf16)
WORKLOADS = {
    "mmdit-1024-bf16": dict(side=64, text=256, fp8=False, metric=METRIC,
                            name="Qwen-Image-shaped dual-stream MMDiT denoise step at 1024x1024, CFG batch 2"),
    "mmdit-2048-fp8": dict(side=128, text=512, fp8=True,
                           metric="s/denoise-step Qwen-Image MMDiT 2048² fp8-e4m3 weights; attention+GEMM % of MFMA peak",
                           name="Qwen-Image-shaped dual-stream MMDiT denoise step at 2048x2048, CFG batch 2, "
                                "fp8-e4m3 linear weights with per-channel scales"),
}
H = W = 64
S = 256
# SDXL-UNet-shaped spatial transformers at 1024x1024 (128x128x4 latent): (stage, token grid side, channels, depth)
SDXL_STAGES = (("A", 64, 640, 2), ("B", 32, 1280, 10))
SDXL_CTX, SDXL_CTX_DIM = 77, 2048
SDXL_METRIC = "s/SDXL spatial-transformer pass 1024² bf16 (stage A depth 2 + stage B depth 10, CFG batch 2)"


# Qwen-Image's VAE decoder (Wan-2.1 layout, base 96, 16 latent channels) on the step's 64 x 64 tokens: a 1024x1024 image
VAE_BASE, VAE_Z, VAE_SIDE = 96, 16, 64
VAE_METRIC = "s/VAE decode 1024² f16 (Qwen-Image decoder, base 96, one frame); conv+attention % of MFMA peak"


def vae_flops(th, tw, b=VAE_BASE, z=VAE_Z):
    """Algorithmic FLOPs of one decode (engine.cpp:862-954; channel padding excluded): 2 k^2 ci co per pixel of each
    conv, 4 n^2 c for the mid block's attention over its n pixels, 2 n c (3c + c) for its 1x1 projections."""
    H, W = 2 * th, 2 * tw
    conv = lambda px, ci, co, k=3: 2 * px * k * k * ci * co
    n, d0 = H * W, 4 * b
    f = conv(n, z, z, 1) + conv(n, z, d0)
    res = lambda px, ci, co: conv(px, ci, co) + conv(px, co, co) + (conv(px, ci, co, 1) if ci != co else 0)
    f += 2 * res(n, d0, d0)
    attn = 4 * n * n * d0
    f += attn + 2 * n * d0 * 4 * d0
    ins, outs = (4 * b, 2 * b, 2 * b, b), (4 * b, 4 * b, 2 * b, b)
    px = n
    for i in range(4):
        f += res(px, ins[i], outs[i]) + 2 * res(px, outs[i], outs[i])
        if i < 3:
            px *= 4
            f += conv(px, outs[i], outs[i] // 2)
    f += conv(px, b, 3)
    return f, attn


def bench_vae(args):
    """The VAE workload: one decode of 64 x 64 tokens to a 1024x1024 image (random-init weights, N(0,1) tokens resident
    on the device), timed with HIP events on the decoder's stream."""
    import numpy as np

    import mkimage as M

    M.call("mk_set_device", 0)
    rng = np.random.default_rng(0)
    vae = M.Vae(VAE_BASE, VAE_Z, mean=rng.standard_normal(VAE_Z) * 0.5, std=1.0 + rng.random(VAE_Z))
    vae.init_random(0)
    th = tw = VAE_SIDE
    tok = M.Dev.from_array(rng.standard_normal((th * tw, 4 * VAE_Z)).astype(np.float32))
    out = M.Dev(16 * th * 16 * tw * 4 * 4)
    stream = vae.stream()
    for _ in range(args.warmup):
        vae.decode_device(tok, th, tw, out)
    M.call("mk_stream_synchronize", stream)
    e0, e1 = M.Event(), M.Event()
    e0.record(stream)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        vae.decode_device(tok, th, tw, out)
    e1.record(stream)
    M.call("mk_stream_synchronize", stream)
    wall = (time.perf_counter() - t0) / args.steps
    sec = e0.elapsed_ms(e1) / 1e3 / args.steps
    img = out.to_array(np.float32, (16 * th, 16 * tw, 4))
    if not np.isfinite(img).all():
        raise RuntimeError("non-finite VAE output")
    fl, fa = vae_flops(th, tw)
    line = {
        "metric": VAE_METRIC, "value": round(sec, 5), "unit": "s/decode", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(sec * 1e3, 3), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "f16",
        "data": "synthetic (random-init weights N(0, 1/fan_in), N(0,1) tokens)",
        "config": {"workload": "Qwen-Image VAE decoder (Wan 2.1 layout), 64x64 tokens -> 1024x1024 RGBA",
                   "base": VAE_BASE, "z": VAE_Z, "tokens": [th, tw], "gflop": round(fl / 1e9, 1),
                   "attention_gflop": round(fa / 1e9, 1),
                   "attention_note": "fp32 keys and values as half hi + lo pairs: the attention's matrix-core work "
                                     "is twice its algorithmic FLOPs"},
        "roofline": {"bound": "mfma", "kernel": "whole decode (implicit-GEMM convs + attention GEMMs)",
                     "achieved": round(fl / sec / 1e12, 1), "peak": PEAK_BF16 / 1e12, "unit": "TFLOP/s",
                     "frac": round(fl / sec / PEAK_BF16, 4), "traffic": None},
        "wall_ms_per_decode": round(wall * 1e3, 3),
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline_vae(args.cpu_seconds, fl)
    print(json.dumps(line), flush=True)


def cpu_baseline_vae(seconds_target, decode_flops):
    """The oracle's decoder (base 96) on 4 x 4 tokens (a 64x64 image) timed on this host, scaled by FLOPs."""
    import numpy as np

    import mkref as R

    v = R.Vae(VAE_BASE, VAE_Z, seed=0)
    tok = np.random.default_rng(0).standard_normal((16, 4 * VAE_Z)).astype(np.float32)
    flops = vae_flops(4, 4)[0]
    reps, t_total = 0, 0.0
    while t_total < seconds_target and reps < 50:
        t0 = time.perf_counter()
        v.decode(tok, 4, 4)
        t_total += time.perf_counter() - t0
        reps += 1
    rate = flops * reps / t_total
    return {"value": decode_flops / rate, "unit": "s/decode", "cores": R.lib().mkref_threads(), "kind": "port",
            "sample": f"oracle (C++/OpenMP, double sums over bf16 weights): {reps} x a 4x4-token decode (64x64 image, "
                      f"{flops / 1e9:.1f} GFLOP each, {t_total:.1f} s, {rate / 1e9:.1f} GFLOP/s), scaled by FLOPs to "
                      f"the 1024x1024 decode"}


def step_flops(blocks=60, D=3072, F=12288, N=4096, S=256, B=2, heads=24):
    """Algorithmic FLOPs of one step (the blocks' GEMMs and attention; padding excluded)."""
    T = N + S
    lin = 2 * (N + S) * D * (3 * D + D + 2 * F)
    attn = 4 * T * T * 128 * heads
    return B * blocks * (lin + attn), B * blocks * lin, B * blocks * attn


def sdxl_flops(n, C, depth, B=2, S=SDXL_CTX):
    """Algorithmic FLOPs of one SDXL spatial-transformer forward (sdxl.cpp:742-796): per block the self-attention's
    QKV and output projections (4 C^2 n), the cross-attention's Q and output projections (2 C^2 n; the context's
    K / V are projected once at begin), GEGLU C -> 8C -> C over 4C (12 C^2 n), self- and cross-attention
    (4 n^2 C + 4 n S C); proj_in and proj_out once (2 C^2 n)."""
    block = 2 * 18 * C * C * n + 4 * n * n * C + 4 * n * S * C
    return B * (depth * block + 2 * 2 * C * C * n), B * depth * (4 * n * n * C + 4 * n * S * C)


def bench_sdxl(args):
    """The SDXL workload: stage A and stage B transformers (random-init bf16 weights, N(0,1) input and context),
    each forward timed whole (mk_sdxl_forward returns after its stream has finished)."""
    import numpy as np

    import mkimage as M

    M.call("mk_set_device", 0)
    rng = np.random.default_rng(0)
    stages, per, tot_s, tot_f, tot_attn, tot_h = {}, {}, 0.0, 0.0, 0.0, 0.0
    for name, side, C, depth in SDXL_STAGES:
        n = side * side
        eng = M.Engine(M.FAMILY_SDXL, blocks=depth, dim=C, heads=C // 64, head_dim=64, ffn=4 * C,
                       text_dim=SDXL_CTX_DIM)
        eng.init_random(0)
        for s in (0, 1):
            eng.begin(rng.standard_normal((SDXL_CTX, SDXL_CTX_DIM)).astype(np.float32), side, side, s)
        x = M.Dev.from_array(rng.standard_normal((2, n, C)).astype(np.float32))
        y = M.Dev(2 * n * C * 4)
        for _ in range(args.warmup):
            eng.sdxl_forward(x, 2, n, y)
        t0 = time.perf_counter()
        for _ in range(args.steps):
            eng.sdxl_forward(x, 2, n, y)
        sec = (time.perf_counter() - t0) / args.steps
        if not np.isfinite(y.to_array(np.float32, (2, n, C))).all():
            raise RuntimeError("non-finite SDXL output")
        eng.set_timing(True)
        for _ in range(args.steps):
            eng.sdxl_forward(x, 2, n, y)
            for k, v in eng.timing().items():
                acc = per.setdefault(k, {"ms": 0.0, "launches": 0, "flops": 0.0})
                acc["ms"] += v["ms"]
                acc["launches"] += v["launches"]
                acc["flops"] += v["flops"]
        eng.set_timing(False)
        eng.close()
        fl, fa = sdxl_flops(n, C, depth)
        # the same stage with half matrices (an F16 checkpoint, as SDXL's are: Engine::matrix keeps them F16)
        eh = M.Engine(M.FAMILY_SDXL, blocks=depth, dim=C, heads=C // 64, head_dim=64, ffn=4 * C,
                      text_dim=SDXL_CTX_DIM, weight_dtype=M.F16)
        eh.init_random(0)
        for s in (0, 1):
            eh.begin(rng.standard_normal((SDXL_CTX, SDXL_CTX_DIM)).astype(np.float32), side, side, s)
        for _ in range(args.warmup):
            eh.sdxl_forward(x, 2, n, y)
        t0 = time.perf_counter()
        for _ in range(args.steps):
            eh.sdxl_forward(x, 2, n, y)
        sec_h = (time.perf_counter() - t0) / args.steps
        if not np.isfinite(y.to_array(np.float32, (2, n, C))).all():
            raise RuntimeError("non-finite SDXL output (half matrices)")
        eh.close()
        stages[name] = {"tokens": n, "channels": C, "heads": C // 64, "depth": depth, "ms": round(sec * 1e3, 3),
                        "tflop": round(fl / 1e12, 3), "tflops": round(fl / sec / 1e12, 1),
                        "ms_f16_matrices": round(sec_h * 1e3, 3)}
        tot_s, tot_f, tot_attn, tot_h = tot_s + sec, tot_f + fl, tot_attn + fa, tot_h + sec_h
    kernels = {k: {"ms_per_pass": round(v["ms"] / args.steps, 3), "launches_per_pass": v["launches"] // args.steps,
                   **({"tflops": round(v["flops"] / (v["ms"] / 1e3) / 1e12, 1)} if v["flops"] else {})}
               for k, v in sorted(per.items(), key=lambda kv: -kv[1]["ms"])}
    g = {"ms": sum(v["ms"] for k, v in per.items() if k.startswith("gemm")),
         "flops": sum(v["flops"] for k, v in per.items() if k.startswith("gemm"))}
    gemm_tf = g["flops"] / (g["ms"] / 1e3) / 1e12 if g["flops"] else None
    line = {
        "metric": SDXL_METRIC, "value": round(tot_s, 5), "unit": "s/pass", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(tot_s * 1e3, 3), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (random-init N(0,0.02) weights, N(0,1) inputs and 77-token contexts)",
        "config": {"workload": "SDXL-UNet-shaped spatial transformers at 1024x1024, CFG batch 2",
                   "stages": stages, "context": [SDXL_CTX, SDXL_CTX_DIM]},
        "roofline": {"bound": "mfma", "kernel": "gemm (bf16 MFMA)", "achieved": round(gemm_tf, 1) if gemm_tf else None,
                     "peak": PEAK_BF16 / 1e12, "unit": "TFLOP/s",
                     "frac": round(gemm_tf * 1e12 / PEAK_BF16, 4) if gemm_tf else None, "traffic": None},
        "pass_tflops": round(tot_f / tot_s / 1e12, 1),
        "pass_mfma_frac": round(tot_f / tot_s / PEAK_BF16, 4),
        "f16_matrices": {"ms_per_pass": round(tot_h * 1e3, 3), "pass_mfma_frac": round(tot_f / tot_h / PEAK_BF16, 4),
                         "note": "weight_dtype F16: proj_in/out, to_out, attn2.to_q and ff as half (half inputs), "
                                 "q|k|v and the context k|v bf16"},
        "kernels": kernels,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline_sdxl(args.cpu_seconds, tot_f)
    print(json.dumps(line), flush=True)


def cpu_baseline_sdxl(seconds_target, pass_flops):
    """The oracle's SDXL transformer timed on this host on one block of each stage at its own shape (stage A: 4096
    tokens x 640 channels; stage B: 1024 x 1280), one sample each; the pass's time at their combined FLOP rate."""
    import numpy as np

    import mkref as R

    rng = np.random.default_rng(0)
    ctx = rng.standard_normal((SDXL_CTX, SDXL_CTX_DIM)).astype(np.float32)
    cases = []
    for _name, side, C, _depth in SDXL_STAGES:
        m = R.Model(R.SDXL, blocks=1, dim=C, heads=C // 64, head_dim=64, ffn=4 * C, text_dim=SDXL_CTX_DIM, seed=0)
        x = rng.standard_normal((side * side, C)).astype(np.float32)
        fl = sdxl_flops(side * side, C, 1, B=1)[0] + 2 * 2 * C * SDXL_CTX_DIM * SDXL_CTX  # + the context K / V
        cases.append((m, x, fl, side, C))
    reps, t_total, done = 0, 0.0, 0.0
    while t_total < seconds_target and reps < 50:
        for m, x, fl, _side, _C in cases:
            t0 = time.perf_counter()
            m.sdxl_trans(x, ctx)
            t_total += time.perf_counter() - t0
            done += fl
        reps += 1
    rate = done / t_total
    shapes = " and ".join(f"{side * side} tokens x {C}" for _m, _x, _fl, side, C in cases)
    return {"value": pass_flops / rate, "unit": "s/pass", "cores": R.lib().mkref_threads(), "kind": "port",
            "sample": f"oracle (C++/OpenMP, fp32 over bf16 weights): {reps} x one block of each stage ({shapes}), one "
                      f"sample ({done / reps / 1e9:.1f} GFLOP a round, {t_total:.1f} s, {rate / 1e9:.1f} GFLOP/s), "
                      f"scaled by FLOPs to the whole batch-2 pass"}


# Qwen-Image 2.1 as the reference runs it (qwen_image.hpp:38; its published numbers, docs/performance.md:5): 32
# blocks of width 4096, 32 heads x 128, SwiGLU 12288, one weight set for text and image rows, 4096 image tokens at
# 1024x1024 and a prompt of 256 rows of width 4096; guidance as two passes (each slot keeps its text K / V).
Q21_CFG = dict(blocks=32, dim=4096, heads=32, head_dim=128, ffn=12288, text_dim=4096)
Q21_METRIC = ("s/denoise-step Qwen-Image 2.1 graph (reference's own model) 1024² bf16, CFG as two passes; "
              "attention+GEMM % of MFMA peak")


def q21_flops(first, N=4096, S=256, blocks=32, D=4096, F=12288, H=32):
    """Algorithmic FLOPs of one guided 2.1 step (two passes): per block the q|k|v, o, gate|up and down projections
    (2 T D (4 D + 3 F)) over T rows (text + image on the first step, image only after) and the attention over
    N (S + N) image query-key pairs plus S (S + 1) / 2 causal text pairs on the first step (4 d per pair a head)."""
    T = N + S if first else N
    lin = 2 * T * D * (4 * D + 3 * F)
    attn = 4 * (N * (N + S) + (S * (S + 1) // 2 if first else 0)) * 128 * H
    return 2 * blocks * (lin + attn), 2 * blocks * lin, 2 * blocks * attn


def bench_q21(args):
    """The 2.1 graph: step 1 (text and image rows, the text K / V kept per slot) and the later steps (image rows
    against the cached K / V), guidance as two passes, each timed with HIP events on the engine's stream."""
    import numpy as np

    import mkimage as M

    M.call("mk_set_device", 0)
    side, S = 64, 256
    N = side * side
    eng = M.Engine(M.FAMILY_Q21, **Q21_CFG)
    eng.init_random(0)
    rng = np.random.default_rng(0)
    prompts = [rng.standard_normal((S, Q21_CFG["text_dim"])).astype(np.float32) for _ in range(2)]
    lat = [M.Dev.from_array(rng.standard_normal((N, 64)).astype(np.float32)), M.Dev(N * 64 * 4)]
    stream = eng.stream()

    def begin():
        for s in (0, 1):
            eng.begin(prompts[s], side, side, s)

    def run(i):
        eng.step_cfg_device(lat[i % 2], 1.0 - 0.02 * i, 0.98 - 0.02 * i, 4.0, lat[(i + 1) % 2], stream)

    def timed(n, first):
        e0, e1 = M.Event(), M.Event()
        tot = 0.0
        for i in range(n):
            if first:
                begin()
            M.call("mk_stream_synchronize", stream)
            e0.record(stream)
            run(i)
            e1.record(stream)
            M.call("mk_stream_synchronize", stream)
            tot += e0.elapsed_ms(e1)
        return tot / n / 1e3

    begin()
    for i in range(args.warmup):
        run(i)
    first_s = timed(max(2, args.steps // 4), True)
    begin()
    run(0)  # step 1 of this generation
    M.call("mk_stream_synchronize", stream)
    e0, e1 = M.Event(), M.Event()
    e0.record(stream)
    for i in range(args.steps):
        run(1 + i)
    e1.record(stream)
    M.call("mk_stream_synchronize", stream)
    later_s = e0.elapsed_ms(e1) / 1e3 / args.steps
    if not np.isfinite(lat[(1 + args.steps) % 2].to_array(np.float32, (N, 64))).all():
        raise RuntimeError("non-finite latents")
    # per-kernel pass over later steps
    eng.set_timing(True)
    per = {}
    for i in range(args.steps):
        run(1 + args.steps + i)
        for k, v in eng.timing().items():
            acc = per.setdefault(k, {"ms": 0.0, "launches": 0, "flops": 0.0})
            for f in ("ms", "launches", "flops"):
                acc[f] += v[f]
    eng.set_timing(False)
    tot, lin, attn = q21_flops(False, N, S)
    tot1 = q21_flops(True, N, S)[0]
    g = {f: sum(v[f] for k, v in per.items() if k.startswith("gemm")) for f in ("ms", "flops")}
    a = per["attention"]
    u = per.get("union:attention+gemm")
    both = (g["flops"] + a["flops"]) / ((u["ms"] if u else g["ms"] + a["ms"]) / 1e3)
    dom = max((k for k, v in per.items() if v["flops"] and (k.startswith("gemm.") or k == "attention")),
              key=lambda k: per[k]["ms"])
    dv = per[dom]
    dl = dv["ms"] / 1e3 / dv["launches"]
    kernels = {k: {"ms_per_step": round(v["ms"] / args.steps, 3), "launches_per_step": v["launches"] // args.steps,
                   **({"tflops": round(v["flops"] / (v["ms"] / 1e3) / 1e12, 1)} if v["flops"] else {})}
               for k, v in sorted(per.items(), key=lambda kv: -kv[1]["ms"])}
    line = {
        "metric": Q21_METRIC, "value": round(later_s, 5), "unit": "s/step", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(later_s * 1e3, 3), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "weight_dtype": "bf16",
        "data": "synthetic (random-init N(0,0.02) weights, N(0,1) latents and prompts)",
        "config": {"workload": "Qwen-Image 2.1 graph (one weight set, SwiGLU, causal text prefix, text K/V cached "
                               "after step 1), 1024x1024, CFG as two passes", **Q21_CFG, "image_tokens": N,
                   "text_tokens": S, "heads_dtype": "f16"},
        "step1_s": round(first_s, 5), "step1_tflop": round(tot1 / 1e12, 2), "step_tflop": round(tot / 1e12, 2),
        "step_mfma_frac": round(tot / later_s / PEAK_BF16, 4),
        "attention_gemm_mfma_frac": round(both / PEAK_BF16, 4),
        "roofline": {"bound": "mfma", "kernel": f"{dom}: {KERNEL_OF_Q21.get(dom, dom)}",
                     "achieved": round(dv["flops"] / dv["launches"] / dl / 1e12, 1), "peak": PEAK_BF16 / 1e12,
                     "unit": "TFLOP/s", "frac": round(dv["flops"] / dv["launches"] / dl / PEAK_BF16, 4),
                     "flops_per_launch": dv["flops"] / dv["launches"], "launch_us": round(dl * 1e6, 1),
                     "traffic": None},
        "kernels": kernels,
        "reference_published": "1.28 s/step at step 2 on an Apple M5 GPU (docs/performance.md:5), other hardware",
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline_q21(args.cpu_seconds, tot)
    print(json.dumps(line), flush=True)


def cpu_baseline_q21(seconds_target, step_flops_):
    """The oracle's 2.1 graph (one block, one pass, at the step's own 64 x 64 image tokens and 256-row prompt: a first
    step, text rows included) timed on this host, scaled by FLOPs to the 32-block guided step with cached text."""
    import numpy as np

    import mkref as R

    m = R.Model(R.Q21, **{**Q21_CFG, "blocks": 1}, seed=0)
    rng = np.random.default_rng(0)
    side, S = 64, 256
    prompt = rng.standard_normal((S, Q21_CFG["text_dim"])).astype(np.float32)
    lat = rng.standard_normal((side * side, 64)).astype(np.float32)
    flops = q21_flops(True, side * side, S, blocks=1)[0] / 2
    reps, t_total = 0, 0.0
    while t_total < seconds_target and reps < 50:
        t0 = time.perf_counter()
        m.q21_step(prompt, lat, side, side, 0.7)
        t_total += time.perf_counter() - t0
        reps += 1
    rate = flops * reps / t_total
    return {"value": step_flops_ / rate, "unit": "s/step", "cores": R.lib().mkref_threads(), "kind": "port",
            "sample": f"oracle (C++/OpenMP, fp32 over bf16 weights): {reps} x one 2.1 block, one pass, {side * side} "
                      f"image + {S} text tokens ({flops / 1e9:.0f} GFLOP each, {t_total:.1f} s, {rate / 1e9:.1f} "
                      f"GFLOP/s), scaled by FLOPs to the 32-block two-pass step at 4096 image tokens (cached text)"}


KERNEL_OF_Q21 = {"gemm.ff1": "gemm_kernel<256, 256, false, 4, 8> (SwiGLU epilogue)",
                 "gemm.ff2": "gemm_sk_kernel<256, 256, false, 2, 8>", "gemm.qkv": "gemm_kernel<256, 256, false, 3, 8>",
                 "gemm.o": "gemm_kernel<256, 256, false, 2, 8>", "attention": "attn2_kernel<128, true, true, false, 4> (half)"}


# The kernel each timing class of the step launches (rocprofv3's name for it), for the traffic figure.
KERNEL_OF = {"gemm.ff2": "gemm_sk_kernel<256, 256, false, 2, 8>",
             "gemm.ff1.img": "gemm_kernel<256, 256, false, 1, 8>", "gemm.ff1.txt": "gemm_kernel<256, 128, false, 129, 4>",
             "gemm.qkv": "gemm_kernel<256, 256, false, 3, 8>", "gemm.o": "gemm_kernel<256, 256, false, 2, 8>",
             "attention": "attn2_kernel<128, true, false, false, 4>"}


def kernel_traffic(kernel):
    """Bytes a launch of `kernel` moves between L2 and the fabric (FETCH_SIZE + WRITE_SIZE, calibrated against a copy
    of known size), from the committed rocprofv3 counter summary of the step; None when absent. The counters see L2
    misses: Infinity Cache (MALL) hits are included, so this bounds the DRAM bytes from above."""
    f = ROOT / "profiles" / "mmdit_step_1024_traffic.md"
    if not f.exists() or not kernel:
        return None
    for line in f.read_text().splitlines():
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) >= 4 and kernel in cells[0]:
            try:
                return int((float(cells[2]) + float(cells[3])) * 2 ** 20)
            except ValueError:
                return None
    return None


def step_bytes_ff2(N=4096, S=256, B=2, D=3072, F=12288):
    """Algorithmic HBM bytes of one grouped FFN-down launch (image + text rows): the bf16 activations and both
    streams' bf16 weights read once, the fp32 residual read and written once."""
    M = B * (N + S)
    return M * F * 2 + 2 * D * F * 2 + 2 * M * D * 4


def cpu_baseline(seconds_target=12.0, fp8=False):
    """The oracle on one dual-stream block of one sample, timed on this host. At 1024x1024 the block runs at the
    step's own sequence (64 x 64 image tokens + the text tokens), so the step is exactly 60 blocks x 2 samples of it;
    larger workloads sample a 64 x 64 block and scale by FLOPs (their attention share differs)."""
    import numpy as np

    import mkref as R

    m = R.Model(R.DUAL, **{**CFG, "blocks": 1}, fp8=fp8, seed=0)
    rng = np.random.default_rng(0)
    n_side = min(H, 64)
    N = n_side * n_side
    img = rng.standard_normal((N, 3072)).astype(np.float32)
    txt = rng.standard_normal((S, 3072)).astype(np.float32)
    mods = (rng.standard_normal((2, 6, 3072)) * 0.02).astype(np.float32)
    cs = R.rope_table(S, n_side, n_side)
    flops = step_flops(blocks=1, N=N, S=S, B=1)[0]
    reps, t_total = 0, 0.0
    while t_total < seconds_target and reps < 50:
        a, b = img.copy(), txt.copy()
        t0 = time.perf_counter()
        m.dual_block(0, a, b, mods[0], mods[1], cs)
        t_total += time.perf_counter() - t0
        reps += 1
    rate = flops * reps / t_total
    return {"value": step_flops(N=H * W, S=S)[0] / rate, "unit": "s/step", "cores": R.lib().mkref_threads(),
            "kind": "port",
            "sample": f"oracle (C++/OpenMP, fp32 over {'fp8' if fp8 else 'bf16'} weights): {reps} x one dual-stream "
                      f"block of one sample at "
                      f"{N} image + {S} text tokens ({flops / 1e9:.0f} GFLOP each, {t_total:.1f} s, "
                      f"{rate / 1e9:.1f} GFLOP/s), "
                      + (f"x 60 blocks x 2 samples (the step's own shape)" if N == H * W else
                         f"scaled by FLOPs to the 60-block batch-2 step at {H * W} + {S} tokens")}


def copy_calibration(args):
    """The traffic counters' calibration: a conversion kernel of known HBM traffic (fp32 -> bf16 over 64 Mi elements:
    reads 256 MiB, writes 128 MiB a launch), three launches. FETCH_SIZE / WRITE_SIZE per dispatch of this kernel give
    the counters' scale."""
    import mkimage as M

    M.call("mk_set_device", 0)
    n = 64 << 20
    x, y = M.Dev(n * 4), M.Dev(n * 2)
    M.call("mk_fill_normal", x.p, n, M.F32, 1, 0.0, 1.0, None)
    M.sync()
    for _ in range(3):
        M.call("mk_f32_to_bf16", x.p, n, y.p, None)
    M.sync()
    print(json.dumps({"calibration": "mk_f32_to_bf16", "elements": n, "read_bytes": 4 * n, "written_bytes": 2 * n}),
          flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    extra = {"sdxl-1024-bf16": bench_sdxl, "vae-1024-decode": bench_vae, "q21-1024": bench_q21,
             "copy-calibration": copy_calibration}
    ap.add_argument("--workload", choices=sorted(WORKLOADS) + sorted(extra), default="mmdit-1024-bf16")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.workload in extra:
        if args.gpus != 1 or world != 1:
            print("bench.py measures one GPU: run it with --gpus 1", file=sys.stderr)
            sys.exit(2)
        extra[args.workload](args)
        return
    wl = WORKLOADS[args.workload]
    global H, W, S
    H = W = wl["side"]
    S = wl["text"]
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: the step runs on one MI355X (asked for {max(args.gpus, world)}); "
              f"run it with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import numpy as np

    import mkimage as M

    M.call("mk_set_device", 0)
    info = M.device_info()
    eng = M.Engine(M.FAMILY_DUAL, **CFG, weight_dtype=M.FP8 if wl["fp8"] else M.BF16)
    t0 = time.perf_counter()
    eng.init_random(0)
    t_init = time.perf_counter() - t0
    rng = np.random.default_rng(0)
    for s in (0, 1):
        eng.begin(rng.standard_normal((S, 3584)).astype(np.float32), H, W, s)
    lat = [M.Dev.from_array(rng.standard_normal((H * W, 64)).astype(np.float32)), M.Dev(H * W * 64 * 4)]
    sigmas = [1.0 - 0.02 * i for i in range(args.warmup + max(args.steps, 4) + 2)]  # (the ragged run takes 4)
    stream = eng.stream()

    def run(i):
        eng.step_cfg_device(lat[i % 2], sigmas[i], sigmas[i + 1], 4.0, lat[(i + 1) % 2], stream)

    for i in range(args.warmup):
        run(i)
    M.call("mk_stream_synchronize", stream)
    e0, e1 = M.Event(), M.Event()
    M.call("mk_synchronize")
    w0 = time.perf_counter()
    e0.record(stream)
    for i in range(args.steps):
        run(args.warmup + i)
    e1.record(stream)
    M.call("mk_stream_synchronize", stream)
    wall = time.perf_counter() - w0
    ms = e0.elapsed_ms(e1) / args.steps
    out = lat[(args.warmup + args.steps) % 2].to_array(np.float32, (H * W, 64))
    if not np.isfinite(out).all():
        raise RuntimeError("non-finite latents after the timed steps")

    # prompts of different lengths (the negative one shorter): still one batch of 2, the shorter prompt padded
    S_neg = S * 25 // 32
    eng.begin(rng.standard_normal((S_neg, 3584)).astype(np.float32), H, W, 1)
    run(args.warmup)
    M.call("mk_stream_synchronize", stream)
    r0, r1 = M.Event(), M.Event()
    r0.record(stream)
    for i in range(3):
        run(args.warmup + 1 + i)
    r1.record(stream)
    M.call("mk_stream_synchronize", stream)
    ragged = {"text_tokens": [S, S_neg], "ms_per_step": round(r0.elapsed_ms(r1) / 3, 3)}
    eng.begin(rng.standard_normal((S, 3584)).astype(np.float32), H, W, 1)

    # per-kernel pass: events around every launch, same steps
    eng.set_timing(True)
    per = {}
    for i in range(args.steps):
        run(args.warmup + i)
        for k, v in eng.timing().items():
            acc = per.setdefault(k, {"ms": 0.0, "launches": 0, "flops": 0.0})
            acc["ms"] += v["ms"]
            acc["launches"] += v["launches"]
            acc["flops"] += v["flops"]
    eng.set_timing(False)
    total, lin, attn = step_flops(N=H * W, S=S)
    g = {"ms": sum(v["ms"] for k, v in per.items() if k.startswith("gemm")),
         "flops": sum(v["flops"] for k, v in per.items() if k.startswith("gemm"))}
    a = per["attention"]
    gemm_tf = g["flops"] / (g["ms"] / 1e3) / 1e12
    attn_tf = a["flops"] / (a["ms"] / 1e3) / 1e12
    # attention + GEMM time: the union of their launches' intervals (the summed durations less any overlap)
    u = per.get("union:attention+gemm")
    both_ms = u["ms"] if u else g["ms"] + a["ms"]
    both = (g["flops"] + a["flops"]) / (both_ms / 1e3)
    # the dominant kernel: the timing class (one launch shape) with the most time a step
    dom = max((k for k, v in per.items() if v["flops"] and (k.startswith("gemm.") or k == "attention")),
              key=lambda k: per[k]["ms"])
    dv = per[dom]
    dom_launch_s = dv["ms"] / 1e3 / dv["launches"]
    dom_flops = dv["flops"] / dv["launches"]
    kernels = {k: {"ms_per_step": round(v["ms"] / args.steps, 3), "launches_per_step": v["launches"] // args.steps,
                   **({"tflops": round(v["flops"] / (v["ms"] / 1e3) / 1e12, 1)} if v["flops"] else {})}
               for k, v in sorted(per.items(), key=lambda kv: -kv[1]["ms"])}
    line = {
        "metric": wl["metric"],
        "value": round(ms / 1e3, 5),
        "unit": "s/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "weight_dtype": "fp8-e4m3" if wl["fp8"] else "bf16",
        "data": "synthetic (random-init N(0,0.02) weights, N(0,1) latents and prompts)",
        "config": {"workload": wl["name"], "blocks": 60, "dim": 3072, "heads": 24, "head_dim": 128, "ffn": 12288,
                   "text_dim": 3584, "image_tokens": H * W, "text_tokens": S, "batch": 2,
                   "weights": "fp8-e4m3" if wl["fp8"] else "bf16"},
        "roofline": {"bound": "mfma", "kernel": f"{dom}: {KERNEL_OF.get(dom, dom)}",
                     "achieved": round(dom_flops / dom_launch_s / 1e12, 1), "peak": PEAK_BF16 / 1e12,
                     "unit": "TFLOP/s", "frac": round(dom_flops / dom_launch_s / PEAK_BF16, 4),
                     "flops_per_launch": dom_flops, "launch_us": round(dom_launch_s * 1e6, 1),
                     "traffic": None if wl["fp8"] else kernel_traffic(KERNEL_OF.get(dom)),
                     "traffic_algorithmic": step_bytes_ff2(H * W, S) if dom == "gemm.ff2" and not wl["fp8"] else None,
                     "traffic_note": "bytes/launch between L2 and the fabric (rocprofv3 FETCH_SIZE + WRITE_SIZE, "
                                     "calibrated; Infinity Cache hits included) from "
                                     "profiles/mmdit_step_1024_traffic.md"},
        "gemm_class": {"achieved": round(gemm_tf, 1), "unit": "TFLOP/s", "frac": round(gemm_tf * 1e12 / PEAK_BF16, 4),
                       "ms_per_step": round(g["ms"] / args.steps, 3)},
        "attention_gemm_mfma_frac": round(both / PEAK_BF16, 4),
        "attention_gemm_ms_per_step": round(both_ms / args.steps, 3),
        "step_mfma_frac": round(total / (ms / 1e3) / PEAK_BF16, 4),
        "attention": {"achieved": round(attn_tf, 1), "unit": "TFLOP/s", "frac": round(attn_tf * 1e12 / PEAK_BF16, 4)},
        "step_tflop": round(total / 1e12, 2),
        "ragged_prompts": ragged,
        "kernels": kernels,
        "wall_s_per_step": round(wall / args.steps, 5),
        "device": info,
        "weights_gb": round(eng.weight_bytes() / 1e9, 2),
        "init_s": round(t_init, 2),
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(args.cpu_seconds, wl["fp8"])
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
