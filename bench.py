"""bench.py -- the dit-step on one MI355X: ms per step at 1024px bf16, and the MFMA roofline.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--resolution 1024] [--no-cpu]
    python bench.py --kernels          # the isolated kernels at 1024px shapes, one line each
    python bench.py --probe NAME       # one kernel three times after a copy, for rocprofv3 --pmc
    python bench.py --denoise 20       # the 20-step on-device denoise loop, eager vs HIP graph

One step is one PixArt-Sigma dit-step forward (28 blocks, hidden 1152, 16 heads x 72, MLP 4608)
at batch 2 (classifier-free guidance) over a 128x128x4 latent (4096 image tokens) and a
300-token caption of width 4096, through the library's fused engine (bh_dit_forward). Weights
(~N(0, 0.02)), latent and caption (~N(0, 1)) are seeded synthetic bf16, resident in HBM before
the timed region. K steps are timed between two HIP events on the engine's stream, bracketed by
device synchronisation.

The JSON line also carries:
  roofline      the dominant kernel (largest share of step time): algorithmic FLOP per launch
                over its average launch duration, timed live with HIP events around one of its
                launches per step in the timed region (every 29th launch: the sampled layer
                moves by one each step), against the 2.5166 PFLOP/s dense bf16 MFMA peak;
                `traffic` is its HBM bytes per launch from the committed rocprofv3 counter
                summary (profiles/flash72_self_1024_traffic.md);
  step          the whole step's algorithmic FLOP (the reference's accounting,
                eval/burnscore/geometry.py:275-367) over the measured step time, same peak;
  kernels       per-class time of one separately profiled step (not the timed region);
  cpu_baseline  the stock oracle's whole dit-step on this host's cores (about 30 s on 16
                threads at 1024px), same workload and seeds.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "dit-step ms @1024px bf16 (1 GPU) + % of MI355X bf16 MFMA roofline"
PEAK_BF16_TFLOPS = 2516.6          # 256 CU x 4096 FLOP/clk x 2.4 GHz, dense
PEAK_HBM_GBS = 8000.0
REFERENCE_5090_MS = 97.85          # eval/cells/BG-1/reference.json:28 (RTX 5090, cuda impl)
HW = {512: 64, 768: 96, 1024: 128, 1152: 144, 2048: 256}


# HBM bytes per launch of a kernel, from the rocprofv3 FETCH_SIZE / WRITE_SIZE summaries committed
# under profiles/ (counter passes cannot run inside this timed program).
TRAFFIC_PROFILES = {"attention_self": ROOT / "profiles" / "flash72_self_1024_traffic.md"}


def traffic_bytes(kernel: str, resolution: int):
    path = TRAFFIC_PROFILES.get(kernel)
    if resolution != 1024 or path is None or not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":", 1)[1])
    return None


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse() -> argparse.Namespace:
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--resolution", type=int, default=1024, choices=sorted(HW))
    p.add_argument("--caption-len", type=int, default=300)
    p.add_argument("--batch", type=int, default=2)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--headline-only", action="store_true",
                   help="time the headline engine only: no device probe, row-split schedule, "
                        "op-by-op plan or other resolutions (implies --no-cpu); for kernel traces "
                        "whose every launch belongs to the headline step")
    p.add_argument("--cpu-threads", type=int, default=0)
    p.add_argument("--probe", choices=sorted(KERNEL_SHAPES),
                   help="for counter collection: run a 256 MiB device copy (calibration) and the "
                        "named kernel at the dit-step shape three times each, then exit")
    p.add_argument("--denoise", type=int, default=0, metavar="STEPS",
                   help="time the whole on-device denoise loop (STEPS sampler steps, CFG 4.5) "
                        "eagerly and as one HIP graph, one JSON line")
    p.add_argument("--vae", action="store_true",
                   help="time the vae-decode stage (SDXL VAE widths, batch 1) at --resolution; "
                        "one JSON line")
    p.add_argument("--t5", action="store_true",
                   help="time the t5-encode stage (T5 v1.1 XXL, [batch, caption-len] ids); one "
                        "JSON line")
    p.add_argument("--kernels", action="store_true",
                   help="time the isolated kernels at 1024px shapes (GEMMs, self- and "
                        "cross-attention, LayerNorm+modulate); one JSON line per kernel")
    return p.parse_args()


def make_kernel(name: str):
    """One isolated kernel of the 1024px dit-step on seeded synthetic
    operands: returns (launch, algorithmic work per launch, unit of that work)."""
    import torch

    import burnisher_amd as bh

    gen = torch.Generator(device="cuda").manual_seed(0)
    randn = lambda *shape, std=1.0: (torch.randn(*shape, device="cuda", generator=gen) * std).bfloat16()
    kind, dims = KERNEL_SHAPES[name]
    if kind == "gemm":
        m, n, k = dims
        a, w, bias = randn(m, k), randn(n, k, std=0.02), randn(n, std=0.02)
        out = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
        launch = lambda: bh.call("bh_gemm", a.data_ptr(), w.data_ptr(), bias.data_ptr(),
                                 out.data_ptr(), m, n, k, 1, 0, bh.BF16, None)
        return launch, 2.0 * m * n * k, "flop", (a, w, bias, out)
    if kind == "attention":
        batch, heads, sq, skv, dh = dims
        q, k, v = randn(batch, sq, heads * dh), randn(batch, skv, heads * dh), randn(batch, skv, heads * dh)
        out = torch.empty_like(q)
        mask = None
        if sq != skv:   # the caption mask of the workload: row 0 keeps 75 tokens, row 1 keeps 150
            mask = torch.zeros(batch, skv, device="cuda")
            mask[0, :75] = 1
            mask[1, :150] = 1
        launch = lambda: bh.call("bh_attention", q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                 out.data_ptr(), batch, heads, sq, skv, dh, 0.0, None,
                                 None if mask is None else mask.data_ptr(), bh.F32, bh.BF16, None)
        return launch, 4.0 * batch * heads * sq * skv * dh, "flop", (q, k, v, out, mask)
    rows, cols = dims   # op-level LayerNorm + chunk + modulate (bh_norm_modulate): read x, write
                        # the result
    x = randn(rows, cols)
    mod = randn(2, 6 * cols, std=0.02)
    table = randn(6, cols, std=0.02)
    out = torch.empty_like(x)
    launch = lambda: bh.call("bh_norm_modulate", x.data_ptr(), mod.data_ptr(), 6, 0, 1,
                             table.data_ptr(), 0, 1, out.data_ptr(), 2, rows // 2, cols, 1e-6,
                             None)
    return launch, 2.0 * rows * cols * 2, "bytes", (x, mod, table, out)


# the isolated kernels of BASELINE.json configs[1] (and the dit-step's norm), 1024px shapes
KERNEL_SHAPES = {
    "gemm_proj": ("gemm", (8192, 1152, 1152)),
    "gemm_qkv": ("gemm", (8192, 3456, 1152)),
    "gemm_ff0": ("gemm", (8192, 4608, 1152)),
    "gemm_ff2": ("gemm", (8192, 1152, 4608)),
    "gemm_8192": ("gemm", (8192, 8192, 8192)),    # the reference probe's GEMM (device.cu:284-318)
    "attention_self": ("attention", (2, 16, 4096, 4096, 72)),
    "attention_cross": ("attention", (2, 16, 4096, 300, 72)),
    "norm_modulate": ("norm", (8192, 1152)),
}


def probe(kernel: str) -> int:
    """Launches for rocprofv3 --pmc passes: a copy of known size, then the kernel, three times
    each."""
    import torch

    import burnisher_amd as bh

    bh.check(bh.lib().bh_init(0), "bh_init")
    src = torch.ones(128 << 20, device="cuda", dtype=torch.bfloat16)   # 256 MiB
    dst = torch.empty_like(src)
    launch, _, _, keep = make_kernel(kernel)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
        launch()
    torch.cuda.synchronize()
    log(f"probe {kernel}: done")
    return 0


def kernels(iters: int) -> int:
    """The isolated kernels: average launch time over `iters` launches between HIP events after
    three warm-up launches; FLOP kernels against the dense bf16 MFMA peak, the norm against HBM."""
    import torch

    import burnisher_amd as bh

    bh.check(bh.lib().bh_init(0), "bh_init")
    for name in KERNEL_SHAPES:
        launch, work, unit, keep = make_kernel(name)
        for _ in range(3):
            launch()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record()
        for _ in range(iters):
            launch()
        stop.record()
        torch.cuda.synchronize()
        us = start.elapsed_time(stop) / iters * 1e3
        rate = work / (us * 1e-6)
        line = {"kernel": name, "shape": list(KERNEL_SHAPES[name][1]), "us_per_launch": round(us, 2)}
        if unit == "flop":
            line.update({"tflops": round(rate / 1e12, 1), "peak": PEAK_BF16_TFLOPS,
                         "frac": round(rate / 1e12 / PEAK_BF16_TFLOPS, 4), "bound": "mfma"})
        else:
            line.update({"gbs": round(rate / 1e9, 1), "peak": PEAK_HBM_GBS,
                         "frac": round(rate / 1e9 / PEAK_HBM_GBS, 4), "bound": "hbm"})
        print(json.dumps(line), flush=True)
        del keep
    return 0


def denoise(args) -> int:
    """The generate loop's denoise stage (pipeline.cpp:110-131) on the device: STEPS x (repeat,
    dit-step, guidance, DPM-Solver++ step), from one seeded N(0,1) latent, timed per image with
    HIP events on the loop's stream, eagerly (every launch from the host) and as one replayed
    HIP graph. Each image restarts from the same noise; the restoring copy is outside the events."""
    import numpy as np
    import torch

    import burnisher_amd as bh
    from burnisher_amd.workload import PIXART_SIGMA, config_struct, dit_step_flops, make_workload

    bh.check(bh.lib().bh_init(0), "bh_init")
    hw = HW[args.resolution]
    steps = args.denoise
    wl = make_workload(PIXART_SIGMA, batch=2, latent_hw=hw, caption_len=args.caption_len)
    top, blocks, _, caption, mask = wl.to_device()
    cfg = config_struct(wl.cfg)
    w, keep = wl.weight_struct(top, blocks)
    engine, sched, den = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
    bh.call("bh_dit_create", ctypes.byref(cfg), ctypes.byref(w), 2, hw, wl.caption_len,
            bh.DIT_FUSED, ctypes.byref(engine))
    scfg = bh.SchedConfig.pinned()
    bh.call("bh_sched_create", ctypes.byref(scfg), ctypes.byref(sched))
    bh.call("bh_sched_set_timesteps", sched, steps)
    bh.call("bh_denoiser_create", engine, sched, 1, 4.5, ctypes.byref(den))
    noise = bh.fill_normal_bf16(4 * hw * hw, "initial_latent", 0, 1.0)
    init = torch.from_numpy(noise.view(np.int16)).cuda()
    latent = torch.empty_like(init)
    stream = torch.cuda.Stream()
    sp = stream.cuda_stream

    def run(graph: bool, reps: int) -> float:
        total = 0.0
        for _ in range(reps):
            with torch.cuda.stream(stream):
                latent.copy_(init)
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record(stream)
                bh.call("bh_denoiser_run", den, latent.data_ptr(), caption.data_ptr(),
                        mask.data_ptr(), bh.F32, int(graph), sp)
                b.record(stream)
            torch.cuda.synchronize()
            total += a.elapsed_time(b)
        return total / reps

    reps = max(1, min(args.steps, 5))
    log(f"denoise {steps} steps at {args.resolution}px: warmup (eager, then graph capture)")
    run(False, 1)
    eager_first = latent.clone()
    t0 = time.perf_counter()
    run(True, 1)
    capture_s = time.perf_counter() - t0
    assert torch.equal(latent, eager_first), "graph loop differs from the eager loop"
    eager_ms = run(False, reps)
    graph_ms = run(True, reps)
    assert torch.equal(latent, eager_first), "graph replay differs from the eager loop"
    res = latent.view(torch.bfloat16).float()
    assert torch.isfinite(res).all() and res.std() > 1e-3, "degenerate denoised latent"
    flops = dit_step_flops(wl.cfg, batch=2, latent_hw=hw, caption_len=wl.caption_len)["total"]
    line = {
        "metric": f"denoise loop ms/image @{args.resolution}px bf16, {steps} steps (1 GPU)",
        "value": round(graph_ms, 3), "unit": "ms", "n_gpus": 1, "steps": reps, "warmup": 1,
        "ms_per_step": round(graph_ms, 3), "higher_is_better": False, "dtype": "bf16",
        "data": "synthetic: seeded N(0,0.02) bf16 weights, N(0,1) caption and initial latent",
        "config": {"workload": f"PixArt-Sigma denoise loop {args.resolution}px, CFG 4.5, "
                               f"{steps} DPM-Solver++ 2M steps, caption {wl.caption_len}",
                   "resolution": args.resolution, "sampler_steps": steps},
        "graph_ms_per_image": round(graph_ms, 3), "eager_ms_per_image": round(eager_ms, 3),
        "graph_ms_per_step": round(graph_ms / steps, 4),
        "eager_ms_per_step": round(eager_ms / steps, 4),
        "graph_capture_s": round(capture_s, 3),
        "step_tflops_graph": round(flops / (graph_ms / steps * 1e-3) / 1e12, 2),
        "output_stats": tensor_stats(latent.view(torch.bfloat16)),
    }
    bh.lib().bh_denoiser_destroy(den)
    bh.lib().bh_sched_destroy(sched)
    bh.lib().bh_dit_destroy(engine)
    print(json.dumps(line), flush=True)
    return 0


def vae(args) -> int:
    """The vae-decode stage (VaeDecoder::forward, vae_decoder.cpp:127-180) at the resolution's
    latent (resolution / 8), batch 1, SDXL VAE widths, seeded synthetic weights, through the
    library's decoder engine. K decodes timed between HIP events on one stream after W warm-up
    decodes; one more decode runs with the launch profiler for the per-class breakdown. The
    roofline is the implicit-GEMM convolution and projection class (MFMA), as that class's
    algorithmic FLOP over its summed launch time. The CPU baseline is the stock oracle's decoder
    on a 128px sample (latent 16) on this host, scaled to the resolution by the FLOP ratio."""
    import numpy as np
    import torch

    import burnisher_amd as bh
    from burnisher_amd.vae import SDXL_VAE, config_struct, make_vae_workload, vae_decode_flops

    bh.check(bh.lib().bh_init(0), "bh_init")
    hw = args.resolution // 8
    wl = make_vae_workload(SDXL_VAE, latent_hw=hw)
    tensors, latent = wl.to_device()
    cfg = config_struct(wl.cfg)
    w, keep = wl.table(tensors)
    h = ctypes.c_void_p()
    bh.call("bh_vae_create", ctypes.byref(cfg), ctypes.byref(w), hw, ctypes.byref(h))
    image = torch.zeros((1, 3, wl.image_hw, wl.image_hw), dtype=torch.bfloat16, device="cuda")
    stream = torch.cuda.Stream()
    sp = stream.cuda_stream
    steps = max(1, min(args.steps, 10))
    for _ in range(max(1, args.warmup)):
        bh.call("bh_vae_decode", h, latent.data_ptr(), image.data_ptr(), sp)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(steps):
            bh.call("bh_vae_decode", h, latent.data_ptr(), image.data_ptr(), sp)
        b.record(stream)
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / steps
    img = image.float()
    assert torch.isfinite(img).all() and img.std() > 1e-3, "degenerate decoded image"
    output_stats = tensor_stats(image)
    # one profiled decode for the breakdown
    bh.check(bh.lib().bh_profile_enable((1 << bh.K_GEMM_QKV + 1) - 1), "bh_profile_enable")
    bh.call("bh_vae_decode", h, latent.data_ptr(), image.data_ptr(), sp)
    torch.cuda.synchronize()
    breakdown = {}
    for cls, name in enumerate(bh.KERNEL_CLASSES[:6]):
        tot, n, work = ctypes.c_double(), ctypes.c_int64(), ctypes.c_double()
        bh.check(bh.lib().bh_profile_read(cls, ctypes.byref(tot), ctypes.byref(n), ctypes.byref(work)))
        if n.value:
            breakdown[name] = {"ms": round(tot.value, 4), "launches": n.value, "work": work.value}
    bh.lib().bh_profile_enable(0)
    bh.lib().bh_vae_destroy(h)
    flops = vae_decode_flops(wl.cfg, hw)
    g = breakdown.get("gemm", {"ms": 0.0, "work": 0.0})
    conv_tflops = g["work"] / (g["ms"] * 1e-3) / 1e12 if g["ms"] else 0.0
    tflops = flops["total"] / (ms * 1e-3) / 1e12
    line = {
        "metric": f"vae-decode ms @{args.resolution}px bf16 (1 GPU)",
        "value": round(ms, 4), "unit": "ms", "n_gpus": 1, "steps": steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded weights (convs N(0, 1/fan_in), GroupNorm affine near identity), "
                "N(0,1) latent",
        "config": {"workload": f"SDXL VAE decoder {args.resolution}px, batch 1",
                   "latent": [1, 4, hw, hw], "image": [1, 3, wl.image_hw, wl.image_hw],
                   "block_out_channels": list(wl.cfg["block_out_channels"])},
        "roofline": {"bound": "mfma", "kernel": "conv3x3 implicit GEMM + projections (class)",
                     "achieved": round(conv_tflops, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(conv_tflops / PEAK_BF16_TFLOPS, 4), "traffic": None},
        "step": {"flop": flops["total"], "tflops": round(tflops, 2),
                 "mfma_frac": round(tflops / PEAK_BF16_TFLOPS, 4),
                 "ceiling_ms": round(flops["total"] / (PEAK_BF16_TFLOPS * 1e12) * 1e3, 3)},
        "kernels": breakdown,
        "output_stats": output_stats,
    }
    if not args.no_cpu:
        import oracle
        threads = args.cpu_threads or min(16, os.cpu_count() or 1)
        sample = make_vae_workload(SDXL_VAE, latent_hw=16)
        scfg = config_struct(sample.cfg)
        sw, skeep = sample.table()
        out = np.zeros((1, 3, sample.image_hw, sample.image_hw), np.uint16)
        log(f"cpu baseline: stock decoder at 128px on {threads} threads")
        t0 = time.perf_counter()
        oracle.call(oracle.stock(), "stock_vae_forward", ctypes.byref(scfg), ctypes.byref(sw),
                    sample.latent.ctypes.data, 16, out.ctypes.data, threads, -1)
        secs = time.perf_counter() - t0
        ratio = flops["total"] / vae_decode_flops(sample.cfg, 16)["total"]
        line["cpu_baseline"] = {"value": round(secs * ratio * 1e3, 1), "unit": "ms", "cores": threads,
                                "kind": "port",
                                "sample": f"stock oracle decoder at 128px (latent 16), {secs:.2f} s, "
                                          f"scaled x{ratio:.1f} by algorithmic FLOP to {args.resolution}px"}
    print(json.dumps(line), flush=True)
    return 0


def t5(args) -> int:
    """The t5-encode stage (T5Encoder::forward, t5_encoder.cpp:132-241): T5 v1.1 XXL on
    [batch, caption_len] token ids (the pipeline's CFG pair: the empty negative prompt, then a
    caption), seeded synthetic weights drawn on the device, through the library's encoder engine.
    K encodes timed between HIP events on one stream after W warm-up encodes (the id upload is
    inside: the engine takes host ids); one more encode runs with the launch profiler for the
    per-class breakdown. The roofline is the GEMM class (MFMA): its algorithmic FLOP over its
    summed launch time. The CPU baseline is the stock oracle's encoder restricted to ONE of the
    layers at the full [batch, caption_len] shape on this host, scaled by the layer count."""
    import numpy as np
    import torch

    import burnisher_amd as bh
    from burnisher_amd.t5 import (T5_XXL, T5Workload, config_struct, make_t5_workload, synthetic_ids,
                                  t5_encode_flops, t5_tensors)

    bh.check(bh.lib().bh_init(0), "bh_init")
    B, S = args.batch, args.caption_len
    cfg = dict(T5_XXL)
    lengths = [1] + [120] * (B - 1)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(20261203)
    tensors = {}
    for name, shape in t5_tensors(cfg).items():
        t = torch.randn(shape, generator=gen, device="cuda", dtype=torch.float32)
        if "layer_norm" in name:
            t = 1.0 + 0.1 * t
        elif name.endswith("SelfAttention.q.weight"):
            t = t / float(np.sqrt(shape[1] * cfg["d_kv"]))
        elif name != "shared.weight" and "relative_attention_bias" not in name:
            t = t / float(np.sqrt(shape[1]))
        tensors[name] = t.to(torch.bfloat16)
        del t
    wl = T5Workload(cfg=cfg, batch=B, seq=S)
    wl.ids = synthetic_ids(B, S, cfg["vocab_size"], lengths, 20261203)
    c = config_struct(cfg)
    w, keep = wl.table(tensors)
    h = ctypes.c_void_p()
    bh.call("bh_t5_create", ctypes.byref(c), ctypes.byref(w), B, S, ctypes.byref(h))
    out = torch.zeros((B, S, cfg["d_model"]), dtype=torch.bfloat16, device="cuda")
    stream = torch.cuda.Stream()
    sp = stream.cuda_stream
    steps = max(1, min(args.steps, 20))
    for _ in range(max(1, args.warmup)):
        bh.call("bh_t5_encode", h, wl.ids.ctypes.data, out.data_ptr(), sp)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(steps):
            bh.call("bh_t5_encode", h, wl.ids.ctypes.data, out.data_ptr(), sp)
        b.record(stream)
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / steps
    o = out.float()
    assert torch.isfinite(o).all() and o.std() > 1e-3, "degenerate encoder output"
    output_stats = tensor_stats(out)
    bh.check(bh.lib().bh_profile_enable((1 << bh.K_GEMM_QKV + 1) - 1), "bh_profile_enable")
    bh.call("bh_t5_encode", h, wl.ids.ctypes.data, out.data_ptr(), sp)
    torch.cuda.synchronize()
    breakdown = {}
    for cls, name in enumerate(bh.KERNEL_CLASSES[:6]):
        tot, n, work = ctypes.c_double(), ctypes.c_int64(), ctypes.c_double()
        bh.check(bh.lib().bh_profile_read(cls, ctypes.byref(tot), ctypes.byref(n), ctypes.byref(work)))
        if n.value:
            breakdown[name] = {"ms": round(tot.value, 4), "launches": n.value, "work": work.value}
    bh.lib().bh_profile_enable(0)
    ws = bh.lib().bh_t5_workspace_bytes(h)
    bh.lib().bh_t5_destroy(h)
    flops = t5_encode_flops(cfg, B, S)
    g = breakdown.get("gemm", {"ms": 0.0, "work": 0.0})
    gemm_tflops = g["work"] / (g["ms"] * 1e-3) / 1e12 if g["ms"] else 0.0
    tflops = flops["total"] / (ms * 1e-3) / 1e12
    line = {
        "metric": f"t5-encode ms bf16 (1 GPU)", "value": round(ms, 4), "unit": "ms", "n_gpus": 1,
        "steps": steps, "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: seeded weights drawn on the device (projections N(0, 1/fan_in), q with a "
                "further 1/sqrt(d_kv), embedding "
                "and relative bias N(0, 1), RMSNorm weights 1 + N(0, 0.01)), seeded token ids",
        "config": {"workload": f"T5 v1.1 XXL encoder, ids [{B}, {S}] (lengths {lengths})",
                   "layers": cfg["num_layers"], "d_model": cfg["d_model"], "d_ff": cfg["d_ff"],
                   "heads": cfg["num_heads"], "engine_device_bytes": ws},
        "roofline": {"bound": "mfma", "kernel": "GEMM class (packed qkv, o, packed wi, wo)",
                     "achieved": round(gemm_tflops, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(gemm_tflops / PEAK_BF16_TFLOPS, 4), "traffic": None},
        "step": {"flop": flops["total"], "tflops": round(tflops, 2),
                 "mfma_frac": round(tflops / PEAK_BF16_TFLOPS, 4),
                 "ceiling_ms": round(flops["total"] / (PEAK_BF16_TFLOPS * 1e12) * 1e3, 3)},
        "kernels": breakdown,
        "output_stats": output_stats,
    }
    del tensors, keep, w
    torch.cuda.empty_cache()
    if not args.no_cpu:
        import oracle
        threads = args.cpu_threads or min(16, os.cpu_count() or 1)
        one = dict(cfg, num_layers=1)
        log(f"cpu baseline: generating one XXL layer on the host")
        sample = make_t5_workload(one, batch=B, seq=S, lengths=lengths)
        sc = config_struct(one)
        sw, skeep = sample.table()
        res = np.zeros((B, S, cfg["d_model"]), np.uint16)
        log(f"cpu baseline: stock encoder, 1 layer at [{B}, {S}], {threads} threads")
        t0 = time.perf_counter()
        oracle.call(oracle.stock(), "stock_t5_forward", ctypes.byref(sc), ctypes.byref(sw),
                    sample.ids.ctypes.data, B, S, res.ctypes.data, threads)
        secs = time.perf_counter() - t0
        line["cpu_baseline"] = {"value": round(secs * cfg["num_layers"] * 1e3, 1), "unit": "ms",
                                "cores": threads, "kind": "port",
                                "sample": f"stock oracle encoder with 1 of the {cfg['num_layers']} layers at "
                                          f"the full [{B}, {S}] shape, {secs:.2f} s, scaled x{cfg['num_layers']}"}
    print(json.dumps(line), flush=True)
    return 0


def stock_step(wl, threads: int):
    """The stock oracle's dit-step (all of wl's blocks) on this host: (output bf16 bits, seconds)."""
    import numpy as np
    import oracle
    from burnisher_amd.workload import config_struct

    cfg = config_struct(wl.cfg)
    w, keep = wl.weight_struct(wl.top, wl.blocks)
    out = np.zeros((wl.batch, wl.cfg["out_channels"], wl.latent_hw, wl.latent_hw), np.uint16)
    t0 = time.perf_counter()
    oracle.call(oracle.stock(), "stock_dit_forward", ctypes.byref(cfg), ctypes.byref(w),
                wl.batch, wl.latent_hw, wl.caption_len, wl.latent.ctypes.data, wl.timestep,
                wl.caption.ctypes.data, wl.mask.ctypes.data, 0, out.ctypes.data, threads, -1)
    return out, time.perf_counter() - t0


def reference_stock_block(wl):
    """The reference's own single-threaded stock dit-step (PixArtDiT::forward with every op
    resolved to `stock`, compiled from /root/reference into oracle/_ref by oracle/Makefile) on
    workload wl, timed on this host; None where that library was not built. Its output is
    checked bit for bit against the port's."""
    import numpy as np
    import oracle
    from burnisher_amd.workload import config_struct

    lib = oracle.ref()
    if lib is None:
        return None
    cfg = config_struct(wl.cfg)
    w, keep = wl.weight_struct(wl.top, wl.blocks)
    out = np.zeros((wl.batch, wl.cfg["out_channels"], wl.latent_hw, wl.latent_hw), np.uint16)
    t0 = time.perf_counter()
    oracle.call(lib, "ref_dit_forward", ctypes.byref(cfg), ctypes.byref(w), wl.batch, wl.latent_hw,
                wl.caption_len, wl.latent.ctypes.data, wl.timestep, wl.caption.ctypes.data,
                wl.mask.ctypes.data, 0, out.ctypes.data, -1)
    secs = time.perf_counter() - t0
    port, _ = stock_step(wl, 1)
    return {"config0_block_512px_b1_cap120_ms": round(secs * 1e3, 1), "cores": 1, "kind": "reference",
            "equals_port": bool(np.array_equal(out, port)),
            "sample": "BASELINE configs[0]: one block at 512px, batch 1, caption 120, the reference's "
                      "stock PixArtDiT::forward (oracle/_ref/libref_stock.so), one thread"}


def tensor_stats(t) -> dict:
    """Mean, standard deviation and largest magnitude of a timed output, as the reference's bench
    line carries them (burnisher_main.cpp:478-480)."""
    f = t.detach().double().cpu()
    return {"mean": float(f.mean()), "std": float(f.std(unbiased=False)), "absmax": float(f.abs().max()),
            "finite": bool(f.isfinite().all())}


def parity(got, want) -> dict:
    """max-abs, relative L2 and cosine of the device output against the oracle's, and the
    configs/tolerance.json dit_step gate they are held to."""
    import numpy as np

    g = (got.astype(np.uint32) << 16).view(np.float32).astype(np.float64).ravel()
    r = (want.astype(np.uint32) << 16).view(np.float32).astype(np.float64).ravel()
    gate = json.loads((ROOT / "configs" / "tolerance.json").read_text())["dit_step"]
    d = g - r
    res = {"max_abs": float(np.max(np.abs(d))),
           "rel_l2": float(np.linalg.norm(d) / np.linalg.norm(r)),
           "cosine": float(np.dot(g, r) / (np.linalg.norm(g) * np.linalg.norm(r))),
           "finite": bool(np.all(np.isfinite(g)))}
    res["gate"] = {k: gate[k] for k in ("max_abs", "rel_l2", "cosine")}
    res["pass"] = (res["finite"] and res["max_abs"] <= gate["max_abs"] and
                   res["rel_l2"] <= gate["rel_l2"] and res["cosine"] >= gate["cosine"])
    return res


def timed_steps(step, stream, steps: int) -> float:
    """ms per step over `steps` back-to-back steps between two HIP events on the stream."""
    import torch
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        start.record(stream)
        for _ in range(steps):
            step()
        stop.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps


def synced_median(step, stream, iters: int) -> float:
    """The reference's method (burnisher_main.cpp:451-464): each iteration timed on the host
    clock from launch to device synchronisation; the median, in ms."""
    import torch
    times = []
    for _ in range(iters):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        with torch.cuda.stream(stream):
            step()
        torch.cuda.synchronize()
        times.append((time.perf_counter() - t0) * 1e3)
    times.sort()
    n = len(times)
    return times[n // 2] if n % 2 else 0.5 * (times[n // 2 - 1] + times[n // 2])


def device_probe() -> dict:
    """What this device sustains (bh_probe_device: a register-only MFMA loop with the shader clock
    it holds, and a 1 GiB device copy), plus this library's GEMM at 8192^3 (the reference's
    `probe` times a vendor GEMM of that size, device.cu:284-318)."""
    import torch

    import burnisher_amd as bh

    src = torch.ones(1 << 29, device="cuda", dtype=torch.bfloat16)   # 1 GiB
    dst = torch.empty_like(src)
    res = bh.ProbeResult()
    bh.call("bh_probe_device", src.data_ptr(), dst.data_ptr(), src.numel() * 2, ctypes.byref(res))
    del src, dst
    out = res.as_dict()
    n = 8192
    gen = torch.Generator(device="cuda").manual_seed(1)
    a = torch.randn(n, n, device="cuda", generator=gen).bfloat16()
    b = (torch.randn(n, n, device="cuda", generator=gen) * 0.02).bfloat16()
    c = torch.empty(n, n, device="cuda", dtype=torch.bfloat16)
    launch = lambda: bh.call("bh_gemm", a.data_ptr(), b.data_ptr(), None, c.data_ptr(), n, n, n, 1, 0,
                             bh.BF16, None)
    launch()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(5):
        launch()
    e1.record()
    torch.cuda.synchronize()
    out["gemm_8192_tflops"] = round(2.0 * n ** 3 / (e0.elapsed_time(e1) / 5 * 1e-3) / 1e12, 1)
    del a, b, c
    torch.cuda.empty_cache()
    return out


class Engine:
    """One bh_dit engine over device weights shared between engines, with its own inputs."""

    def __init__(self, wl, top, blocks, mode, stream):
        import numpy as np
        import torch

        import burnisher_amd as bh
        from burnisher_amd.workload import config_struct

        self.bh, self.wl, self.stream = bh, wl, stream
        t = lambda a: torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).cuda()
        self.latent, self.caption = t(wl.latent), t(wl.caption)
        self.mask = torch.from_numpy(wl.mask).cuda()
        self.cfg = config_struct(wl.cfg)
        self.w, self._keep = wl.weight_struct(top, blocks)
        self.handle = ctypes.c_void_p()
        bh.call("bh_dit_create", ctypes.byref(self.cfg), ctypes.byref(self.w), wl.batch,
                wl.latent_hw, wl.caption_len, mode, ctypes.byref(self.handle))
        self.out = torch.zeros((wl.batch, self.cfg.out_channels, wl.latent_hw, wl.latent_hw),
                               dtype=torch.bfloat16, device="cuda")

    def step(self):
        self.bh.call("bh_dit_forward", self.handle, self.latent.data_ptr(), self.wl.timestep,
                     self.caption.data_ptr(), self.mask.data_ptr(), self.bh.F32,
                     self.out.data_ptr(), self.stream.cuda_stream)

    def workspace(self) -> int:
        return int(self.bh.lib().bh_dit_workspace_bytes(self.handle))

    def input_bytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.latent, self.caption, self.mask, self.out))

    def output(self):
        import numpy as np
        import torch
        torch.cuda.synchronize()
        return self.out.cpu().view(torch.int16).numpy().view(np.uint16).copy()

    def close(self):
        if self.handle:
            self.bh.lib().bh_dit_destroy(self.handle)
            self.handle = ctypes.c_void_p()


def main() -> int:
    args = parse()
    if args.probe:
        return probe(args.probe)
    if args.kernels:
        return kernels(max(args.steps, 10))
    if args.denoise:
        return denoise(args)
    if args.vae:
        return vae(args)
    if args.t5:
        return t5(args)
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the dit-step would shard on the CFG batch: one batch row per GPU)", file=sys.stderr)
        return 2
    import numpy as np
    import torch

    import burnisher_amd as bh
    from burnisher_amd.workload import PIXART_SIGMA, dit_step_flops, make_workload

    bh.check(bh.lib().bh_init(0), "bh_init")
    if args.headline_only:
        args.no_cpu = True
    probed = {"mfma_tflops": None} if args.headline_only else device_probe()
    log(f"device probe: {json.dumps(probed)}")
    hw = HW[args.resolution]
    log(f"generating the {args.resolution}px workload (seeded synthetic bf16)")
    wl = make_workload(PIXART_SIGMA, batch=args.batch, latent_hw=hw, caption_len=args.caption_len)
    free0 = torch.cuda.mem_get_info()[0]
    # the checkpoint loader's layout (bh_dit_weights_load): packed Q/K/V and caption K/V, which
    # the engine reads in place
    top, blocks = wl.weights_to_device()
    weight_bytes = sum(x.numel() * 2 for x in top.values()) + \
        sum(x.numel() * 2 for b in blocks for x in b.values())
    stream = torch.cuda.Stream()
    eng = Engine(wl, top, blocks, bh.DIT_FUSED, stream)
    torch.cuda.synchronize()
    driver_used = free0 - torch.cuda.mem_get_info()[0]
    peak_bytes = weight_bytes + eng.input_bytes() + eng.workspace()

    flops = dit_step_flops(wl.cfg, batch=wl.batch, latent_hw=hw, caption_len=wl.caption_len)
    with torch.cuda.stream(stream):
        for _ in range(max(1, args.warmup)):
            eng.step()
    torch.cuda.synchronize()
    log("warmup done")

    # one profiled step, every class, for the breakdown and to name the dominant kernel
    classes = {name: i for i, name in enumerate(bh.KERNEL_CLASSES)}
    bh.call("bh_profile_enable", (1 << len(classes)) - 1)
    with torch.cuda.stream(stream):
        eng.step()
    torch.cuda.synchronize()
    breakdown = {}
    for name, i in classes.items():
        ms, n, work = ctypes.c_double(), ctypes.c_int64(), ctypes.c_double()
        bh.call("bh_profile_read", i, ctypes.byref(ms), ctypes.byref(n), ctypes.byref(work))
        if n.value:
            breakdown[name] = {"ms": round(ms.value, 4), "launches": n.value, "work": work.value}
    bh.call("bh_profile_enable", 0)
    exclusive = ["attention_self", "attention_cross", "gemm_ff0", "gemm_ff2", "gemm_qkv", "norm"]
    dominant = max((c for c in exclusive if c in breakdown), key=lambda c: breakdown[c]["ms"])
    log(f"profiled step: {json.dumps(breakdown)}; dominant kernel {dominant}")

    # the timed region: K steps, HIP events around one launch of the dominant kernel per step.
    # Every (layers + 1)-th launch is bracketed, so the sampled layer moves by one each step and
    # the other launches run with no event beside them.
    sample_every = wl.cfg["num_layers"] + 1
    bh.call("bh_profile_sample", sample_every)
    bh.call("bh_profile_enable", 1 << classes[dominant])
    ms_per_step = timed_steps(eng.step, stream, args.steps)
    dms, dn, dwork = ctypes.c_double(), ctypes.c_int64(), ctypes.c_double()
    bh.call("bh_profile_read", classes[dominant], ctypes.byref(dms), ctypes.byref(dn), ctypes.byref(dwork))
    bh.call("bh_profile_enable", 0)
    bh.call("bh_profile_sample", 1)
    avg_launch_ms = dms.value / max(1, dn.value)
    work_per_launch = dwork.value / max(1, dn.value)
    achieved = work_per_launch / (avg_launch_ms * 1e-3) / 1e12
    log(f"timed {args.steps} steps: {ms_per_step:.3f} ms/step; {dominant}: {dn.value} launches, "
        f"{avg_launch_ms * 1e3:.1f} us avg, {achieved:.1f} TFLOP/s")
    got = eng.output()
    gf = (got.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    output_stats = {"mean": float(gf.mean()), "std": float(gf.std()), "absmax": float(np.abs(gf).max()),
                    "finite": bool(np.all(np.isfinite(gf)))}

    # the same steps with no event inside a step, and the reference's synchronised median
    plain_ms = timed_steps(eng.step, stream, args.steps)
    median_ms = synced_median(eng.step, stream, max(5, min(args.steps, 20)))
    log(f"profiler off: {plain_ms:.3f} ms/step; synchronised median {median_ms:.3f} ms")

    # the engine's other row schedule: the two CFG rows on two streams (bh_dit_set_rows)
    split_ms, split_equal = None, None
    if wl.batch >= 2 and not args.headline_only:
        bh.call("bh_dit_set_rows", eng.handle, bh.ROWS_SPLIT)
        with torch.cuda.stream(stream):
            eng.step()
        split_ms = timed_steps(eng.step, stream, args.steps)
        split_equal = bool(np.array_equal(eng.output(), got))
        bh.call("bh_dit_set_rows", eng.handle, bh.ROWS_JOINED)
        log(f"rows split over two streams: {split_ms:.3f} ms/step, output identical: {split_equal}")

    step_tflops = flops["total"] / (ms_per_step * 1e-3) / 1e12
    line = {
        "metric": METRIC,
        "value": round(ms_per_step, 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": round(ms_per_step / REFERENCE_5090_MS, 4) if args.resolution == 1024 else None,
        "vs_baseline_basis": "value / 97.85 ms, the reference's published dit-step at this config "
                             "on an RTX 5090 (eval/cells/BG-1/reference.json:28); lower is better",
        "dtype": "bf16",
        "data": "synthetic: seeded N(0,0.02) bf16 weights, N(0,1) latent and caption, timestep 500",
        "config": {"workload": f"PixArt-Sigma dit-step {args.resolution}px, batch {wl.batch} (CFG), "
                               f"caption {wl.caption_len}, 28 blocks",
                   "resolution": args.resolution, "latent": [wl.batch, 4, hw, hw],
                   "tokens": wl.tokens, "batch": wl.batch, "caption_len": wl.caption_len,
                   "layers": wl.cfg["num_layers"], "engine": "bh_dit_forward (fused plan)"},
        "timing": {"ms_per_step_events": round(ms_per_step, 4),
                   "ms_per_step_profiler_off": round(plain_ms, 4),
                   "sync_median_ms": round(median_ms, 4),
                   "ms_per_step_rows_split": None if split_ms is None else round(split_ms, 4),
                   "rows_split_output_identical": split_equal,
                   "basis": "value: K back-to-back steps between HIP events on the engine's stream, "
                            "with HIP events also around one launch of the dominant kernel per step "
                            f"(every {sample_every}th launch, so the sampled layer moves by one each "
                            "step: the roofline's live measurement); profiler_off: the same with no "
                            "event inside a step; sync_median: the reference's method, each step timed "
                            "on the host clock from launch to device synchronisation, median; "
                            "rows_split: the same engine with its two CFG rows on two streams "
                            "(BH_DIT_ROWS_SPLIT), profiler off -- not the value, whose per-launch "
                            "roofline needs each launch to run alone"},
        "roofline": {"bound": "mfma", "kernel": dominant,
                     "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "probed_peak": probed["mfma_tflops"],
                     "probed_frac": (round(achieved / probed["mfma_tflops"], 4)
                                     if probed["mfma_tflops"] else None),
                     "traffic": traffic_bytes(dominant, args.resolution),
                     "traffic_basis": "HBM bytes per launch: rocprofv3 FETCH_SIZE (x2.000) + "
                                      "WRITE_SIZE (x1.000), each scaled by a 256 MiB copy; "
                                      "profiles/flash72_self_1024_traffic.md",
                     "avg_launch_us": round(avg_launch_ms * 1e3, 2), "launches": dn.value,
                     "launch_sample": f"1 in {sample_every} launches of the timed region",
                     "flop_per_launch": work_per_launch},
        "step": {"flop": flops["total"], "tflops": round(step_tflops, 2),
                 "mfma_frac": round(step_tflops / PEAK_BF16_TFLOPS, 4),
                 "ceiling_ms": round(flops["total"] / (PEAK_BF16_TFLOPS * 1e12) * 1e3, 3),
                 "probed_frac": (round(step_tflops / probed["mfma_tflops"], 4)
                                 if probed["mfma_tflops"] else None)},
        "probe": probed,
        "memory": {"peak_device_bytes": int(peak_bytes), "weights_bytes": int(weight_bytes),
                   "engine_workspace_bytes": eng.workspace(),
                   "driver_used_bytes": int(driver_used),
                   "basis": "peak_device_bytes: what the runtime asked for (weights + inputs + "
                            "output + the engine's intermediates, all allocated before the first "
                            "forward; forward allocates nothing), as the reference's "
                            "device::peak_allocated_bytes counts it (device.h:31-35); "
                            "driver_used_bytes: the drop in the driver's free memory over the same "
                            "allocations, allocator granularity included"},
        "kernels": breakdown,
        "output_stats": output_stats,
    }
    eng.close()
    if args.headline_only:
        print(json.dumps(line), flush=True)
        return 0

    # the op-by-op plan (the registry drop-in path: one bh_* op per reference op), same steps
    op = Engine(wl, top, blocks, bh.DIT_OPWISE, stream)
    with torch.cuda.stream(stream):
        op.step()
    opwise_ms = timed_steps(op.step, stream, max(3, args.steps // 2))
    line["opwise_ms_per_step"] = round(opwise_ms, 4)
    opwise_out = op.output()
    op.close()
    log(f"op-by-op plan: {opwise_ms:.3f} ms/step")
    line["opwise_equals_fused"] = bool(np.array_equal(opwise_out, got))

    # the other full-step configs on the same device weights: BASELINE configs[2] and [4], and
    # the reference's held-out scoring shapes (768 and 1152 px; caption 300 and 128 --
    # configs/axes.json:10-24)
    others = {}
    for res, cap in ((512, wl.caption_len), (768, wl.caption_len), (1152, wl.caption_len), (1152, 128),
                     (2048, wl.caption_len)):
        if res == args.resolution and cap == wl.caption_len:
            continue
        owl = make_workload(PIXART_SIGMA, batch=wl.batch, latent_hw=HW[res], caption_len=cap,
                            layers=0)
        owl.cfg["num_layers"] = wl.cfg["num_layers"]
        owl.top, owl.blocks = wl.top, wl.blocks
        oe = Engine(owl, top, blocks, bh.DIT_FUSED, stream)
        with torch.cuda.stream(stream):
            oe.step()
        o_ms = timed_steps(oe.step, stream, 5 if res > 1024 else 10)
        of = dit_step_flops(owl.cfg, batch=owl.batch, latent_hw=HW[res], caption_len=owl.caption_len)
        ores = oe.output()
        oe.close()
        fo = (ores.astype(np.uint32) << 16).view(np.float32)
        key = f"{res}px" if cap == wl.caption_len else f"{res}px_cap{cap}"
        others[key] = {"ms_per_step": round(o_ms, 4), "flop": of["total"],
                       "mfma_frac": round(of["total"] / (o_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                       "finite": bool(np.all(np.isfinite(fo)))}
        log(f"{key}: {o_ms:.3f} ms/step")
    # one block at 512px, batch 1, a 120-token caption (block 0's weights)
    cwl = make_workload(PIXART_SIGMA, batch=1, latent_hw=64, caption_len=120, layers=0)
    cwl.cfg["num_layers"] = 1
    ce = Engine(cwl, top, blocks[:1], bh.DIT_FUSED, stream)
    with torch.cuda.stream(stream):
        ce.step()
    c_ms = timed_steps(ce.step, stream, 20)
    c_med = synced_median(ce.step, stream, 20)
    cf = dit_step_flops(cwl.cfg, batch=1, latent_hw=64, caption_len=120)
    cres = ce.output()
    ce.close()
    others["config0_block_512px_b1_cap120"] = {
        "ms_per_step": round(c_ms, 4), "sync_median_ms": round(c_med, 4), "flop": cf["total"],
        "mfma_frac": round(cf["total"] / (c_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
        "finite": bool(np.all(np.isfinite((cres.astype(np.uint32) << 16).view(np.float32))))}
    log(f"configs[0] (one block, 512px, B=1, caption 120): {c_ms:.3f} ms, median {c_med:.3f} ms")
    line["other_configs"] = others
    del top, blocks
    torch.cuda.empty_cache()

    status = 0
    if not args.no_cpu:
        threads = args.cpu_threads or min(16, os.cpu_count() or 1)
        log(f"cpu baseline on {threads} threads: the full {args.resolution}px step")
        want, secs = stock_step(wl, threads)
        log(f"cpu baseline: one full dit-step in {secs:.2f} s")
        line["cpu_baseline"] = {
            "value": round(secs * 1e3, 1), "unit": "ms", "cores": threads, "kind": "port",
            "sample": (f"one whole dit-step of the stock oracle (oracle/stock.cpp, the reference's "
                       f"stock numerics) at the same {args.resolution}px B={wl.batch} workload and "
                       f"seeds, {threads} threads, not extrapolated")}
        line["parity"] = parity(got, want)
        log(f"parity vs the stock oracle: {json.dumps(line['parity'])}")
        if not line["parity"]["pass"]:
            status = 1
        # BASELINE configs[0] (one block, 512px, batch 1, caption 120) and configs[2] (the full
        # 512px step), timed on the same host
        cpu_cfg = {}
        c0 = make_workload(PIXART_SIGMA, batch=1, latent_hw=64, caption_len=120, layers=1)
        _, s0 = stock_step(c0, threads)
        cpu_cfg["config0_block_512px_b1_cap120_ms"] = round(s0 * 1e3, 1)
        if args.resolution != 512:
            c2 = make_workload(PIXART_SIGMA, batch=2, latent_hw=64, caption_len=wl.caption_len)
            _, s2 = stock_step(c2, threads)
            cpu_cfg["config2_step_512px_ms"] = round(s2 * 1e3, 1)
        line["cpu_baseline"]["other_configs"] = cpu_cfg
        log(f"cpu baseline, other configs: {cpu_cfg}")
        # the reference's own stock path (oracle/_ref, built from its sources; single-threaded as
        # the reference is), on configs[0] only: its full step would take many minutes
        ref = reference_stock_block(c0)
        if ref is not None:
            line["cpu_baseline"]["reference_single_thread"] = ref
            log(f"cpu baseline, the reference's own stock on configs[0]: {json.dumps(ref)}")
    print(json.dumps(line), flush=True)
    return status


if __name__ == "__main__":
    sys.exit(main())
