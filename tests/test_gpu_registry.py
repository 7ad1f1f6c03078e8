"""The drop-in, end to end on the GPU: the reference's own `PixArtDiT::forward`
(/root/reference/src/models/pixart_dit.cpp:112-304, compiled from its sources into
oracle/_ref/registry_main together with the repository's registry adapter and HIP device layer)
runs on the MI355X with ImplSelection::from_request("hip-gfx950", Device::CUDA), so every op of
the graph goes through `register_impl` into libburnisher_hip.so, and every intermediate through
the HIP `device::alloc`. Its output must equal, bit for bit, the library's op-by-op engine and its
fused engine on the same seeded workload: the reference graph calls the same ops in the same
order, and fusion moves no rounding point."""
import ctypes
import json
import subprocess

import numpy as np
import pytest

import oracle
from burnisher_amd.workload import PIXART_SIGMA, config_struct, make_workload
from helpers import F32

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def driver():
    path = oracle.registry_main()
    assert path is not None, "oracle/_ref/registry_main was not built (build() builds it beside the reference)"
    return path


def engine_output(wl, mode):
    import torch
    import burnisher_amd as bh
    top, blocks, latent, caption, mask = wl.to_device()
    cfg = config_struct(wl.cfg)
    w, keep = wl.weight_struct(top, blocks)
    h = ctypes.c_void_p()
    bh.call("bh_dit_create", ctypes.byref(cfg), ctypes.byref(w), wl.batch, wl.latent_hw, wl.caption_len,
            mode, ctypes.byref(h))
    try:
        out = torch.zeros((wl.batch, cfg.out_channels, wl.latent_hw, wl.latent_hw), dtype=torch.bfloat16,
                          device="cuda")
        bh.call("bh_dit_forward", h, latent.data_ptr(), wl.timestep, caption.data_ptr(), mask.data_ptr(),
                F32, out.data_ptr(), None)
        torch.cuda.synchronize()
        return out.cpu().view(torch.int16).numpy().view(np.uint16).copy()
    finally:
        bh.lib().bh_dit_destroy(h)


def reference_graph(driver, tmp_path, layers, batch, latent_hw, caption_len, iters=0):
    out = tmp_path / "dit_out.bin"
    print(f"registry_main dit-step {layers} {batch} {latent_hw} {caption_len} iters={iters}", flush=True)
    proc = subprocess.run([str(driver), "dit-step", str(layers), str(batch), str(latent_hw), str(caption_len),
                           str(out), str(iters)], capture_output=True, text=True, timeout=240)
    assert proc.returncode == 0, proc.stderr + proc.stdout
    line = json.loads(proc.stdout.strip().splitlines()[-1])
    print("reference graph through the registry:", json.dumps(line), flush=True)
    got = np.fromfile(out, dtype=np.uint16).reshape(batch, 8, latent_hw, latent_hw)
    return got, line


@pytest.mark.parametrize("layers,batch,latent_hw,caption_len", [
    (1, 1, 64, 120),      # BASELINE configs[0]'s shape
    (2, 2, 64, 300),      # 512px, the CFG batch
], ids=["512px_b1_1block", "512px_b2_2blocks"])
def test_reference_graph_through_registry_equals_engines(driver, tmp_path, hip, layers, batch, latent_hw,
                                                         caption_len):
    got, line = reference_graph(driver, tmp_path, layers, batch, latent_hw, caption_len)
    assert all(v == "hip-gfx950" for k, v in line["effective"].items() if k != "device")
    wl = make_workload(PIXART_SIGMA, batch=batch, latent_hw=latent_hw, caption_len=caption_len, layers=layers)
    opwise = engine_output(wl, 1)
    assert np.array_equal(got, opwise), f"{np.sum(got != opwise)} of {got.size} values differ from the op-wise engine"
    assert np.array_equal(got, engine_output(wl, 0)), "differs from the fused engine"


def engine_median_ms(wl, mode, iters):
    # the reference bench's method (burnisher_main.cpp:451-464): each forward timed on the host
    # clock from launch to device synchronisation, median of `iters` after one warm-up
    import time
    import torch
    import burnisher_amd as bh
    top, blocks, latent, caption, mask = wl.to_device()
    cfg = config_struct(wl.cfg)
    w, keep = wl.weight_struct(top, blocks)
    h = ctypes.c_void_p()
    bh.call("bh_dit_create", ctypes.byref(cfg), ctypes.byref(w), wl.batch, wl.latent_hw, wl.caption_len,
            mode, ctypes.byref(h))
    try:
        out = torch.zeros((wl.batch, cfg.out_channels, wl.latent_hw, wl.latent_hw), dtype=torch.bfloat16,
                          device="cuda")
        ms = []
        for i in range(iters + 1):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            bh.call("bh_dit_forward", h, latent.data_ptr(), wl.timestep, caption.data_ptr(), mask.data_ptr(),
                    F32, out.data_ptr(), None)
            torch.cuda.synchronize()
            if i:
                ms.append((time.perf_counter() - t0) * 1e3)
        return float(np.median(ms))
    finally:
        bh.lib().bh_dit_destroy(h)


def test_reference_graph_1024px_full_depth_equals_engine_and_is_timed(driver, tmp_path, hip):
    # The headline configuration through the reference's own graph and the registry: the output
    # equals the fused engine's, and the driver reports the reference bench's median and peak,
    # printed beside the library's op-by-op and fused engines timed the same way in this process.
    got, line = reference_graph(driver, tmp_path, 28, 2, 128, 300, iters=10)
    wl = make_workload(PIXART_SIGMA, batch=2, latent_hw=128, caption_len=300)
    assert np.array_equal(got, engine_output(wl, 0))
    assert line["median_ms"] > 0 and line["peak_vram_bytes"] >= line["weights_bytes"] > 1_000_000_000
    opwise, fused = engine_median_ms(wl, 1, 10), engine_median_ms(wl, 0, 10)
    print("registry path vs engines (host-clock median, ms):", json.dumps({
        "registry_ms_per_step": line["median_ms"], "opwise_ms_per_step": round(opwise, 4),
        "fused_ms_per_step": round(fused, 4), "registry_over_opwise": round(line["median_ms"] / opwise, 4),
        "registry_peak_vram_bytes": line["peak_vram_bytes"], "effective": line["effective"]}), flush=True)
