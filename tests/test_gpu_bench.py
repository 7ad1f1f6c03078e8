"""bench.py's stage modes (--t5, --vae, --denoise) run end to end on the GPU and print one JSON
line with the contract's fields. The default dit-step mode is what the round's bench run times;
these modes are only run by hand, so a test keeps them working. Each runs bench.main() in this
process with the CPU baseline off and the smallest step counts."""
import json
import sys

import pytest

pytestmark = pytest.mark.gpu

CONTRACT = ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
            "dtype", "data", "config", "output_stats")


def run_bench(capsys, argv):
    import bench
    old = sys.argv
    sys.argv = ["bench.py"] + argv
    try:
        rc = bench.main()
    finally:
        sys.argv = old
    out = capsys.readouterr().out.strip().splitlines()
    assert rc == 0, f"bench.py {' '.join(argv)} exited {rc}"
    line = json.loads(out[-1])
    for key in CONTRACT:
        assert key in line, f"bench.py {' '.join(argv)}: no '{key}' in its line"
    assert line["value"] > 0 and line["output_stats"]["finite"]
    assert line["output_stats"]["std"] > 0
    return line


@pytest.mark.parametrize("argv", [
    ["--t5", "--steps", "1", "--warmup", "1", "--no-cpu"],
    ["--vae", "--resolution", "512", "--steps", "1", "--warmup", "1", "--no-cpu"],
    ["--denoise", "2", "--resolution", "512", "--steps", "1", "--warmup", "1", "--no-cpu"],
], ids=["t5", "vae_512px", "denoise_2_steps_512px"])
def test_bench_stage_modes(hip, capsys, argv):
    print(f"bench.py {' '.join(argv)}", file=sys.stderr, flush=True)
    line = run_bench(capsys, argv)
    assert line["unit"] == "ms" and line["n_gpus"] == 1
    if "--denoise" not in argv:   # the stage kernels' MFMA class against the dense bf16 peak
        assert 0 < line["roofline"]["frac"] < 1
