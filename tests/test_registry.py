"""The registry drop-in from the reference's side, on the CPU: the reference runtime's own
registry and selection code (/root/reference/include/burnisher/registry.h:34-100,
src/core/impl_select.cpp:57-67, src/models/weights.cpp:329-362) linked with this repository's
adapter (burnisher_amd/registry/ops_hip.cpp). Registration touches no device, so this runs on a
host without a GPU, as the reference's own CUDA registration test does (tests/test_ops.cpp:
310-339)."""
import subprocess

import pytest

import oracle


@pytest.fixture(scope="module")
def driver():
    path = oracle.registry_main()
    if path is None:
        pytest.skip("oracle/_ref/registry_main was not built (it needs /root/reference at build time)")
    return path


def test_every_op_registers_and_resolves_to_hip_gfx950(driver):
    proc = subprocess.run([str(driver), "check"], capture_output=True, text=True, timeout=120)
    assert proc.returncode == 0, proc.stderr + proc.stdout
    assert '"failures": 0' in proc.stdout and '"ops": 15' in proc.stdout


def test_driver_refuses_bad_usage(driver):
    proc = subprocess.run([str(driver), "nonsense"], capture_output=True, text=True, timeout=60)
    assert proc.returncode == 2 and "usage" in proc.stderr
