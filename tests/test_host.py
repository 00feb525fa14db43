"""The C++ host interface (sharpinference_amd/host/si_host.hpp) through its
own test runner, tests/host/test_host (built by tests/host/Makefile).

The CPU group covers the instruction contract, the registry and the program
binding rules, and that the executor fails loudly without a device; the GPU
group runs quantized mat-vec and gather-row programs through the executor
against the oracle (GpuMatVecTests.cs analogues).  The GPU group runs in one
process.
"""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
RUNNER = os.path.join(HERE, "host", "test_host")


def _run(group, timeout):
    proc = subprocess.run([RUNNER, group], capture_output=True, text=True, timeout=timeout)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout[-4000:] + proc.stderr[-2000:]
    assert "0 failed" in proc.stdout


def test_host_contract_registry_and_binding():
    subprocess.run(["make", "-s", "-C", os.path.join(HERE, "host")], check=True)
    _run("cpu", 120)


@pytest.mark.gpu
def test_host_executor_runs_quantized_programs():
    if not os.path.exists(RUNNER):
        pytest.fail(f"{RUNNER} is not built: run make -C tests/host after building the libraries")
    _run("gpu", 300)
