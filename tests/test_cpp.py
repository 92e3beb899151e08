"""The C++ tests of the qwen3:: layer (tests/cpp/), built by build(): CPU
contract tests here, GPU op tests under the gpu marker.  A GPU test may print
PARITY lines (JSON: case, elements, failures, ulp histogram); they go to the
parity report with the Python tests' comparisons."""
import json
import os
import subprocess

import pytest

import gpu_util

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(REPO, "tests", "cpp", "build")
CPU_TESTS = ["core_metadata_test", "tensor_view_test", "buffer_cpu_test", "tensor_cpu_test", "ops_validation_cpu_test",
             "io_cpu_test", "io_contract_cpu_test", "copy_crew_cpu_test",
             "sample_finish_cpu_test", "launch_limits_cpu_test", "dispatch_cpu_test", "row_crew_cpu_test",
             "model_config_cpu_test"]
GPU_TESTS = ["buffer_gpu_test", "ops_gpu_test", "fused_gpu_test", "chain_oracle_gpu_test", "kv_cache_gpu_test",
             "sampling_gpu_test", "io_gpu_test", "decode_alloc_gpu_test"]


def _run(name, env=None, timeout=120):
    exe = os.path.join(BIN, name)
    if not os.path.exists(exe):
        pytest.fail(f"{exe} is not built; run __graft_entry__.build()")
    proc = subprocess.run([exe], capture_output=True, text=True, timeout=timeout, env=env)
    for line in proc.stdout.splitlines():
        if line.startswith("PARITY "):
            gpu_util.record(json.loads(line[len("PARITY "):]))
    assert proc.returncode == 0, f"{name} failed ({proc.returncode}):\n{proc.stdout}\n{proc.stderr}"
    assert "passed" in proc.stdout


@pytest.mark.parametrize("name", CPU_TESTS)
def test_cpp_cpu(name):
    _run(name)


@pytest.mark.gpu
@pytest.mark.parametrize("name", GPU_TESTS)
def test_cpp_gpu(name):
    _run(name, timeout=300)


@pytest.mark.gpu
def test_cpp_gpu_block_cache_off():
    """Buffer with the small-block cache turned off (QWEN3_DEVICE_BLOCK_CACHE=0): every small block goes through
    hipMalloc and hipFree, as the reference's Buffer does."""
    _run("buffer_gpu_test", env=dict(os.environ, QWEN3_DEVICE_BLOCK_CACHE="0"), timeout=300)
