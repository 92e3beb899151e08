"""The host-side C++ tests rebuilt with AddressSanitizer +
UndefinedBehaviorSanitizer, and the loader's copy crew with ThreadSanitizer
(g++, host code only; CPU only)."""
import glob
import os
import shutil
import subprocess
import tempfile

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

def test_cpp_cpu_under_sanitizers():
    """Core tensor layer + host tests rebuilt with -fsanitize=address,undefined."""
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    core = sorted(glob.glob(os.path.join(REPO, "qwen3-runtime-byyourself_amd", "csrc", "core", "*.cpp")))
    inc = [f"-I{os.path.join(REPO, 'include')}", "-I/opt/rocm/include", f"-I{os.path.join(REPO, 'oracle')}",
           f"-I{os.path.join(REPO, 'tests', 'cpp')}"]
    flags = ["-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-omit-frame-pointer",
             "-fno-sanitize-recover=undefined", "-D__HIP_PLATFORM_AMD__"]
    libs = [os.path.join(REPO, "oracle", "build", "libq3k_oracle.so"), "-L/opt/rocm/lib", "-lamdhip64",
            "-Wl,-rpath,/opt/rocm/lib", "-Wl,-rpath," + os.path.join(REPO, "oracle", "build"), "-pthread"]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0", UBSAN_OPTIONS="print_stacktrace=1")
    with tempfile.TemporaryDirectory() as tmp:
        for name in ["core_metadata_test", "tensor_view_test", "buffer_cpu_test", "tensor_cpu_test", "copy_crew_cpu_test"]:
            exe = os.path.join(tmp, name)
            src = os.path.join(REPO, "tests", "cpp", name + ".cpp")
            build = subprocess.run(["g++", *flags, *inc, src, *core, "-o", exe, *libs], capture_output=True, text=True)
            assert build.returncode == 0, build.stderr[-3000:]
            proc = subprocess.run([exe], capture_output=True, text=True, timeout=120, env=env)
            assert proc.returncode == 0, f"{name} under sanitizers:\n{proc.stdout}\n{proc.stderr[-3000:]}"


def test_host_runtime_tests_under_sanitizers():
    """The safetensors contract and IO tests, the sampler's host finish and rules, and the launch-limit decisions,
    with every host source of the runtime (core, ops, model, generation, io) rebuilt with
    -fsanitize=address,undefined; the kernels come from the built libq3k.so (nothing here launches one)."""
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    lib_dir = os.path.join(REPO, "qwen3-runtime-byyourself_amd", "lib")
    if not os.path.exists(os.path.join(lib_dir, "libq3k.so")):
        pytest.skip("libq3k.so is not built")
    host = []
    for d in ("core", "ops", "model", "generation", "io"):
        host += sorted(glob.glob(os.path.join(REPO, "qwen3-runtime-byyourself_amd", "csrc", d, "*.cpp")))
    inc = [f"-I{os.path.join(REPO, 'include')}", "-I/opt/rocm/include", f"-I{os.path.join(REPO, 'oracle')}",
           f"-I{os.path.join(REPO, 'tests', 'cpp')}"]
    flags = ["-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-omit-frame-pointer",
             "-fno-sanitize-recover=undefined", "-D__HIP_PLATFORM_AMD__"]
    libs = [os.path.join(REPO, "oracle", "build", "libq3k_oracle.so"), f"-L{lib_dir}", "-lq3k", "-L/opt/rocm/lib",
            "-lamdhip64", "-Wl,-rpath," + lib_dir, "-Wl,-rpath,/opt/rocm/lib",
            "-Wl,-rpath," + os.path.join(REPO, "oracle", "build"), "-pthread"]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0", UBSAN_OPTIONS="print_stacktrace=1",
               Q3K_GOLDEN_DIR=os.path.join(REPO, "tests", "golden"))
    with tempfile.TemporaryDirectory() as tmp:
        objs = []
        for src in host:
            obj = os.path.join(tmp, os.path.relpath(src, REPO).replace(os.sep, "_") + ".o")
            build = subprocess.run(["g++", *flags, *inc, "-c", src, "-o", obj], capture_output=True, text=True)
            assert build.returncode == 0, build.stderr[-3000:]
            objs.append(obj)
        for name in ["io_contract_cpu_test", "io_cpu_test", "sample_finish_cpu_test", "launch_limits_cpu_test"]:
            exe = os.path.join(tmp, name)
            src = os.path.join(REPO, "tests", "cpp", name + ".cpp")
            build = subprocess.run(["g++", *flags, *inc, src, *objs, "-o", exe, *libs], capture_output=True, text=True)
            assert build.returncode == 0, build.stderr[-3000:]
            proc = subprocess.run([exe], capture_output=True, text=True, timeout=300, env=env)
            assert proc.returncode == 0, f"{name} under sanitizers:\n{proc.stdout}\n{proc.stderr[-3000:]}"


@pytest.mark.parametrize("name", ["copy_crew_cpu_test", "row_crew_cpu_test"])
def test_crews_under_thread_sanitizer(name):
    """The staging copy crew (helper threads publishing and finishing copies through atomics) and the sampler's row
    crew (helpers woken per run by a condition variable) under -fsanitize=thread."""
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    inc = [f"-I{os.path.join(REPO, 'include')}", f"-I{os.path.join(REPO, 'oracle')}",
           f"-I{os.path.join(REPO, 'tests', 'cpp')}"]
    libs = [os.path.join(REPO, "oracle", "build", "libq3k_oracle.so"),
            "-Wl,-rpath," + os.path.join(REPO, "oracle", "build"), "-pthread"]
    with tempfile.TemporaryDirectory() as tmp:
        exe = os.path.join(tmp, name + "_tsan")
        src = os.path.join(REPO, "tests", "cpp", name + ".cpp")
        build = subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-fsanitize=thread", *inc, src, "-o", exe, *libs],
                               capture_output=True, text=True)
        assert build.returncode == 0, build.stderr[-3000:]
        env = dict(os.environ, TSAN_OPTIONS="halt_on_error=1")
        proc = subprocess.run([exe], capture_output=True, text=True, timeout=300, env=env)
        assert proc.returncode == 0, f"{name} under ThreadSanitizer:\n{proc.stdout}\n{proc.stderr[-3000:]}"
