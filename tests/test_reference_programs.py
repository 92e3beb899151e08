"""The reference's own test programs, run against this library.

`oracle/reference_programs.mk` compiles them from the reference's sources
(its tests/unit programs for every component this library provides, and the
two tests/integration programs that need only a safetensors file) against
this repository's headers and libraries, with only the CUDA-runtime spellings
changed (`oracle/cuda_to_hip.sed`), into `oracle/_ref/`.  A program passes
when it exits 0, as under the reference's own build.  CPU programs run here,
GPU programs under the gpu marker; the two safetensors programs read a
Qwen3-0.6B-shaped file written by the test (the embedding left as a hole)."""
import json
import os
import struct
import subprocess

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(REPO, "oracle", "_ref")
CONFIGS = os.path.join(REPO, "tests", "golden", "model_config")

CPU_PROGRAMS = ["core_metadata_test", "tensor_view_test", "tensor_cpu_test", "buffer_cpu_test", "mapped_file_test",
                "safetensors_file_test", "safetensors_checkpoint_test"]
GPU_PROGRAMS = ["buffer_cuda_test", "tensor_cuda_test", "embedding_cuda_test", "rms_norm_cuda_test", "rope_cuda_test",
                "elementwise_cuda_test", "kv_cache_cuda_test", "gqa_attention_cuda_test", "argmax_cuda_test",
                "sampler_cuda_test"]


def _run(name, args=(), timeout=120):
    exe = os.path.join(BIN, name)
    if not os.path.exists(exe):
        # build() compiles these only where the reference's sources are present
        pytest.skip(f"{exe} is not built: this tree was built without the reference's sources")
    print(f"running {name} {' '.join(args)}", flush=True)
    proc = subprocess.run([exe, *args], capture_output=True, text=True, timeout=timeout)
    assert proc.returncode == 0, f"{name} failed ({proc.returncode}):\n{proc.stdout}\n{proc.stderr}"
    return proc.stdout


@pytest.mark.parametrize("name", CPU_PROGRAMS)
def test_reference_program_cpu(name):
    _run(name)


def test_reference_model_config_program():
    out = _run("model_config_test", [os.path.join(CONFIGS, "qwen3_0_6b.json"), os.path.join(CONFIGS, "qwen3_8b.json")])
    assert "8B: layers=36, hidden=4096, tied=0" in out


@pytest.mark.gpu
@pytest.mark.parametrize("name", GPU_PROGRAMS)
def test_reference_program_gpu(name):
    _run(name, timeout=300)


def _qwen3_0_6b_shaped_file(path):
    """model.safetensors with the tensors the two integration programs read, at Qwen3-0.6B shapes: the small ones
    filled with seeded bytes, the [151936, 1024] embedding left as a hole at the end of the file."""
    rng = np.random.default_rng(7)
    small = [("model.layers.0.self_attn.q_proj.weight", [2048, 1024]),
             ("model.layers.0.self_attn.k_proj.weight", [1024, 1024]),
             ("model.layers.0.mlp.gate_proj.weight", [3072, 1024]),
             ("model.layers.0.mlp.up_proj.weight", [3072, 1024]),
             ("model.norm.weight", [1024])]
    header, offset, blobs = {}, 0, []
    for name, shape in small:
        n = 2 * int(np.prod(shape))
        header[name] = {"dtype": "BF16", "shape": shape, "data_offsets": [offset, offset + n]}
        blobs.append(rng.integers(0, 256, n, dtype=np.uint8).tobytes())
        offset += n
    emb = 2 * 151936 * 1024
    header["model.embed_tokens.weight"] = {"dtype": "BF16", "shape": [151936, 1024],
                                           "data_offsets": [offset, offset + emb]}
    text = json.dumps(header).encode()
    text += b" " * (-len(text) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(text)) + text)
        for b in blobs:
            f.write(b)
        f.truncate(8 + len(text) + offset + emb)
    return path


def test_reference_safetensors_metadata_program(tmp_path):
    out = _run("safetensors_metadata_smoke", [_qwen3_0_6b_shaped_file(str(tmp_path / "model.safetensors"))])
    assert "Tensor count: 6" in out


@pytest.mark.gpu
def test_reference_safetensors_loader_program(tmp_path):
    _run("safetensors_loader_smoke", [_qwen3_0_6b_shaped_file(str(tmp_path / "model.safetensors"))], timeout=300)
