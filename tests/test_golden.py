"""The oracle reproduces the committed golden fixtures bit for bit (CPU), and
the generator that wrote them regenerates identical arrays; the GPU kernels
are checked against the same fixtures in test_gpu_golden (gpu marker)."""
import glob
import importlib.util
import os

import numpy as np
import pytest

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with np.load(os.path.join(HERE, name + ".npz"), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def test_fixture_set_is_complete():
    names = {os.path.basename(p)[:-4] for p in glob.glob(os.path.join(HERE, "*.npz"))}
    assert names == {"kat_rms_norm_2x3x1024", "kat_rms_norm_2x3x4x128", "kat_rope", "kat_elementwise",
                     "kat_embedding", "config1_rms_norm"}


def test_oracle_reproduces_fixtures(oracle):
    spec = importlib.util.spec_from_file_location("make_golden", os.path.join(HERE, "make_golden.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    fresh = mod.fixtures(oracle)
    for name, arrays in fresh.items():
        stored = load(name)
        assert set(stored) == set(arrays), name
        for key, value in arrays.items():
            assert np.array_equal(stored[key], value), f"{name}.{key} drifted"


def test_config1_fixture_matches_baseline_spec(synth, configs):
    f = load("config1_rms_norm")
    assert f["x"].shape == (16, 1024) and f["w"].shape == (1024,)
    x = synth.bf16_to_f32(f["x"])
    w = synth.bf16_to_f32(f["w"])
    assert abs(float(x.mean())) < 0.05 and 0.9 < float(x.std()) < 1.1
    assert abs(float(w.mean()) - 1.0) < 0.01 and 0.08 < float(w.std()) < 0.12


@pytest.mark.gpu
def test_gpu_golden(q3k, hip, oracle):
    from gpu_util import Guarded, check_band, check_exact

    for name in ("kat_rms_norm_2x3x1024", "kat_rms_norm_2x3x4x128", "config1_rms_norm"):
        f = load(name)
        X, W, Y = Guarded(hip, f["x"]), Guarded(hip, f["w"]), Guarded(hip, nbytes=f["x"].nbytes)
        q3k.rms_norm(X, W, Y, f["x"].size // f["w"].size, f["w"].size, 1e-6)
        hip.synchronize()
        check_band(oracle, "golden " + name, Y.get(np.uint16, f["x"].shape), f["y"], f["lo"], f["hi"])
    f = load("kat_elementwise")
    A, B = Guarded(hip, f["residual"]), Guarded(hip, f["delta"])
    q3k.add_inplace(A, B, f["residual"].size)
    G, U, O = Guarded(hip, f["gate"]), Guarded(hip, f["up"]), Guarded(hip, nbytes=f["gate"].nbytes)
    q3k.silu_mul(G, U, O, f["gate"].size)
    hip.synchronize()
    check_exact("golden add", A.get(np.uint16, f["residual"].shape), f["add_out"])
    check_band(oracle, "golden silu", O.get(np.uint16, f["gate"].shape), f["silu_out"], f["silu_lo"], f["silu_hi"])
    f = load("kat_embedding")
    I, T, O = Guarded(hip, f["ids"]), Guarded(hip, f["table"]), Guarded(hip, nbytes=f["out"].nbytes)
    q3k.embedding(I, f["ids"].size, T, f["table"].shape[0], f["table"].shape[1], O)
    hip.synchronize()
    check_exact("golden embedding", O.get(np.uint16, f["out"].shape), f["out"])
    f = load("kat_rope")
    for key, heads in (("q", 2), ("k", 1)):
        X, C = Guarded(hip, f[key]), Guarded(hip, f["cache"])
        q3k.rope(X, 1, 3, heads, 8, C, f["cache"].shape[0], 5)
        hip.synchronize()
        check_band(oracle, "golden rope " + key, X.get(np.uint16, f[key].shape), f[key + "_out"], f[key + "_lo"],
                   f[key + "_hi"])
