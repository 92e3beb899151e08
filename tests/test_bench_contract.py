"""bench.py's command-line contract on the CPU: one GPU only, so --gpus N > 1
exits with a message and a non-zero status before touching a device."""
import os
import subprocess
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_bench_refuses_more_than_one_gpu():
    proc = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"], capture_output=True,
                          text=True, timeout=120, cwd=REPO)
    assert proc.returncode != 0
    assert "one GPU only" in proc.stdout + proc.stderr
    assert proc.stdout.strip() == "" or not proc.stdout.lstrip().startswith("{"), "no JSON line for --gpus 2"


def test_traffic_provenance_parses_the_committed_profile():
    """roofline.traffic comes with the profile's file, commit and kernel-source hash, and a stale flag that
    compares that hash with the kernels in the tree."""
    import bench
    value, source = bench.read_traffic("silu_mul")
    assert isinstance(value, int) and value > 0
    assert source["file"] == bench.TRAFFIC_PROFILE
    assert source["commit"] and all(c in "0123456789abcdef" for c in source["commit"])
    assert len(source["kernel_sources"]) == 16 and len(source["current_kernel_sources"]) == 16
    assert source["stale"] == (source["kernel_sources"] != source["current_kernel_sources"])


def test_kernel_source_hash_follows_code_not_comments(tmp_path):
    """The provenance hash changes with the kernels' code and not with their comments or layout, so a comment
    edit does not mark a measured traffic figure stale while a code edit does."""
    import bench
    code = ('// header\n#include "x.hpp"\n__global__ void k(float *p) { p[0] = 1.0f / 2.0f; } /* tail */\n'
            'const char *s = "a // kept";\n')
    (tmp_path / "a.hip").write_text(code)
    (tmp_path / "notes.txt").write_text("not a kernel source")
    base = bench.kernel_source_hash(str(tmp_path))
    assert len(base) == 16 and base == bench.kernel_source_hash(str(tmp_path))
    (tmp_path / "a.hip").write_text("/* new */ " + code.replace("{ p", "{\n    p").replace("// header", "// other"))
    assert bench.kernel_source_hash(str(tmp_path)) == base, "comment and layout edits changed the hash"
    for edit in (code.replace("2.0f", "3.0f"), code.replace('"a // kept"', '"a // kept!"'), code + "int y;\n"):
        (tmp_path / "a.hip").write_text(edit)
        assert bench.kernel_source_hash(str(tmp_path)) != base, "a code edit left the hash unchanged"
    (tmp_path / "a.hip").write_text(code)
    (tmp_path / "b.hpp").write_text("int z;\n")
    assert bench.kernel_source_hash(str(tmp_path)) != base, "a new header left the hash unchanged"
