"""q3k_argmax_bf16_noalloc, the argmax entry point that allocates nothing (its
slice results live in a fixed device array held by the library), against
q3k_argmax_bf16 with a caller workspace and against the oracle, bit for bit:
several calls in a row on one GPU, each after the first with a smaller input
(sliced rows, one long row, then enough rows to skip slicing), plus the
ties-across-slices, NaN and -0 rows of the workspace form's tests.  The
device's free memory is the same before and after each call."""
import numpy as np
import pytest

from gpu_util import Guarded, announce, check_exact

pytestmark = pytest.mark.gpu

# rows, columns: the first call is the largest; later ones are smaller
CALLS = [(64, 151936), (9, 40000), (1, 151936), (2, 8192), (600, 2048)]


def _logits(synth, i, rows, N):
    x = synth.normal_bf16(300 + i, N, (rows, N), std=4.0)
    big = synth.f32_to_bf16(np.array([70.0], np.float32))[0]
    x[0, N // 2] = x[0, N - 1] = big           # the maximum tied across slices: the first index wins
    if rows > 3:
        x[1, :] = 0x7fc0                       # NaN counts as -inf: index 0
        x[2, :] = 0x8000                       # -0 everywhere but one +0: -0 == +0, index 0
        x[2, N - 1] = 0
    return x


def test_noalloc_argmax_matches_workspace_form(q3k, hip, oracle, synth):
    for i, (rows, N) in enumerate(CALLS):
        name = f"argmax noalloc call {i}: rows={rows} N={N} (workspace {q3k.argmax_workspace_bytes(rows, N)} B)"
        announce(name)
        x = _logits(synth, i, rows, N)
        X = Guarded(hip, x)
        want = Guarded(hip, nbytes=rows * 4)
        got = Guarded(hip, nbytes=rows * 4)
        ws = q3k.argmax_workspace_bytes(rows, N)
        W = Guarded(hip, nbytes=ws) if ws else None
        q3k.argmax(X, want, rows, N, N, workspace=W, workspace_bytes=ws)
        hip.synchronize()
        free_before, _ = hip.mem_info()
        q3k.argmax_noalloc(X, got, rows, N, N)
        hip.synchronize()
        free_after, _ = hip.mem_info()
        assert free_after == free_before, f"{name}: device free memory {free_before} -> {free_after}"
        assert X.guards_intact() and got.guards_intact() and want.guards_intact()
        g = got.get(np.int32, (rows,))
        check_exact(name + " vs workspace form", g.view(np.uint32), want.get(np.int32, (rows,)).view(np.uint32))
        check_exact(name + " vs oracle", g.view(np.uint32), oracle.argmax(x).view(np.uint32))
        for b in (X, want, got, W):
            if b is not None:
                b.free()


def test_noalloc_argmax_argument_errors(q3k, hip):
    """The workspace form's checks, with the same errors."""
    X = hip.DeviceBuffer(64)
    O = hip.DeviceBuffer(64)
    with pytest.raises(ValueError):
        q3k.argmax_noalloc(X, O, -1, 8, 8)
    with pytest.raises(ValueError):
        q3k.argmax_noalloc(X, O, 1, 8, 9)
    with pytest.raises(ValueError):
        q3k.argmax_noalloc(None, O, 1, 8, 8)
    q3k.argmax_noalloc(None, None, 0, 8, 8)   # no rows: nothing to do
    X.free()
    O.free()


def test_noalloc_argmax_captured_in_graph(q3k, hip, oracle, synth):
    """The entry point captured into a HIP graph, for callers that record their decode step: the first call on
    the GPU (made eagerly, before the capture) resolves the array's device address; the captured call then
    replays three times, each replay preceded by an eager call on other logits that overwrites the same array,
    and every replay's result equals the oracle's."""
    rows, N = 9, 40000
    rows2, N2 = 2, 151936
    assert q3k.argmax_workspace_bytes(rows, N) > 0 and q3k.argmax_workspace_bytes(rows2, N2) > 0, "sliced shapes"
    announce(f"argmax noalloc in a graph: rows={rows} N={N}, eager rows={rows2} N={N2} between replays")
    x, x2 = _logits(synth, 10, rows, N), _logits(synth, 11, rows2, N2)
    want, want2 = oracle.argmax(x).view(np.uint32), oracle.argmax(x2).view(np.uint32)
    X, X2 = hip.DeviceBuffer.from_array(x), hip.DeviceBuffer.from_array(x2)
    O, O2 = hip.DeviceBuffer(rows * 4), hip.DeviceBuffer(rows2 * 4)
    stream = hip.Stream()
    q3k.argmax_noalloc(X, O, rows, N, N, stream)   # the first call on this GPU: before any capture
    stream.synchronize()
    graph = hip.Graph(stream, lambda: q3k.argmax_noalloc(X, O, rows, N, N, stream))
    try:
        for replay in range(3):
            O.fill_bytes(0xFF)
            q3k.argmax_noalloc(X2, O2, rows2, N2, N2, stream)
            stream.synchronize()
            check_exact(f"eager call before replay {replay}", O2.download(np.int32, (rows2,)).view(np.uint32), want2)
            graph.launch(stream)
            stream.synchronize()
            check_exact(f"graph replay {replay}", O.download(np.int32, (rows,)).view(np.uint32), want)
    finally:
        graph.destroy()
        for b in (X, X2, O, O2):
            b.free()
        stream.destroy()
