"""Helpers for the GPU parity tests: guarded device buffers and the oracle
comparison with a readable failure message."""
import json
import os
import sys

import numpy as np

GUARD = 4096
GUARD_BYTE = 0xA5

_REPORT = []


class Guarded:
    """A device buffer with GUARD bytes of a fixed pattern on both sides.

    ``offset`` shifts the data start by that many bytes to exercise the
    kernels' unaligned paths."""

    def __init__(self, hip, arr=None, nbytes=None, offset=0):
        self.hip = hip
        self.n = int(arr.nbytes if arr is not None else nbytes)
        self.offset = offset
        self.buf = hip.DeviceBuffer(self.n + 2 * GUARD + offset)
        self.buf.fill_bytes(GUARD_BYTE)
        self.ptr = self.buf.ptr + GUARD + offset
        if arr is not None:
            self.buf.upload(np.ascontiguousarray(arr), GUARD + offset)

    def get(self, dtype, shape):
        return self.buf.download(dtype, shape, GUARD + self.offset)

    def guards_intact(self):
        head = self.buf.download(np.uint8, (GUARD + self.offset,), 0)
        tail = self.buf.download(np.uint8, (GUARD,), GUARD + self.offset + self.n)
        return bool(np.all(head == GUARD_BYTE) and np.all(tail == GUARD_BYTE))

    def free(self):
        self.buf.free()


def announce(name):
    print(f"[gpu case] {name}", file=sys.stderr, flush=True)


def check_band(oracle, name, got, prim, lo, hi, max_fail=0):
    st = oracle.compare(got, prim, lo, hi)
    st["case"] = name
    _REPORT.append(st)
    if st["fail"] > max_fail:
        i = st["first_fail"]
        g, p = np.ravel(got)[i], np.ravel(prim)[i]
        l = np.ravel(lo)[i] if lo is not None else p
        h = np.ravel(hi)[i] if hi is not None else p
        raise AssertionError(f"{name}: {st['fail']} of {st['n']} elements outside the 1-ulp band; first at {i}: "
                             f"got 0x{g:04x} primary 0x{p:04x} band [0x{l:04x}, 0x{h:04x}] stats {st}")
    return st


def check_exact(name, got, want):
    got, want = np.ravel(got), np.ravel(want)
    diff = got != want
    _REPORT.append({"case": name, "n": int(got.size), "fail": int(diff.sum()), "exact": True})
    if diff.any():
        i = int(np.argmax(diff))
        raise AssertionError(f"{name}: {int(diff.sum())} of {got.size} differ; first at {i}: "
                             f"got 0x{int(got[i]):04x} want 0x{int(want[i]):04x}")


def record(stats):
    """Add a comparison made elsewhere (a C++ test's PARITY line) to the report."""
    _REPORT.append(stats)


def write_report():
    path = os.environ.get("Q3K_PARITY_REPORT")
    if path and _REPORT:
        os.makedirs(os.path.dirname(path) or ".", exist_ok=True)
        with open(path, "w") as f:
            json.dump(_REPORT, f, indent=1)
