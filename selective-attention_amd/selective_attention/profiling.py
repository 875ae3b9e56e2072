"""Live per-kernel timing of the HIP kernels (HIP events on the launch stream).

    with kernel_timer() as kt:
        ...launches...
    kt.stats  ->  {kernel_name: {"count": n, "total_ms": t, "avg_us": a}}

The events bracket each launch on the stream it runs on, so the durations
are what the device spent between the two records (launch gaps excluded).
"""
from __future__ import annotations

import ctypes
from contextlib import contextmanager

from . import _lib

_MAX = 64


def collect() -> dict:
    lib = _lib.load()
    names = ctypes.create_string_buffer(64 * _MAX)
    tot = (ctypes.c_float * _MAX)()
    cnt = (ctypes.c_int * _MAX)()
    n = lib.sa_profile_collect(names, len(names), tot, cnt, _MAX)
    if n < 0:
        raise RuntimeError("sa_profile_collect failed")
    raw = names.raw.split(b"\0")
    out = {}
    for k in range(min(n, _MAX)):
        name = raw[k].decode()
        out[name] = {"count": int(cnt[k]), "total_ms": float(tot[k]),
                     "avg_us": 1000.0 * float(tot[k]) / max(1, int(cnt[k]))}
    return out


class _Timer:
    stats: dict

    def __init__(self):
        self.stats = {}


@contextmanager
def kernel_timer():
    lib = _lib.load()
    collect()  # drop stale records
    lib.sa_profile_enable(1)
    t = _Timer()
    try:
        yield t
    finally:
        lib.sa_profile_enable(0)
        t.stats = collect()
