"""Per-kernel event timing (sa_profile_enable / sa_profile_collect) used from
several host threads: every launch's record is collected exactly once, with
a finite, non-negative duration, while another thread collects concurrently."""
import threading

import pytest
import torch

from tests.test_ssu import _small


@pytest.mark.gpu
def test_profile_collect_concurrent_with_launches():
    from selective_attention import _lib, profiling
    from selective_attention.ops import SSUFn
    print("profiling: 2 launching threads, 1 collecting thread", flush=True)
    x = {k: (v.cuda() if v is not None else None) for k, v in _small().items()}
    lib = _lib.load()
    profiling.collect()                 # drop stale records
    n_launch, n_threads = 150, 2
    seen, errors = [], []
    done = threading.Event()

    def launcher():
        try:
            s = torch.cuda.Stream()     # default priority
            with torch.cuda.stream(s):
                h = x["h"].clone()
                for _ in range(n_launch):
                    SSUFn.forward(x["u"], x["A"], x["B"], x["C"], x["delta_raw"],
                                  x["delta_bias"], h)
            s.synchronize()
        except Exception as e:          # noqa: BLE001 - reported below
            errors.append(e)

    def collector():
        try:
            while not done.is_set():
                seen.append(profiling.collect())
        except Exception as e:          # noqa: BLE001
            errors.append(e)

    lib.sa_profile_enable(1)
    try:
        ts = [threading.Thread(target=launcher) for _ in range(n_threads)]
        c = threading.Thread(target=collector)
        c.start()
        for t in ts:
            t.start()
        for t in ts:
            t.join()
        done.set()
        c.join()
    finally:
        lib.sa_profile_enable(0)
    torch.cuda.synchronize()
    seen.append(profiling.collect())
    assert not errors, errors
    total = 0
    for st in seen:
        for name, r in st.items():
            assert name == "ssu_fwd", st
            assert r["count"] > 0 and r["total_ms"] >= 0.0 and r["total_ms"] < 1e4, st
            total += r["count"]
    assert total == n_launch * n_threads, (total, len(seen))
