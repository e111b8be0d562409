"""Kernel cache semantics (compile_cache.py:13-37 of the reference): one factory call per
key, reset empties it; here also safe under concurrent first use."""

from __future__ import annotations

import threading

from tiledattention.kernels import compile_cache as cc


def test_get_kernel_hit_miss_and_reset():
    cc.reset_cache_for_tests()
    calls = []
    k1 = cc.get_kernel(("a", 1), lambda: calls.append(1) or "kernel-a")
    k2 = cc.get_kernel(("a", 1), lambda: calls.append(2) or "other")
    k3 = cc.get_kernel(("b", 1), lambda: calls.append(3) or "kernel-b")
    assert (k1, k2, k3) == ("kernel-a", "kernel-a", "kernel-b")
    assert calls == [1, 3]
    assert cc.cache_size() == 2
    cc.reset_cache_for_tests()
    assert cc.cache_size() == 0
    assert cc.get_kernel(("a", 1), lambda: "fresh") == "fresh"
    cc.reset_cache_for_tests()


def test_get_kernel_builds_once_under_contention():
    cc.reset_cache_for_tests()
    calls = []
    barrier = threading.Barrier(8)
    out = []

    def worker():
        barrier.wait()
        out.append(cc.get_kernel(("k",), lambda: calls.append(1) or object()))

    threads = [threading.Thread(target=worker) for _ in range(8)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert len(calls) == 1
    assert all(o is out[0] for o in out)
    cc.reset_cache_for_tests()
