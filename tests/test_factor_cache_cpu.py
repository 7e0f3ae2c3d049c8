"""The derived-factor caches key on tensor identity, not on storage address.

A per-layer loop (nar/e17_v2_fold_verify.py:139-185 DownHooks,
nar/e17_v3.py:206-251 benchmark_model) frees one layer's factors and loads the
next; the caching allocator can hand the next factor the same block, and a
fresh tensor starts again at version 0.  Such a tensor must never hit the
previous layer's entry.  CPU tensors exercise the cache logic; the GPU test
(test_gpu_factor_cache.py) runs the launchers through it.
"""

from __future__ import annotations

import gc

import pytest

torch = pytest.importorskip("torch")

from narhip.factors import IdentityCache  # noqa: E402


def counted(cache, src, extra=()):
    calls = []

    def make():
        calls.append(1)
        return src.sum().reshape(1).clone()
    return cache.get((src,), extra, make), len(calls)


def test_hit_on_same_object_and_state():
    cache = IdentityCache()
    a = torch.arange(12.0).reshape(3, 4)
    v1, c1 = counted(cache, a)
    v2, c2 = counted(cache, a)
    assert (c1, c2) == (1, 0) and v1 is v2


def test_in_place_update_misses():
    cache = IdentityCache()
    a = torch.ones(8)
    v1, _ = counted(cache, a)
    a.add_(1.0)
    v2, c2 = counted(cache, a)
    assert c2 == 1 and float(v2) == 16.0 and float(v1) == 8.0


def test_freed_source_drops_entry_and_reused_address_misses():
    cache = IdentityCache()
    a = torch.full((1024,), 1.0)
    ptr = a.data_ptr()
    counted(cache, a)
    assert len(cache) == 1
    del a
    gc.collect()
    assert len(cache) == 0, "the finalizer of a freed source must drop its entry"
    # try to get the same block back (the CPU allocator often reuses it)
    b = None
    for _ in range(64):
        b = torch.full((1024,), 2.0)
        if b.data_ptr() == ptr:
            break
    v, c = counted(cache, b)
    assert c == 1 and float(v) == 2048.0


def test_same_address_different_object_misses_even_without_gc():
    # a second view object on the same storage is a different source
    cache = IdentityCache()
    base = torch.arange(6.0)
    a = base.view(2, 3)
    counted(cache, a)
    b = base.view(2, 3)
    assert b.data_ptr() == a.data_ptr() and b._version == a._version
    _, c = counted(cache, b)
    assert c == 1


def test_derived_value_does_not_keep_source_alive():
    cache = IdentityCache()
    a = torch.ones(4)
    ref = __import__("weakref").ref(a)
    counted(cache, a)
    del a
    gc.collect()
    assert ref() is None and len(cache) == 0


def test_pair_sources_and_none():
    cache = IdentityCache()
    a, b = torch.ones(3), torch.full((3,), 2.0)
    calls = []

    def make():
        calls.append(1)
        return (a if a is not None else 0) + b
    cache.get((a, b), (3,), make)
    cache.get((a, b), (3,), make)
    cache.get((None, b), (3,), lambda: b.clone())
    assert len(calls) == 1 and len(cache) == 2
    del b
    gc.collect()
    assert len(cache) == 0


def test_bounded_size_and_eviction_detaches_finalizers():
    cache = IdentityCache(max_entries=4)
    keep = [torch.full((2,), float(i)) for i in range(10)]
    for t in keep:
        counted(cache, t)
    assert len(cache) == 4
    del keep, t
    gc.collect()
    assert len(cache) == 0
