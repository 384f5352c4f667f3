"""Bookkeeping of the drop-in layer's packed-operand cache (kan_amd/functional.py),
on the CPU: entries are found by tensor identity and key (version, storage,
dtype, shape, precision, basis), never by tensor equality, and leave with
their tensor.  The GPU test test_packed_operand_cache_reuse_and_invalidation
covers reuse and invalidation through the layer."""
import gc

import torch

from kan_amd import functional as F


def test_lookup_by_identity_and_key():
    a, b = torch.zeros(3), torch.zeros(3)  # equal values, different tensors
    F._cache_put(a, ("k", 1), "packed-a")
    assert F._cache_get(a, ("k", 1)) == "packed-a"
    assert F._cache_get(a, ("k", 2)) is None       # another key (e.g. a newer version)
    assert F._cache_get(b, ("k", 1)) is None       # equal values are not the same tensor
    assert F.cached_pack(a) == "packed-a"
    F.clear_pack_cache()
    assert F.cached_pack(a) is None


def test_key_tracks_in_place_updates():
    c = torch.zeros(4, 3, 9)
    k0 = F._pack_key(c, "bf16", None, None)
    c.add_(1.0)  # an in-place update advances the version counter
    assert F._pack_key(c, "bf16", None, None) != k0
    assert F._pack_key(c, "fp32", None, None) != F._pack_key(c, "bf16", None, None)


def test_entry_dies_with_its_tensor():
    a = torch.zeros(5)
    F._cache_put(a, ("k",), "packed")
    ida = id(a)
    del a
    gc.collect()
    assert ida not in F._pack_cache
