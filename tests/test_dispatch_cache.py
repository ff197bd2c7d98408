"""The module's "this mask is tril(L)" verdict and its concatenated generator
weights are cached per live tensor object: a new tensor that the allocator
places at a freed tensor's address never inherits the verdict (the reference
re-checks every call, kernel/attention_kernel.py:203-208)."""
from __future__ import annotations

import gc

import pytest
import torch

from holonomyawareattention_amd.attention_kernel import PathOrderedGeometricMHA


def _same_address_mask(L, ptr, device, tries=200):
    """A fresh (L, L) all-true mask, preferably at address `ptr`."""
    keep = []
    for _ in range(tries):
        m = torch.ones(L, L, dtype=torch.bool, device=device)
        if m.data_ptr() == ptr:
            return m, True
        keep.append(m)
    return torch.ones(L, L, dtype=torch.bool, device=device), False


def _check_alias(device):
    L = 96
    mod = PathOrderedGeometricMHA(48, n_heads=2)
    tril = torch.ones(L, L, dtype=torch.bool, device=device).tril()
    assert mod._tril_path(tril, L)
    assert mod._tril_path(tril, L)                      # cached verdict for the same object
    ptr = tril.data_ptr()
    del tril
    gc.collect()
    ones, reused = _same_address_mask(L, ptr, device)
    assert not mod._tril_path(ones, L)
    return reused


def test_freed_tril_mask_does_not_alias_cpu():
    _check_alias(torch.device("cpu"))


def test_modified_mask_is_rechecked():
    L = 64
    mod = PathOrderedGeometricMHA(48, n_heads=2)
    mask = torch.ones(L, L, dtype=torch.bool).tril()
    assert mod._tril_path(mask, L)
    mask[0, 5] = True                                    # in place: the version counter moves
    assert not mod._tril_path(mask, L)


def test_weight_cache_follows_the_tensors():
    mod = PathOrderedGeometricMHA(48, n_heads=2)
    w1 = mod._cat_weight((mod.gqproj, mod.gkproj))
    assert mod._cat_weight((mod.gqproj, mod.gkproj)) is w1
    with torch.no_grad():
        mod.gqproj.weight.add_(1.0)                      # in-place update
    w2 = mod._cat_weight((mod.gqproj, mod.gkproj))
    assert w2 is not w1 and torch.equal(w2[:mod.gqproj.weight.shape[0]], mod.gqproj.weight)
    mod.gkproj.weight = torch.nn.Parameter(torch.zeros_like(mod.gkproj.weight))   # a new tensor
    w3 = mod._cat_weight((mod.gqproj, mod.gkproj))
    assert torch.equal(w3[mod.gqproj.weight.shape[0]:], mod.gkproj.weight)


@pytest.mark.gpu
def test_freed_tril_mask_does_not_alias_gpu():
    """On the GPU the caching allocator hands a freed block of the same size
    straight back: the new all-true mask lands at the old tril mask's address."""
    reused = _check_alias(torch.device("cuda:0"))
    assert reused
