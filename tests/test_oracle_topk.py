"""The top-k selection oracle (oracle.topk_indices / order_keys) pinned without the GPU, and
the C ABI's argument checks of dsa_topk_indices (no launch on these paths).

The reference has no top-k step (its kernels take the caller's lists,
opus_attn/dsa_v4/README.md:185), so the oracle is pinned against independent
statements of what a top-k selection must return:
- the key order against numpy's own float sort of the special values;
- on rows without ties, the selected set against torch.topk (which also ranks
  NaN above every number);
- on rows full of ties, the defining invariants: min(k, n) positions,
  ascending, every unselected key <= every selected key, and at the threshold
  key the selected positions are the lowest ones.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import oracle
from opfoundry_amd import abi

SPECIALS = np.array([-np.inf, -3.4e38, -1.0, -1e-40, -0.0, 0.0, 1e-45, 1e-40, 1.0, 3.4e38, np.inf],
                    np.float32)


def test_order_keys_follow_float_order():
    k = oracle.order_keys(SPECIALS).astype(np.int64)
    assert (np.diff(k) >= 0).all()
    # equal keys exactly where the floats compare equal (-0 == +0)
    assert [bool(d == 0) for d in np.diff(k)] == [bool(a == b) for a, b in zip(SPECIALS[:-1], SPECIALS[1:])]
    nan = oracle.order_keys(np.array([np.nan, -np.nan], np.float32))
    assert (nan == 0xFFFFFFFF).all() and (nan > k.max()).all()
    rng = np.random.default_rng(5)
    x = rng.standard_normal(100_000).astype(np.float32) * np.float32(1e3)
    order = np.argsort(x, kind="stable")
    assert (np.diff(oracle.order_keys(x[order]).astype(np.int64)) >= 0).all()


@pytest.mark.parametrize("n,k", [(1, 1), (100, 7), (5000, 2048), (70_000, 2048), (3000, 2999)])
def test_matches_torch_topk_without_ties(n, k):
    rng = np.random.default_rng(n + k)
    s = rng.permutation(np.arange(n, dtype=np.float32) - n / 3)[None] * np.float32(0.37)
    got = oracle.topk_indices(s, None, k)[0]
    ref = np.sort(torch.topk(torch.from_numpy(s[0]), min(k, n)).indices.numpy())
    assert np.array_equal(got[:min(k, n)], ref) and (got[min(k, n):] == -1).all()


def test_nan_ranks_first_as_in_torch():
    rng = np.random.default_rng(9)
    s = rng.standard_normal(4000).astype(np.float32)
    s[[17, 900, 3999]] = np.nan
    s[[5, 6]] = np.inf
    got = oracle.topk_indices(s[None], None, 10)[0]
    ref = np.sort(torch.topk(torch.from_numpy(s), 10).indices.numpy())
    assert np.array_equal(got, ref) and {17, 900, 3999, 5, 6} <= set(got.tolist())


@pytest.mark.parametrize("levels,n,k", [(1, 4096, 1000), (2, 333, 100), (8, 5000, 2048), (8, 5000, 1)])
def test_tie_invariants(levels, n, k):
    rng = np.random.default_rng(levels * 7 + k)
    s = rng.integers(0, levels, n).astype(np.float32)
    s[rng.integers(0, n, n // 10)] = -0.0            # -0 ties with +0
    got = oracle.topk_indices(s[None], None, k)[0]
    sel = got[got >= 0]
    assert sel.size == min(k, n) and (np.diff(sel) > 0).all()
    unsel = np.setdiff1d(np.arange(n), sel)
    thr = s[sel].min()
    assert unsel.size == 0 or s[unsel].max() <= thr
    at_thr = np.flatnonzero(s == thr)
    taken = np.intersect1d(sel, at_thr)
    assert np.array_equal(taken, at_thr[:taken.size])   # lowest positions at the threshold


def test_lengths_and_short_rows():
    s = np.arange(40, dtype=np.float32).reshape(4, 10)[:, ::-1].copy()   # row t: 9..0 descending
    got = oracle.topk_indices(s, np.array([0, 3, -2, 99], np.int32), 5)
    assert (got[0] == -1).all() and (got[2] == -1).all()
    assert got[1].tolist() == [0, 1, 2, -1, -1]
    assert got[3].tolist() == [0, 1, 2, 3, 4]


# ---------------------------------------------------------------- C ABI checks, no launch

@pytest.fixture(scope="module")
def lib():
    return abi.load_library()


def test_abi_validation(lib):
    E = {name: code for code, name in abi.ERRORS.items()}
    f = lib.dsa_topk_indices
    buf = (ctypes.c_int32 * 64)()
    sc = (ctypes.c_float * 64)()
    a16 = ctypes.addressof(sc) + (-ctypes.addressof(sc)) % 16
    out = ctypes.addressof(buf)
    assert f(None, 16, None, -1, 16, 4, out, 4, None) == E["DSA_ERR_BAD_SHAPE"]
    assert f(None, 16, None, 1, 16, -1, out, 4, None) == E["DSA_ERR_BAD_SHAPE"]
    assert f(None, 16, None, 1, 0x7ffffff1, 4, out, 4, None) == E["DSA_ERR_BAD_SHAPE"]
    assert f(None, 16, None, 0, 16, 4, None, 4, None) == 0      # nothing to do: no launch
    assert f(None, 16, None, 4, 16, 0, None, 0, None) == 0
    assert f(a16, 16, None, 1, 16, 4, None, 4, None) == E["DSA_ERR_NULL_POINTER"]
    assert f(None, 16, None, 1, 16, 4, out, 4, None) == E["DSA_ERR_NULL_POINTER"]
    assert f(a16, 16, None, 1, 16, 8, out, 4, None) == E["DSA_ERR_BAD_SHAPE"]   # idx_stride < topk
    assert f(a16, 12, None, 1, 16, 4, out, 4, None) == E["DSA_ERR_BAD_SHAPE"]   # stride < n_max
    assert f(a16, 18, None, 1, 16, 4, out, 4, None) == E["DSA_ERR_BAD_STRIDE"]
    assert f(a16 + 4, 16, None, 1, 16, 4, out, 4, None) == E["DSA_ERR_BAD_STRIDE"]
