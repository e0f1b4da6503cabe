"""CPU unit test of the index rules the forward kernel applies (opfoundry_amd/csrc/dsa_rows.h).

The header is compiled here with g++ (tests/native/rows_check.cpp), so these are the
device functions' own source.  Every accepted entry must address a row inside the pool
it will be gathered from:
- V4 prefix ids (unified_kv, mla_v4_host.cc:482-532) checked against total_pages,
  including ids in [2^30, 2^31) whose bit 30 is the second-pool tag;
- V4 extend ids checked against total_tokens and tagged;
- CSR rows (host.cc:482,526) against total_tokens;
- top-k positions through the block table (paged) or a flat batch base, with the
  seq_len / causal bound and a bad block-table entry.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
POOL2 = 1 << 30


@pytest.fixture(scope="module")
def rl(tmp_path_factory):
    so = str(tmp_path_factory.mktemp("rows") / "librows_check.so")
    subprocess.run(["g++", "-O1", "-std=c++17", "-shared", "-fPIC", "-Wall", "-Werror",
                    os.path.join(HERE, "native", "rows_check.cpp"), "-o", so], check=True)
    L = ctypes.CDLL(so)
    i32, i64, vp = ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p
    for name, args, res in [("rows_v4_prefix", [i32, i64], i32), ("rows_v4_extend", [i32, i64], i32),
                            ("rows_csr", [i32, i64], i32), ("rows_in_pool2", [i32], ctypes.c_int),
                            ("rows_index", [i32], i32), ("rows_max_pool", [], i64),
                            ("rows_topk", [i32, i64, vp, i32, i32, i64, i64], i64),
                            ("rows_v4_list", [vp, ctypes.c_int, vp, ctypes.c_int, i64, i64, vp, vp],
                             ctypes.c_int)]:
        f = getattr(L, name)
        f.argtypes, f.restype = args, res
    return L


EDGE_IDS = [-(2 ** 31), -POOL2, -2, -1, 0, 1, 7, 999, 1000, 1001, POOL2 - 1, POOL2, POOL2 + 1,
            POOL2 + 7, POOL2 + 999, 2 ** 31 - 1]


@pytest.mark.parametrize("pages", [0, 1, 1000, POOL2 - 1])
def test_v4_prefix_rule(rl, pages):
    """A prefix id is a first-pool row iff 0 <= id < total_pages: never tagged, whatever its bit 30."""
    rng = np.random.default_rng(pages % 97)
    ids = EDGE_IDS + list(rng.integers(-(2 ** 31), 2 ** 31, 2000, dtype=np.int64))
    for j in ids:
        r = rl.rows_v4_prefix(int(j), pages)
        if 0 <= j < pages:
            assert r == j and not rl.rows_in_pool2(r) and rl.rows_index(r) == j
        else:
            assert r == -1, (j, pages, r)


@pytest.mark.parametrize("tokens", [0, 1, 1000, POOL2 - 1])
def test_v4_extend_rule(rl, tokens):
    """An extend id is tagged as a second-pool row iff 0 <= id < total_tokens."""
    rng = np.random.default_rng(tokens % 89 + 1)
    for j in EDGE_IDS + list(rng.integers(-(2 ** 31), 2 ** 31, 2000, dtype=np.int64)):
        r = rl.rows_v4_extend(int(j), tokens)
        if 0 <= j < tokens:
            assert rl.rows_in_pool2(r) and rl.rows_index(r) == j and r >= 0
        else:
            assert r == -1, (j, tokens, r)


def test_v4_list_high_prefix_ids(rl):
    """The case the tag once leaked through: prefix ids in [2^30, 2^31) with a small extend
    pool.  Every kept entry names its own pool and a row inside it; the kept list equals
    the oracle's filter (mla_v4_host.cc:482-532 with rows outside their pool skipped)."""
    rng = np.random.default_rng(5)
    pages, tokens = 5000, 64
    pre = np.concatenate([rng.integers(0, pages, 300), rng.integers(POOL2, 2 ** 31, 200),
                          [POOL2, POOL2 + 3, POOL2 + tokens - 1, -1, pages, 2 ** 31 - 1]]).astype(np.int32)
    rng.shuffle(pre)
    ext = np.concatenate([np.arange(tokens), [tokens, -5, POOL2 + 1]]).astype(np.int32)
    pool = np.zeros(pre.size + ext.size, np.int32)
    row = np.zeros_like(pool)
    n = rl.rows_v4_list(pre.ctypes.data, pre.size, ext.ctypes.data, ext.size, pages, tokens,
                        pool.ctypes.data, row.ctypes.data)
    want = [(1, int(j)) for j in pre if 0 <= j < pages] + [(2, int(j)) for j in ext if 0 <= j < tokens]
    got = list(zip(pool[:n].tolist(), row[:n].tolist()))
    assert got == want
    for p, r in got:
        assert 0 <= r < (pages if p == 1 else tokens)


def test_pool_limit(rl):
    """The tag needs every pool below 2^30 rows; the host entries enforce that bound."""
    assert rl.rows_max_pool() == POOL2
    assert rl.rows_v4_prefix(POOL2 - 1, POOL2) == POOL2 - 1
    assert not rl.rows_in_pool2(rl.rows_v4_prefix(POOL2 - 1, POOL2))


def test_csr_rule(rl):
    for rows in (0, 1, 65536):
        for j in EDGE_IDS:
            assert rl.rows_csr(j, rows) == (j if 0 <= j < rows else -1)


def test_topk_rule_paged_and_flat(rl):
    """Logical position -> physical row: block table (power-of-two and other block sizes),
    flat batches, the seq_len / causal bound, and block-table entries outside the cache."""
    rng = np.random.default_rng(9)
    for bs, shift in ((64, 6), (1, 0), (48, -1), (16, 4)):
        rows = 4096
        nblk = 40
        bt = rng.integers(0, rows // bs, nblk).astype(np.int32)
        bt[3] = -1                     # a bad block id: its positions are skipped
        bt[5] = rows // bs + 2         # beyond the cache
        jmax = min(nblk * bs, 1500)
        for j in list(range(-3, 3)) + list(range(jmax - 3, jmax + 3)) + list(rng.integers(0, jmax, 300)):
            j = int(j)
            got = rl.rows_topk(j, jmax, bt.ctypes.data, bs, shift, 0, rows)
            if j < 0 or j >= jmax:
                want = -1
            else:
                r = int(bt[j // bs]) * bs + j % bs
                want = r if 0 <= r < rows else -1
            assert got == want, (bs, j, got, want)
    # flat: batch base + j, bounded by the cache
    for j in (-1, 0, 10, 99, 100):
        assert rl.rows_topk(j, 100, None, 1, 0, 3900, 4000) == (3900 + j if 0 <= j < 100 else -1)
    assert rl.rows_topk(50, 200, None, 1, 0, 3990, 4000) == -1     # past the last cache row
