"""GPU parity of split-K prefill (num_splits on dsa_mla_prefill, dsa_mla_prefill_v4 and
dsa_mla_prefill_v4_fp8).

Few query tokens with long lists leave most CUs idle when every token runs in one
workgroup.  Split-K cuts each token's list into contiguous parts of whole 32-row tiles
(prefix rows first, then extend rows: the reference's split layout,
opus_attn/dsa_v4/common/mla_prefill_split.h:7-54), runs one workgroup per (token, part),
and merges the fp32 partials (O and LSE) in a combine kernel, which folds the attention
sink into the denominator once (mla_v4_host.cc:469-472), not once per part.

Cases:
- the V4 harness at -n 16 -topk 0 over 65536 pages (every page, scattered, plus a 128-row
  extend window: 65,536-65,552 rows per query), bf16 and fp8 rows: automatic splits (16
  per query), and 8 and 64 explicit ones, all 16 queries against the V4 oracle;
- sink and range edges with forced splits: a sink far above and far below every score, an
  empty list (O = 0, LSE = +inf), lists shorter than the split count (empty parts), and a
  list longer than max_rows (NaN, never a silently cut attention);
- the V3.2 prefill (top-k form) with 8 queries of top-k 8192 over 16384 rows, causal:
  automatic splits against the oracle.

Bar: O max-abs <= 2e-2 (or one bf16 step where |O| >= 4), LSE within 1e-3 * (1 + |LSE|).
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import oracle
from _cases import D_QK, assert_parity, bf16_rows
from opfoundry_amd import abi, dsa
from test_long_lists_gpu import v4_lists

pytestmark = pytest.mark.gpu
H, D = 128, 512


def t16(a: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(dev)


def ts(a: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def v4_workspace_splits(N, max_rows):
    """The automatic split count the library picks, read back from its workspace size."""
    a = abi.PrefillV4Args()
    a.q = a.unified_kv = a.kv = a.out = 0x1000
    a.kv_indptr_prefix = a.kv_indices_prefix = a.kv_indptr_extend = a.kv_indices_extend = 0x1000
    a.N, a.H, a.D, a.total_pages, a.total_tokens = N, H, D, 1, 1
    a.stride_qo_n, a.stride_qo_h, a.stride_kv_page = H * D, D, D
    a.max_rows, a.num_splits = max_rows, 0
    n = ctypes.c_size_t(0)
    assert abi.load_library().dsa_mla_prefill_v4_workspace_size(ctypes.byref(a), ctypes.byref(n)) == 0
    return 1 if n.value == 0 else (n.value - 256) // (N * H * 513 * 4)


@pytest.mark.parametrize("fp8", [False, True])
def test_v4_split_topk0_65536_pages(dev, fp8):
    N, pages, window = 16, 65536, 128
    rng = np.random.default_rng(81 + fp8)
    sink = rng.normal(0.5, 1.0, H).astype(np.float32)
    lists = v4_lists(rng, N, pages, 0, window)
    ipp, ipe = lists[0], lists[2]
    max_rows = int(((ipp[1:] - ipp[:-1]) + (ipe[1:] - ipe[:-1])).max())
    auto = v4_workspace_splits(N, max_rows)
    assert auto >= 8, auto
    scale = 1.0 / np.sqrt(D)
    print(f"[case] V4 {'fp8' if fp8 else 'bf16'} -n {N} -topk 0 over {pages} pages: longest list "
          f"{max_rows}, automatic splits {auto}", flush=True)
    if fp8:
        qn, qr = oracle.v4fp8_rows(rng, N * H)
        qn, qr = qn.reshape(N, H, 512), qr.reshape(N, H, 64)
        un, ur = oracle.v4fp8_rows(rng, pages)
        xn, xr = oracle.v4fp8_rows(rng, N)
        o_ref, l_ref = oracle.mla_prefill_v4_fp8(qn, qr, un, ur, xn, xr, sink, *lists, scale)
        args = (ts(qn, dev), t16(qr, dev), ts(un, dev), t16(ur, dev), ts(xn, dev), t16(xr, dev))
        fn = dsa.mla_prefill_v4_fp8
    else:
        q = oracle.normal_bf16(rng, (N, H, D))
        ukv = oracle.normal_bf16(rng, (pages, D))
        xkv = oracle.normal_bf16(rng, (N, D))
        o_ref, l_ref = oracle.mla_prefill_v4(q, ukv, xkv, sink, *lists, scale)
        args = (t16(q, dev), t16(ukv, dev), t16(xkv, dev))
        fn = dsa.mla_prefill_v4
    ls = [ts(x, dev) for x in lists]
    for ns in (0, 8, 64):
        out, lse = fn(*args, ts(sink, dev), *ls, scale, num_splits=ns)
        torch.cuda.synchronize()
        e = assert_parity(bits(out), lse.cpu().numpy(), o_ref, l_ref, f"V4 split {ns}")
        print(f"[case] splits {ns or auto}: max|dO|={e[0]:.3e} max rel dLSE={e[1]:.3e}", flush=True)


@pytest.mark.parametrize("fp8", [False, True])
def test_v4_split_sink_and_edges(dev, fp8):
    """Forced splits (4 and 16) on short pools: sinks far above and below every score, an
    empty list, lists shorter than the split count, and one list past max_rows (NaN)."""
    rng = np.random.default_rng(83 + fp8)
    pages, N = 700, 6
    lens = [600, 0, 3, 45, 650, 700]       # query 5: longer than max_rows below
    ipp, idp = [0], []
    for n in lens:
        idp += list(rng.permutation(pages)[:n])
        ipp.append(len(idp))
    ipe = np.array([0, 1, 1, 2, 2, 3, 4], np.int32)[:N + 1]
    ide = np.arange(ipe[-1], dtype=np.int32)
    lists = [np.array(ipp, np.int32), np.array(idp, np.int32), ipe, ide]
    max_rows = 655                          # query 5 has 700 + 1 rows: cut, NaN
    scale = 1.0 / np.sqrt(D)
    for sink_mu in (80.0, -80.0, 0.3):
        sink = (sink_mu + rng.normal(0.0, 1.0, H)).astype(np.float32)
        if fp8:
            qn, qr = oracle.v4fp8_rows(rng, N * H)
            qn, qr = qn.reshape(N, H, 512), qr.reshape(N, H, 64)
            un, ur = oracle.v4fp8_rows(rng, pages)
            xn, xr = oracle.v4fp8_rows(rng, 8)
            o_ref, l_ref = oracle.mla_prefill_v4_fp8(qn, qr, un, ur, xn, xr, sink, *lists, scale)
            args = (ts(qn, dev), t16(qr, dev), ts(un, dev), t16(ur, dev), ts(xn, dev), t16(xr, dev))
            fn = dsa.mla_prefill_v4_fp8
        else:
            q = oracle.normal_bf16(rng, (N, H, D))
            ukv = oracle.normal_bf16(rng, (pages, D))
            xkv = oracle.normal_bf16(rng, (8, D))
            o_ref, l_ref = oracle.mla_prefill_v4(q, ukv, xkv, sink, *lists, scale)
            args = (t16(q, dev), t16(ukv, dev), t16(xkv, dev))
            fn = dsa.mla_prefill_v4
        for ns in (4, 16):
            print(f"[case] V4 {'fp8' if fp8 else 'bf16'} edges: sink ~{sink_mu}, splits {ns}", flush=True)
            out, lse = fn(*args, ts(sink, dev), *(ts(x, dev) for x in lists), scale, num_splits=ns,
                          max_rows=max_rows)
            torch.cuda.synchronize()
            o, l = bits(out), lse.cpu().numpy()
            assert np.isnan(l[5]).all() and np.isnan(oracle.bf16_to_f32(o[5])).all()
            assert np.isinf(l[1]).all() and (l[1] > 0).all() and (o[1] == 0).all()
            keep = [0, 2, 3, 4]
            assert_parity(o[keep], l[keep], o_ref[keep], l_ref[keep], f"V4 edges sink {sink_mu} splits {ns}")


def test_prefill_topk_split(dev):
    """The V3.2 prefill (top-k form) with few queries and long lists: 8 queries (positions near
    the end of a 16384-row cache) of top-k 8192, causal, -1 padded; automatic splits."""
    rng = np.random.default_rng(85)
    rows, topk = 16384, 8192
    pos = np.array([100, 5000, 8191, 9000, 12000, 16000, 16382, 16383], np.int64)
    N = len(pos)
    q = oracle.normal_bf16(rng, (N, H, D_QK))
    kv = bf16_rows(rng, rows)
    idx = np.full((N, topk), -1, np.int32)
    for i, t in enumerate(pos):
        n = min(topk, int(t) + 1)
        idx[i, :n] = oracle.distinct_indices(rng, int(t) + 1, n)
    sm = 1.0 / np.sqrt(192.0)
    # (each list already keeps to its query's causal bound j <= pos, so the call runs
    # without the causal rule)
    o_ref, l_ref = oracle.mla_prefill(q, kv, idx, sm)
    for ns in (0, 5):
        out, lse = dsa.mla_prefill(t16(q, dev), t16(kv, dev), ts(idx, dev), sm, num_splits=ns)
        torch.cuda.synchronize()
        e = assert_parity(bits(out), lse.cpu().numpy(), o_ref, l_ref, f"prefill top-k split {ns}")
        print(f"[case] prefill top-k 8192, splits {ns}: max|dO|={e[0]:.3e} max rel dLSE={e[1]:.3e}", flush=True)
