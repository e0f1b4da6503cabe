"""GPU parity of the 32-head forward kernel (dsa_mla_fwd_narrow_kernel) on the cases its
selection rule sends it, beyond the low-batch decodes the other tests already run on it.

The library runs bf16 rows on 32-head workgroups when H <= 32, or when 128-head
workgroups would number fewer than 128 even after splitting.  Cases:
- a 5000-entry paged list, unsplit (one query token, three 2048-entry chunks of the
  row list in one workgroup), bf16, top-k form;
- the V4 prefill at H = 16 with a sink far above every score and lists longer than one
  chunk (2300 prefix pages + window), unsplit and 3 splits;
- the CSR form with uniform splits and a list longer than max_kv_len (NaN for that
  token only), bf16.
(Head counts that leave a partial last group, H = 40 and 200, with sentinel-filled outputs,
run in tests/test_heads_gpu.py.)

Bar: O max-abs <= 2e-2 (or one bf16 step where |O| >= 4), LSE within 1e-3 * (1 + |LSE|).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from _cases import D_QK, SM_SCALE, assert_parity, bf16_rows, paged_case
from opfoundry_amd import dsa

pytestmark = pytest.mark.gpu
D = 512


def t16(a: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(dev)


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def run_decode(c, dev, num_splits):
    out_t, lse_t = dsa.mla_decode(t16(c.q, dev), t16(c.kv, dev), torch.from_numpy(c.indices).to(dev),
                                  c.sm_scale, seq_lens=torch.from_numpy(c.seq_lens).to(dev),
                                  block_table=torch.from_numpy(c.block_table).to(dev),
                                  block_size=c.block_size, causal=c.causal, num_splits=num_splits)
    torch.cuda.synchronize()
    return out_t, lse_t


def test_long_list_one_workgroup(dev):
    c = paged_case(seed=91, B=1, s_q=1, seq_len=6000, topk=5000)
    print("[case] narrow: one token, 5000 entries, unsplit (3 chunks)", flush=True)
    o_ref, l_ref = c.oracle()
    o, l = run_decode(c, dev, 1)
    e = assert_parity(bits(o), l.cpu().numpy(), o_ref, l_ref, "narrow long list")
    print(f"[case] max|dO|={e[0]:.3e} max rel dLSE={e[1]:.3e}", flush=True)


def test_v4_h16_sink_long_lists(dev):
    H, N, pages, window = 16, 5, 2600, 64
    rng = np.random.default_rng(93)
    ipp, idp, ipe, ide = [0], [], [0], []
    for i in range(N):
        idp += list(rng.permutation(pages)[:2300 - 37 * i])
        ipp.append(len(idp))
        n = min(i + 1, window)
        ide += list(range(i + 1 - n, i + 1))
        ipe.append(len(ide))
    lists = [np.array(x, np.int32) for x in (ipp, idp, ipe, ide)]
    q = oracle.normal_bf16(rng, (N, H, D))
    ukv = oracle.normal_bf16(rng, (pages, D))
    xkv = oracle.normal_bf16(rng, (N, D))
    sink = (40.0 + rng.normal(0.0, 1.0, H)).astype(np.float32)
    scale = 1.0 / np.sqrt(D)
    o_ref, l_ref = oracle.mla_prefill_v4(q, ukv, xkv, sink, *lists, scale)
    ts = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    for ns in (1, 3):
        print(f"[case] narrow V4: H=16, sink ~40, lists of ~2300 rows, splits {ns}", flush=True)
        out, lse = dsa.mla_prefill_v4(t16(q, dev), t16(ukv, dev), t16(xkv, dev), ts(sink),
                                      *(ts(x) for x in lists), scale, num_splits=ns)
        torch.cuda.synchronize()
        e = assert_parity(bits(out), lse.cpu().numpy(), o_ref, l_ref, f"narrow V4 splits {ns}")
        print(f"[case] max|dO|={e[0]:.3e} max rel dLSE={e[1]:.3e}", flush=True)


def test_csr_uniform_splits_cut_list(dev):
    H = 128
    rng = np.random.default_rng(94)
    total = 3000
    lens = [900, 1500]
    kv = bf16_rows(rng, total)
    indptr = np.array([0, lens[0], lens[0] + lens[1]], np.int32)
    indices = rng.integers(0, total, sum(lens)).astype(np.int32)
    q = oracle.normal_bf16(rng, (2, H, D_QK))
    max_kv_len = 1200                      # batch 1's 1500 entries are cut: NaN
    print("[case] narrow CSR: uniform splits (2), one list past max_kv_len", flush=True)
    out, lse = dsa.mla_decode_csr(t16(q, dev), t16(kv, dev), torch.from_numpy(indptr).to(dev),
                                  torch.from_numpy(indices).to(dev), SM_SCALE, s_q=1,
                                  max_kv_len=max_kv_len, num_splits=2)
    torch.cuda.synchronize()
    o, l = bits(out), lse.cpu().numpy()
    assert np.isnan(l[1]).all() and np.isnan(oracle.bf16_to_f32(o[1])).all()
    idx = np.full((1, 1, lens[0]), -1, np.int32)
    idx[0, 0] = indices[:lens[0]]
    o_ref, l_ref = oracle.mla_decode(q[:1].reshape(1, 1, H, D_QK), kv, idx, np.full(1, total, np.int32), SM_SCALE)
    e = assert_parity(o[:1], l[:1], o_ref.reshape(1, H, -1), l_ref.reshape(1, H), "narrow CSR kept row")
    print(f"[case] max|dO|={e[0]:.3e} max rel dLSE={e[1]:.3e}", flush=True)
