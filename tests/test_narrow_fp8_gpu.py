"""GPU parity of the 32-head forward kernel on 656-byte fp8 rows
(dsa_mla_fwd_narrow_kernel<DSA_KV_FP8_656>).

The library runs fp8 rows on 32-head workgroups under the same rule as bf16 rows: H <= 32,
or fewer than 128 workgroups of 128 heads even after splitting.  The kernel gathers raw
656-byte tiles into a ring of three slots and dequantises each into one of two fp16 tile
buffers (fp16(code * 2^e) * fp16(mantissa), as the 128-head kernel does); the NoPE part of
QK^T and PV run on fp16 operands.  Cases:
- the C1 shape on fp8 rows (B = 2, H = 128, top-k 2048 with 256 padding entries), automatic
  splits (16);
- one query token with a 5000-entry paged list, unsplit: three 2048-entry chunks of the row
  list walked in one workgroup through the raw ring;
- H = 16 (one 32-head group, half of it padding) at B = 32 with MTP (s_q = 2, causal),
  paged, automatic splits;
- the prefill entry on fp8 rows at H = 16 (causal lists, the first queries' lists short);
- the CSR form on fp8 rows with uniform splits and a list past max_kv_len (NaN for that
  token only).
The range rules of the fp8 path (|q| up to 1e5, scales at and past the limit) run on this
kernel in tests/test_fp8_range_gpu.py, whose B = 4 cases select it.

Bar: O max-abs <= 2e-2 (or one bf16 step where |O| >= 4), LSE within 1e-3 * (1 + |LSE|).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from _cases import D_QK, SM_SCALE, assert_parity, flat_case, fp8_rows, paged_case
from opfoundry_amd import dsa

pytestmark = pytest.mark.gpu


def t16(a: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(dev)


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def run_decode(c, dev, num_splits):
    bt = None if c.block_table is None else torch.from_numpy(c.block_table).to(dev)
    out_t, lse_t = dsa.mla_decode(t16(c.q, dev), torch.from_numpy(c.kv).to(dev), torch.from_numpy(c.indices).to(dev),
                                  c.sm_scale, seq_lens=torch.from_numpy(c.seq_lens).to(dev), block_table=bt,
                                  block_size=c.block_size, kv_batch_stride=c.kv_batch_stride, causal=c.causal,
                                  num_splits=num_splits)
    torch.cuda.synchronize()
    return bits(out_t), lse_t.cpu().numpy()


def test_fp8_c1_shape(dev):
    c = flat_case(seed=2027, fp8=True)
    print("[case] fp8 narrow: C1 shape (B=2, H=128, top-k 2048, 256 padding), automatic splits", flush=True)
    o_ref, l_ref = c.oracle()
    o, l = run_decode(c, dev, 0)
    e = assert_parity(o, l, o_ref, l_ref, "fp8 C1 shape")
    print(f"[case] max|dO|={e[0]:.3e} max rel dLSE={e[1]:.3e}", flush=True)


def test_fp8_long_list_one_workgroup(dev):
    c = paged_case(seed=95, B=1, s_q=1, seq_len=6000, topk=5000, fp8=True)
    print("[case] fp8 narrow: one token, 5000 entries, unsplit (3 chunks)", flush=True)
    o_ref, l_ref = c.oracle()
    o, l = run_decode(c, dev, 1)
    e = assert_parity(o, l, o_ref, l_ref, "fp8 narrow long list")
    print(f"[case] max|dO|={e[0]:.3e} max rel dLSE={e[1]:.3e}", flush=True)


def test_fp8_h16_mtp_batch(dev):
    c = paged_case(seed=96, B=32, s_q=2, H=16, seq_len=4096, topk=1024, fp8=True, causal=True)
    print("[case] fp8 narrow: H=16, B=32, s_q=2 causal, paged, automatic splits", flush=True)
    o_ref, l_ref = c.oracle()
    o, l = run_decode(c, dev, 0)
    e = assert_parity(o, l, o_ref, l_ref, "fp8 narrow H=16")
    print(f"[case] max|dO|={e[0]:.3e} max rel dLSE={e[1]:.3e}", flush=True)


def test_fp8_prefill_h16(dev):
    rng = np.random.default_rng(97)
    N, H, topk = 300, 16, 256
    q = oracle.normal_bf16(rng, (N, H, D_QK))
    kv = fp8_rows(rng, N)
    idx = np.full((N, topk), -1, np.int32)
    for t in range(N):
        n = min(topk, t + 1)
        idx[t, :n] = oracle.distinct_indices(rng, t + 1, n)
    print(f"[case] fp8 narrow prefill: N={N} H={H} top-k {topk} causal", flush=True)
    o_ref, l_ref = oracle.mla_prefill(q, kv, idx, SM_SCALE, causal=True)
    out, lse = dsa.mla_prefill(t16(q, dev), torch.from_numpy(kv).to(dev), torch.from_numpy(idx).to(dev),
                               SM_SCALE, causal=True)
    torch.cuda.synchronize()
    e = assert_parity(bits(out), lse.cpu().numpy(), o_ref, l_ref, "fp8 narrow prefill")
    print(f"[case] max|dO|={e[0]:.3e} max rel dLSE={e[1]:.3e}", flush=True)


def test_fp8_csr_uniform_splits_cut_list(dev):
    H = 128
    rng = np.random.default_rng(98)
    total = 3000
    lens = [900, 1500]
    kv = fp8_rows(rng, total)
    indptr = np.array([0, lens[0], lens[0] + lens[1]], np.int32)
    indices = rng.integers(0, total, sum(lens)).astype(np.int32)
    q = oracle.normal_bf16(rng, (2, H, D_QK))
    max_kv_len = 1200                      # batch 1's 1500 entries are cut: NaN
    print("[case] fp8 narrow CSR: uniform splits (2), one list past max_kv_len", flush=True)
    out, lse = dsa.mla_decode_csr(t16(q, dev), torch.from_numpy(kv).to(dev), torch.from_numpy(indptr).to(dev),
                                  torch.from_numpy(indices).to(dev), SM_SCALE, s_q=1,
                                  max_kv_len=max_kv_len, num_splits=2)
    torch.cuda.synchronize()
    o, l = bits(out), lse.cpu().numpy()
    assert np.isnan(l[1]).all() and np.isnan(oracle.bf16_to_f32(o[1])).all()
    idx = np.full((1, 1, lens[0]), -1, np.int32)
    idx[0, 0] = indices[:lens[0]]
    o_ref, l_ref = oracle.mla_decode(q[:1].reshape(1, 1, H, D_QK), kv, idx, np.full(1, total, np.int32), SM_SCALE)
    e = assert_parity(o[:1], l[:1], o_ref.reshape(1, H, -1), l_ref.reshape(1, H), "fp8 narrow CSR kept row")
    print(f"[case] max|dO|={e[0]:.3e} max rel dLSE={e[1]:.3e}", flush=True)
