"""Pins the oracle's attention core, index handling, combine and prefill (CPU only).

The oracle restates opus_attn/dsa_v32/common/host.cc:431-548 (decode),
opus_attn/dsa_v4/common/mla_v4_host.cc:482-532 (prefill, no sink) and
opus_attn/dsa_v32/common/mla_reduce.hpp:6-156 (combine).  Each check below
states the expected answer independently of the oracle's code:

- fp64 numpy brute force of the same semantics on small shapes (scores over
  all 576 dims, sm_scale, max-subtracted softmax, P rounded to bf16 through
  torch, O = P.V over the first 512 dims, natural-log LSE);
- closed forms: one valid index -> O = bf16(V_j), LSE = s_j; identical rows ->
  O = V, LSE = s + ln n; q = 0 -> O = mean(V), LSE = ln n; no valid index ->
  O = 0, LSE = +inf (host.cc:486-489);
- index handling: -1 anywhere, j >= seq_len, j < -1, causal violations and
  bad block-table entries give exactly the output of the filtered list;
  permutation invariance; a duplicated index counts twice;
- combine: split partials merged == unsplit result; a single split passes
  through; empty splits are ignored; all-empty -> O = 0, LSE = +inf.
A plausible oracle mistake (RoPE dims dropped, scale applied twice or not at
all, V taken from the wrong dims, LSE in log2, causal bound off by one) fails
at least one of these.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from _cases import D_QK, D_VO, SM_SCALE, flat_case, paged_case

H_SMALL = 4


def f32(bits):
    return oracle.bf16_to_f32(bits).astype(np.float64)


def bf16_round64(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16).to(torch.float64).numpy()


def brute(q64: np.ndarray, rows64: np.ndarray, scale: float):
    """q64 [H, 576], rows64 [n, 576] -> (O fp64 [H, 512], LSE fp64 [H])."""
    if rows64.shape[0] == 0:
        return np.zeros((q64.shape[0], D_VO)), np.full(q64.shape[0], np.inf)
    s = (q64 @ rows64.T) * scale
    m = s.max(axis=1, keepdims=True)
    e = np.exp(s - m)
    den = e.sum(axis=1, keepdims=True)
    p = bf16_round64(e / den)
    return p @ rows64[:, :D_VO], (m + np.log(den))[:, 0]


def bf16_bits_of(x64: np.ndarray) -> np.ndarray:
    return oracle.bf16_bits(x64.astype(np.float32))


def small_decode(seed, B=2, s_q=2, seq_len=200, block_size=16, topk=40, fp8=False, causal=True,
                 poison_unused=True):
    c = paged_case(seed=seed, B=B, s_q=s_q, H=H_SMALL, seq_len=seq_len, block_size=block_size,
                   topk=topk, fp8=fp8, causal=causal, poison_unused=poison_unused)
    return c


def rows_of(c, b, t):
    """Gather valid rows of (b, t) in list order as fp64 (dequantised for fp8)."""
    L = int(c.seq_lens[b])
    out = []
    for j in c.indices[b, t]:
        if j < 0 or j >= L:
            continue
        if c.causal and j > L - c.q.shape[1] + t:
            continue
        if c.block_table is not None:
            blk = c.block_table[b, j // c.block_size]
            row = int(blk) * c.block_size + j % c.block_size
        else:
            row = b * c.kv_batch_stride + j
        if row < 0 or row >= c.kv.shape[0]:
            continue
        out.append(row)
    out = np.array(out, np.int64)
    if c.kv.dtype == np.uint16:
        return f32(c.kv[out])
    return oracle.dequant_rows_656(c.kv[out]).astype(np.float64)


@pytest.mark.parametrize("fp8", [False, True])
def test_decode_vs_fp64_brute_force(fp8):
    c = small_decode(seed=100 + fp8, fp8=fp8)
    o, l = c.oracle(num_threads=2)
    B, s_q = c.q.shape[:2]
    for b in range(B):
        for t in range(s_q):
            ob, lb = brute(f32(c.q[b, t]), rows_of(c, b, t), c.sm_scale)
            got_o = oracle.bf16_to_f32(o[b, t]).astype(np.float64)
            # oracle accumulates in fp32 and rounds O to bf16 once: <= 1 bf16 ulp + fp32 noise
            assert np.all(np.abs(got_o - ob) <= np.abs(ob) * 2.0 ** -8 + 1e-6), (b, t)
            assert np.allclose(l[b, t], lb, rtol=2e-6, atol=2e-6), (b, t, l[b, t], lb)


def test_prefill_vs_fp64_brute_force():
    rng = np.random.default_rng(7)
    N, topk = 24, 10
    q = oracle.normal_bf16(rng, (N, H_SMALL, D_QK))
    kv = oracle.normal_bf16(rng, (N, D_QK))
    idx = np.full((N, topk), -1, np.int32)
    for t in range(N):
        n = min(topk, t + 1)
        idx[t, :n] = oracle.distinct_indices(rng, t + 1, n)
    idx[5, 3] = 20          # future position: masked by causality
    o, l = oracle.mla_prefill(q, kv, idx, SM_SCALE, causal=True, num_threads=2)
    for t in range(N):
        sel = [j for j in idx[t] if 0 <= j <= t]
        ob, lb = brute(f32(q[t]), f32(kv[np.array(sel, np.int64)]), SM_SCALE)
        assert np.all(np.abs(oracle.bf16_to_f32(o[t]) - ob) <= np.abs(ob) * 2.0 ** -8 + 1e-6)
        assert np.allclose(l[t], lb, rtol=2e-6, atol=2e-6)
    # non-causal + causal_offset: offset 100 admits every index
    o2, l2 = oracle.mla_prefill(q, kv, idx, SM_SCALE, causal=True, causal_offset=100)
    o3, l3 = oracle.mla_prefill(q, kv, idx, SM_SCALE, causal=False)
    assert np.array_equal(o2, o3) and np.array_equal(l2, l3)
    assert not np.array_equal(l2[5], l[5])


def _single_row_case(fp8=False):
    rng = np.random.default_rng(9)
    c = flat_case(seed=9, B=1, s_q=1, H=H_SMALL, kv_len=64, topk=8, pad=0, fp8=fp8,
                  poison_unused=False)
    c.indices[:] = -1
    return c, rng


def test_closed_form_single_index():
    c, _ = _single_row_case()
    c.indices[0, 0, 3] = 17
    o, l = c.oracle()
    v = c.kv[17]
    assert np.array_equal(o[0, 0], np.broadcast_to(v[:D_VO], (H_SMALL, D_VO)))
    s = (f32(c.q[0, 0]) @ f32(v)) * SM_SCALE
    assert np.allclose(l[0, 0], s, rtol=1e-6, atol=1e-6)


def test_closed_form_identical_rows():
    c, _ = _single_row_case()
    n = 8
    c.kv[:n] = c.kv[0]
    c.indices[0, 0, :] = np.arange(n)
    o, l = c.oracle()
    assert np.array_equal(o[0, 0], np.broadcast_to(c.kv[0, :D_VO], (H_SMALL, D_VO)))
    s = (f32(c.q[0, 0]) @ f32(c.kv[0])) * SM_SCALE
    assert np.allclose(l[0, 0], s + math.log(n), rtol=1e-6, atol=1e-6)


def test_closed_form_zero_query():
    c, _ = _single_row_case()
    c.q[:] = 0
    n = 8                                              # power of two: P = 1/8 exactly in bf16
    c.indices[0, 0, :] = np.arange(10, 10 + n)
    o, l = c.oracle()
    mean = f32(c.kv[10:10 + n, :D_VO]).mean(axis=0)
    assert np.all(np.abs(oracle.bf16_to_f32(o[0, 0]) - mean) <= np.abs(mean) * 2.0 ** -8 + 1e-6)
    assert np.allclose(l[0, 0], math.log(n), rtol=1e-6)


def test_closed_form_no_valid_index():
    c, _ = _single_row_case()
    c.indices[0, 0, :] = [-1, -2, 64, 65, 1 << 30, -1, -1, -(1 << 30)]
    o, l = c.oracle()
    assert (o == 0).all() and np.isposinf(l).all()


def test_fp8_dequant_feeds_attention():
    """fp8 rows: oracle output equals the bf16-free fp64 evaluation on dequantised rows."""
    c, _ = _single_row_case(fp8=True)
    c.indices[0, 0, 0] = 5
    o, l = c.oracle()
    deq = oracle.dequant_rows_656(c.kv[5:6])[0]
    assert np.array_equal(o[0, 0], np.broadcast_to(bf16_bits_of(deq[:D_VO]), (H_SMALL, D_VO)))
    assert np.allclose(l[0, 0], (f32(c.q[0, 0]) @ deq.astype(np.float64)) * SM_SCALE, rtol=1e-6)


def test_invalid_entries_equal_filtered_list():
    # junk entries may name valid positions outside the drawn list: no poisoned rows here
    c = small_decode(seed=11, B=3, s_q=2, seq_len=150, topk=50, causal=True, poison_unused=False)
    c.block_table = c.block_table.copy()
    c.block_table[2, 1] = 10 ** 7                         # beyond the pool -> invalid
    c.block_table[2, 2] = -4
    rng = np.random.default_rng(12)
    dirty = c.indices.copy()
    junk = rng.choice(np.array([-1, -9, 150, 151, 149, 1 << 29], np.int32), size=dirty.shape)
    mask = rng.random(dirty.shape) < 0.3
    dirty[mask] = junk[mask]
    c.indices = dirty
    o1, l1 = c.oracle()
    filt = np.full_like(dirty, -1)
    bs = c.block_size
    for b in range(3):
        L = int(c.seq_lens[b])
        for t in range(2):
            keep = []
            for j in dirty[b, t]:
                if not (0 <= j < L and j <= L - 2 + t):
                    continue
                blk = int(c.block_table[b, j // bs])
                if blk < 0 or blk * bs + j % bs >= c.kv.shape[0]:
                    continue
                keep.append(j)
            filt[b, t, :len(keep)] = keep
    c.indices = filt
    o2, l2 = c.oracle()
    assert np.array_equal(o1, o2) and np.array_equal(l1, l2)
    # causal bound is inclusive: position L - s_q + t is attended, L - s_q + t + 1 is not
    c.indices[:] = -1
    L = int(c.seq_lens[0])
    c.indices[0, 0, 0] = L - 2
    c.indices[0, 0, 1] = L - 1
    o3, l3 = c.oracle()
    c.indices[0, 0, 1] = -1
    o4, l4 = c.oracle()
    assert np.array_equal(o3[0, 0], o4[0, 0]) and np.array_equal(l3[0, 0], l4[0, 0])
    assert np.isfinite(l4[0, 0]).all()


def test_permutation_invariance_and_duplicates():
    c = small_decode(seed=13, B=1, s_q=1, seq_len=300, topk=64, causal=False)
    o1, l1 = c.oracle()
    c2 = small_decode(seed=13, B=1, s_q=1, seq_len=300, topk=64, causal=False)
    c2.indices = c.indices[:, :, ::-1].copy()
    o2, l2 = c2.oracle()
    ob1 = oracle.bf16_to_f32(o1)
    ob2 = oracle.bf16_to_f32(o2)
    assert np.allclose(ob1, ob2, rtol=2.0 ** -7, atol=1e-6)
    assert np.allclose(l1, l2, rtol=1e-6, atol=1e-6)
    # a duplicated index counts twice: LSE grows by ln(1 + p_j) for the duplicated row
    c3 = small_decode(seed=13, B=1, s_q=1, seq_len=300, topk=64, causal=False)
    base = c3.indices.copy()
    c3.indices = np.concatenate([base, base[:, :, :1]], axis=2)
    o3, l3 = c3.oracle()
    rows = rows_of(c, 0, 0)
    s = (f32(c.q[0, 0]) @ rows.T) * SM_SCALE
    lse = np.log(np.exp(s).sum(axis=1))
    lse_dup = np.log(np.exp(s).sum(axis=1) + np.exp(s[:, 0]))
    assert np.allclose(l1[0, 0], lse, rtol=2e-6)
    assert np.allclose(l3[0, 0], lse_dup, rtol=2e-6)


def test_combine_split_identity():
    c = small_decode(seed=21, B=2, s_q=2, seq_len=400, topk=96, causal=True)
    o_full, l_full = c.oracle()
    bounds = [0, 10, 41, 41, 96]                       # includes an empty split
    po, pl = [], []
    for k0, k1 in zip(bounds[:-1], bounds[1:]):
        a, b = oracle.mla_decode_partial(c.q, c.kv, c.indices, c.seq_lens, c.sm_scale, k0, k1,
                                         block_table=c.block_table, block_size=c.block_size,
                                         causal=True)
        po.append(a)
        pl.append(b)
    po, pl = np.stack(po), np.stack(pl)
    assert (pl[2] == -np.finfo(np.float32).max).all()   # the empty split
    o, l = oracle.mla_combine(po, pl)
    H = c.q.shape[2]
    ref_o = oracle.bf16_to_f32(o_full.reshape(-1, H, D_VO))
    got_o = oracle.bf16_to_f32(o)
    assert np.all(np.abs(got_o - ref_o) <= np.abs(ref_o) * 2.0 ** -7 + 2e-3)
    assert np.allclose(l, l_full.reshape(-1, H), rtol=1e-5, atol=1e-5)
    # one split passes through: partial over the whole list == final result
    a, b = oracle.mla_decode_partial(c.q, c.kv, c.indices, c.seq_lens, c.sm_scale, 0, 96,
                                     block_table=c.block_table, block_size=c.block_size,
                                     causal=True)
    o1, l1 = oracle.mla_combine(a[None], b[None])
    assert np.array_equal(o1, o_full.reshape(-1, H, D_VO))
    assert np.allclose(l1, l_full.reshape(-1, H), rtol=1e-6)


def test_combine_closed_form():
    rng = np.random.default_rng(22)
    S, rows, H = 3, 2, 4
    po = rng.standard_normal((S, rows, H, D_VO)).astype(np.float32)
    pl = rng.standard_normal((S, rows, H)).astype(np.float32)
    pl[0, 1, :] = -np.finfo(np.float32).max
    pl[:, 0, 2] = -np.finfo(np.float32).max
    o, l = oracle.mla_combine(po, pl)
    for r in range(rows):
        for h in range(H):
            lv = pl[:, r, h].astype(np.float64)
            ok = lv > -np.finfo(np.float32).max
            if not ok.any():
                assert np.isposinf(l[r, h]) and (o[r, h] == 0).all()
                continue
            w = np.exp(lv[ok])
            want = (w[:, None] * po[ok, r, h].astype(np.float64)).sum(0) / w.sum()
            assert np.array_equal(o[r, h], bf16_bits_of(want))
            assert np.isclose(l[r, h], np.log(w.sum()), rtol=1e-6, atol=1e-6)


def test_thread_count_does_not_change_results():
    c = small_decode(seed=31, B=3, s_q=2, seq_len=120, topk=30)
    o1, l1 = c.oracle(num_threads=1)
    o2, l2 = c.oracle(num_threads=5)
    assert np.array_equal(o1, o2) and np.array_equal(l1, l2)


@pytest.mark.parametrize("fp8", [False, True])
def test_power_of_two_query_scale_is_exact(fp8):
    """q * 2^k with sm_scale * 2^-k gives bit-identical O and LSE: the scores (q . k) * sm_scale
    are the same fp32 values.  The GPU's 656-B path relies on exactly this to bring a head
    with |q| >= 2^15 into fp16's range; here q reaches about 2^16 * 3, past fp16's 65504."""
    c = small_decode(31, fp8=fp8)
    o1, l1 = c.oracle()
    k = 16
    q2 = oracle.bf16_bits(oracle.bf16_to_f32(c.q) * np.float32(2.0 ** k))
    assert np.abs(oracle.bf16_to_f32(q2)).max() > 6.5e4
    o2, l2 = oracle.mla_decode(q2, c.kv, c.indices, c.seq_lens, np.float32(c.sm_scale * 2.0 ** -k),
                               block_table=c.block_table, block_size=c.block_size, causal=c.causal)
    assert np.array_equal(o1, o2) and np.array_equal(l1, l2)
