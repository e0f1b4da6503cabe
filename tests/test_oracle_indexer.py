"""The index scorer's oracle (oracle.indexer_scores), pinned without retyping its formula:
- brute force with pure-Python loops over (head, dim) on tiny shapes, pages included;
- closed forms: one head with weight 1 and q = e_d gives max(0, k[j][d]); negated q gives
  the negative part; scaling the weights scales the scores;
- ReLU: a head whose dot products are all negative contributes nothing;
- rows outside the cache score -inf, positions past a list are NaN (not scored)."""
from __future__ import annotations

import numpy as np

import oracle

rng = np.random.default_rng(61)


def brute(q, w, k, seq_lens, bt, bs, causal, n_cols):
    qf = oracle.bf16_to_f32(q)
    kf = oracle.bf16_to_f32(k)
    B, s_q, H_I, D = q.shape
    out = np.full((B, s_q, n_cols), np.nan)
    for b in range(B):
        for t in range(s_q):
            n = min(max(int(seq_lens[b]) - ((s_q - 1 - t) if causal else 0), 0), n_cols)
            for j in range(n):
                phys = int(bt[b][j // bs]) * bs + j % bs if bt is not None else j
                if not 0 <= phys < k.shape[0]:
                    out[b, t, j] = -np.inf
                    continue
                acc = 0.0
                for h in range(H_I):
                    dot = 0.0
                    for d in range(D):
                        dot += float(qf[b, t, h, d]) * float(kf[phys, d])
                    acc += float(w[b, t, h]) * max(dot, 0.0)
                out[b, t, j] = acc
    return out


def test_brute_force_paged_causal():
    B, s_q, H_I, D, bs = 2, 2, 3, 128, 4
    q = oracle.normal_bf16(rng, (B, s_q, H_I, D))
    w = rng.normal(size=(B, s_q, H_I)).astype(np.float32)
    k = oracle.normal_bf16(rng, (24, D))
    bt = np.array([[5, 1, 0, 2], [3, 4, 7, 2]], np.int32)     # block 7: rows 28.. outside the cache
    seq_lens = np.array([13, 15], np.int32)
    got = oracle.indexer_scores(q, w, k, seq_lens, block_table=bt, block_size=bs, causal=True, n_cols=16)
    ref = brute(q, w, k, seq_lens, bt, bs, True, 16)
    assert np.array_equal(np.isnan(got), np.isnan(ref)) and np.array_equal(np.isinf(got), np.isinf(ref))
    fin = np.isfinite(ref)
    assert np.allclose(got[fin], ref[fin], rtol=1e-12, atol=1e-12)
    assert np.isinf(got[1, :, 8:12]).all()                     # the block outside the cache
    assert np.isnan(got[0, 0, 12:]).all() and not np.isnan(got[0, 1, 12])   # causal lengths 12, 13


def test_closed_forms():
    D, n = 128, 40
    k = oracle.normal_bf16(rng, (n, D))
    kf = oracle.bf16_to_f32(k).astype(np.float64)
    q = np.zeros((1, 1, 2, D), np.uint16)
    d = 17
    q[0, 0, 0, d] = 0x3F80                                     # e_d (bf16 1.0)
    q[0, 0, 1, d] = 0xBF80                                     # -e_d
    lens = np.array([n], np.int32)
    one = oracle.indexer_scores(q[:, :, :1], np.ones((1, 1, 1), np.float32), k, lens)
    assert np.array_equal(one[0, 0], np.maximum(kf[:, d], 0))
    neg = oracle.indexer_scores(q[:, :, 1:], np.ones((1, 1, 1), np.float32), k, lens)
    assert np.array_equal(neg[0, 0], np.maximum(-kf[:, d], 0))
    both = oracle.indexer_scores(q, np.full((1, 1, 2), 2.5, np.float32), k, lens)
    assert np.allclose(both[0, 0], 2.5 * np.abs(kf[:, d]))


def test_relu_drops_negative_heads():
    D, n = 128, 30
    k = oracle.normal_bf16(rng, (n, D))
    kf = oracle.bf16_to_f32(k).astype(np.float64)
    # head 1's query is -(sum of all k rows), scaled: negative against most rows
    q = oracle.normal_bf16(rng, (1, 1, 2, D))
    neg = -kf.sum(0)
    neg = neg / np.abs(neg).max()
    q[0, 0, 1] = oracle.bf16_bits(neg.astype(np.float32))
    qf = oracle.bf16_to_f32(q[0, 0, 1]).astype(np.float64)
    lens = np.array([n], np.int32)
    w = np.array([[[1.0, 7.0]]], np.float32)
    got = oracle.indexer_scores(q, w, k, lens)[0, 0]
    alone = oracle.indexer_scores(q[:, :, :1], w[:, :, :1], k, lens)[0, 0]
    negrow = qf @ kf.T < 0
    assert negrow.sum() > n // 2
    assert np.allclose(got[negrow], alone[negrow])
