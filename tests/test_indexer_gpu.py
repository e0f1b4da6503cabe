"""GPU parity of the index scorer (dsa_indexer_scores) against oracle.indexer_scores.

Bar: fp32 scores within 2e-5 * (sum_h |w_h| * |q_h . k| + 1e-3) of the float64 oracle
(bf16 products are exact in fp32; only the summation order differs), -inf exactly where the
row lies outside the cache, and no position past a list written.

Cases: the DeepSeek-V3.2 shape (H_I = 64, MTP s_q = 2, causal, paged cache of 64-row
blocks, lists crossing 2048-position spans and 128-position chunks); H_I = 32 (four tokens
per workgroup, a partial last group) and H_I = 128; a flat cache with padded rows; block
table entries outside the cache; and the end-to-end step: scores -> dsa_topk_indices ->
dsa_mla_decode on the selected rows.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from _cases import SM_SCALE, assert_parity
from opfoundry_amd import dsa

pytestmark = pytest.mark.gpu


def t16(a: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(dev)


def check(got, q, w, k, ref, what):
    got = got.cpu().numpy().astype(np.float64)
    fin = np.isfinite(ref)
    assert np.array_equal(np.isneginf(got), np.isneginf(ref)), f"{what}: -inf mismatch"
    assert np.isnan(got[np.isnan(ref)]).all(), f"{what}: a position past a list was written"
    # scale of each score: sum_h |w| |q.k| bounded by sum_h |w| |q| |k|
    err = np.abs(got[fin] - ref[fin])
    tol = 2e-5 * (np.abs(ref[fin]) + 1.0) + 1e-4
    worst = float((err / tol).max()) if err.size else 0.0
    assert worst <= 1.0, f"{what}: score error {float(err.max())} (worst ratio {worst:.2f})"
    return float(err.max()) if err.size else 0.0


def paged(rng, B, seq, bs, H_I, s_q, bad_blocks=0):
    mb = -(-seq.max() // bs)
    nblk = B * mb
    perm = rng.permutation(nblk).astype(np.int32)
    bt = perm.reshape(B, mb)
    if bad_blocks:
        bt.flat[rng.choice(bt.size, bad_blocks, replace=False)] = nblk + 5     # outside the cache
    k = oracle.normal_bf16(rng, (nblk * bs, 128))
    q = oracle.normal_bf16(rng, (B, s_q, H_I, 128))
    w = (rng.normal(size=(B, s_q, H_I)) / np.sqrt(H_I)).astype(np.float32)
    return q, w, k, bt


@pytest.mark.parametrize("H_I,s_q", [(64, 2), (32, 5), (128, 1)])
def test_indexer_paged_causal(dev, H_I, s_q):
    rng = np.random.default_rng(400 + H_I)
    seq = np.array([5000, 130, 2049, 1, 4096], np.int32)
    bs = 64
    q, w, k, bt = paged(rng, len(seq), seq, bs, H_I, s_q, bad_blocks=3)
    n_cols = int(seq.max())
    print(f"[case] indexer H_I={H_I} s_q={s_q} lens={list(seq)}", flush=True)
    ref = oracle.indexer_scores(q, w, k, seq, block_table=bt, block_size=bs, causal=True, n_cols=n_cols)
    got = dsa.indexer_scores(t16(q, dev), torch.from_numpy(w).to(dev), t16(k, dev), torch.from_numpy(seq).to(dev),
                             block_table=torch.from_numpy(bt).to(dev), block_size=bs, causal=True, n_cols=n_cols)
    torch.cuda.synchronize()
    e = check(got, q, w, k, ref, f"indexer H_I={H_I}")
    print(f"[case] max |d score| = {e:.3e}", flush=True)


def test_indexer_flat_padded_rows_and_short_n_cols(dev):
    """Flat per-sequence caches with padded k rows (stride 192 elements), not causal, and
    n_cols shorter than the lists (positions at or past n_cols are not scored)."""
    rng = np.random.default_rng(410)
    B, s_q, H_I, L = 3, 2, 64, 3000
    q = oracle.normal_bf16(rng, (B, s_q, H_I, 128))
    w = rng.normal(size=(B, s_q, H_I)).astype(np.float32)
    kpad = oracle.normal_bf16(rng, (B * L, 192))
    seq = np.array([3000, 2500, 17], np.int32)
    n_cols = 2600
    ref = oracle.indexer_scores(q, w, kpad[:, :128], seq, k_batch_stride=L, n_cols=n_cols)
    kd = t16(kpad, dev)[:, :128]
    got = dsa.indexer_scores(t16(q, dev), torch.from_numpy(w).to(dev), kd, torch.from_numpy(seq).to(dev),
                             k_batch_stride=L, n_cols=n_cols)
    torch.cuda.synchronize()
    check(got, q, w, kpad[:, :128], ref, "indexer flat")


def test_indexer_topk_decode_end_to_end(dev):
    """One DSA attention step on the GPU: index scores -> top-k positions -> sparse MLA decode
    over the selected rows, against the oracle at each stage (top-k selection of the GPU's
    own scores is exact)."""
    rng = np.random.default_rng(420)
    B, s_q, H_I, bs, topk = 2, 2, 64, 64, 256
    seq = np.array([3000, 1500], np.int32)
    q, w, k, bt = paged(rng, B, seq, bs, H_I, s_q)
    n_cols = int(seq.max())
    sl = torch.from_numpy(seq).to(dev)
    btd = torch.from_numpy(bt).to(dev)
    scores = dsa.indexer_scores(t16(q, dev), torch.from_numpy(w).to(dev), t16(k, dev), sl, block_table=btd,
                                block_size=bs, causal=True, n_cols=n_cols)
    lens = torch.tensor([int(seq[b]) - (s_q - 1 - t) for b in range(B) for t in range(s_q)], dtype=torch.int32,
                        device=dev)
    idx = dsa.topk_indices(scores.view(B * s_q, n_cols), topk, lens)
    torch.cuda.synchronize()
    idx_ref = oracle.topk_indices(scores.view(B * s_q, n_cols).cpu().numpy(), lens.cpu().numpy(), topk)
    assert np.array_equal(idx.cpu().numpy(), idx_ref)
    # the decode over the selected positions of the MLA latent cache (same paging)
    qm = oracle.normal_bf16(rng, (B, s_q, 128, 576))
    kv = oracle.normal_bf16(rng, (k.shape[0], 576))
    indices = idx.view(B, s_q, topk)
    out, lse = dsa.mla_decode(t16(qm, dev), t16(kv, dev), indices, SM_SCALE, seq_lens=sl, block_table=btd,
                              block_size=bs, causal=True)
    torch.cuda.synchronize()
    o_ref, l_ref = oracle.mla_decode(qm, kv, indices.cpu().numpy(), seq, SM_SCALE, block_table=bt, block_size=bs,
                                     causal=True)
    assert_parity(out.cpu().contiguous().view(torch.int16).numpy().view(np.uint16), lse.cpu().numpy(), o_ref,
                  l_ref, "indexer -> topk -> decode")
