"""dsa_topk_indices on the GPU against the CPU oracle (oracle.topk_indices): bit-exact index
rows.  Cases:
- the C3 shape (256 query tokens, causal lengths up to 65536, top-k 2048);
- rows full of ties (scores drawn from a few integers, -0 mixed with +0);
- all-equal rows;
- a narrow band of values (1 + tiny noise), which needs every refinement pass;
- NaN, +-inf, +-0 and subnormals;
- lengths that are clamped (negative, 0, 1, k - 1, k, k + 1, over n_max);
- top-k above the row length (-1 padding), top-k 1;
- a row stride above n_max whose padding holds NaN (never read);
- an output stride above top-k whose extra columns must stay untouched.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from opfoundry_amd import dsa

pytestmark = pytest.mark.gpu


def run_case(dev, scores, lengths, k, out_cols=None, stride=None):
    T, n = scores.shape
    stride = stride or ((n + 3) // 4) * 4
    buf = torch.full((T, stride), float("nan"), dtype=torch.float32)
    buf[:, :n] = torch.from_numpy(scores)
    s_dev = buf.to(dev)[:, :n]
    ln = None if lengths is None else torch.from_numpy(np.asarray(lengths, np.int32)).to(dev)
    cols = out_cols or k
    out = torch.full((T, cols), -7, dtype=torch.int32, device=dev)
    dsa.topk_indices(s_dev, k, ln, out=out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    ref = oracle.topk_indices(scores, lengths, k)
    bad = np.argwhere(got[:, :k] != ref)
    assert bad.size == 0, f"{bad.shape[0]} entries differ, first (token, slot) {bad[0].tolist()}"
    assert (got[:, k:] == -7).all(), "columns past top-k were written"
    return got


def test_topk_c3_shape(dev):
    print("[case] topk c3 shape T=256 n=65536 k=2048", flush=True)
    rng = np.random.default_rng(71)
    T, n, s_q = 256, 65536, 2
    scores = rng.standard_normal((T, n), dtype=np.float32)
    lengths = np.array([n - s_q + (t % s_q) + 1 for t in range(T)], np.int32)
    got = run_case(dev, scores, lengths, 2048)
    assert (got >= 0).all()


@pytest.mark.parametrize("levels,k", [(1, 1000), (3, 100), (8, 2048), (8, 1)])
def test_topk_ties(dev, levels, k):
    print(f"[case] topk ties levels={levels} k={k}", flush=True)
    rng = np.random.default_rng(levels * 31 + k)
    T, n = 12, 6000
    scores = rng.integers(0, levels, (T, n)).astype(np.float32)
    scores[rng.random((T, n)) < 0.1] = -0.0
    run_case(dev, scores, None, k)


def test_topk_narrow_band(dev):
    print("[case] topk narrow band", flush=True)
    rng = np.random.default_rng(73)
    T, n = 8, 20000
    scores = (1.0 + rng.integers(0, 4000, (T, n)) * np.float32(2.0 ** -23)).astype(np.float32)
    run_case(dev, scores, None, 777)


def test_topk_special_values(dev):
    print("[case] topk special values", flush=True)
    rng = np.random.default_rng(74)
    T, n = 6, 3001
    scores = rng.standard_normal((T, n)).astype(np.float32)
    pick = rng.random((T, n))
    scores[pick < 0.02] = np.nan
    scores[(pick >= 0.02) & (pick < 0.04)] = np.inf
    scores[(pick >= 0.04) & (pick < 0.06)] = -np.inf
    scores[(pick >= 0.06) & (pick < 0.10)] = 0.0
    scores[(pick >= 0.10) & (pick < 0.14)] = -0.0
    scores[(pick >= 0.14) & (pick < 0.18)] = np.float32(1e-42)
    scores[(pick >= 0.18) & (pick < 0.22)] = -np.float32(1e-42)
    for k in (37, 600):
        run_case(dev, scores, None, k)


def test_topk_lengths_padding_and_strides(dev):
    print("[case] topk lengths, -1 padding, strides", flush=True)
    rng = np.random.default_rng(75)
    n, k = 3001, 64
    lengths = np.array([-5, 0, 1, k - 1, k, k + 1, 1000, n, n + 10], np.int32)
    scores = rng.standard_normal((lengths.size, n)).astype(np.float32)
    run_case(dev, scores, lengths, k, out_cols=k + 5, stride=3012)
    run_case(dev, scores[:3], None, 5000)        # top-k above the row: every position, then -1
    run_case(dev, scores[:2, :1], None, 1)


def test_topk_feeds_decode(dev):
    """The selected rows drive the decode entry: decoding the GPU-selected lists (int32
    [T, k] viewed as [B, s_q, k]) matches the oracle decode of the same lists."""
    print("[case] topk -> decode", flush=True)
    from _cases import assert_parity, paged_case
    c = paged_case(seed=76, B=2, s_q=2, seq_len=3000, block_size=64, topk=256, fp8=False, causal=True,
                   varlen=False, pad_to=256, poison_unused=False)
    rng = np.random.default_rng(76)
    B, s_q = c.q.shape[:2]
    scores = rng.standard_normal((B * s_q, int(c.seq_lens.max()))).astype(np.float32)
    lengths = np.array([int(c.seq_lens[t // s_q]) - s_q + (t % s_q) + 1 for t in range(B * s_q)], np.int32)
    got = run_case(dev, scores, lengths, 256)
    c.indices = got.reshape(B, s_q, 256)
    o_ref, l_ref = c.oracle()
    kv = torch.from_numpy(np.ascontiguousarray(c.kv).view(np.int16)).view(torch.bfloat16).to(dev)
    q = torch.from_numpy(np.ascontiguousarray(c.q).view(np.int16)).view(torch.bfloat16).to(dev)
    o, lse = dsa.mla_decode(q, kv, torch.from_numpy(c.indices).to(dev), c.sm_scale,
                            seq_lens=torch.from_numpy(c.seq_lens).to(dev),
                            block_table=torch.from_numpy(c.block_table).to(dev), block_size=c.block_size,
                            causal=True)
    torch.cuda.synchronize()
    o = o.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
    assert_parity(o, lse.cpu().numpy(), o_ref, l_ref, "decode of GPU-selected top-k lists")


@pytest.mark.parametrize("n,k", [(65536, 2048), (65537, 2048), (100003, 2048), (100003, 5000)])
def test_topk_row_length_paths(dev, n, k):
    """Rows of at most 65536 positions are selected from registers, longer rows by the
    two-read kernel (with its multi-pass path above 4096): both sides of the switch,
    and ties at the threshold, against the oracle."""
    print(f"[case] topk row length n={n} k={k}", flush=True)
    rng = np.random.default_rng(n + k)
    T = 6
    scores = rng.standard_normal((T, n)).astype(np.float32)
    scores[1] = np.round(scores[1] * 4.0)       # heavy ties
    lengths = np.array([n, n - 1, n // 2, k + 1, k, 3], np.int32)
    run_case(dev, scores, lengths, k)
