"""Pinning of the V4 prefill oracle (oracle.mla_prefill_v4), CPU only.

The oracle restates mla_v4_attention_compute / mla_v4_attention_ref
(opus_attn/dsa_v4/common/mla_v4_host.cc:455-532) with softmax_scale as a
parameter. It is checked against:
- fp64 numpy brute force with a sink, prefix and extend pools, and rows
  outside a pool;
- closed forms: q = 0, a single row, and a sink that dominates;
- the V3.2 prefill oracle, an independent code path, on the same rows with no
  sink and zero RoPE.
"""
from __future__ import annotations

import numpy as np

import oracle
from _cases import D_QK

D = 512
H_SMALL = 3


def f32(bits):
    return oracle.bf16_to_f32(bits).astype(np.float64)


def bf16_round64(x: np.ndarray) -> np.ndarray:
    return f32(oracle.bf16_bits(x.astype(np.float32)))


def brute_v4(q64, rows64, scale, sink):
    """q64 [H, 512], rows64 [n, 512], sink [H] (or None) -> (O fp64 [H, 512], LSE fp64 [H])."""
    H = q64.shape[0]
    if rows64.shape[0] == 0:
        return np.zeros((H, D)), np.full(H, np.inf)
    s = (q64 @ rows64.T) * scale
    sk = np.full(H, -np.inf) if sink is None else sink.astype(np.float64)
    m = np.maximum(s.max(axis=1), sk)[:, None]
    e = np.exp(s - m)
    den = e.sum(axis=1, keepdims=True) + np.exp(sk[:, None] - m)
    p = bf16_round64(e / den)
    return p @ rows64, (m + np.log(den))[:, 0]


def v4_case(seed, N=12, total_pages=60, total_tokens=30, n_pre=7, window=4, sink=True, bad=True):
    rng = np.random.default_rng(seed)
    q = oracle.normal_bf16(rng, (N, H_SMALL, D))
    ukv = oracle.normal_bf16(rng, (total_pages, D))
    xkv = oracle.normal_bf16(rng, (total_tokens, D))
    ipp, idp, ipe, ide = [0], [], [0], []
    for i in range(N):
        pre = rng.choice(total_pages, n_pre, replace=False).astype(np.int32)
        ext = np.arange(max(0, i + 1 - window), i + 1, dtype=np.int32) % total_tokens
        if bad and i % 5 == 2:
            pre[0] = -3
            pre[1] = total_pages + 7        # outside the prefix pool: skipped
        idp += list(pre)
        ide += list(ext)
        ipp.append(len(idp))
        ipe.append(len(ide))
    s = rng.normal(0.0, 1.0, H_SMALL).astype(np.float32) if sink else None
    arr = lambda x: np.array(x, np.int32)  # noqa: E731
    return q, ukv, xkv, s, arr(ipp), arr(idp), arr(ipe), arr(ide)


def rows_for(case, i):
    q, ukv, xkv, s, ipp, idp, ipe, ide = case
    pre = [j for j in idp[ipp[i]:ipp[i + 1]] if 0 <= j < ukv.shape[0]]
    ext = [j for j in ide[ipe[i]:ipe[i + 1]] if 0 <= j < xkv.shape[0]]
    return np.concatenate([f32(ukv[np.array(pre, np.int64)]).reshape(-1, D),
                           f32(xkv[np.array(ext, np.int64)]).reshape(-1, D)])


def test_v4_vs_fp64_brute_force():
    case = v4_case(3)
    q, ukv, xkv, s, ipp, idp, ipe, ide = case
    scale = 1.0 / np.sqrt(D)
    o, l = oracle.mla_prefill_v4(q, ukv, xkv, s, ipp, idp, ipe, ide, scale, num_threads=2)
    for i in range(q.shape[0]):
        ob, lb = brute_v4(f32(q[i]), rows_for(case, i), scale, s)
        assert np.all(np.abs(f32(o[i]) - ob) <= np.abs(ob) * 2.0 ** -8 + 1e-6), i
        assert np.allclose(l[i], lb, rtol=2e-6, atol=2e-6), i


def test_v4_no_sink_equals_v32_prefill_oracle():
    """With no sink and no extend rows, V4 on 512-value rows is the V3.2 prefill on the same
    rows padded with a zero RoPE: an independent code path of the oracle."""
    case = v4_case(4, sink=False, window=0, bad=False)
    q, ukv, xkv, s, ipp, idp, ipe, ide = case
    scale = 0.07
    o4, l4 = oracle.mla_prefill_v4(q, ukv, xkv, None, ipp, idp, ipe, ide, scale)
    N = q.shape[0]
    q576 = np.zeros((N, H_SMALL, D_QK), np.uint16)
    q576[..., :D] = q
    kv576 = np.zeros((ukv.shape[0], D_QK), np.uint16)
    kv576[:, :D] = ukv
    topk = int((ipp[1:] - ipp[:-1]).max())
    idx = np.full((N, topk), -1, np.int32)
    for i in range(N):
        idx[i, :ipp[i + 1] - ipp[i]] = idp[ipp[i]:ipp[i + 1]]
    o3, l3 = oracle.mla_prefill(q576, kv576, idx, scale)
    assert np.array_equal(o4, o3)
    assert np.array_equal(l4, l3)


def test_v4_closed_forms():
    case = v4_case(5, N=3)
    q, ukv, xkv, s, ipp, idp, ipe, ide = case
    # q = 0: every score is 0, P = 1 / (n + e^sink) per row, LSE = ln(n + e^sink)
    qz = np.zeros_like(q)
    o, l = oracle.mla_prefill_v4(qz, ukv, xkv, s, ipp, idp, ipe, ide, 0.05)
    for i in range(3):
        rows = rows_for(case, i)
        n = rows.shape[0]
        p = bf16_round64(1.0 / (n + np.exp(s.astype(np.float64))))
        expect = p[:, None] * rows.sum(axis=0)[None, :]
        assert np.all(np.abs(f32(o[i]) - expect) <= np.abs(expect) * 2.0 ** -8 + 1e-5)
        assert np.allclose(l[i], np.log(n + np.exp(s.astype(np.float64))), rtol=1e-6)
    # a sink far above every score takes all the weight: O = 0 (LSE = sink)
    big = np.full(H_SMALL, 1e4, np.float32)
    o, l = oracle.mla_prefill_v4(q, ukv, xkv, big, ipp, idp, ipe, ide, 0.05)
    assert (f32(o) == 0).all()
    assert np.allclose(l, 1e4)
    # one row and no sink: O = bf16(row), LSE = its score
    one = (np.array([0, 1], np.int32), np.array([9], np.int32), np.array([0, 0], np.int32),
           np.zeros(0, np.int32))
    o, l = oracle.mla_prefill_v4(q[:1], ukv, xkv, None, *one, 0.05)
    assert np.array_equal(o[0], np.broadcast_to(ukv[9], (H_SMALL, D)))
    assert np.allclose(l[0], (f32(q[0]) @ f32(ukv[9])) * 0.05, rtol=1e-5, atol=1e-6)


def test_v4_empty_query():
    case = v4_case(6, N=2, n_pre=0, window=0)
    q, ukv, xkv, s, ipp, idp, ipe, ide = case
    o, l = oracle.mla_prefill_v4(q, ukv, xkv, s, ipp, idp, ipe, ide, 0.05)
    assert (o == 0).all() and np.isinf(l).all()
