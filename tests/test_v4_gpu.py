"""GPU parity of the DeepSeek-V4 prefill entry (dsa_mla_prefill_v4) against the V4 oracle.

Inputs follow the reference harness (opus_attn/dsa_v4/common/mla_v4_host.cc:243-283,
README "-topk" / "-window"):
- each query selects scattered prefix rows of the unified cache;
- and its last min(i + 1, window) rows of the extend tensor;
- D = 512, where K and V are the same row;
- a per-head attention sink in the softmax denominator.

Extra cases:
- queries whose whole list fits one 32-row tile (the normalised-P fold);
- empty prefix or extend ranges;
- rows outside their pool;
- no sink.

Bar: bf16 O max-abs <= 2e-2 and LSE within 1e-3 * (1 + |LSE|).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from _cases import assert_parity
from opfoundry_amd import dsa

pytestmark = pytest.mark.gpu
H, D = 128, 512


def t16(a: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(dev)


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def v4_inputs(seed, N=96, total_pages=8192, topk=512, window=128):
    rng = np.random.default_rng(seed)
    q = oracle.normal_bf16(rng, (N, H, D))
    ukv = oracle.normal_bf16(rng, (total_pages, D))
    xkv = oracle.normal_bf16(rng, (N, D))
    ipp, idp, ipe, ide = [0], [], [0], []
    for i in range(N):
        n_pre = 0 if i % 7 == 3 else (20 if i % 7 == 5 else topk)   # empty / one-tile prefixes
        pre = rng.choice(total_pages, n_pre, replace=False).astype(np.int32)
        ext = np.arange(max(0, i + 1 - window), i + 1, dtype=np.int32)
        if i % 11 == 4 and n_pre > 2:
            pre[0], pre[1] = -1, total_pages + 3     # outside the prefix pool: skipped
        if i % 13 == 6:
            ext = ext[:0]                            # empty extend range
        idp += list(pre)
        ide += list(ext)
        ipp.append(len(idp))
        ipe.append(len(ide))
    sink = rng.normal(0.5, 1.0, H).astype(np.float32)
    return q, ukv, xkv, sink, *(np.array(x, np.int32) for x in (ipp, idp, ipe, ide))


@pytest.mark.parametrize("with_sink", [True, False])
def test_prefill_v4_parity(dev, with_sink):
    print(f"[case] V4 prefill sink={with_sink}", flush=True)
    q, ukv, xkv, sink, ipp, idp, ipe, ide = v4_inputs(41 + with_sink)
    scale = 1.0 / np.sqrt(D)
    s = sink if with_sink else None
    o_ref, l_ref = oracle.mla_prefill_v4(q, ukv, xkv, s, ipp, idp, ipe, ide, scale)
    ts = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    out, lse = dsa.mla_prefill_v4(t16(q, dev), t16(ukv, dev), t16(xkv, dev),
                                  None if s is None else ts(s), ts(ipp), ts(idp), ts(ipe), ts(ide),
                                  scale)
    torch.cuda.synchronize()
    e = assert_parity(bits(out), lse.cpu().numpy(), o_ref, l_ref, f"V4 prefill sink={with_sink}")
    print(f"[case] max|dO|={e[0]:.3e} max rel dLSE={e[1]:.3e}", flush=True)
    # queries with no rows at all (i % 7 == 3 and i % 13 == 6): O = 0
    empty = [i for i in range(q.shape[0]) if ipp[i + 1] == ipp[i] and ipe[i + 1] == ipe[i]]
    for i in empty:
        assert (bits(out[i]) == 0).all()


def test_prefill_v4_padded_row_stride(dev):
    """Cache rows stride_kv_page = 520 elements apart (a padded cache), same results."""
    print("[case] V4 prefill padded row stride", flush=True)
    q, ukv, xkv, sink, ipp, idp, ipe, ide = v4_inputs(43, N=24, total_pages=1024, topk=100,
                                                      window=40)
    scale = 0.05
    o_ref, l_ref = oracle.mla_prefill_v4(q, ukv, xkv, sink, ipp, idp, ipe, ide, scale)
    pad = lambda a: np.concatenate([a, np.zeros((a.shape[0], 8), np.uint16)], axis=1)  # noqa: E731
    ukv_t = t16(pad(ukv), dev)[:, :D]
    xkv_t = t16(pad(xkv), dev)[:, :D]
    ts = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    out, lse = dsa.mla_prefill_v4(t16(q, dev), ukv_t, xkv_t, ts(sink), ts(ipp), ts(idp), ts(ipe),
                                  ts(ide), scale)
    torch.cuda.synchronize()
    assert_parity(bits(out), lse.cpu().numpy(), o_ref, l_ref, "V4 prefill padded stride")


def test_prefill_v4_reference_restart(dev):
    """The fixed-reference softmax's rerun on 512-value rows with a sink: query 8 gets an
    all-ones Q and two prefix rows (list entries 40 and 75, tiles 1 and 2) holding 8.0 in
    dims 0..255 (score 2048) and 256..510 (score 2040), about 126 log2 units above the rest.
    8.0 is exact in bf16, so the output must also be the closed-form mixture
    1 : e^(-8 scale) of the two V halves (the sink's weight is negligible).
    The two rows are appended to the pool so that no other query's list names them:
    a random query against them would give outputs near 8, where one bf16 step is
    0.03 to 0.06 and the 2e-2 bar no longer applies."""
    print("[case] V4 prefill reference restart", flush=True)
    q, ukv, xkv, sink, ipp, idp, ipe, ide = v4_inputs(47)
    scale = 1.0 / np.sqrt(D)
    i0 = 8
    qf = oracle.bf16_to_f32(q)
    qf[i0] = 1.0
    q = oracle.bf16_bits(qf)
    spike = np.zeros((2, D), np.float32)
    spike[0, :256] = 8.0
    spike[1, 256:511] = 8.0
    ra, rb = ukv.shape[0], ukv.shape[0] + 1
    ukv = np.concatenate([ukv, oracle.bf16_bits(spike)])
    idp[ipp[i0] + 40], idp[ipp[i0] + 75] = ra, rb
    o_ref, l_ref = oracle.mla_prefill_v4(q, ukv, xkv, sink, ipp, idp, ipe, ide, scale)
    ts = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    out, lse = dsa.mla_prefill_v4(t16(q, dev), t16(ukv, dev), t16(xkv, dev), ts(sink), ts(ipp), ts(idp),
                                  ts(ipe), ts(ide), scale)
    torch.cuda.synchronize()
    o = bits(out)
    e = assert_parity(o, lse.cpu().numpy(), o_ref, l_ref, "V4 prefill reference restart")
    print(f"[case] max|dO|={e[0]:.3e} max rel dLSE={e[1]:.3e}", flush=True)
    w = 8.0 * np.exp(-8 * scale) / (1 + np.exp(-8 * scale))
    oi = oracle.bf16_to_f32(o)[i0]
    assert np.allclose(oi[:, :256], 8.0 - w, atol=2e-2) and np.allclose(oi[:, 256:511], w, atol=2e-2)


def test_prefill_v4_high_prefix_ids_are_skipped(dev):
    """Prefix ids in [2^30, 2^31) beside a small extend pool.  Bit 30 is the kernel's
    second-pool tag; a prefix id is checked against total_pages before any tag exists, so
    these ids are skipped like any other id outside the prefix pool (the oracle skips them
    too), whether or not their low 30 bits name an extend row."""
    print("[case] V4 prefill prefix ids >= 2^30", flush=True)
    q, ukv, xkv, sink, ipp, idp, ipe, ide = v4_inputs(45, N=40, total_pages=2048, topk=300, window=16)
    rng = np.random.default_rng(46)
    pos = rng.choice(idp.size, 200, replace=False)
    high = np.concatenate([(1 << 30) + rng.integers(0, xkv.shape[0], 100),   # low bits: an extend row
                           rng.integers(1 << 30, 2 ** 31, 100)])             # anywhere up to 2^31 - 1
    idp[pos] = high.astype(np.int32)
    scale = 1.0 / np.sqrt(D)
    o_ref, l_ref = oracle.mla_prefill_v4(q, ukv, xkv, sink, ipp, idp, ipe, ide, scale)
    ts = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    out, lse = dsa.mla_prefill_v4(t16(q, dev), t16(ukv, dev), t16(xkv, dev), ts(sink), ts(ipp), ts(idp),
                                  ts(ipe), ts(ide), scale)
    torch.cuda.synchronize()
    e = assert_parity(bits(out), lse.cpu().numpy(), o_ref, l_ref, "V4 prefill high prefix ids")
    print(f"[case] max|dO|={e[0]:.3e} max rel dLSE={e[1]:.3e}", flush=True)


def test_prefill_v4_extreme_sink(dev):
    """Sinks far above every score (+200, +60 natural-log units), far below (-200) and near
    the scores: the maximum is taken over the scores and the sink together
    (mla_v4_host.cc:469), so O stays finite (about 0 under a dominant sink) and LSE is about
    the sink.  Lists of one tile (the normalised-P fold) and of many."""
    print("[case] V4 prefill extreme sink", flush=True)
    q, ukv, xkv, sink, ipp, idp, ipe, ide = v4_inputs(48, N=48, total_pages=4096, topk=400, window=8)
    sink = sink.copy()
    sink[:32], sink[32:64], sink[64:96] = 200.0, -200.0, 60.0
    sink[96:128] = np.linspace(-3.0, 6.0, 32)
    scale = 1.0 / np.sqrt(D)
    o_ref, l_ref = oracle.mla_prefill_v4(q, ukv, xkv, sink, ipp, idp, ipe, ide, scale)
    ts = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    out, lse = dsa.mla_prefill_v4(t16(q, dev), t16(ukv, dev), t16(xkv, dev), ts(sink), ts(ipp), ts(idp),
                                  ts(ipe), ts(ide), scale)
    torch.cuda.synchronize()
    l = lse.cpu().numpy()
    assert np.isfinite(oracle.bf16_to_f32(bits(out))).all()
    e = assert_parity(bits(out), l, o_ref, l_ref, "V4 prefill extreme sink")
    print(f"[case] max|dO|={e[0]:.3e} max rel dLSE={e[1]:.3e}", flush=True)
    nonempty = [i for i in range(q.shape[0]) if ipp[i + 1] > ipp[i] or ipe[i + 1] > ipe[i]]
    assert np.allclose(l[nonempty, :32], 200.0, rtol=1e-6)


def test_prefill_v4_rows_beyond_max_rows_are_nan(dev):
    """max_rows below a query's prefix + extend entries: that query's O and LSE are NaN;
    queries within the bound are exact."""
    print("[case] V4 prefill underestimated max_rows", flush=True)
    q, ukv, xkv, sink, ipp, idp, ipe, ide = v4_inputs(49, N=16, total_pages=2048, topk=300, window=40)
    n_rows = (ipp[1:] - ipp[:-1]) + (ipe[1:] - ipe[:-1])
    bound = 305
    scale = 1.0 / np.sqrt(D)
    o_ref, l_ref = oracle.mla_prefill_v4(q, ukv, xkv, sink, ipp, idp, ipe, ide, scale)
    ts = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    out, lse = dsa.mla_prefill_v4(t16(q, dev), t16(ukv, dev), t16(xkv, dev), ts(sink), ts(ipp), ts(idp),
                                  ts(ipe), ts(ide), scale, max_rows=bound)
    torch.cuda.synchronize()
    l = lse.cpu().numpy()
    over = n_rows > bound
    assert over.any() and (~over).any()
    assert np.isnan(l[over]).all() and torch.isnan(out[torch.from_numpy(over).to(dev)].float()).all()
    assert_parity(bits(out)[~over], l[~over], o_ref[~over], l_ref[~over], "V4 prefill within bound")
