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
