"""GPU parity of the DeepSeek-V4 fp8 prefill entry (dsa_mla_prefill_v4_fp8).

Inputs follow the reference harness (opus_attn/dsa_v4/common/mla_v4_host.cc):
- rows and Q heads drawn as init_fp8_dsa_split (:208-240): 448 e4m3 values with
  14 E8M0 scales in a 512-byte stream row padded with 0xFF, plus 64 bf16 RoPE;
- scattered prefix rows, a sliding window of extend rows, a per-head sink;
- rows the lists never name poisoned with NaN in both streams (:312-322), so a
  stray read shows.

The kernel is checked against the CPU oracle (oracle.mla_prefill_v4_fp8,
pinned in tests/test_oracle_v4fp8.py): bf16 O max-abs <= 2e-2 and LSE within
1e-3 * (1 + |LSE|). The dequantised values are bf16 values, so the outputs
must also equal the bf16 V4 entry's on the dequantised rows bit for bit.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from _cases import assert_parity
from opfoundry_amd import dsa

pytestmark = pytest.mark.gpu
H = 128


def t16(a: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(dev)


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def v4fp8_inputs(seed, N=64, total_pages=4096, topk=512, window=128):
    rng = np.random.default_rng(seed)
    qn, qr = oracle.v4fp8_rows(rng, N * H)
    q = (qn.reshape(N, H, 512), qr.reshape(N, H, 64))
    ukv = oracle.v4fp8_rows(rng, total_pages)
    xkv = oracle.v4fp8_rows(rng, N)
    ipp, idp, ipe, ide = [0], [], [0], []
    for i in range(N):
        n_pre = 0 if i % 7 == 3 else (20 if i % 7 == 5 else topk)
        pre = rng.choice(total_pages, n_pre, replace=False).astype(np.int32)
        ext = np.arange(max(0, i + 1 - window), i + 1, dtype=np.int32)
        if i % 11 == 4 and n_pre > 2:
            pre[0], pre[1] = -1, total_pages + 3
        if i % 13 == 6:
            ext = ext[:0]
        idp += list(pre)
        ide += list(ext)
        ipp.append(len(idp))
        ipe.append(len(ide))
    lists = [np.array(x, np.int32) for x in (ipp, idp, ipe, ide)]
    # poison the prefix rows no list names (mla_v4_host.cc:312-322)
    used = np.zeros(total_pages, bool)
    ok = (lists[1] >= 0) & (lists[1] < total_pages)
    used[lists[1][ok]] = True
    ukv[0][~used] = 0xFF
    ukv[1][~used] = 0x7FC0                       # bf16 NaN
    sink = rng.normal(0.5, 1.0, H).astype(np.float32)
    return q, ukv, xkv, sink, lists


def to_dev(q, ukv, xkv, dev):
    u8 = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    return (u8(q[0]), t16(q[1], dev)), (u8(ukv[0]), t16(ukv[1], dev)), (u8(xkv[0]), t16(xkv[1], dev))


def run(qd, ud, xd, sink, lists, scale, dev):
    ts = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    out, lse = dsa.mla_prefill_v4_fp8(*qd, *ud, *xd, None if sink is None else ts(sink),
                                      *(ts(x) for x in lists), scale)
    torch.cuda.synchronize()
    return bits(out), lse.cpu().numpy()


@pytest.mark.parametrize("with_sink", [True, False])
def test_prefill_v4_fp8_parity(dev, with_sink):
    print(f"[case] V4 fp8 prefill sink={with_sink}", flush=True)
    q, ukv, xkv, sink, lists = v4fp8_inputs(61 + with_sink)
    s = sink if with_sink else None
    scale = 1.0 / np.sqrt(512)
    o_ref, l_ref = oracle.mla_prefill_v4_fp8(*q, *ukv, *xkv, s, *lists, scale)
    o, l = run(*to_dev(q, ukv, xkv, dev), s, lists, scale, dev)
    e = assert_parity(o, l, o_ref, l_ref, f"V4 fp8 prefill sink={with_sink}")
    print(f"[case] max|dO|={e[0]:.3e} max rel dLSE={e[1]:.3e}", flush=True)
    ipp, _, ipe, _ = lists
    for i in range(q[0].shape[0]):
        if ipp[i + 1] == ipp[i] and ipe[i + 1] == ipe[i]:
            assert (o[i] == 0).all()


def test_prefill_v4_fp8_equals_bf16_entry_bitwise(dev):
    """The fp8 entry and the bf16 entry on the dequantised rows run the same 128-head kernel
    arithmetic: identical bits.  (128 queries of short lists: with fewer, the bf16 entry runs
    32-head workgroups, whose QK^T sums in another order.)"""
    print("[case] V4 fp8 vs bf16 V4 entry, bitwise", flush=True)
    q, ukv, xkv, sink, lists = v4fp8_inputs(63, N=128, total_pages=1024, topk=200, window=40)
    scale = 0.05
    o8, l8 = run(*to_dev(q, ukv, xkv, dev), sink, lists, scale, dev)
    deq = lambda nr: oracle.bf16_bits(oracle.dequant_rows_v4fp8(*nr))  # noqa: E731
    q16 = deq((q[0].reshape(-1, 512), q[1].reshape(-1, 64))).reshape(q[0].shape[0], H, 512)
    ts = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    with np.errstate(invalid="ignore"):
        u16, x16 = deq(ukv), deq(xkv)
    out, lse = dsa.mla_prefill_v4(t16(q16, dev), t16(u16, dev), t16(x16, dev), ts(sink),
                                  *(ts(x) for x in lists), scale)
    torch.cuda.synchronize()
    assert (bits(out) == o8).all()
    assert np.array_equal(lse.cpu().numpy(), l8)


def test_prefill_v4_fp8_padded_streams(dev):
    """Row strides of 528 bytes (nope) and 72 elements (rope), Q heads likewise: same results."""
    print("[case] V4 fp8 padded streams", flush=True)
    q, ukv, xkv, sink, lists = v4fp8_inputs(64, N=16, total_pages=512, topk=100, window=20)
    scale = 0.05
    qd, ud, xd = to_dev(q, ukv, xkv, dev)
    o0, l0 = run(qd, ud, xd, sink, lists, scale, dev)

    def pad(t, w):
        z = torch.zeros(*t.shape[:-1], w, dtype=t.dtype, device=dev)
        z[..., :t.shape[-1]] = t
        return z[..., :t.shape[-1]]

    o1, l1 = run((pad(qd[0], 528), pad(qd[1], 72)), (pad(ud[0], 528), pad(ud[1], 72)),
                 (pad(xd[0], 528), pad(xd[1], 72)), sink, lists, scale, dev)
    assert (o1 == o0).all() and np.array_equal(l1, l0)


def test_prefill_v4_fp8_reference_restart(dev):
    """The rerun of the fixed-reference softmax on V4 fp8 rows: query 8 gets Q = 1 (code 1.0,
    scale 2^0; RoPE bf16 1.0) and two prefix rows (list entries 40 and 75, tiles 1 and 2)
    holding 8.0 (code 1.0 under an E8M0 scale of 2^3) in dims 0..255 and in dims 256..447 plus
    bf16 8.0 in RoPE dims 448..510: scores 2048 and 2040, about 126 log2 units above the
    rest.  Every value is exact, so the output must also be the closed-form mixture.
    The two rows are appended to the pool so that no other query's list names them
    (outputs near 8 would put one bf16 step above the 2e-2 bar)."""
    print("[case] V4 fp8 prefill reference restart", flush=True)
    q, ukv, xkv, sink, lists = v4fp8_inputs(67)
    scale = 1.0 / np.sqrt(512)
    ipp, idp = lists[0], lists[1]
    i0 = 8
    q[0][i0] = 0
    q[0][i0, :, :448] = 0x38          # e4m3 1.0
    q[0][i0, :, 448:462] = 127        # E8M0 2^0
    q[1][i0] = 0x3F80                 # bf16 1.0
    codes = np.zeros((2,) + ukv[0].shape[1:], ukv[0].dtype)
    rope = np.zeros((2,) + ukv[1].shape[1:], ukv[1].dtype)
    codes[:, 448:462] = 130           # E8M0 2^3
    codes[0, :256] = 0x38             # 8.0 in dims 0..255
    codes[1, 256:448] = 0x38          # 8.0 in dims 256..447
    rope[1, :63] = 0x4100             # bf16 8.0 in dims 448..510
    ra, rb = ukv[0].shape[0], ukv[0].shape[0] + 1
    ukv = (np.concatenate([ukv[0], codes]), np.concatenate([ukv[1], rope]))
    idp[ipp[i0] + 40], idp[ipp[i0] + 75] = ra, rb
    o_ref, l_ref = oracle.mla_prefill_v4_fp8(*q, *ukv, *xkv, sink, *lists, scale)
    o, l = run(*to_dev(q, ukv, xkv, dev), sink, lists, scale, dev)
    e = assert_parity(o, l, o_ref, l_ref, "V4 fp8 prefill reference restart")
    print(f"[case] max|dO|={e[0]:.3e} max rel dLSE={e[1]:.3e}", flush=True)
    w = 8.0 * np.exp(-8 * scale) / (1 + np.exp(-8 * scale))
    oi = oracle.bf16_to_f32(o)[i0]
    assert np.allclose(oi[:, :256], 8.0 - w, atol=2e-2) and np.allclose(oi[:, 256:511], w, atol=2e-2)


def test_prefill_v4_fp8_high_prefix_ids_are_skipped(dev):
    """As the bf16 V4 case: prefix ids in [2^30, 2^31) next to a small extend pool are outside
    the prefix pool and skipped; the oracle skips them too."""
    print("[case] V4 fp8 prefill prefix ids >= 2^30", flush=True)
    q, ukv, xkv, sink, lists = v4fp8_inputs(65, N=32, total_pages=1024, topk=200, window=16)
    rng = np.random.default_rng(66)
    idp = lists[1]
    pos = rng.choice(idp.size, 150, replace=False)
    idp[pos] = np.concatenate([(1 << 30) + rng.integers(0, xkv[0].shape[0], 75),
                               rng.integers(1 << 30, 2 ** 31, 75)]).astype(np.int32)
    scale = 1.0 / np.sqrt(512)
    o_ref, l_ref = oracle.mla_prefill_v4_fp8(*q, *ukv, *xkv, sink, *lists, scale)
    o, l = run(*to_dev(q, ukv, xkv, dev), sink, lists, scale, dev)
    e = assert_parity(o, l, o_ref, l_ref, "V4 fp8 prefill high prefix ids")
    print(f"[case] max|dO|={e[0]:.3e} max rel dLSE={e[1]:.3e}", flush=True)


def test_prefill_v4_fp8_extreme_sink(dev):
    """Sinks far above and far below every score, on fp8 rows: finite O, LSE about the sink."""
    print("[case] V4 fp8 prefill extreme sink", flush=True)
    q, ukv, xkv, sink, lists = v4fp8_inputs(67, N=32, total_pages=2048, topk=300, window=8)
    sink = sink.copy()
    sink[:64], sink[64:96] = 150.0, -150.0
    scale = 1.0 / np.sqrt(512)
    o_ref, l_ref = oracle.mla_prefill_v4_fp8(*q, *ukv, *xkv, sink, *lists, scale)
    o, l = run(*to_dev(q, ukv, xkv, dev), sink, lists, scale, dev)
    assert np.isfinite(oracle.bf16_to_f32(o)).all()
    e = assert_parity(o, l, o_ref, l_ref, "V4 fp8 prefill extreme sink")
    print(f"[case] max|dO|={e[0]:.3e} max rel dLSE={e[1]:.3e}", flush=True)
