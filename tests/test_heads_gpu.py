"""GPU parity at head counts other than 128.

The kernel runs 128 heads per workgroup; a query with H heads takes
ceil(H / 128) workgroups, and the last one computes its heads past H on a copy
of head H-1 and never stores them.  The reference dispatches H = 16 / 40 / 96 /
128 for the V3.2 decode (opus_attn/dsa_v32/README.md:83, host.cc:870-891) and
any positive H for V4 (opus_attn/dsa_v4/README.md:174).

Cases: decode (paged, bf16 and fp8 rows) at H = 16, 40, 64, 200, unsplit and
split; the CSR entry at H = 16; the V3.2 prefill at H = 64; the V4 prefill
(bf16 and fp8 rows, with a sink) at H = 16, 64 and 200.  Outputs and LSEs live
inside larger sentinel-filled buffers: the heads past H must stay untouched.

Bar: O max-abs <= 2e-2 (or one bf16 step where |O| >= 4) and LSE within
1e-3 * (1 + |LSE|), as for H = 128.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from _cases import D_QK, SM_SCALE, assert_parity, bf16_rows, paged_case
from opfoundry_amd import dsa

pytestmark = pytest.mark.gpu
SENT_O = 0x7BCD          # a finite bf16 sentinel
SENT_L = -12345.0
EXTRA = 8                # sentinel heads past H in each output row


def t16(a: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(dev)


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def guarded_out(lead, H, dev):
    """(out view [..., H, 512], lse view [..., H], full out buffer, full lse buffer)."""
    full_o = torch.full((*lead, H + EXTRA, 512), 0, dtype=torch.int16, device=dev)
    full_o.fill_(SENT_O - 65536 if SENT_O > 32767 else SENT_O)
    full_o = full_o.view(torch.bfloat16)
    n = int(np.prod(lead)) * H
    full_l = torch.full((n + 64,), SENT_L, dtype=torch.float32, device=dev)
    return full_o[..., :H, :], full_l[:n].view(*lead, H), full_o, full_l


def check_guards(full_o, full_l, H, n):
    tail = bits(full_o[..., H:, :])
    assert (tail == SENT_O).all(), "a head past H was written"
    assert (full_l[n:].cpu().numpy() == SENT_L).all(), "LSE written past H"


@pytest.mark.parametrize("H", [16, 40, 64, 200])
@pytest.mark.parametrize("fp8", [False, True])
def test_decode_heads(dev, H, fp8):
    c = paged_case(seed=300 + H, B=3, s_q=2, H=H, seq_len=1500, topk=700, fp8=fp8, causal=True)
    o_ref, l_ref = c.oracle()
    q = t16(c.q, dev)
    kv = torch.from_numpy(c.kv).to(dev) if fp8 else t16(c.kv, dev)
    idx = torch.from_numpy(c.indices).to(dev)
    sl = torch.from_numpy(c.seq_lens).to(dev)
    bt = torch.from_numpy(c.block_table).to(dev)
    for ns in (0, 1, 4):
        print(f"[case] decode H={H} fp8={fp8} splits={ns}", flush=True)
        out, lse, full_o, full_l = guarded_out((3, 2), H, dev)
        dsa.mla_decode(q, kv, idx, c.sm_scale, out, lse, seq_lens=sl, block_table=bt,
                       block_size=c.block_size, causal=True, num_splits=ns)
        torch.cuda.synchronize()
        e = assert_parity(bits(out), lse.cpu().numpy(), o_ref, l_ref, f"decode H={H} splits={ns}")
        print(f"[case] max|dO|={e[0]:.3e} max rel dLSE={e[1]:.3e}", flush=True)
        check_guards(full_o, full_l, H, 3 * 2 * H)


def test_csr_heads(dev):
    H = 16
    rng = np.random.default_rng(311)
    lens = [900, 2500, 1, 0]
    total = 4000
    q = oracle.normal_bf16(rng, (len(lens), H, D_QK))
    kv = bf16_rows(rng, total)
    indptr = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    indices = np.concatenate([rng.permutation(total)[:n] for n in lens]).astype(np.int32)
    idx = np.full((len(lens), 1, max(lens)), -1, np.int32)
    for b, n in enumerate(lens):
        idx[b, 0, :n] = indices[indptr[b]:indptr[b + 1]]
    o_ref, l_ref = oracle.mla_decode(q.reshape(len(lens), 1, H, D_QK), kv, idx,
                                     np.full(len(lens), total, np.int32), SM_SCALE)
    o_ref, l_ref = o_ref.reshape(len(lens), H, -1), l_ref.reshape(len(lens), H)
    for ns in (0, 1):
        print(f"[case] CSR H={H} splits={ns}", flush=True)
        out, lse, full_o, full_l = guarded_out((len(lens),), H, dev)
        dsa.mla_decode_csr(t16(q, dev), t16(kv, dev), torch.from_numpy(indptr).to(dev),
                           torch.from_numpy(indices).to(dev), SM_SCALE, out, lse, s_q=1, num_splits=ns)
        torch.cuda.synchronize()
        assert_parity(bits(out), lse.cpu().numpy(), o_ref, l_ref, f"CSR H={H} splits={ns}")
        check_guards(full_o, full_l, H, len(lens) * H)


def test_prefill_heads(dev):
    H, N, topk = 64, 200, 128
    rng = np.random.default_rng(312)
    q = oracle.normal_bf16(rng, (N, H, D_QK))
    kv = bf16_rows(rng, N)
    idx = np.full((N, topk), -1, np.int32)
    for t in range(N):
        n = min(topk, t + 1)
        idx[t, :n] = oracle.distinct_indices(rng, t + 1, n)
    o_ref, l_ref = oracle.mla_prefill(q, kv, idx, SM_SCALE, causal=True)
    print(f"[case] prefill H={H}", flush=True)
    out, lse, full_o, full_l = guarded_out((N,), H, dev)
    dsa.mla_prefill(t16(q, dev), t16(kv, dev), torch.from_numpy(idx).to(dev), SM_SCALE, out, lse,
                    causal=True)
    torch.cuda.synchronize()
    assert_parity(bits(out), lse.cpu().numpy(), o_ref, l_ref, f"prefill H={H}")
    check_guards(full_o, full_l, H, N * H)


def v4_lists(rng, N, pages, topk, window):
    ipp, idp, ipe, ide = [0], [], [0], []
    for i in range(N):
        idp += list(rng.permutation(pages)[:topk].astype(np.int32))
        ide += list(range(max(0, i + 1 - window), i + 1))
        ipp.append(len(idp))
        ipe.append(len(ide))
    return [np.array(x, np.int32) for x in (ipp, idp, ipe, ide)]


@pytest.mark.parametrize("H", [16, 64, 200])
def test_prefill_v4_heads(dev, H):
    N, pages = 40, 2048
    rng = np.random.default_rng(320 + H)
    q = oracle.normal_bf16(rng, (N, H, 512))
    ukv = oracle.normal_bf16(rng, (pages, 512))
    xkv = oracle.normal_bf16(rng, (N, 512))
    sink = rng.normal(0.5, 1.0, H).astype(np.float32)
    lists = v4_lists(rng, N, pages, 300, 16)
    scale = 1.0 / np.sqrt(512)
    o_ref, l_ref = oracle.mla_prefill_v4(q, ukv, xkv, sink, *lists, scale)
    print(f"[case] V4 bf16 H={H}", flush=True)
    ts = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    out, lse = dsa.mla_prefill_v4(t16(q, dev), t16(ukv, dev), t16(xkv, dev), ts(sink),
                                  *(ts(x) for x in lists), scale)
    torch.cuda.synchronize()
    e = assert_parity(bits(out), lse.cpu().numpy(), o_ref, l_ref, f"V4 H={H}")
    print(f"[case] max|dO|={e[0]:.3e} max rel dLSE={e[1]:.3e}", flush=True)


@pytest.mark.parametrize("H", [16, 200])
def test_prefill_v4_fp8_heads(dev, H):
    N, pages = 24, 1024
    rng = np.random.default_rng(330 + H)
    qn, qr = oracle.v4fp8_rows(rng, N * H)
    qn, qr = qn.reshape(N, H, 512), qr.reshape(N, H, 64)
    un, ur = oracle.v4fp8_rows(rng, pages)
    xn, xr = oracle.v4fp8_rows(rng, N)
    sink = rng.normal(0.5, 1.0, H).astype(np.float32)
    lists = v4_lists(rng, N, pages, 200, 8)
    scale = 1.0 / np.sqrt(512)
    o_ref, l_ref = oracle.mla_prefill_v4_fp8(qn, qr, un, ur, xn, xr, sink, *lists, scale)
    print(f"[case] V4 fp8 H={H}", flush=True)
    ts = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    out, lse = dsa.mla_prefill_v4_fp8(ts(qn), t16(qr, dev), ts(un), t16(ur, dev), ts(xn), t16(xr, dev),
                                      ts(sink), *(ts(x) for x in lists), scale)
    torch.cuda.synchronize()
    e = assert_parity(bits(out), lse.cpu().numpy(), o_ref, l_ref, f"V4 fp8 H={H}")
    print(f"[case] max|dO|={e[0]:.3e} max rel dLSE={e[1]:.3e}", flush=True)
