"""GPU parity of lists longer than one 2048-entry chunk of the row list.

A workgroup resolves its list 2048 entries at a time and carries the softmax
state and the O accumulators from one chunk to the next, so the prefill
entries (which run one workgroup per query) take lists of any length:
- the V4 harness at -topk 2048 -window 128: 2048 scattered prefix pages plus
  the last min(i + 1, 128) extend rows, up to 2176 rows
  (opus_attn/dsa_v4/common/mla_v4_host.cc:243-283, README "-topk" / "-window");
- the V4 harness at -topk 0: every page of a small pool (4500 pages), in a
  scattered order (mla_v4_host.cc:252, 819-820), plus the window;
- the same two lists on the fp8 V4 entry;
- the V3.2 prefill at top-k 4096 (config-5 shape with twice the list): query t
  attends min(4096, t + 1) distinct positions <= t, -1 padded;
- a skewed CSR batch: one 200,000-row list (longer than 64 splits x 2048
  entries) beside short and empty ones, through the device work plan and
  through uniform splits.

Extra cases: a chunk with no valid row between two valid ones, invalid entries
straddling a chunk boundary, and a query whose only valid rows lie in its
second chunk (the softmax reference is set by the first tile that has rows).

Bar: O max-abs <= 2e-2 (or one bf16 step where |O| >= 4) and LSE within
1e-3 * (1 + |LSE|), as for every other entry.
"""
from __future__ import annotations

from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch

import oracle
from _cases import D_QK, SM_SCALE, assert_parity, bf16_rows, fp8_rows
from opfoundry_amd import dsa

pytestmark = pytest.mark.gpu
H, D = 128, 512


def t16(a: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(dev)


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def v4_lists(rng, N, total_pages, topk, window):
    """Prefix: `topk` scattered pages (all pages when topk <= 0); extend: the last
    min(i + 1, window) rows ending at row i (mla_v4_host.cc:244-283)."""
    budget = total_pages if topk <= 0 or topk > total_pages else topk
    ipp, idp, ipe, ide = [0], [], [0], []
    for i in range(N):
        pre = rng.permutation(total_pages)[:budget].astype(np.int32)
        if i % 5 == 2:
            # invalid entries around the first chunk boundary (entry 2048)
            pre[2040:2056] = -1
        if i % 5 == 4:
            # the whole first chunk invalid: the rows start in the second chunk
            pre[:2048] = total_pages + 7
        if i % 5 == 3 and budget > 4096:
            # an empty chunk between two chunks with rows
            pre[2048:4096] = -1
        ext = np.arange(max(0, i + 1 - window), i + 1, dtype=np.int32)
        idp += list(pre)
        ide += list(ext)
        ipp.append(len(idp))
        ipe.append(len(ide))
    return [np.array(x, np.int32) for x in (ipp, idp, ipe, ide)]


CASES = {
    # name: (N, total_pages, topk, window)
    "topk2048_window128": (136, 8192, 2048, 128),
    "topk0_pool4500": (24, 4500, 0, 128),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_prefill_v4_long_lists(dev, name):
    N, pages, topk, window = CASES[name]
    rng = np.random.default_rng(71)
    q = oracle.normal_bf16(rng, (N, H, D))
    ukv = oracle.normal_bf16(rng, (pages, D))
    xkv = oracle.normal_bf16(rng, (N, D))
    sink = rng.normal(0.5, 1.0, H).astype(np.float32)
    lists = v4_lists(rng, N, pages, topk, window)
    ipp, ipe = lists[0], lists[2]
    longest = int(((ipp[1:] - ipp[:-1]) + (ipe[1:] - ipe[:-1])).max())
    assert longest > 2048
    print(f"[case] V4 bf16 {name}: N={N} longest list {longest}", flush=True)
    scale = 1.0 / np.sqrt(D)
    o_ref, l_ref = oracle.mla_prefill_v4(q, ukv, xkv, sink, *lists, scale)
    ts = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    out, lse = dsa.mla_prefill_v4(t16(q, dev), t16(ukv, dev), t16(xkv, dev), ts(sink),
                                  *(ts(x) for x in lists), scale)
    torch.cuda.synchronize()
    e = assert_parity(bits(out), lse.cpu().numpy(), o_ref, l_ref, f"V4 {name}")
    print(f"[case] max|dO|={e[0]:.3e} max rel dLSE={e[1]:.3e}", flush=True)


@pytest.mark.parametrize("name", sorted(CASES))
def test_prefill_v4_fp8_long_lists(dev, name):
    N, pages, topk, window = CASES[name]
    N = min(N, 40)
    rng = np.random.default_rng(72)
    qn, qr = oracle.v4fp8_rows(rng, N * H)
    qn, qr = qn.reshape(N, H, 512), qr.reshape(N, H, 64)
    un, ur = oracle.v4fp8_rows(rng, pages)
    xn, xr = oracle.v4fp8_rows(rng, N)
    sink = rng.normal(0.5, 1.0, H).astype(np.float32)
    lists = v4_lists(rng, N, pages, topk, window)
    print(f"[case] V4 fp8 {name}: N={N}", flush=True)
    scale = 1.0 / np.sqrt(D)
    o_ref, l_ref = oracle.mla_prefill_v4_fp8(qn, qr, un, ur, xn, xr, sink, *lists, scale)
    ts = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    out, lse = dsa.mla_prefill_v4_fp8(ts(qn), t16(qr, dev), ts(un), t16(ur, dev), ts(xn), t16(xr, dev),
                                      ts(sink), *(ts(x) for x in lists), scale)
    torch.cuda.synchronize()
    e = assert_parity(bits(out), lse.cpu().numpy(), o_ref, l_ref, f"V4 fp8 {name}")
    print(f"[case] max|dO|={e[0]:.3e} max rel dLSE={e[1]:.3e}", flush=True)


@pytest.mark.parametrize("fp8", [False, True])
def test_prefill_topk4096(dev, fp8):
    """Config-5 shape with a 4096-entry list: 8192 cache rows, query t (its
    position) attends min(4096, t + 1) distinct positions <= t, -1 padded.
    Queries are taken across the whole range: short padded lists, lists that end
    inside the second chunk, and full ones."""
    rng = np.random.default_rng(73)
    rows, topk = 8192, 4096
    pos = np.concatenate([[0, 1, 31, 2047, 2048, 2049, 3000, 4095, 4096],
                          rng.choice(np.arange(4097, rows), 23, replace=False)]).astype(np.int64)
    N = len(pos)
    q = oracle.normal_bf16(rng, (N, H, D_QK))
    kv = fp8_rows(rng, rows) if fp8 else bf16_rows(rng, rows)
    idx = np.full((N, topk), -1, np.int32)
    for i, t in enumerate(pos):
        n = min(topk, int(t) + 1)
        idx[i, :n] = oracle.distinct_indices(rng, int(t) + 1, n)
    print(f"[case] prefill top-k 4096 fp8={fp8} N={N}", flush=True)
    o_ref, l_ref = oracle.mla_prefill(q, kv, idx, SM_SCALE)
    kvd = torch.from_numpy(kv).to(dev) if fp8 else t16(kv, dev)
    out, lse = dsa.mla_prefill(t16(q, dev), kvd, torch.from_numpy(idx).to(dev), SM_SCALE)
    torch.cuda.synchronize()
    e = assert_parity(bits(out), lse.cpu().numpy(), o_ref, l_ref, "prefill top-k 4096")
    print(f"[case] max|dO|={e[0]:.3e} max rel dLSE={e[1]:.3e}", flush=True)


def test_csr_decode_beyond_64_chunks(dev):
    """A skewed CSR batch: one list of 200,000 rows (more than 64 splits x 2048
    entries) beside short and empty ones, with MTP (s_q = 2, count-based
    causality).  Automatic splits run the device work plan; 4 and 64 uniform
    splits run the per-token split path."""
    rng = np.random.default_rng(74)
    pool, lens, s_q = 220_000, [200_000, 300, 2_100, 0], 2
    B = len(lens)
    q = oracle.normal_bf16(rng, (B * s_q, H, D_QK))
    kv = bf16_rows(rng, pool)
    indptr = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    indices = np.concatenate([rng.permutation(pool)[:n] for n in lens]).astype(np.int32)
    indices[5000:5100] = -1                  # skipped rows
    print(f"[case] CSR decode lists {lens}, s_q={s_q}", flush=True)
    # The oracle on the top-k form of the same lists (query token t of batch b
    # sees the first len - (s_q - 1 - t) entries), in ranges of 10,000 entries
    # run side by side (one oracle task is one whole list), merged by the
    # oracle's split combine.
    width = max(lens)
    idx = np.full((B, s_q, width), -1, np.int32)
    for b, n in enumerate(lens):
        for t in range(s_q):
            m = max(0, n - (s_q - 1 - t))
            idx[b, t, :m] = indices[indptr[b]:indptr[b] + m]
    q4 = q.reshape(B, s_q, H, D_QK)
    sl = np.full(B, pool, np.int32)

    def part(r0):
        sub = np.ascontiguousarray(idx[:, :, r0:r0 + 10_000])
        return oracle.mla_decode_partial(q4, kv, sub, sl, SM_SCALE, 0, sub.shape[2], num_threads=2)

    with ThreadPoolExecutor(8) as ex:
        parts = list(ex.map(part, range(0, width, 10_000)))
    o_ref, l_ref = oracle.mla_combine(np.stack([p[0] for p in parts]), np.stack([p[1] for p in parts]))
    for ns in (0, 4, 64):
        out, lse = dsa.mla_decode_csr(t16(q, dev), t16(kv, dev), torch.from_numpy(indptr).to(dev),
                                      torch.from_numpy(indices).to(dev), SM_SCALE, s_q=s_q,
                                      max_kv_len=max(lens), num_splits=ns)
        torch.cuda.synchronize()
        e = assert_parity(bits(out), lse.cpu().numpy(), o_ref, l_ref, f"CSR skewed splits={ns}")
        print(f"[case] splits={ns}: max|dO|={e[0]:.3e} max rel dLSE={e[1]:.3e}", flush=True)
