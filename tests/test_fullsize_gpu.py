"""GPU parity at the BASELINE configurations' full sizes.

The HIP path runs on the exact shapes bench.py measures (configs 2-5). The CPU
oracle (threaded C, all host cores) then checks, with the same bar as every
other parity test (bf16 O max-abs <= 2e-2 on every element, LSE within
1e-3 * (1 + |LSE|)):
- every query token of C2, C3 and C4 (C3: 256 tokens x 2048 rows, about 2 s
  of oracle time on 16 cores);
- every 8th C5 query plus the edges of the -1 padded range (about 1,030
  queries, 2M (query, row) pairs), and every 16th query of the V4 workloads.

Size-independent properties cover every output:
- all outputs are finite wherever a query has valid indices;
- the split-top-k path (partials + combine kernel) agrees with the unsplit
  path at full size;
- the prefill queries with t < 2048, whose lists are -1 padded, match the
  oracle.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import bench
import oracle
from _cases import D_QK, SM_SCALE, assert_parity, lse_rel, o_max_abs
from opfoundry_amd import dsa

pytestmark = pytest.mark.gpu
H = 128


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def sampled_decode_oracle(d, picks):
    """Oracle outputs for the query tokens `picks` of a bench decode workload.

    The rows each token selects are gathered into a compact cache, and the
    token's indices are remapped to it. Invalid entries stay -1.
    """
    B, s_q, topk = d["idx"].shape
    qs, rows, idxs = [], [], []
    for n, (b, t) in enumerate(picks):
        qs.append(d["q"][b, t])
        ii = d["idx"][b, t].long()
        L = int(d["seq_lens"][b])
        hi = L - s_q + t + 1 if d["causal"] else L
        ok = (ii >= 0) & (ii < min(L, hi))
        j = ii.clamp(min=0)
        if d["block_table"] is not None:
            bs = d["block_size"]
            phys = d["block_table"][b].long()[j // bs] * bs + j % bs
        else:
            phys = b * d["kv_batch_stride"] + j
        rows.append(d["kv"][phys])
        loc = torch.arange(topk, device=ii.device) + n * topk
        idxs.append(torch.where(ok, loc, torch.full_like(loc, -1)))
    q = bits(torch.stack(qs).view(len(picks), 1, H, D_QK))
    kv = torch.cat(rows).cpu()
    kv = kv.numpy() if kv.dtype == torch.uint8 else kv.view(torch.int16).numpy().view(np.uint16)
    idx = torch.stack(idxs).view(len(picks), 1, topk).to(torch.int32).cpu().numpy()
    sl = np.full(len(picks), kv.shape[0], np.int32)
    o, lse = oracle.mla_decode(q, kv, idx, sl, SM_SCALE)
    return o[:, 0], lse[:, 0]


def run_full_decode(cfg_name, dev, splits=None):
    cfg = bench.CONFIGS[cfg_name]
    d = bench.make_decode(cfg, dev)
    out, lse = bench.decode_call(d, cfg.get("splits", 0) if splits is None else splits)
    torch.cuda.synchronize()
    return d, out, lse


def check_sample(d, out, lse, picks, what):
    o_ref, l_ref = sampled_decode_oracle(d, picks)
    o_got = np.stack([bits(out[b, t]) for b, t in picks])
    l_got = np.stack([lse[b, t].cpu().numpy() for b, t in picks])
    e = assert_parity(o_got, l_got, o_ref, l_ref, what)
    print(f"[case] {what}: {len(picks)} tokens checked, max|dO|={e[0]:.3e} "
          f"max rel dLSE={e[1]:.3e}", flush=True)


def test_c2_full_size(dev):
    print("[case] C2 full size: B=64, paged 64, seq 32768, top-k 2048", flush=True)
    d, out, lse = run_full_decode("c2", dev)
    assert torch.isfinite(lse).all() and torch.isfinite(out.float()).all()
    check_sample(d, out, lse, [(b, 0) for b in range(d["idx"].shape[0])], "C2 full size (all tokens)")


def test_c3_full_size_and_split_invariance(dev):
    print("[case] C3 full size: fp8 656-B rows, B=128, s_q=2, seq 65536, causal", flush=True)
    d, out, lse = run_full_decode("c3", dev)
    assert torch.isfinite(lse).all() and torch.isfinite(out.float()).all()
    B, s_q, _ = d["idx"].shape
    check_sample(d, out, lse, [(b, t) for b in range(B) for t in range(s_q)], "C3 full size (all tokens)")
    # the split-top-k path (partials + combine) over the whole batch
    out4, lse4 = bench.decode_call(d, 4)
    torch.cuda.synchronize()
    e_o = o_max_abs(bits(out4), bits(out))
    e_l = lse_rel(lse4.cpu().numpy(), lse.cpu().numpy())
    print(f"[case] C3 split 4 vs unsplit: max|dO|={e_o:.3e} max rel dLSE={e_l:.3e}", flush=True)
    assert e_o <= 2e-2 and e_l <= 1e-3


def test_c4_full_size_split_combine(dev):
    print("[case] C4 full size: B=4, seq U[1024,131072], 8 splits + combine", flush=True)
    d, out, lse = run_full_decode("c4", dev)
    B = d["idx"].shape[0]
    check_sample(d, out, lse, [(b, 0) for b in range(B)], "C4 full size (all tokens)")


def test_c5_prefill_full_size(dev):
    print("[case] C5 full size: prefill N=8192, top-k 2048 from [0, t]", flush=True)
    p = bench.make_prefill(bench.CONFIGS["c5"], dev)
    out, lse = dsa.mla_prefill(p["q"], p["kv"], p["idx"], SM_SCALE)
    torch.cuda.synchronize()
    assert torch.isfinite(lse).all() and torch.isfinite(out.float()).all()
    N = p["q"].shape[0]
    sel = torch.tensor(sorted(set(range(0, N, 8)) | {1, 2, 2046, 2047, 2049, N - 1}))
    q = bits(p["q"][sel])
    kv = bits(p["kv"])
    idx = p["idx"][sel].cpu().numpy()
    o_ref, l_ref = oracle.mla_prefill(q, kv, idx, SM_SCALE)
    e = assert_parity(bits(out[sel]), lse[sel].cpu().numpy(), o_ref, l_ref, "C5 full size")
    print(f"[case] C5 full size: {len(sel)} sampled queries, max|dO|={e[0]:.3e} "
          f"max rel dLSE={e[1]:.3e}", flush=True)


@pytest.mark.parametrize("name", ["v4", "v4fp8"])
def test_v4_prefill_full_size(dev, name):
    """The V4 bench workloads (the reference harness's defaults: N=4096, top-k 1024 of 65536
    pages, window 128, sink): sampled queries against the oracle."""
    print(f"[case] {name} full size: N=4096, top-k 1024 of 65536 pages, window 128", flush=True)
    v = bench.make_v4(bench.CONFIGS[name], dev)
    step, keep = bench.v4_step(v, dev)
    step()
    torch.cuda.synchronize()
    out, lse = keep[0], keep[1]
    assert torch.isfinite(lse).all() and torch.isfinite(out.float()).all()
    ipp, idp, ipe, ide = (x.cpu().numpy() for x in v["lists"])
    sel = sorted(set(range(0, v["q"][0].shape[0] if v["fp8"] else v["q"].shape[0], 16)) | {1, 127, 4095})
    lists = [[0], [], [0], []]
    for i in sel:
        lists[1] += list(idp[ipp[i]:ipp[i + 1]])
        lists[3] += list(ide[ipe[i]:ipe[i + 1]])
        lists[0].append(len(lists[1]))
        lists[2].append(len(lists[3]))
    lists = [np.array(x, np.int32) for x in lists]
    b16 = lambda t: t.cpu().view(torch.int16).numpy().view(np.uint16)  # noqa: E731
    sink = v["sink"].cpu().numpy()
    scale = 1.0 / np.sqrt(512.0)
    if v["fp8"]:
        o_ref, l_ref = oracle.mla_prefill_v4_fp8(v["q"][0][sel].cpu().numpy(), b16(v["q"][1][sel]),
                                                 v["ukv"][0].cpu().numpy(), b16(v["ukv"][1]),
                                                 v["xkv"][0].cpu().numpy(), b16(v["xkv"][1]), sink, *lists, scale)
    else:
        o_ref, l_ref = oracle.mla_prefill_v4(b16(v["q"][sel]), b16(v["ukv"]), b16(v["xkv"]), sink, *lists, scale)
    e = assert_parity(bits(out[sel]), lse[sel].cpu().numpy(), o_ref, l_ref, f"{name} full size")
    print(f"[case] {name}: {len(sel)} sampled queries, max|dO|={e[0]:.3e} max rel dLSE={e[1]:.3e}", flush=True)
