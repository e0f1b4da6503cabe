"""Benchmark of the DSA sparse-MLA hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c3]

A "step" is one sparse-MLA decode call over one batch of synthetic inputs that
are already resident in HBM.  Default workload: BASELINE config 3 (the one the
north-star target is quoted on) - fp8 656-byte KV rows, batch 128, MTP s_q = 2,
128 heads, top-k 2048, seq_len 65536 paged at 64 rows, causal.  The JSON line
also carries configs 1, 2 and 4 (bf16 decode; 1 and 4 timed as HIP-graph
replays), config 5 (bf16 sparse prefill, 8192 x 128 heads x top-k 2048) in
TFLOP/s, the same decode on MXFP8 split streams (the reference's own -dtype fp8
format, C3-shaped: B=128, s_q=2, 2048 rows per token), the DeepSeek-V4
prefill (bf16 and fp8 rows) at the reference harness's default shape, the
top-k index selection that produces config 3's lists (256 tokens, lengths up to
65536, top-k 2048), the dominant kernel's roofline for each, and the CPU oracle
timed on a bounded sample of each workload on this host.

Warm-up: by default at least 10 steps and 0.15 s of back-to-back calls per
workload before the timed steps (the GPU takes tens of ms of sustained load to
settle; the first ~30 ms of a decode run are up to 30 % slower).  The JSON line
reports the warm-up step count used.

Algorithmic work (V = valid (query, index) pairs):
  FLOPs = 2 * 128 * (576 + 512) * V
  bytes = Q + V * row_bytes + O + LSE + indices   (row_bytes 656 fp8 / 1152 bf16)
  top-k selection: bytes = 4 * (sum of row lengths) + 4 * tokens * top-k
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

H, D_QK, D_VO = 128, 576, 512
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
SM_SCALE = 1.0 / math.sqrt(192.0)
FLOP_PER_PAIR = 2 * H * (D_QK + D_VO)


def bf16_fwd_kernel(tokens, splits, heads=H, d512=False):
    """Name of the forward kernel the library runs for bf16 rows: 32-head workgroups when
    heads <= 32 or when the 128-head kernel would run fewer than 128 workgroups, else the
    128-head one.  (splits: the 128-head kernel's split count.)"""
    narrow = heads <= 32 or tokens * ((heads + 127) // 128) * splits < 128
    if narrow:
        return "dsa_mla_fwd_narrow_kernel<" + ("512" if d512 else "576") + ">"
    return "dsa_mla_fwd_kernel<" + ("bf16_d512" if d512 else "bf16") + ">"

def fp8_fwd_kernel(tokens, splits, heads=H):
    """The same for 656-B fp8 rows (the same selection rule)."""
    narrow = heads <= 32 or tokens * ((heads + 127) // 128) * splits < 128
    return "dsa_mla_fwd_narrow_kernel<fp8>" if narrow else "dsa_mla_fwd_kernel<fp8>"


CONFIGS = {
    "c1": dict(kind="decode", B=2, s_q=1, seq=8192, block=None, topk=2048, pad=256, fp8=False,
               causal=False),
    "c2": dict(kind="decode", B=64, s_q=1, seq=32768, block=64, topk=2048, pad=0, fp8=False,
               causal=False),
    # three (Q, top-k) sets alternate step by step: one set's 417 MB could partly stay in
    # the 256 MB MALL between steps
    "c3": dict(kind="decode", B=128, s_q=2, seq=65536, block=64, topk=2048, pad=0, fp8=True,
               causal=True, sets=3),
    "c4": dict(kind="decode", B=4, s_q=1, seq=None, block=64, topk=2048, pad=0, fp8=False,
               causal=False, splits=8),
    "c5": dict(kind="prefill", N=8192, topk=2048),
    # MXFP8 split streams (the reference's -dtype fp8 format), C3-shaped: the two tokens of an
    # MTP pair see 2047 and 2048 rows of their batch's CSR list (count-based causality)
    "mx": dict(kind="mxfp8", B=128, s_q=2, rows=2048),
    # DeepSeek-V4 prefill at the reference harness's defaults (mla_v4_host.cc:779-830): N=4096
    # queries, 1024 scattered prefix rows of 65536 pages plus a 128-row extend window, D=512
    "v4": dict(kind="v4", N=4096, topk=1024, pages=65536, window=128, fp8=False),
    "v4fp8": dict(kind="v4", N=4096, topk=1024, pages=65536, window=128, fp8=True),
    # split-K prefill: the harness at -n 16 -topk 0 (every one of 65536 pages, scattered, plus the
    # 128-row window): 16 queries would leave 240 of 256 CUs idle unsplit
    "v4split": dict(kind="v4", N=16, topk=65536, pages=65536, window=128, fp8=False),
    "v4fp8split": dict(kind="v4", N=16, topk=65536, pages=65536, window=128, fp8=True),
    # top-k index selection producing the c3 step's lists: 256 query tokens (B=128, s_q=2),
    # causal lengths n - s_q + j + 1; five score sets (320 MB) alternate, above the 256 MB MALL
    "topk": dict(kind="topk", T=256, n=65536, s_q=2, topk=2048, sets=5),
    # the reference harness's --varlen lists (host.cc:238-261): 8 batches, lengths U[5, 131072]
    "csr_skew": dict(kind="csr", B=8, s_q=1, s=131072),
    # the index scorer in front of the c3 step's top-k: DeepSeek-V3.2 indexer shape (64 index
    # heads of 128), B=128, MTP s_q=2, seq 65536 paged at 64, causal
    "indexer": dict(kind="indexer", B=128, s_q=2, H_I=64, seq=65536, block=64),
}
NAMES = {
    "c1": "bf16 sparse MLA decode B=2 H=128 top-k 2048 (256 pad) flat KV 8192",
    "c2": "bf16 sparse MLA decode B=64 H=128 top-k 2048 paged(64) seq 32768",
    "c3": "fp8-KV(656B) sparse MLA decode B=128 s_q=2 (MTP) H=128 top-k 2048 paged(64) seq 65536 causal"
          " (3 Q / top-k sets alternate step by step)",
    "c4": "bf16 split-top-k decode B=4 H=128 top-k<=2048 seq U[1024,131072] 8 splits + combine",
    "c5": "bf16 sparse MLA prefill N=8192 H=128 top-k 2048 from [0,t]",
    "mx": ("MXFP8 split-stream sparse MLA decode (E8M0 per 32, CSR) B=128 s_q=2 (MTP) H=128, "
           "2048-row lists from a shuffled page table (2 disjoint index sets alternate step by step)"),
    "v4": "DeepSeek-V4 bf16 prefill N=4096 H=128 D=512, top-k 1024 of 65536 pages + window 128, sink",
    "v4fp8": ("DeepSeek-V4 fp8 prefill (448 e4m3 + 14 E8M0 | 64 bf16) N=4096 H=128, top-k 1024 of "
              "65536 pages + window 128, sink"),
    "v4split": "DeepSeek-V4 bf16 prefill N=16 H=128 D=512, -topk 0 (all 65536 pages) + window 128, sink",
    "v4fp8split": "DeepSeek-V4 fp8 prefill N=16 H=128, -topk 0 (all 65536 pages) + window 128, sink",
    "topk": ("top-k index selection for the c3 step: 256 query tokens (B=128 s_q=2), fp32 scores, "
             "causal lengths up to 65536, top-k 2048 (5 score sets alternate step by step)"),
    "csr_skew": ("bf16 CSR decode on the reference's --varlen lists: B=8, lengths U[5, 131072], "
                 "shuffled page table; device work plan against uniform splits"),
    "indexer": ("DSA index scores (sum_h w * relu(q.k)), bf16 in / fp32 out: B=128, s_q=2 (MTP), 64 index "
                "heads of 128, seq 65536 paged at 64, causal (the c3 step's score rows)"),
}


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# CPU baselines run after every GPU timing (see main): (message, leg dict, job)
CPU_JOBS = []


def defer_cpu(args, msg, leg, job):
    """Queue leg["cpu_baseline"] = job() for after the GPU legs and the headline, so that no
    GPU leg starts on a GPU left idle by seconds of CPU work."""
    if not args.no_cpu:
        CPU_JOBS.append((msg, leg, job))


def run_cpu_jobs():
    for msg, leg, job in CPU_JOBS:
        log(msg)
        leg["cpu_baseline"] = job()
    CPU_JOBS.clear()


# ------------------------------------------------------------------ inputs

def make_decode(cfg, dev, seed=2026):
    import torch
    from opfoundry_amd import dsa
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    B, s_q, topk = cfg["B"], cfg["s_q"], cfg["topk"]
    if cfg["seq"] is None:   # config 4: seq_lens ~ U[1024, 131072]
        seq_lens = torch.randint(1024, 131073, (B,), generator=g, device=dev, dtype=torch.int32)
    else:
        seq_lens = torch.full((B,), cfg["seq"], dtype=torch.int32, device=dev)
    max_len = int(seq_lens.max())
    q = torch.randn((B, s_q, H, D_QK), generator=g, device=dev).to(torch.bfloat16)
    bs = cfg["block"]
    if bs:
        mb = (max_len + bs - 1) // bs
        nblk = B * mb
        rows = nblk * bs
        block_table = torch.randperm(nblk, generator=g, device=dev).to(torch.int32).view(B, mb)
    else:
        rows = B * max_len
        block_table = None
    # latent rows ~N(0,1): bf16 cache directly, or quantised by the fp8 cache writer
    if cfg["fp8"]:
        kv = torch.empty((rows, 656), dtype=torch.uint8, device=dev)
        chunk = 1 << 20
        for r0 in range(0, rows, chunk):
            n = min(chunk, rows - r0)
            src = torch.randn((n, D_QK), generator=g, device=dev).to(torch.bfloat16)
            dsa.quantize_kv_fp8(src, kv[r0:r0 + n])
    else:
        kv = torch.randn((rows, D_QK), generator=g, device=dev).to(torch.bfloat16)
    # distinct top-k positions per query token (scattered order), causal bound, -1 padding
    def top_k_set():
        idx = torch.full((B, s_q, topk), -1, dtype=torch.int32, device=dev)
        for b in range(B):
            L = int(seq_lens[b])
            for t in range(s_q):
                hi = L - s_q + t + 1 if cfg["causal"] else L
                n = min(topk - cfg["pad"], hi)
                r = torch.rand((hi,), generator=g, device=dev)
                idx[b, t, :n] = torch.topk(r, n).indices.to(torch.int32)
        return idx
    idx = top_k_set()
    # further (Q, top-k) sets for the rotated timing loop; set 0 is (q, idx)
    sets = [(q, idx)]
    for _ in range(cfg.get("sets", 1) - 1):
        q_k = torch.randn((B, s_q, H, D_QK), generator=g, device=dev).to(torch.bfloat16)
        sets.append((q_k, top_k_set()))
    torch.cuda.synchronize()
    return dict(q=q, kv=kv, idx=idx, seq_lens=seq_lens, block_table=block_table, block_size=bs or 1,
                kv_batch_stride=0 if bs else max_len, causal=cfg["causal"], sets=sets)


def decode_call(d, splits=0, out=None, lse=None, ws=None):
    from opfoundry_amd import dsa
    return dsa.mla_decode(d["q"], d["kv"], d["idx"], SM_SCALE, out, lse, seq_lens=d["seq_lens"],
                          block_table=d["block_table"], block_size=d["block_size"],
                          causal=d["causal"], num_splits=splits,
                          kv_batch_stride=d["kv_batch_stride"], workspace=ws)


def make_prefill(cfg, dev, seed=2031):
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    N, topk = cfg["N"], cfg["topk"]
    q = torch.randn((N, H, D_QK), generator=g, device=dev).to(torch.bfloat16)
    kv = torch.randn((N, D_QK), generator=g, device=dev).to(torch.bfloat16)
    idx = torch.empty((N, topk), dtype=torch.int32, device=dev)
    for r0 in range(0, N, 1024):
        n = min(1024, N - r0)
        r = torch.rand((n, N), generator=g, device=dev)
        t = torch.arange(r0, r0 + n, device=dev)[:, None]
        col = torch.arange(N, device=dev)[None, :]
        r = torch.where(col <= t, r, torch.full_like(r, -1.0))
        v, i = torch.topk(r, topk, dim=1)
        idx[r0:r0 + n] = torch.where(v >= 0, i, torch.full_like(i, -1)).to(torch.int32)
    torch.cuda.synchronize()
    return dict(q=q, kv=kv, idx=idx)


def prefill_step(p, dev):
    """(step, buffers) for one c5 prefill call through the C ABI."""
    import torch
    from opfoundry_amd import dsa
    N = p["q"].shape[0]
    pout = torch.empty((N, H, D_VO), dtype=torch.bfloat16, device=dev)
    plse = torch.empty((N, H), dtype=torch.float32, device=dev)
    a = dsa.make_prefill_args(p["q"], p["kv"], p["idx"], SM_SCALE, pout, plse)
    nbytes = dsa.prefill_workspace_size(a)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev) if nbytes else None
    return prepared_prefill(a, ws), (pout, plse, a, ws)


MX_SETS = 2


def make_mx(cfg, dev, seed=2041):
    """MXFP8 split streams drawn as init_fp8_mla_split (opus_attn/dsa_v32/common/host.cc:207-237):
    per 32-value block e in [0, 3], scale byte e + 127, codes e4m3(N(0,1) * 2^-e); RoPE N(0,1)
    bf16.  The page table is a shuffled permutation of all rows (host.cc:239-262).  For HBM
    honesty the pool holds MX_SETS times the rows one step references, and MX_SETS disjoint
    index sets alternate step by step: consecutive steps touch MX_SETS x 172 MB of distinct rows,
    more than the 256 MB MALL holds (one set alone would stay cache-resident)."""
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    B, s_q, L = cfg["B"], cfg["s_q"], cfg["rows"]

    def streams(n):
        e = torch.randint(0, 4, (n, 16), generator=g, device=dev)
        x = torch.randn((n, 16, 32), generator=g, device=dev) * torch.exp2(-e.float())[:, :, None]
        nope = x.reshape(n, 512).to(torch.float8_e4m3fn).view(torch.uint8)
        rope = torch.randn((n, 64), generator=g, device=dev).to(torch.bfloat16)
        return nope, (e + 127).to(torch.uint8), rope

    total = MX_SETS * B * L
    kv = streams(total)
    qn, qs, qr = streams(B * s_q * H)
    q = (qn.view(B * s_q, H, 512), qs.view(B * s_q, H, 16), qr.view(B * s_q, H, 64))
    indptr = (torch.arange(B + 1, device=dev, dtype=torch.int32) * L)
    perm = torch.randperm(total, generator=g, device=dev).to(torch.int32)
    sets = [perm[i * B * L:(i + 1) * B * L].contiguous() for i in range(MX_SETS)]
    torch.cuda.synchronize()
    return dict(q=q, kv=kv, indptr=indptr, indices=sets[0], sets=sets, s_q=s_q, L=L)


def prepared_mx(args, ws):
    """Steps alternate over the prepared argument blocks (one per index set)."""
    import ctypes
    import torch
    from opfoundry_amd.abi import check, load_library
    fn = load_library().dsa_mla_decode_mxfp8
    aps = [ctypes.byref(a) for a in args]
    turn = [0]
    wp, wb = (ws.data_ptr(), ws.numel()) if ws is not None else (None, 0)
    st = torch.cuda.current_stream().cuda_stream

    def step():
        rc = fn(aps[turn[0]], wp, wb, st)
        turn[0] = (turn[0] + 1) % len(aps)
        if rc:
            check(rc, "dsa_mla_decode_mxfp8")
    return step


def mx_step(m, dev):
    """(step, buffers, plan step) for one MXFP8 decode call through the C ABI.  The CSR work
    plan of the lists is built once (dsa_mla_csr_plan; the index sets share kv_indptr, so one
    plan serves every set) and the timed step reuses it (num_splits = DSA_MLA_SPLITS_PLANNED),
    as the reference harness runs get_mla_metadata_kernel once before its timed loop
    (opus_attn/dsa_v32/common/host.cc:266-272).  The plan step, timed apart, rebuilds it."""
    import ctypes
    import torch
    from opfoundry_amd import abi, dsa
    from opfoundry_amd.abi import check, load_library
    T = m["q"][0].shape[0]
    out = torch.empty((T, H, D_VO), dtype=torch.bfloat16, device=dev)
    lse = torch.empty((T, H), dtype=torch.float32, device=dev)
    args = [dsa.make_decode_mxfp8_args(*m["q"], *m["kv"], m["indptr"], ix, SM_SCALE, out, lse,
                                       s_q=m["s_q"], max_kv_len=m["L"], num_splits=abi.SPLITS_PLANNED)
            for ix in m["sets"]]
    nb = T // m["s_q"]
    ws = dsa.csr_plan(m["indptr"], nb, m["s_q"], H, m["L"])
    lib = load_library()
    st = torch.cuda.current_stream().cuda_stream
    wb = ws.numel()

    def plan_step():
        check(lib.dsa_mla_csr_plan(m["indptr"].data_ptr(), nb, m["s_q"], H, m["L"], ws.data_ptr(), wb, st),
              "dsa_mla_csr_plan")
    return prepared_mx(args, ws), (out, lse, args, ws), plan_step


def cpu_baseline_mx(m, sample_batches):
    """The C oracle on the first `sample_batches` batches (both MTP tokens, all heads),
    scaled to the full step."""
    import numpy as np
    import torch
    import oracle
    s_q, L = m["s_q"], m["L"]
    B = m["indptr"].numel() - 1
    nb = min(sample_batches, B)
    q = tuple(x[:nb * s_q].cpu().numpy() for x in m["q"][:2]) + \
        (m["q"][2][:nb * s_q].cpu().view(torch.int16).numpy().view(np.uint16),)
    kv = (m["kv"][0].cpu().numpy(), m["kv"][1].cpu().numpy(),
          m["kv"][2].cpu().view(torch.int16).numpy().view(np.uint16))
    ip = m["indptr"][:nb + 1].cpu().numpy()
    ix = m["indices"][:nb * L].cpu().numpy()
    nt = oracle.num_threads()
    t0 = time.perf_counter()
    oracle.mla_decode_mxfp8(*q, *kv, ip, ix, s_q, SM_SCALE, num_threads=nt)
    dt = time.perf_counter() - t0
    return dict(value=dt * B / nb * 1e6, unit="us/step", cores=nt, kind="port", cpu_model=cpu_model(),
                sample=f"{nb} of {B} batches ({nb * s_q} query tokens, all 128 heads), {dt:.2f} s "
                       f"measured, scaled x{B / nb:.1f} to one step")


def make_v4(cfg, dev, seed=2051):
    """V4 prefill inputs as the reference harness draws them (mla_v4_host.cc:208-290): per query
    `topk` distinct scattered prefix pages and its last min(i + 1, window) extend rows; values
    N(0,1) (bf16), or init_fp8_dsa_split rows (fp8: 14 blocks of e4m3(N(0,1) * 2^-e), e in
    [0, 3], scale bytes e + 127, pad 0xFF; RoPE N(0,1) bf16); per-head sink N(0,1)."""
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    N, topk, pages, window = cfg["N"], cfg["topk"], cfg["pages"], cfg["window"]
    idp = torch.empty((N, topk), dtype=torch.int32, device=dev)
    for r0 in range(0, N, 256):
        n = min(256, N - r0)
        idp[r0:r0 + n] = torch.rand((n, pages), generator=g, device=dev).argsort(dim=1)[:, :topk].to(torch.int32)
    ipp = torch.arange(N + 1, device=dev, dtype=torch.int32) * topk
    ne = torch.clamp(torch.arange(N, device=dev) + 1, max=window)
    ipe = torch.zeros(N + 1, dtype=torch.int32, device=dev)
    ipe[1:] = torch.cumsum(ne, 0).to(torch.int32)
    qi = torch.repeat_interleave(torch.arange(N, device=dev), ne)
    ide = (qi - (ipe[:-1].long()[qi] + ne[qi] - 1 - torch.arange(qi.numel(), device=dev))).to(torch.int32)

    def rows(n):
        if not cfg["fp8"]:
            return torch.randn((n, 512), generator=g, device=dev).to(torch.bfloat16)
        e = torch.randint(0, 4, (n, 14), generator=g, device=dev)
        x = torch.randn((n, 14, 32), generator=g, device=dev) * torch.exp2(-e.float())[:, :, None]
        nope = torch.full((n, 512), 0xFF, dtype=torch.uint8, device=dev)
        nope[:, :448] = x.reshape(n, 448).to(torch.float8_e4m3fn).view(torch.uint8)
        nope[:, 448:462] = (e + 127).to(torch.uint8)
        return nope, torch.randn((n, 64), generator=g, device=dev).to(torch.bfloat16)

    q, ukv, xkv = rows(N * H), rows(pages), rows(N)
    if cfg["fp8"]:
        q = (q[0].view(N, H, 512), q[1].view(N, H, 64))
    else:
        q = q.view(N, H, 512)
    sink = torch.randn((H,), generator=g, device=dev)
    torch.cuda.synchronize()
    return dict(q=q, ukv=ukv, xkv=xkv, sink=sink, lists=(ipp, idp.view(-1), ipe, ide), fp8=cfg["fp8"],
                rows=N * topk + int(ne.sum()), N=N)


def v4_step(v, dev, splits=0):
    """(step, buffers) for one V4 prefill call through the C ABI (arguments built once), with
    num_splits = splits (0 = the library's automatic choice) and its workspace."""
    import ctypes
    import torch
    from opfoundry_amd import abi
    from opfoundry_amd.abi import check, load_library
    N = v["N"]
    out = torch.empty((N, H, 512), dtype=torch.bfloat16, device=dev)
    lse = torch.empty((N, H), dtype=torch.float32, device=dev)
    ipp, idp, ipe, ide = v["lists"]
    mr = int(((ipp[1:] - ipp[:-1]) + (ipe[1:] - ipe[:-1])).max())
    if v["fp8"]:
        a = abi.PrefillV4Fp8Args()
        a.q_nope, a.q_rope = v["q"][0].data_ptr(), v["q"][1].data_ptr()
        a.unified_kv_nope, a.unified_kv_rope = v["ukv"][0].data_ptr(), v["ukv"][1].data_ptr()
        a.kv_nope, a.kv_rope = v["xkv"][0].data_ptr(), v["xkv"][1].data_ptr()
        a.total_pages, a.total_tokens = v["ukv"][0].shape[0], v["xkv"][0].shape[0]
        a.stride_q_nope_n, a.stride_q_nope_h = H * 512, 512
        a.stride_q_rope_n, a.stride_q_rope_h = H * 64, 64
        a.stride_o_n, a.stride_o_h = H * 512, 512
        a.stride_kv_nope_page, a.stride_kv_rope_page = 512, 64
        fn, name = load_library().dsa_mla_prefill_v4_fp8, "dsa_mla_prefill_v4_fp8"
    else:
        a = abi.PrefillV4Args()
        a.q, a.unified_kv, a.kv = v["q"].data_ptr(), v["ukv"].data_ptr(), v["xkv"].data_ptr()
        a.D = 512
        a.total_pages, a.total_tokens = v["ukv"].shape[0], v["xkv"].shape[0]
        a.stride_qo_n, a.stride_qo_h = H * 512, 512
        a.stride_kv_page = 512
        fn, name = load_library().dsa_mla_prefill_v4, "dsa_mla_prefill_v4"
    a.attn_sink, a.out, a.lse = v["sink"].data_ptr(), out.data_ptr(), lse.data_ptr()
    a.kv_indptr_prefix, a.kv_indices_prefix = ipp.data_ptr(), idp.data_ptr()
    a.kv_indptr_extend, a.kv_indices_extend = ipe.data_ptr(), ide.data_ptr()
    a.N, a.H, a.max_rows = N, H, mr
    a.softmax_scale = 1.0 / math.sqrt(512.0)
    a.num_splits = splits
    ap = ctypes.byref(a)
    st = torch.cuda.current_stream().cuda_stream
    n = ctypes.c_size_t(0)
    check(getattr(load_library(), name + "_workspace_size")(ap, ctypes.byref(n)), name + "_workspace_size")
    ws = torch.empty(max(n.value, 16), dtype=torch.uint8, device=dev)
    wp, wb = ws.data_ptr(), n.value

    def step():
        rc = fn(ap, wp, wb, st)
        if rc:
            check(rc, name)
    return step, (out, lse, a, ws)


def cpu_baseline_v4(v, sample):
    """The C oracle on the first `sample` queries of the V4 step, scaled to the whole step."""
    import numpy as np
    import torch
    import oracle
    N = v["N"]
    n = min(sample, N)
    ipp, idp, ipe, ide = (x.cpu().numpy() for x in v["lists"])
    lists = (ipp[:n + 1], idp[:ipp[n]], ipe[:n + 1], ide[:ipe[n]])
    b16 = lambda t: t.cpu().view(torch.int16).numpy().view(np.uint16)  # noqa: E731
    sink = v["sink"].cpu().numpy()
    scale = 1.0 / math.sqrt(512.0)
    nt = oracle.num_threads()
    if v["fp8"]:
        args = (v["q"][0][:n].cpu().numpy(), b16(v["q"][1][:n]), v["ukv"][0].cpu().numpy(), b16(v["ukv"][1]),
                v["xkv"][0].cpu().numpy(), b16(v["xkv"][1]), sink, *lists, scale)
        t0 = time.perf_counter()
        oracle.mla_prefill_v4_fp8(*args, num_threads=nt)
    else:
        args = (b16(v["q"][:n]), b16(v["ukv"]), b16(v["xkv"]), sink, *lists, scale)
        t0 = time.perf_counter()
        oracle.mla_prefill_v4(*args, num_threads=nt)
    dt = time.perf_counter() - t0
    rows = int(ipp[n] + ipe[n])
    return dict(value=4.0 * H * rows * 512 / dt / 1e12, unit="TFLOP/s", cores=nt, kind="port", cpu_model=cpu_model(),
                sample=f"{n} of {N} queries ({rows} rows), {dt:.2f} s")


def make_topk(cfg, dev, seed=2061):
    """Index-score rows for the top-k leg: `sets` tensors fp32 [T, n] ~ N(0, 1), the causal
    lengths of a B x s_q decode step, and the int32 [T, topk] output."""
    import torch
    g = torch.Generator(device=dev).manual_seed(seed)
    T, n, s_q = cfg["T"], cfg["n"], cfg["s_q"]
    sets = [torch.randn((T, n), generator=g, device=dev, dtype=torch.float32) for _ in range(cfg["sets"])]
    lengths = torch.tensor([n - s_q + (t % s_q) + 1 for t in range(T)], dtype=torch.int32, device=dev)
    out = torch.empty((T, cfg["topk"]), dtype=torch.int32, device=dev)
    return dict(T=T, n=n, topk=cfg["topk"], sets=sets, lengths=lengths, out=out)


def topk_step(tk):
    """One selection call per step through the C ABI, arguments built once; the score sets
    alternate step by step."""
    import torch
    from opfoundry_amd.abi import check, load_library
    f = load_library().dsa_topk_indices
    stream = torch.cuda.current_stream().cuda_stream
    args = [(x.data_ptr(), tk["n"], tk["lengths"].data_ptr(), tk["T"], tk["n"], tk["topk"],
             tk["out"].data_ptr(), tk["topk"], stream) for x in tk["sets"]]
    state = [0]

    def step():
        a = args[state[0] % len(args)]
        state[0] += 1
        rc = f(*a)
        if rc:
            check(rc, "dsa_topk_indices")
    return step


def cpu_baseline_topk(tk, sample):
    """numpy oracle (one core) on the first `sample` tokens of one score set, scaled to the step."""
    import oracle
    n_s = min(sample, tk["T"])
    scores = tk["sets"][0][:n_s].cpu().numpy()
    lengths = tk["lengths"][:n_s].cpu().numpy()
    t0 = time.perf_counter()
    oracle.topk_indices(scores, lengths, tk["topk"])
    dt = time.perf_counter() - t0
    return dict(value=round(dt / n_s * tk["T"] * 1e6, 1), unit="us/step", cores=1, kind="port", cpu_model=cpu_model(),
                sample=f"{n_s} of {tk['T']} tokens, {dt:.2f} s, scaled to the step")


def measured_peaks(dev):
    """Achievable rates on this GPU, beside the spec peaks: a STREAM-like 2 GiB device copy
    (read + write bytes / time) and a large dense bf16 GEMM through torch (hipBLASLt)."""
    import torch
    n = 2 << 30
    src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    copy_ms = time_steps(lambda: dst.copy_(src), 20, None)
    del src, dst
    m = 8192
    a = torch.randn((m, m), device=dev).to(torch.bfloat16)
    b = torch.randn((m, m), device=dev).to(torch.bfloat16)
    c = torch.empty((m, m), device=dev, dtype=torch.bfloat16)
    gemm_ms = time_steps(lambda: torch.matmul(a, b, out=c), 20, None)
    del a, b, c
    torch.cuda.empty_cache()
    return {"hbm_copy_GBps": round(2 * n / (copy_ms * 1e-3) / 1e9, 1),
            "bf16_gemm_TFLOPs": round(2 * m ** 3 / (gemm_ms * 1e-3) / 1e12, 1),
            "how": "device copy of 2 GiB (read + write bytes); torch.matmul bf16 8192^3"}


def count_valid(d) -> int:
    import torch
    idx = d["idx"].long()
    if "seq_lens" not in d:
        return int((idx >= 0).sum())
    B, s_q, _ = idx.shape
    L = d["seq_lens"].long().view(B, 1, 1)
    hi = L - s_q + torch.arange(s_q, device=idx.device).view(1, s_q, 1) + 1 if d["causal"] else L
    return int(((idx >= 0) & (idx < torch.minimum(L, hi))).sum())


def prepared_decode(a, ws):
    """One decode step as a direct C-ABI call with arguments built once: the timed loop
    measures the library, not Python argument checking.  `a` may be a list of argument
    blocks (rotated input sets), used in turn."""
    import ctypes
    import torch
    from opfoundry_amd.abi import check, load_library
    fn = load_library().dsa_mla_decode
    aps = [ctypes.byref(x) for x in (a if isinstance(a, list) else [a])]
    wp, wb = ws.data_ptr(), ws.numel()
    st = torch.cuda.current_stream().cuda_stream
    turn = [0]

    def step():
        rc = fn(aps[turn[0]], wp, wb, st)
        turn[0] = (turn[0] + 1) % len(aps)
        if rc:
            check(rc, "dsa_mla_decode")
    return step


def prepared_prefill(a, ws):
    import ctypes
    import torch
    from opfoundry_amd.abi import check, load_library
    fn = load_library().dsa_mla_prefill
    ap = ctypes.byref(a)
    wp, wb = (ws.data_ptr(), ws.numel()) if ws is not None else (None, 0)
    st = torch.cuda.current_stream().cuda_stream

    def step():
        rc = fn(ap, wp, wb, st)
        if rc:
            check(rc, "dsa_mla_prefill")
    return step


def profiled_traffic(name):
    """HBM bytes per launch of a kernel from the committed rocprofv3 PMC summary
    profiles/<name>: the line 'traffic_bytes_per_launch: N' (FETCH_SIZE and
    WRITE_SIZE scaled by a plain copy's reading).  None if there is no such summary."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


# ------------------------------------------------------------------ timing

WARM_SECONDS = 0.15


def warm_up(fn, warmup):
    """Untimed warm-up: exactly `warmup` steps, or (None) at least 10 steps and WARM_SECONDS of
    back-to-back calls.  The MI355X takes tens of ms of sustained load to settle: the first
    ~30 ms of a decode run are up to 30 % slower than its steady state.  Returns the count."""
    import torch
    if warmup is not None:
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        return warmup
    n, t0 = 0, time.perf_counter()
    while n < 10 or time.perf_counter() - t0 < WARM_SECONDS:
        for _ in range(10):
            fn()
        n += 10
        torch.cuda.synchronize()
    return n


def time_steps(fn, steps, warmup):
    import torch
    warm_up(fn, warmup)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps  # ms per step


def kernel_avg_ms(fn, reps):
    """Average duration of one launch of the dominant kernel, from HIP events recorded on the
    stream the kernel is launched on (torch's current stream), one event pair per launch."""
    import torch
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(reps)]
    torch.cuda.synchronize()
    for a, b in evs:
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    return sum(a.elapsed_time(b) for a, b in evs) / reps


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), for the cpu_baseline records."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def reference_figures(T, s_q, V, row_bytes, ms):
    """The reference harness's own throughput figures (opus_attn/dsa_v32/common/host.cc:
    301-316): flops = 2 * s_q * H * total_kv * (576 + 512) and bytes = q + o + kv with
    q = tokens * H * row_bytes, o = tokens * H * 512 * 2, kv = total_kv * row_bytes, where
    total_kv is the summed per-batch list length (the s_q tokens of a batch share its list
    there).  Here total_kv = V / s_q.  Unlike the algorithmic bytes, kv counts a row once per
    batch although each query token gathers its own list, and q counts Q at the KV row width."""
    total_kv = V / s_q
    q_b = T * H * row_bytes
    o_b = T * H * D_VO * 2
    kv_b = total_kv * row_bytes
    flops = 2.0 * s_q * H * total_kv * (D_QK + D_VO)
    return {"q_o_kv_bytes": int(q_b + o_b + kv_b), "TBps": round((q_b + o_b + kv_b) / (ms * 1e-3) / 1e12, 3),
            "TFLOPs": round(flops / (ms * 1e-3) / 1e12, 1)}


def graph_replay(make_step, calls):
    """Capture `calls` back-to-back steps into one HIP graph and return its replay function.
    For steps of a few microseconds, where timing launches from Python would time the host.
    `make_step` is called with the capture stream current (the step binds that stream)."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step = make_step()
        for _ in range(3):
            step()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for _ in range(calls):
            step()
    torch.cuda.synchronize()
    return g.replay, g


def decode_leg(name, args, dev, dst):
    """One decode configuration (c1, c2, c4) as a leg of the JSON line (dst[name]): step time,
    the fused kernel's roofline, the reference's own figures and the CPU oracle on the same
    inputs.  c1 and c4 (a few microseconds per step) are timed as HIP-graph replays of 20
    steps; c2 as stream launches like the headline.  Unsplit, the step is the fused kernel;
    c4's step also holds the combine kernel, and its roofline is taken over the whole step.
    A generator: inputs are built up to the yield, the timing follows."""
    import torch
    from opfoundry_amd import dsa
    cfg = CONFIGS[name]
    d = make_decode(cfg, dev)
    splits = cfg.get("splits", 0)
    out, lse = decode_call(d, splits)
    torch.cuda.synchronize()
    ref_out, ref_lse = out.clone(), lse.clone()
    a = dsa.make_decode_args(d["q"], d["kv"], d["idx"], SM_SCALE, out, lse, seq_lens=d["seq_lens"],
                             block_table=d["block_table"], block_size=d["block_size"],
                             causal=d["causal"], num_splits=splits, kv_batch_stride=d["kv_batch_stride"])
    ns = dsa.decode_num_splits(a)
    ws = torch.empty(max(dsa.decode_workspace_size(a), 1), dtype=torch.uint8, device=dev)
    graphed = name in ("c1", "c4")
    if graphed:
        calls = 20
        replay, g = graph_replay(lambda: prepared_decode(a, ws), calls)
    yield
    if graphed:
        reps = max(5, args.steps // 4)
        ms = time_steps(replay, reps, args.warmup) / calls
        timing = f"HIP graph of {calls} steps, replayed {reps} times"
    else:
        g = None
        ms = time_steps(prepared_decode(a, ws), args.steps, args.warmup)
        timing = f"{args.steps} stream launches"
    torch.cuda.synchronize()
    # the replayed / launched steps rewrote out and lse: they must equal the eager call's
    same = bool(torch.equal(out.view(torch.int16), ref_out.view(torch.int16)) and torch.equal(lse, ref_lse))
    B, s_q, topk = d["idx"].shape
    V = count_valid(d)
    row_bytes = 656 if cfg["fp8"] else 1152
    T = B * s_q
    alg_bytes = T * H * D_QK * 2 + V * row_bytes + T * H * D_VO * 2 + T * H * 4 + T * topk * 4
    ach = alg_bytes / (ms * 1e-3) / 1e9
    leg = {"workload": f"{name}: {NAMES[name]}", "us_per_step": round(ms * 1e3, 3), "timing": timing,
           "num_splits": ns, "valid_pairs": V, "replay_equals_eager": same,
           "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(ach / HBM_PEAK_GBS, 4),
                        "traffic": profiled_traffic(f"dsa_mla_fwd_bf16_{name}_traffic.txt"),
                        "kernel": bf16_fwd_kernel(T, ns) + (" + dsa_mla_combine_kernel (whole step)"
                                                        if ns > 1 else ""),
                        "kernel_avg_us": round(ms * 1e3, 3), "alg_bytes": alg_bytes,
                        "mfma_frac": round(FLOP_PER_PAIR * V / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4)},
           "reference_figures": reference_figures(T, s_q, V, row_bytes, ms)}
    del g, a, ws, out, lse
    defer_cpu(args, f"CPU baseline (oracle) on {name}", leg,
              lambda: cpu_baseline_decode(d, cfg["fp8"], min(args.cpu_sample, 64), T))
    dst[name] = leg


def make_csr_skew(cfg, dev, seed=2071):
    """CSR lists drawn as the reference harness's --varlen mode (init_kv_page_table,
    opus_attn/dsa_v32/common/host.cc:238-261): each batch's length uniform in [min(5, s), s],
    kv_indices one shuffled permutation of every row; Q and rows ~N(0,1) bf16."""
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    B, s_q, s = cfg["B"], cfg["s_q"], cfg["s"]
    lens = torch.randint(min(5, s), s + 1, (B,), generator=g, device=dev)
    indptr = torch.zeros(B + 1, dtype=torch.int32, device=dev)
    indptr[1:] = torch.cumsum(lens, 0).to(torch.int32)
    total = int(indptr[-1])
    indices = torch.randperm(total, generator=g, device=dev).to(torch.int32)
    q = torch.randn((B * s_q, H, D_QK), generator=g, device=dev).to(torch.bfloat16)
    kv = torch.randn((total, D_QK), generator=g, device=dev).to(torch.bfloat16)
    torch.cuda.synchronize()
    return dict(q=q, kv=kv, indptr=indptr, indices=indices, lens=lens.cpu().tolist(), s_q=s_q, total=total)


def csr_skew_leg(args, dev, dst):
    """The skewed CSR batch through the device work plan (built once, reused by the timed
    calls) and through uniform splits (32 per row: the 256 workgroups the per-row rule gives 8
    rows), timed as stream launches in three alternating rounds (the median of each), with
    the plan's own time, the planned call's roofline and a CPU oracle sample."""
    import ctypes
    import numpy as np
    import torch
    from opfoundry_amd import dsa
    from opfoundry_amd.abi import check, load_library
    c = make_csr_skew(CONFIGS["csr_skew"], dev)
    T = c["q"].shape[0]
    out = torch.empty((T, H, D_VO), dtype=torch.bfloat16, device=dev)
    lse = torch.empty((T, H), dtype=torch.float32, device=dev)
    lib = load_library()
    st = torch.cuda.current_stream().cuda_stream
    steps = {}
    outs = {}
    B, mx_len = len(c["lens"]), max(c["lens"])
    for name, ns in (("plan", -1), ("uniform_32", 32)):
        a = dsa.make_decode_csr_args(c["q"], c["kv"], c["indptr"], c["indices"], SM_SCALE, out, lse,
                                     s_q=c["s_q"], max_kv_len=mx_len, num_splits=ns)
        n = ctypes.c_size_t(0)
        check(lib.dsa_mla_decode_csr_workspace_size(ctypes.byref(a), ctypes.byref(n)), "workspace")
        ws = torch.empty(max(n.value, 1), dtype=torch.uint8, device=dev)
        if ns < 0:
            dsa.csr_plan(c["indptr"], B, c["s_q"], H, mx_len, ws)   # built once, reused by the timed calls
            plan_ws = ws
        ap = ctypes.byref(a)

        def step(ap=ap, ws=ws, nb=n.value):
            rc = lib.dsa_mla_decode_csr(ap, ws.data_ptr(), nb, st)
            if rc:
                check(rc, "dsa_mla_decode_csr")
        step()
        torch.cuda.synchronize()
        outs[name] = (out.clone(), lse.clone())
        steps[name] = (step, ws, a)
    yield
    # a comparison: three alternating rounds, the median of each
    times = {name: [] for name in steps}
    for _ in range(3):
        for name, (step, _, _) in steps.items():
            times[name].append(time_steps(step, args.steps, args.warmup))
    res = {name: sorted(v)[1] for name, v in times.items()}

    def plan_step():
        check(lib.dsa_mla_csr_plan(c["indptr"].data_ptr(), B, c["s_q"], H, mx_len, plan_ws.data_ptr(),
                                   plan_ws.numel(), st), "dsa_mla_csr_plan")
    plan_ms = time_steps(plan_step, args.steps, args.warmup)
    del steps
    V = c["total"]
    alg = T * H * D_QK * 2 + V * 1152 + T * H * D_VO * 2 + T * H * 4 + V * 4
    ms = res["plan"]
    ach = alg / (ms * 1e-3) / 1e9
    d_o = (outs["plan"][0].float() - outs["uniform_32"][0].float()).abs().max().item()
    leg = {"workload": f"csr_skew: {NAMES['csr_skew']}", "lengths": c["lens"],
           "us_per_step": round(ms * 1e3, 3), "uniform_32_us_per_step": round(res["uniform_32"] * 1e3, 3),
           "plan_us": round(plan_ms * 1e3, 3),
           "plan": "built once (dsa_mla_csr_plan) and reused by the timed calls, as the reference "
                   "runs get_mla_metadata before its timed loop; plan_us is one rebuild",
           "plan_speedup": round(res["uniform_32"] / ms, 3), "plan_vs_uniform_max_abs_dO": d_o,
           "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None,
                        "kernel": "dsa_mla_fwd_kernel<bf16> + dsa_mla_combine_plan_kernel (whole step)", "kernel_avg_us": round(ms * 1e3, 3), "alg_bytes": alg}}
    def cpu():
        # the oracle on the first 16384 entries of the longest list, scaled to every entry
        import oracle
        b = int(np.argmax(c["lens"]))
        n = min(16384, c["lens"][b])
        ip = c["indptr"].cpu().numpy()
        rows = c["indices"][ip[b]:ip[b] + n].long()
        q = c["q"][b:b + 1].cpu().view(torch.int16).numpy().view(np.uint16).reshape(1, 1, H, D_QK)
        kv = c["kv"][rows].cpu().view(torch.int16).numpy().view(np.uint16)
        idx = np.arange(n, dtype=np.int32).reshape(1, 1, n)
        nt = oracle.num_threads()
        t0 = time.perf_counter()
        oracle.mla_decode(q, kv, idx, np.full(1, n, np.int32), SM_SCALE, num_threads=nt)
        dt = time.perf_counter() - t0
        return dict(value=dt * V / n * 1e6, unit="us/step", cores=1, kind="port",
                    cpu_model=cpu_model(),
                    sample=f"{n} entries of one row ({dt:.2f} s; one row is one oracle task), "
                           f"scaled x{V / n:.1f} to the step's {V} entries")
    defer_cpu(args, "CPU baseline (oracle) on csr_skew", leg, cpu)
    del out, lse
    dst["csr_skew"] = leg


def make_indexer(cfg, dev, seed=2081):
    """Index-scorer inputs: q bf16 [B, s_q, H_I, 128] and k rows bf16 ~N(0, 1), weights
    N(0, 1/H_I) fp32, the k cache paged at `block` rows through a shuffled block table."""
    import torch
    g = torch.Generator(device=dev).manual_seed(seed)
    B, s_q, H_I, seq, bs = cfg["B"], cfg["s_q"], cfg["H_I"], cfg["seq"], cfg["block"]
    mb = seq // bs
    bt = torch.randperm(B * mb, generator=g, device=dev).to(torch.int32).view(B, mb)
    k = torch.randn((B * mb * bs, 128), generator=g, device=dev).to(torch.bfloat16)
    q = torch.randn((B, s_q, H_I, 128), generator=g, device=dev).to(torch.bfloat16)
    w = torch.randn((B, s_q, H_I), generator=g, device=dev) / math.sqrt(H_I)
    sl = torch.full((B,), seq, dtype=torch.int32, device=dev)
    scores = torch.empty((B, s_q, seq), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    return dict(q=q, w=w, k=k, bt=bt, sl=sl, scores=scores, bs=bs, seq=seq)


def indexer_leg(args, dev, dst):
    """The index scorer on the c3 step's shape: step time, HBM roofline (k rows read once per
    sequence, scores written), MFMA share, and numpy's float64 oracle on a sample."""
    import ctypes
    import numpy as np
    import torch
    from opfoundry_amd import abi
    from opfoundry_amd.abi import check, load_library
    cfg = CONFIGS["indexer"]
    x = make_indexer(cfg, dev)
    B, s_q, H_I, seq = cfg["B"], cfg["s_q"], cfg["H_I"], cfg["seq"]
    a = abi.IndexerArgs()
    a.q, a.weights, a.k_cache = x["q"].data_ptr(), x["w"].data_ptr(), x["k"].data_ptr()
    a.q_stride_b, a.q_stride_t, a.q_stride_h = x["q"].stride(0), x["q"].stride(1), x["q"].stride(2)
    a.k_total_rows, a.k_stride_row = x["k"].shape[0], 128
    a.block_table, a.block_table_stride, a.block_size = x["bt"].data_ptr(), x["bt"].stride(0), x["bs"]
    a.seq_lens, a.scores, a.score_stride = x["sl"].data_ptr(), x["scores"].data_ptr(), seq
    a.B, a.s_q, a.H_I, a.n_cols, a.causal = B, s_q, H_I, seq, 1
    fn = load_library().dsa_indexer_scores
    ap = ctypes.byref(a)
    st = torch.cuda.current_stream().cuda_stream

    def step():
        rc = fn(ap, st)
        if rc:
            check(rc, "dsa_indexer_scores")
    yield
    ms = time_steps(step, args.steps, args.warmup)
    pairs = sum(seq - (s_q - 1 - t) for t in range(s_q)) * B        # (token, position) pairs
    alg = B * seq * 256 + pairs * 4 + x["q"].numel() * 2 + x["w"].numel() * 4
    flops = 2 * 128 * H_I * pairs
    ach = alg / (ms * 1e-3) / 1e9
    leg = {"workload": f"indexer: {NAMES['indexer']}", "us_per_step": round(ms * 1e3, 3),
           "tflops": round(flops / (ms * 1e-3) / 1e12, 1),
           "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": profiled_traffic("dsa_indexer_traffic.txt"),
                        "kernel": "dsa_indexer_kernel<64>", "kernel_avg_us": round(ms * 1e3, 3), "alg_bytes": alg,
                        "mfma_frac": round(flops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4)}}
    def cpu():
        import oracle
        try:
            from threadpoolctl import threadpool_info
            nt = max([i.get("num_threads", 1) for i in threadpool_info() if i.get("user_api") == "blas"] or [1])
        except Exception:
            nt = 1
        nb = 4
        qn = x["q"][:nb].cpu().view(torch.int16).numpy().view(np.uint16)
        wn = x["w"][:nb].cpu().numpy()
        rows = (x["bt"][:nb].long()[:, :, None] * x["bs"] + torch.arange(x["bs"], device=dev)).view(nb, -1)
        kn = x["k"][rows.view(-1)].cpu().view(torch.int16).numpy().view(np.uint16)
        t0 = time.perf_counter()
        oracle.indexer_scores(qn, wn, kn, x["sl"][:nb].cpu().numpy(), k_batch_stride=seq, causal=True, n_cols=seq)
        dt = time.perf_counter() - t0
        return dict(value=dt * B / nb * 1e6, unit="us/step", cores=nt, kind="port",
                    cpu_model=cpu_model(),
                    sample=f"{nb} of {B} sequences (both tokens, all positions; float64 numpy, "
                           f"{nt} BLAS threads), {dt:.2f} s, scaled x{B / nb:.0f}")
    defer_cpu(args, "CPU baseline (numpy float64 oracle) on the indexer", leg, cpu)
    dst["indexer"] = leg


# -------------------------------------------------------------- CPU baseline

def cpu_baseline_decode(d, fmt_fp8, sample_queries, unit_scale):
    """Time the C oracle on `sample_queries` query tokens of the same workload (their rows
    gathered into a compact cache, indices remapped), scaled to the full step."""
    import numpy as np
    import torch
    import oracle
    B, s_q, topk = d["idx"].shape
    picks = [(b, t) for b in range(B) for t in range(s_q)][:sample_queries]
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
    q = torch.stack(qs).view(len(picks), 1, H, D_QK).cpu().view(torch.int16).numpy().view(np.uint16)
    kv = torch.cat(rows).cpu()
    kv = kv.numpy() if fmt_fp8 else kv.view(torch.int16).numpy().view(np.uint16)
    idx = torch.stack(idxs).view(len(picks), 1, topk).to(torch.int32).cpu().numpy()
    sl = np.full(len(picks), kv.shape[0], np.int32)
    nt = oracle.num_threads()
    t0 = time.perf_counter()
    oracle.mla_decode(q, kv, idx, sl, SM_SCALE, num_threads=nt)
    dt = time.perf_counter() - t0
    per_query = dt / len(picks)
    scale = unit_scale / len(picks)
    how = "the whole step" if len(picks) == unit_scale else f"scaled x{scale:.1f} to one step"
    return dict(value=per_query * unit_scale * 1e6, unit="us/step", cores=nt, kind="port", cpu_model=cpu_model(),
                sample=f"{len(picks)} of {B * s_q} query tokens (all 128 heads, full top-k), "
                       f"{dt:.2f} s measured, {how}")


def cpu_baseline_prefill(p, sample_queries, total_pairs):
    import numpy as np
    import torch
    import oracle
    N = p["q"].shape[0]
    sel = torch.linspace(0, N - 1, sample_queries).long()
    q = p["q"][sel].cpu().view(torch.int16).numpy().view(np.uint16)
    kv = p["kv"].cpu().view(torch.int16).numpy().view(np.uint16)
    idx = p["idx"][sel].cpu().numpy()
    pairs = int((p["idx"][sel] >= 0).sum())
    nt = oracle.num_threads()
    t0 = time.perf_counter()
    oracle.mla_prefill(q, kv, idx, SM_SCALE, num_threads=nt)
    dt = time.perf_counter() - t0
    tflops = FLOP_PER_PAIR * pairs / dt / 1e12
    return dict(value=tflops, unit="TFLOP/s", cores=nt, kind="port", cpu_model=cpu_model(),
                sample=f"{sample_queries} of {N} queries ({pairs} pairs), {dt:.2f} s; "
                       f"full step would take {dt * total_pairs / pairs:.0f} s")


# ------------------------------------------------------------- gather floor

def gather_floor(args, dev):
    """The memory floor of the c3 step: libdsa_gather_floor.so moves each query token's 2048
    656-B rows into LDS with the forward kernel's LDS-DMA loads and tile ring, and computes
    nothing.  The three input sets' row lists (block table applied) alternate step by step as
    in the headline; each launch's per-token word sums are checked against torch's."""
    import ctypes
    import torch
    from opfoundry_amd.abi import bind_torch_hip_runtime
    from opfoundry_amd.build import PROBE_LIB_PATH
    if not os.path.exists(PROBE_LIB_PATH):
        raise RuntimeError(f"{PROBE_LIB_PATH} not built: python -m opfoundry_amd.build")
    bind_torch_hip_runtime()
    lib = ctypes.CDLL(PROBE_LIB_PATH)
    lib.dsa_gather_floor.restype = ctypes.c_int
    lib.dsa_gather_floor.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    cfg = CONFIGS["c3"]
    log("building c3 inputs")
    d = make_decode(cfg, dev)
    B, s_q, topk = d["idx"].shape
    ntok, bs, row_bytes = B * s_q, d["block_size"], 656
    kv = d["kv"]
    # per-row sums of the 164 32-bit words, then the expected per-token sums of each set
    words = row_bytes // 4
    rsum = torch.empty(kv.shape[0], dtype=torch.int64, device=dev)
    for r0 in range(0, kv.shape[0], 1 << 20):
        rsum[r0:r0 + (1 << 20)] = kv[r0:r0 + (1 << 20)].view(torch.int32).view(-1, words).long().sum(1)
    sets = []
    for _, idx in d["sets"]:
        assert bool((idx >= 0).all()), "c3 lists hold no padding"
        j = idx.long().view(B, s_q * topk)
        phys = torch.gather(d["block_table"].long(), 1, j // bs) * bs + j % bs
        rows = phys.view(ntok, topk).to(torch.int32).contiguous()
        sets.append((rows, rsum[rows.long()].sum(1) & 0xFFFFFFFF))
    sums = torch.zeros(ntok, dtype=torch.int32, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    row_bytes_step = ntok * topk * row_bytes
    out = {"probe": "gather_floor", "workload": "c3", "tokens": ntok, "rows_per_token": topk,
           "row_bytes": row_bytes, "row_bytes_per_step": row_bytes_step, "results": []}
    for slots in (2, 3, 4):
        turn = [0]

        def step():
            rows = sets[turn[0]][0]
            rc = lib.dsa_gather_floor(kv.data_ptr(), rows.data_ptr(), ntok, topk, row_bytes, slots,
                                      sums.data_ptr(), st)
            if rc:
                raise RuntimeError(f"dsa_gather_floor returned {rc}")
            turn[0] = (turn[0] + 1) % len(sets)
        ok = True
        for k in range(len(sets)):      # one checked launch per set
            turn[0] = k
            step()
            torch.cuda.synchronize()
            ok = ok and bool(torch.equal(sums.long() & 0xFFFFFFFF, sets[k][1]))
        turn[0] = 0
        log(f"gather floor: {slots} tiles in LDS, checksums {'ok' if ok else 'WRONG'}")
        ms = time_steps(step, args.steps, args.warmup)
        out["results"].append({"slots": slots, "us_per_step": ms * 1e3, "checksums_ok": ok,
                               "row_TBps": row_bytes_step / (ms * 1e-3) / 1e12})
    return out


# ------------------------------------------------------------- issue probe

ISSUE_MODES = ("4 independent f16 MFMAs per trip (AGPR accumulators)",
               "+ one 656-B dequant piece after the 4 MFMAs",
               "+ the same piece split between the single MFMAs",
               "+ the split piece and its ds_write_b128",
               "+ 4 v_fma_f32 after every MFMA",
               "one dependent chain of 36 f16 MFMAs (register operands)",
               "four interleaved chains of the same 36 MFMAs",
               "mode 0's MFMAs as compiler builtins (VGPR accumulators)",
               "mode 0 without the s_nop before each MFMA")


def issue_probe(args, dev):
    """What one wave per SIMD hides under its own MFMAs: libdsa_issue_probe.so runs 256
    workgroups of 256 threads (one wave per SIMD) through the modes of ISSUE_MODES; each
    mode's time per trip (4 MFMAs, or 36 for the chain modes) against mode 0's."""
    import ctypes
    import torch
    from opfoundry_amd.abi import bind_torch_hip_runtime
    from opfoundry_amd.build import ISSUE_PROBE_LIB_PATH
    if not os.path.exists(ISSUE_PROBE_LIB_PATH):
        raise RuntimeError(f"{ISSUE_PROBE_LIB_PATH} not built: python -m opfoundry_amd.build")
    bind_torch_hip_runtime()
    lib = ctypes.CDLL(ISSUE_PROBE_LIB_PATH)
    lib.dsa_issue_probe.restype = ctypes.c_int
    lib.dsa_issue_probe.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    out_buf = torch.empty(256 * 256, dtype=torch.float32, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    res = []
    for mode, what in enumerate(ISSUE_MODES):
        chain = mode in (5, 6)
        iters = 2000 if chain else 20000

        def step():
            rc = lib.dsa_issue_probe(mode, iters, out_buf.data_ptr(), st)
            if rc:
                raise RuntimeError(f"dsa_issue_probe returned {rc}")
        ms = time_steps(step, 10, 3)
        mfmas = iters * (36 if chain else 4)
        res.append({"mode": mode, "what": what, "ns_per_mfma": round(ms * 1e6 / mfmas, 2),
                    "ms": round(ms, 4)})
    for r in res:
        if r["mode"] not in (5, 6):
            r["vs_mode0"] = round(r["ns_per_mfma"] / res[0]["ns_per_mfma"], 3)
    return {"probe": "issue", "workgroups": 256, "threads": 256, "results": res}


# --------------------------------------------------------------------- main

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed warm-up steps (default: at least 10 steps and 0.15 s of "
                         "back-to-back calls, until the GPU's clocks have settled)")
    ap.add_argument("--config", default="c3", choices=list(CONFIGS),
                    help="decode workload of the JSON line (c5 only with --kernel-only)")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-legs", action="store_true", help="skip the c1 / c2 / c4 decode legs")
    ap.add_argument("--no-mx", action="store_true")
    ap.add_argument("--no-v4", action="store_true")
    ap.add_argument("--no-topk", action="store_true")
    ap.add_argument("--cpu-topk-sample", type=int, default=64,
                    help="query tokens of the topk step the CPU oracle runs")
    ap.add_argument("--no-peaks", action="store_true")
    ap.add_argument("--cpu-v4-sample", type=int, default=128,
                    help="V4 prefill queries the CPU oracle runs")
    ap.add_argument("--cpu-mx-sample", type=int, default=64,
                    help="batches of the mx step (both MTP tokens) the CPU oracle runs")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-sample", type=int, default=256,
                    help="query tokens of the decode step the CPU oracle runs (256 = all of c3)")
    ap.add_argument("--cpu-prefill-sample", type=int, default=2048,
                    help="prefill queries (evenly spaced over [0, N)) the CPU oracle runs")
    ap.add_argument("--kernel-only", action="store_true",
                    help="only run the timed steps of --config (for profiler runs)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="instead: run --steps plain device copies of MIB MiB (the reference "
                         "kernel that scales rocprof FETCH_SIZE / WRITE_SIZE readings)")
    ap.add_argument("--gather-floor", action="store_true",
                    help="instead: time the gather-only probe (libdsa_gather_floor.so) on the "
                         "c3 step's rows, 2, 3 and 4 tiles in LDS")
    ap.add_argument("--issue-probe", action="store_true",
                    help="instead: run the one-wave-per-SIMD issue probe (libdsa_issue_probe.so): "
                         "which instructions hide under a wave's own MFMAs")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); "
              "multi-GPU runs are not part of this build", file=sys.stderr)
        sys.exit(2)

    import torch
    from opfoundry_amd.abi import load_library
    load_library()
    dev = torch.device("cuda:0")
    cfg = CONFIGS[args.config]

    if args.calibrate_copy:
        n = args.calibrate_copy << 20
        src = torch.randint(0, 255, (n,), dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        ms = time_steps(lambda: dst.copy_(src), args.steps, args.warmup)
        print(json.dumps({"copy_bytes": n, "ms_per_copy": ms,
                          "GBps_read_plus_write": 2 * n / (ms * 1e-3) / 1e9}))
        return
    if args.issue_probe:
        print(json.dumps(issue_probe(args, dev)))
        return
    if args.gather_floor:
        print(json.dumps(gather_floor(args, dev)))
        return
    if cfg["kind"] == "v4":
        if not args.kernel_only:
            ap.error("--config v4 / v4fp8 are reported inside the default JSON line; use them with --kernel-only")
        log(f"building {args.config} inputs")
        v = make_v4(cfg, dev)
        ms = time_steps(v4_step(v, dev)[0], args.steps, args.warmup)
        print(json.dumps({"config": args.config, "ms_per_step": ms}))
        return
    if cfg["kind"] == "indexer":
        if not args.kernel_only:
            ap.error("--config indexer is reported inside the default JSON line; use it with --kernel-only")
        args.no_cpu = True
        out = {}
        for _ in indexer_leg(args, dev, out):
            pass
        print(json.dumps({"config": args.config, "ms_per_step": out["indexer"]["us_per_step"] / 1e3}))
        return
    if cfg["kind"] == "topk":
        if not args.kernel_only:
            ap.error("--config topk is reported inside the default JSON line; use it with --kernel-only")
        log("building topk inputs")
        tk = make_topk(cfg, dev)
        ms = time_steps(topk_step(tk), args.steps, args.warmup)
        print(json.dumps({"config": args.config, "ms_per_step": ms}))
        return
    if cfg["kind"] == "mxfp8":
        if not args.kernel_only:
            ap.error("--config mx is reported inside the default JSON line; use it with --kernel-only")
        log("building mx inputs")
        m = make_mx(cfg, dev)
        ms = time_steps(mx_step(m, dev)[0], args.steps, args.warmup)
        print(json.dumps({"config": args.config, "ms_per_step": ms}))
        return
    if cfg["kind"] == "prefill":
        if not args.kernel_only:
            ap.error("--config c5 is reported inside the default JSON line; use it with --kernel-only")
        log("building c5 prefill inputs")
        p = make_prefill(cfg, dev)
        ms = time_steps(prefill_step(p, dev)[0], args.steps, args.warmup)
        print(json.dumps({"config": args.config, "ms_per_step": ms}))
        return

    log(f"building {args.config} inputs")
    d = make_decode(cfg, dev)
    splits = cfg.get("splits", 0)
    out, lse = decode_call(d, splits)
    from opfoundry_amd import dsa
    a_sets = [dsa.make_decode_args(q_k, d["kv"], idx_k, SM_SCALE, out, lse, seq_lens=d["seq_lens"],
                                   block_table=d["block_table"], block_size=d["block_size"],
                                   causal=d["causal"], num_splits=splits,
                                   kv_batch_stride=d["kv_batch_stride"]) for q_k, idx_k in d["sets"]]
    a = a_sets[0]
    ns = dsa.decode_num_splits(a)
    ws_bytes = dsa.decode_workspace_size(a)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    step = prepared_decode(a_sets, ws)

    if args.kernel_only:
        log(f"timing {args.steps} steps after warm-up (splits={ns})")
        warm_up(step, args.warmup)
        ms = time_steps(step, args.steps, 0)
        print(json.dumps({"config": args.config, "ms_per_step": ms}))
        return

    res = {}
    legs_before_headline(args, dev, res)

    # The headline is timed right after the other legs, before any CPU baseline: its W
    # warm-up steps then start on a GPU whose clocks have settled under sustained load.  From a cold start (or after ~2 s idle) the first ~100 c3 steps run
    # up to 30 % slower while the GPU's power management settles, whatever the kernel.
    log(f"timing {args.steps} steps after warm-up (splits={ns})")
    n_warm = warm_up(step, args.warmup)
    ms = time_steps(step, args.steps, 0)
    B, s_q, topk = d["idx"].shape
    V = count_valid(d)
    row_bytes = 656 if cfg["fp8"] else 1152
    alg_bytes = (B * s_q * H * D_QK * 2 + V * row_bytes + B * s_q * H * D_VO * 2 + B * s_q * H * 4
                 + B * s_q * topk * 4)
    flops = FLOP_PER_PAIR * V
    # dominant kernel: the fused decode kernel.  Unsplit, a step is that one kernel and its
    # launch duration is the HIP-event average over the timed region (event pairs around
    # single launches would add a cache flush to each).  Split, the step also holds the
    # combine kernel: time the fused kernel alone with per-launch events.
    dom_ms = ms if ns == 1 else kernel_avg_ms(step, max(10, args.steps // 2))
    achieved = alg_bytes / (dom_ms * 1e-3) / 1e9
    if cfg["fp8"] and not args.no_legs:
        # the headline's lists (set 0) with fewer heads, the per-GPU head counts of tensor-
        # parallel DeepSeek-V3.2 serving (128 heads over 8 or 4 GPUs): 32-head workgroups
        res["decode_heads"] = heads_leg(d, args, dev)
    legs = res
    res = {
        "metric": "sparse-MLA decode us/step + achieved HBM TB/s; prefill TFLOP/s (1 MI355X)",
        "value": round(ms * 1e3, 3),
        "unit": "us/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": n_warm,
        "ms_per_step": round(ms, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3 KV -> f16 MFMA, f32 accumulate" if cfg["fp8"] else "bf16 MFMA, f32 accumulate",
        "data": "synthetic",
        "config": {"workload": f"{args.config}: {NAMES[args.config]}", "kv_format":
                   "fp8_e4m3_656B" if cfg["fp8"] else "bf16_1152B", "num_splits": ns,
                   "valid_pairs": V, "parallelism": "none (1 GPU)"},
        "hbm_TBps": round(alg_bytes / (ms * 1e-3) / 1e12, 3),
        "tflops": round(flops / (ms * 1e-3) / 1e12, 1),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": profiled_traffic(f"dsa_mla_fwd_{'fp8' if cfg['fp8'] else 'bf16'}_"
                                                 f"{args.config}_traffic.txt"),
                     "kernel": "dsa_mla_fwd_kernel<fp8>" if cfg["fp8"] else "dsa_mla_fwd_kernel<bf16>",
                     "kernel_avg_us": round(dom_ms * 1e3, 3), "alg_bytes": alg_bytes,
                     "mfma_frac": round(flops / (dom_ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4)},
    }
    del out, lse, ws, step, a
    res.update(legs)
    res["reference_figures"] = reference_figures(B * s_q, s_q, V, row_bytes, ms)
    # every CPU baseline, after all GPU timing
    defer_cpu(args, "CPU baseline (oracle) on a bounded sample of the headline", res,
              lambda: cpu_baseline_decode(d, cfg["fp8"], args.cpu_sample, B * s_q))
    run_cpu_jobs()
    del d
    torch.cuda.empty_cache()
    if not args.no_peaks:
        log("measured peaks (copy, bf16 GEMM)")
        pk = measured_peaks(dev)
        # information only: every roofline fraction is taken against the spec peaks
        res["measured_peaks"] = pk
    print(json.dumps(res))


def heads_leg(d, args, dev):
    """The headline's fp8 lists (set 0: its Q's first H heads, its top-k lists, its cache) at
    H = 16 and 32.  HBM-bound like the headline: the fraction counts the rows each token
    attends once, plus Q, O, LSE and the lists of H heads."""
    import torch
    from opfoundry_amd import dsa
    q0, idx0 = d["sets"][0]
    B, s_q, topk = idx0.shape
    V = count_valid(d)
    out = {}
    for Hs in (16, 32):
        qh = q0[:, :, :Hs].contiguous()
        hout = torch.empty((B, s_q, Hs, D_VO), dtype=torch.bfloat16, device=dev)
        hlse = torch.empty((B, s_q, Hs), dtype=torch.float32, device=dev)
        a = dsa.make_decode_args(qh, d["kv"], idx0, SM_SCALE, hout, hlse, seq_lens=d["seq_lens"],
                                 block_table=d["block_table"], block_size=d["block_size"], causal=d["causal"],
                                 num_splits=0, kv_batch_stride=d["kv_batch_stride"])
        ns = dsa.decode_num_splits(a)
        ws = torch.empty(max(dsa.decode_workspace_size(a), 1), dtype=torch.uint8, device=dev)
        step = prepared_decode([a], ws)
        ms = time_steps(step, args.steps, args.warmup)
        alg = (B * s_q * Hs * D_QK * 2 + V * 656 + B * s_q * Hs * D_VO * 2 + B * s_q * Hs * 4
               + B * s_q * topk * 4)
        dom_ms = ms if ns == 1 else kernel_avg_ms(step, max(10, args.steps // 2))
        ach = alg / (dom_ms * 1e-3) / 1e9
        out[f"H{Hs}"] = {
            "workload": f"c3 lists (set 0), H={Hs}", "us_per_step": round(ms * 1e3, 3), "num_splits": ns,
            "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None,
                         "kernel": fp8_fwd_kernel(B * s_q, ns, heads=Hs), "kernel_avg_us": round(dom_ms * 1e3, 3),
                         "alg_bytes": alg}}
        del ws, hout, hlse
    return out


def legs_before_headline(args, dev, res):
    """Every leg but the headline, into res: the decode legs, csr_skew, top-k, the indexer, the
    V4 prefills (split-K rows first), mx and the c5 prefill.  Each leg is a generator that
    builds its inputs up to a yield: every input is built first, then the legs are timed back
    to back, so no leg starts on a GPU left idle by input generation or CPU work.  The CPU
    baselines are queued (defer_cpu) and run after the headline."""
    import torch
    gens = []
    # order: light legs first, the MFMA-heavy ones last and c5 right before the headline.  A
    # change from light to heavy load costs ~20 ms of lower clocks while the GPU's power
    # management settles (the first ~100 c3 steps after a light leg run up to 30 % slower);
    # heavy after heavy does not.
    if not args.no_legs:
        res["decode_legs"] = {}
        for name in ("c1", "c4", "c2"):
            if name != args.config:
                gens.append((f"decode leg {name}", decode_leg(name, args, dev, res["decode_legs"])))
        gens.append(("csr_skew leg (device work plan against uniform splits)", csr_skew_leg(args, dev, res)))
    if not args.no_topk:
        gens.append(("topk leg", topk_leg(args, dev, res)))
    if not args.no_legs:
        gens.append(("indexer leg", indexer_leg(args, dev, res)))
    if not args.no_v4:
        res["v4_prefill"] = {}
        for name in ("v4split", "v4fp8split"):
            gens.append((f"{name} leg (split-K against unsplit)", v4_split_leg(name, args, dev, res["v4_prefill"])))
        for name in ("v4", "v4fp8"):
            gens.append((f"{name} leg", v4_leg(name, args, dev, res["v4_prefill"])))
    if not args.no_mx:
        gens.append(("mx (MXFP8 split-stream) leg", mx_leg(args, dev, res)))
    if not args.no_prefill:
        gens.append(("c5 prefill", c5_leg(args, dev, res)))
    for msg, g in gens:
        log(f"building inputs: {msg}")
        next(g)
    torch.cuda.synchronize()
    for msg, g in gens:
        log(f"timing: {msg}")
        for _ in g:
            pass


def c5_leg(args, dev, res):
    p = make_prefill(CONFIGS["c5"], dev)
    pstep, keep = prefill_step(p, dev)
    psteps = max(3, args.steps // 5)
    yield
    pms = time_steps(pstep, psteps, args.warmup)
    pk_ms = pms       # one kernel per step: the timed region's average launch
    del keep
    pV = int((p["idx"] >= 0).sum())
    pfl = FLOP_PER_PAIR * pV
    res["prefill"] = {"workload": f"c5: {NAMES['c5']}", "ms_per_step": round(pms, 4),
                      "tflops": round(pfl / (pms * 1e-3) / 1e12, 1), "valid_pairs": pV,
                      "roofline": {"bound": "mfma", "achieved": round(pfl / (pk_ms * 1e-3) / 1e12, 1),
                                   "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                   "frac": round(pfl / (pk_ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
                                   "traffic": profiled_traffic("dsa_mla_fwd_bf16_c5_traffic.txt"),
                                   "kernel": "dsa_mla_fwd_kernel<bf16>",
                                   "kernel_avg_us": round(pk_ms * 1e3, 1)}}
    defer_cpu(args, "CPU baseline (oracle) on a c5 sample", res["prefill"],
              lambda: cpu_baseline_prefill(p, args.cpu_prefill_sample, pV))
    # The c5 lists with fewer heads (the first H heads of c5's Q): H <= 32 runs on 32-head
    # workgroups, H = 64 on 128-head ones; the fraction is of useful flops (H heads).
    import torch
    from opfoundry_amd import dsa
    res["prefill_heads"] = {}
    for Hs in (16, 32, 64):
        qh = p["q"][:, :Hs].contiguous()
        hout = torch.empty((qh.shape[0], Hs, D_VO), dtype=torch.bfloat16, device=dev)
        hlse = torch.empty((qh.shape[0], Hs), dtype=torch.float32, device=dev)
        a = dsa.make_prefill_args(qh, p["kv"], p["idx"], SM_SCALE, hout, hlse)
        nb = dsa.prefill_workspace_size(a)
        hws = torch.empty(nb, dtype=torch.uint8, device=dev) if nb else None
        hstep = prepared_prefill(a, hws)
        hms = time_steps(hstep, psteps, args.warmup)
        hfl = pfl * Hs / H
        res["prefill_heads"][f"H{Hs}"] = {
            "workload": f"c5 lists, H={Hs}", "ms_per_step": round(hms, 4),
            "tflops": round(hfl / (hms * 1e-3) / 1e12, 1),
            "vs_c5_time": round(hms / pms, 3), "ideal_vs_c5_time": round(Hs / H, 3),
            "roofline": {"bound": "mfma", "achieved": round(hfl / (hms * 1e-3) / 1e12, 1),
                         "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(hfl / (hms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
                         "traffic": None, "kernel": bf16_fwd_kernel(qh.shape[0], 1, heads=Hs),
                         "kernel_avg_us": round(hms * 1e3, 1)}}
        del hws, hout, hlse


def mx_leg(args, dev, res):
    m = make_mx(CONFIGS["mx"], dev)
    mstep, keep, mplan = mx_step(m, dev)
    yield
    mms = time_steps(mstep, args.steps, args.warmup)   # warm-up as the decode leg
    plan_ms = time_steps(mplan, args.steps, args.warmup)
    del keep
    T = m["q"][0].shape[0]
    L = m["L"]
    mV = sum(L - (m["s_q"] - 1 - t) for t in range(m["s_q"])) * (T // m["s_q"])
    # both tokens of an MTP pair share their batch's list: each row counts once
    nb = T // m["s_q"]
    m_bytes = T * H * (512 + 16 + 128) + nb * L * (656 + 4) + T * H * D_VO * 2 + T * H * 4
    mach = m_bytes / (mms * 1e-3) / 1e9
    res["mxfp8"] = {"workload": f"mx: {NAMES['mx']}", "us_per_step": round(mms * 1e3, 3),
                    "plan": "CSR work plan built once and reused (num_splits = DSA_MLA_SPLITS_PLANNED), "
                            "as the reference times its decode after get_mla_metadata",
                    "plan_us": round(plan_ms * 1e3, 3),
                    "dtype": "MXFP8 (e4m3 + E8M0) KV and Q -> exact bf16 dequant, bf16 MFMA, f32 accumulate",
                    "valid_pairs": mV, "hbm_TBps": round(m_bytes / (mms * 1e-3) / 1e12, 3),
                    "roofline": {"bound": "hbm", "achieved": round(mach, 1), "peak": HBM_PEAK_GBS,
                                 "unit": "GB/s", "frac": round(mach / HBM_PEAK_GBS, 4),
                                 "traffic": profiled_traffic("dsa_mla_fwd_mxfp8_mx_traffic.txt"),
                                 "kernel": "dsa_mla_fwd_kernel<mxfp8>",
                                 "kernel_avg_us": round(mms * 1e3, 3), "alg_bytes": m_bytes,
                                 "mfma_frac": round(FLOP_PER_PAIR * mV / (mms * 1e-3) / 1e12
                                                    / BF16_PEAK_TFLOPS, 4)}}
    defer_cpu(args, "CPU baseline (oracle) on an MXFP8 sample", res["mxfp8"],
              lambda: cpu_baseline_mx(m, args.cpu_mx_sample))


def v4_leg(name, args, dev, dst):
    v = make_v4(CONFIGS[name], dev)
    vstep, keep = v4_step(v, dev)
    vsteps = max(5, args.steps // 5)
    yield
    vms = time_steps(vstep, vsteps, args.warmup)    # one kernel per step
    vfl = 4.0 * H * v["rows"] * 512                   # the reference's count (mla_v4_host.cc:358)
    leg = {"workload": f"{name}: {NAMES[name]}", "ms_per_step": round(vms, 4),
           "tflops": round(vfl / (vms * 1e-3) / 1e12, 1), "rows": v["rows"],
           "roofline": {"bound": "mfma", "achieved": round(vfl / (vms * 1e-3) / 1e12, 1),
                        "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                        "frac": round(vfl / (vms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
                        "traffic": profiled_traffic(f"dsa_mla_fwd_{name}_traffic.txt"),
                        "kernel": "dsa_mla_fwd_kernel<mxfp8_v4>" if v["fp8"] else bf16_fwd_kernel(v["N"], 1, d512=True),
                        "kernel_avg_us": round(vms * 1e3, 1)}}
    del keep
    defer_cpu(args, f"CPU baseline (oracle) on a {name} sample", leg,
              lambda: cpu_baseline_v4(v, args.cpu_v4_sample))
    dst[name] = leg


def v4_split_leg(name, args, dev, dst):
    """Split-K: few queries with long lists (the harness at -n 16 -topk 0), the automatic split
    count against one workgroup per query, in three alternating rounds (the median of each)."""
    import torch
    v = make_v4(CONFIGS[name], dev)
    runs = {"split": v4_step(v, dev, 0), "unsplit": v4_step(v, dev, 1)}
    ws = runs["split"][1][3]
    ns = (ws.numel() - 256) // (v["N"] * H * 513 * 4) if ws.numel() > 16 else 1
    vsteps = max(5, args.steps // 5)
    yield
    times = {k: [] for k in runs}
    for _ in range(3):
        for k, (st_, _) in runs.items():
            times[k].append(time_steps(st_, vsteps, args.warmup))
    t = {k: sorted(x)[1] for k, x in times.items()}
    torch.cuda.synchronize()
    d_o = (runs["split"][1][0].float() - runs["unsplit"][1][0].float()).abs().max().item()
    vfl = 4.0 * H * v["rows"] * 512
    tf = vfl / (t["split"] * 1e-3) / 1e12
    dst[name] = {
        "workload": f"{name}: {NAMES[name]}", "num_splits": ns, "rows": v["rows"],
        "ms_per_step": round(t["split"], 4), "unsplit_ms_per_step": round(t["unsplit"], 4),
        "split_speedup": round(t["unsplit"] / t["split"], 2), "split_vs_unsplit_max_abs_dO": d_o,
        "tflops": round(tf, 1),
        "roofline": {"bound": "mfma", "achieved": round(tf, 1), "peak": BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tf / BF16_PEAK_TFLOPS, 4), "traffic": None,
                     "kernel": ("dsa_mla_fwd_kernel<mxfp8_v4>" if v["fp8"] else bf16_fwd_kernel(v["N"], ns, d512=True))
                               + " + dsa_mla_combine_kernel (whole step)",
                     "kernel_avg_us": round(t["split"] * 1e3, 1)}}


def topk_leg(args, dev, res):
    tk = make_topk(CONFIGS["topk"], dev)
    tstep = topk_step(tk)
    yield
    tms = time_steps(tstep, args.steps, args.warmup)
    tk_ms = tms       # one kernel per step: the timed region's average launch
    t_bytes = 4 * int(tk["lengths"].sum().item()) + 4 * tk["T"] * tk["topk"]
    tach = t_bytes / (tk_ms * 1e-3) / 1e9
    res["topk"] = {"workload": f"topk: {NAMES['topk']}", "us_per_step": round(tms * 1e3, 3),
                   "dtype": "fp32 scores -> int32 positions",
                   "roofline": {"bound": "hbm", "achieved": round(tach, 1), "peak": HBM_PEAK_GBS,
                                "unit": "GB/s", "frac": round(tach / HBM_PEAK_GBS, 4),
                                "traffic": profiled_traffic("dsa_topk_traffic.txt"),
                                "kernel": "dsa_topk_reg_kernel", "kernel_avg_us": round(tk_ms * 1e3, 3),
                                "alg_bytes": t_bytes}}
    defer_cpu(args, "CPU baseline (oracle) on a topk sample", res["topk"],
              lambda: cpu_baseline_topk(tk, args.cpu_topk_sample))


if __name__ == "__main__":
    main()
