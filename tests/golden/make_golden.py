"""Seeded, library-independent generators for the golden fixtures, and the
script that writes them.

    python tests/golden/make_golden.py        # rewrites tests/golden/*.npz

Inputs are never stored: they are regenerated bit-exactly from a seed by a
counter-based generator (splitmix64 over (seed, stream, index), Box-Muller
for N(0,1), partial Fisher-Yates for distinct top-k positions as in
opus_attn/dsa_v4/common/mla_v4_host.cc:270-281), so the fixture files only
hold expected outputs plus a SHA-256 of the inputs they belong to.  The
expected outputs are written by the CPU oracle (oracle/dsa_oracle.c), whose
arithmetic is pinned independently by tests/test_oracle_*.py.

Fixtures:
  c1_bf16.npz      BASELINE config 1 at full size: B=2, s_q=1, H=128, flat KV
                   [2, 8192, 576] bf16, top-k 2048 distinct of [0, 8192) with
                   the last 256 entries = -1, sm_scale = 1/sqrt(192)
  c3s_fp8.npz      config 3 scaled down: B=1, s_q=2 (MTP), H=128, fp8 656-B
                   rows, seq_len 4096 paged at 64 (shuffled block table),
                   top-k 1024 distinct of [0, L - 2 + t], causal
"""
from __future__ import annotations

import hashlib
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

M64 = np.uint64(0xFFFFFFFFFFFFFFFF)
SM_SCALE = 1.0 / math.sqrt(192.0)


def splitmix64(x: np.ndarray) -> np.ndarray:
    x = x.astype(np.uint64)
    with np.errstate(over="ignore"):
        x = x + np.uint64(0x9E3779B97F4A7C15)
        z = x
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def raw_u64(seed: int, stream: int, n: int) -> np.ndarray:
    base = splitmix64(np.array([seed * 1_000_003 + stream], np.uint64))[0]
    with np.errstate(over="ignore"):
        return splitmix64(np.arange(n, dtype=np.uint64) + base)


def uniform(seed: int, stream: int, n: int) -> np.ndarray:
    """n doubles in (0, 1)."""
    return ((raw_u64(seed, stream, n) >> np.uint64(11)).astype(np.float64) + 0.5) * 2.0 ** -53


def normal(seed: int, stream: int, n: int) -> np.ndarray:
    """n N(0,1) float32 values (Box-Muller over two uniform streams)."""
    u1 = uniform(seed, 2 * stream, n)
    u2 = uniform(seed, 2 * stream + 1, n)
    return (np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)).astype(np.float32)


def distinct(seed: int, stream: int, high: int, k: int) -> np.ndarray:
    """k distinct positions of [0, high) in scattered order (partial Fisher-Yates)."""
    r = raw_u64(seed, stream, k)
    perm = np.arange(high, dtype=np.int64)
    for i in range(k):
        j = i + int(r[i] % np.uint64(high - i))
        perm[i], perm[j] = perm[j], perm[i]
    return perm[:k].astype(np.int32)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns, round to nearest even (finite inputs)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)
    return u.astype(np.uint16)


def sha256(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        if a is None:
            h.update(b"none")
            continue
        a = np.ascontiguousarray(a)
        h.update(str(a.dtype).encode() + str(a.shape).encode())
        h.update(a.tobytes())
    return h.hexdigest()


def c1_inputs(seed: int = 2026):
    B, H, L, topk, pad = 2, 128, 8192, 2048, 256
    q = bf16_bits(normal(seed, 2, B * H * 576)).reshape(B, 1, H, 576)
    kv = bf16_bits(normal(seed, 4, B * L * 576)).reshape(B * L, 576)
    idx = np.full((B, 1, topk), -1, np.int32)
    for b in range(B):
        idx[b, 0, :topk - pad] = distinct(seed, 100 + b, L, topk - pad)
    seq_lens = np.full(B, L, np.int32)
    return dict(q=q, kv=kv, indices=idx, seq_lens=seq_lens, block_table=None, block_size=1,
                kv_batch_stride=L, causal=False)


def c3s_inputs(seed: int = 2027):
    import oracle
    B, s_q, H, L, bs, topk = 1, 2, 128, 4096, 64, 1024
    q = bf16_bits(normal(seed, 2, B * s_q * H * 576)).reshape(B, s_q, H, 576)
    nblk = B * L // bs
    src = oracle.bf16_to_f32(bf16_bits(normal(seed, 4, nblk * bs * 576))).reshape(-1, 576)
    kv = oracle.quantize_rows_656(src)
    order = np.argsort(raw_u64(seed, 6, nblk), kind="stable").astype(np.int32)
    block_table = order.reshape(B, L // bs)
    idx = np.full((B, s_q, topk), -1, np.int32)
    for b in range(B):
        for t in range(s_q):
            hi = L - s_q + t + 1
            idx[b, t] = distinct(seed, 100 + 2 * b + t, hi, topk)
    seq_lens = np.full(B, L, np.int32)
    return dict(q=q, kv=kv, indices=idx, seq_lens=seq_lens, block_table=block_table,
                block_size=bs, kv_batch_stride=0, causal=True)


CASES = {"c1_bf16": c1_inputs, "c3s_fp8": c3s_inputs}


def input_digest(d) -> str:
    return sha256(d["q"], d["kv"], d["indices"], d["seq_lens"], d["block_table"])


def run_oracle(d):
    import oracle
    return oracle.mla_decode(d["q"], d["kv"], d["indices"], d["seq_lens"], SM_SCALE,
                             block_table=d["block_table"], block_size=d["block_size"],
                             kv_batch_stride=d["kv_batch_stride"], causal=d["causal"])


def load(name: str):
    z = np.load(os.path.join(HERE, name + ".npz"), allow_pickle=False)
    return {k: z[k] for k in z.files}


def main():
    for name, fn in CASES.items():
        d = fn()
        o, lse = run_oracle(d)
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, o=o, lse=lse, input_sha256=np.array(input_digest(d)),
                            sm_scale=np.array(SM_SCALE, np.float64))
        print(f"{path}: O {o.shape} LSE {lse.shape} inputs {input_digest(d)[:16]}")


if __name__ == "__main__":
    main()
