"""Seeded input builders and comparison helpers shared by the tests.

Inputs follow the generation conventions of the reference harnesses: N(0,1)
q / KV rounded to bf16, distinct uniformly drawn top-k positions in scattered
order (opus_attn/dsa_v4/common/mla_v4_host.cc:243-283), -1 padding, paged
caches with a random permutation of physical blocks, and NaN-poisoned rows
the index list never selects (mla_v4_host.cc:295-323) so a wrong gather
shows up as NaN.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

import oracle

D_QK, D_VO = 576, 512
SM_SCALE = 1.0 / math.sqrt(192.0)
O_ATOL = 2e-2          # bf16 O: max-abs error bound (every element; one bf16 step where |O| >= 4, o_bound)
LSE_RTOL = 1e-3        # LSE: |got - ref| <= LSE_RTOL * (1 + |ref|), see lse_rel


@dataclass
class DecodeCase:
    q: np.ndarray                 # uint16 bf16 [B, s_q, H, 576]
    kv: np.ndarray                # uint16 [rows, 576] (bf16) or uint8 [rows, 656] (fp8)
    indices: np.ndarray           # int32 [B, s_q, topk]
    seq_lens: np.ndarray          # int32 [B]
    block_table: np.ndarray | None = None
    block_size: int = 1
    kv_batch_stride: int = 0
    causal: bool = False
    sm_scale: float = SM_SCALE
    extra: dict = field(default_factory=dict)

    @property
    def shape(self):
        return tuple(self.q.shape[:3]) + (self.indices.shape[2],)

    def oracle(self, num_threads=0):
        return oracle.mla_decode(self.q, self.kv, self.indices, self.seq_lens, self.sm_scale,
                                 block_table=self.block_table, block_size=self.block_size,
                                 kv_batch_stride=self.kv_batch_stride, causal=self.causal,
                                 num_threads=num_threads)


def bf16_rows(rng, n):
    return oracle.normal_bf16(rng, (n, D_QK))


def fp8_rows(rng, n):
    """656-byte rows: NoPE ~N(0,1) quantised per 128 (scale amax/448), bf16 RoPE."""
    src = oracle.bf16_to_f32(bf16_rows(rng, n))
    return oracle.quantize_rows_656(src)


def poison(kv: np.ndarray, keep_rows: np.ndarray) -> None:
    """Overwrite every cache row not in keep_rows with NaN (bf16 0x7FC0 / fp8 0xFF)."""
    mask = np.ones(kv.shape[0], bool)
    mask[keep_rows] = False
    if kv.dtype == np.uint16:
        kv[mask] = 0x7FC0
    else:
        kv[mask] = 0xFF


def flat_case(seed=2026, B=2, s_q=1, H=128, kv_len=8192, topk=2048, pad=256, fp8=False,
              causal=False, poison_unused=True):
    """Per-batch flat caches [B, kv_len, row] (BASELINE config 1 shape by default)."""
    rng = np.random.default_rng(seed)
    q = oracle.normal_bf16(rng, (B, s_q, H, D_QK))
    kv = fp8_rows(rng, B * kv_len) if fp8 else bf16_rows(rng, B * kv_len)
    idx = np.full((B, s_q, topk), -1, np.int32)
    for b in range(B):
        for t in range(s_q):
            hi = kv_len - s_q + t + 1 if causal else kv_len
            n = min(topk - pad, hi)
            idx[b, t, :n] = oracle.distinct_indices(rng, hi, n)
    seq_lens = np.full(B, kv_len, np.int32)
    if poison_unused:
        used = (idx + (np.arange(B, dtype=np.int64)[:, None, None] * kv_len))[idx >= 0]
        poison(kv, np.unique(used))
    return DecodeCase(q, kv, idx, seq_lens, None, 1, kv_len, causal)


def paged_case(seed=7, B=4, s_q=1, H=128, seq_len=4096, block_size=64, topk=2048, fp8=False,
               causal=False, varlen=False, pad_to=None, poison_unused=True):
    """Paged cache: every sequence owns seq_len/block_size blocks of one shuffled pool."""
    rng = np.random.default_rng(seed)
    q = oracle.normal_bf16(rng, (B, s_q, H, D_QK))
    if varlen:
        seq_lens = rng.integers(1, seq_len + 1, size=B).astype(np.int32)
    else:
        seq_lens = np.full(B, seq_len, np.int32)
    mb = (seq_len + block_size - 1) // block_size
    nblk = B * mb
    perm = rng.permutation(nblk).astype(np.int32)
    block_table = perm.reshape(B, mb)
    rows = nblk * block_size
    kv = fp8_rows(rng, rows) if fp8 else bf16_rows(rng, rows)
    width = pad_to or topk
    idx = np.full((B, s_q, width), -1, np.int32)
    for b in range(B):
        L = int(seq_lens[b])
        for t in range(s_q):
            hi = L - s_q + t + 1 if causal else L
            n = max(0, min(topk, hi))
            if n:
                idx[b, t, :n] = oracle.distinct_indices(rng, hi, n)
    if poison_unused:
        used = []
        for b in range(B):
            j = idx[b][idx[b] >= 0].astype(np.int64)
            used.append(block_table[b][j // block_size].astype(np.int64) * block_size + j % block_size)
        poison(kv, np.unique(np.concatenate(used)) if used else np.zeros(0, np.int64))
    return DecodeCase(q, kv, idx, seq_lens, block_table, block_size, 0, causal)


def o_max_abs(got_bits: np.ndarray, ref_bits: np.ndarray) -> float:
    g = oracle.bf16_to_f32(got_bits)
    r = oracle.bf16_to_f32(ref_bits)
    if np.isnan(g).any():
        return float("inf")
    return float(np.max(np.abs(g - r))) if g.size else 0.0


def lse_rel(got: np.ndarray, ref: np.ndarray) -> float:
    """Largest |got - ref| / (1 + |ref|) over finite entries (inf if an infinity or NaN differs).

    Bounding this by 1e-3 is the reference's own LSE check, |got - ref| <= atol + rtol * |ref|
    with rtol = atol = 1e-3 (validate_mla_decode_lse, opus_attn/dsa_v32/common/host.cc:379-416):
    relative for |LSE| >= 1 and absolute near 0, where the LSE of a one-row list is a single
    score and a relative error is not defined.
    """
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    inf_r, inf_g = np.isinf(ref), np.isinf(got)
    if (inf_r != inf_g).any() or (np.sign(ref[inf_r]) != np.sign(got[inf_r])).any():
        return float("inf")
    fin = ~inf_r
    if not fin.any():
        return 0.0
    if np.isnan(got[fin]).any():
        return float("inf")
    return float(np.max(np.abs(got[fin] - ref[fin]) / (1.0 + np.abs(ref[fin]))))


def bf16_step(x: np.ndarray) -> np.ndarray:
    """Spacing of bf16 values at |x| (2^(e - 7) for |x| in [2^e, 2^(e+1)))."""
    ax = np.maximum(np.abs(np.asarray(x, np.float64)), np.finfo(np.float32).tiny)
    return np.exp2(np.floor(np.log2(ax)) - 7)


def o_bound(ref: np.ndarray) -> np.ndarray:
    """Per-element O bound: 2e-2, or one bf16 step where a step is larger.

    The outputs are bf16, so two of them differ by 0 or by at least one step.  For
    |O| >= 4 a step is 2^-5 = 0.031 > 2e-2: there the 2e-2 bar would demand the
    identical bf16 value, and a result that differs from the reference by any rounding
    error (the fp8 656-B path dequantises to fp16, 2^-11 relative) may round to the
    neighbouring value.  One step is the bound at those elements; below |O| = 4 the
    bound is 2e-2.
    """
    return np.maximum(O_ATOL, bf16_step(ref))


def assert_parity(o_got, lse_got, o_ref, lse_ref, what=""):
    g = oracle.bf16_to_f32(o_got)
    r = oracle.bf16_to_f32(o_ref)
    # O is a convex mix of finite V rows: a NaN or infinity on either side is a mismatch
    # (the comparisons below are False for NaN, so they would let it pass)
    assert np.isfinite(r).all(), f"{what}: the reference O holds {int((~np.isfinite(r)).sum())} non-finite values"
    assert np.isfinite(g).all(), f"{what}: O holds {int((~np.isfinite(g)).sum())} non-finite values"
    e_o = o_max_abs(o_got, o_ref)
    e_l = lse_rel(lse_got, lse_ref)
    if g.size and not np.isnan(g).any():
        d = np.abs(g.astype(np.float64) - r)
        over = d > o_bound(r)
        assert not over.any(), (f"{what}: O error {float(d[over].max())} above the bound at "
                                f"{int(over.sum())} elements (2e-2, or one bf16 step where |O| >= 4)")
        stepped = int((d > O_ATOL).sum())
        if stepped:
            print(f"[parity] {what}: {stepped} of {d.size} elements (|O| >= 4) differ by one bf16 step",
                  flush=True)
    else:
        assert e_o <= O_ATOL, f"{what}: O max-abs error {e_o} > {O_ATOL}"
    assert e_l <= LSE_RTOL, f"{what}: LSE error {e_l} > {LSE_RTOL} (relative to 1 + |LSE|)"
    return e_o, e_l
