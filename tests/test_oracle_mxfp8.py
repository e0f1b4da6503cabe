"""Pinning of the MXFP8 decode oracle (oracle.mla_decode_mxfp8), CPU only.

The oracle restates the reference's fp8 CPU path:
- dequant_mla_row_fp8, opus_attn/dsa_v32/common/host.cc:418-429;
- mla_decode_attention_ref_fp8, host.cc:459-506 (CSR rows, count-based MTP
  causality).

It is checked against:
- the dequant: every e4m3 code under several E8M0 bytes, against torch's own
  float8_e4m3fn decode times 2^(e - 127); per-block scales pin the block of
  each of the 512 dims (d / 32);
- the attention: reduction to the bf16 top-k decode oracle, which is pinned
  separately. Each MXFP8 value is a bf16 value, so running the bf16 oracle on
  torch-dequantised rows and queries must give the same bits. The CSR lists
  are mapped to the top-k form by hand, as a dsa_v32 harness would, covering
  MTP causality, empty ranges and rows outside the cache.
"""
from __future__ import annotations

import numpy as np
import torch

import oracle
from _cases import SM_SCALE

H_SMALL = 4


def torch_dequant(nope: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """fp8 codes [..., 512] and E8M0 bytes [..., 16] -> fp32, by torch's e4m3fn decode."""
    v = torch.from_numpy(np.ascontiguousarray(nope)).view(torch.float8_e4m3fn).float().numpy()
    e = np.repeat(scale.astype(np.int32) - 127, 32, axis=-1)
    with np.errstate(over="ignore"):   # 448 * 2^127 overflows fp32, as in the oracle
        return (v.astype(np.float64) * np.ldexp(1.0, e)).astype(np.float32)


def test_dequant_every_code_and_block():
    codes = np.arange(256, dtype=np.uint8)
    rope = np.zeros(64, np.uint16)
    for e in (0, 1, 100, 127, 130, 200, 254):
        nope = np.tile(codes, 2)
        sc = np.full(16, e, np.uint8)
        got = oracle.dequant_rows_mxfp8(nope, sc, rope)[0, :512]
        want = torch_dequant(nope, sc)
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(got), nan)
        assert np.array_equal(got[~nan], want[~nan]), f"E8M0 byte {e}"
    # distinct scale per block: dim d must take block d // 32
    rng = np.random.default_rng(5)
    nope = np.full(512, 0x38, np.uint8)           # e4m3 1.0
    sc = rng.permutation(np.arange(120, 136)).astype(np.uint8)
    got = oracle.dequant_rows_mxfp8(nope, sc, rope)[0, :512]
    assert np.array_equal(got, np.ldexp(1.0, np.repeat(sc.astype(int) - 127, 32)).astype(np.float32))


def test_dequant_rope_is_bf16():
    rng = np.random.default_rng(6)
    nope, sc, rope = oracle.mxfp8_rows(rng, 3)
    got = oracle.dequant_rows_mxfp8(nope, sc, rope)
    assert np.array_equal(got[:, 512:], oracle.bf16_to_f32(rope))


def mx_case(seed, lens, s_q, total, bad=0):
    rng = np.random.default_rng(seed)
    B = len(lens)
    kn, ks, kr = oracle.mxfp8_rows(rng, total)
    qn, qs, qr = oracle.mxfp8_rows(rng, B * s_q * H_SMALL)
    q = (qn.reshape(B * s_q, H_SMALL, 512), qs.reshape(B * s_q, H_SMALL, 16), qr.reshape(B * s_q, H_SMALL, 64))
    indptr = np.zeros(B + 1, np.int32)
    indptr[1:] = np.cumsum(lens)
    indices = rng.integers(0, total, int(indptr[-1])).astype(np.int32)
    if bad:
        pos = rng.choice(indices.size, bad, replace=False)
        indices[pos] = np.where(np.arange(bad) % 2 == 0, -2, total + 5).astype(np.int32)
    return q, (kn, ks, kr), indptr, indices


def as_bf16(x: np.ndarray) -> np.ndarray:
    bits = oracle.bf16_bits(x)
    assert np.array_equal(oracle.bf16_to_f32(bits), x), "MXFP8 values must be bf16-exact"
    return bits


def topk_oracle(q, kv, indptr, indices, s_q):
    """bf16 top-k decode oracle on torch-dequantised MXFP8 data (the CSR lists mapped by hand)."""
    (qn, qs, qr), (kn, ks, kr) = q, kv
    T, H = qn.shape[:2]
    q16 = as_bf16(np.concatenate([torch_dequant(qn, qs), oracle.bf16_to_f32(qr)], axis=-1))
    kv16 = as_bf16(np.concatenate([torch_dequant(kn, ks), oracle.bf16_to_f32(kr)], axis=-1))
    B = indptr.size - 1
    maxc = max(int(indptr[b + 1] - indptr[b]) for b in range(B))
    idx = np.full((B, s_q, max(maxc, 1)), -1, np.int32)
    for b in range(B):
        for t in range(s_q):
            n = int(indptr[b + 1] - indptr[b]) - (s_q - 1 - t)
            if n > 0:
                idx[b, t, :n] = indices[indptr[b]:indptr[b] + n]
    sl = np.full(B, kv16.shape[0], np.int32)
    o, lse = oracle.mla_decode(q16.reshape(B, s_q, H, 576), kv16, idx, sl, SM_SCALE)
    return o.reshape(T, H, -1), lse.reshape(T, H)


def run_mx(q, kv, indptr, indices, s_q):
    return oracle.mla_decode_mxfp8(*q, *kv, indptr, indices, s_q, SM_SCALE)


def test_mx_oracle_equals_bf16_oracle_mtp():
    lens = [40, 1, 0, 77, 3]
    q, kv, indptr, indices = mx_case(11, lens, 2, 300, bad=6)
    o, lse = run_mx(q, kv, indptr, indices, 2)
    o_ref, l_ref = topk_oracle(q, kv, indptr, indices, 2)
    assert np.array_equal(o, o_ref)
    assert np.array_equal(lse, l_ref)
    # batch 2 is empty; batch 1's token 0 sees no row (count-based causality)
    assert np.isinf(lse[4:6]).all() and (o[4:6] == 0).all()
    assert np.isinf(lse[2]).all() and not np.isinf(lse[3]).any()


def test_mx_oracle_single_token_reference_shape():
    q, kv, indptr, indices = mx_case(12, [200, 150], 1, 1000)
    o, lse = run_mx(q, kv, indptr, indices, 1)
    o_ref, l_ref = topk_oracle(q, kv, indptr, indices, 1)
    assert np.array_equal(o, o_ref) and np.array_equal(lse, l_ref)


def test_mx_oracle_scale_matters():
    """A planted mistake fails: dropping the E8M0 scales changes the result."""
    q, kv, indptr, indices = mx_case(13, [64], 1, 128)
    o, lse = run_mx(q, kv, indptr, indices, 1)
    kn, ks, kr = kv
    o2, l2 = run_mx(q, (kn, np.full_like(ks, 127), kr), indptr, indices, 1)
    assert not np.array_equal(lse, l2)
