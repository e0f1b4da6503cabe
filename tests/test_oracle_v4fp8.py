"""Pinning of the V4 fp8 prefill oracle (oracle.mla_prefill_v4_fp8), CPU only.

The oracle restates the reference's fp8 V4 CPU path:
- decode_dsa_row_fp8, opus_attn/dsa_v4/common/mla_v4_host.cc:443-453;
- mla_v4_attention_ref_fp8, mla_v4_host.cc:535-588.

It is checked against:
- the dequant: every e4m3 code under several E8M0 bytes, against torch's own
  float8_e4m3fn decode times 2^(e - 127). Distinct per-block scales pin the
  block of each of the 448 fp8 values (d / 32, scales at byte 448 + d / 32).
  RoPE becomes values 448..511, and the pad bytes are ignored;
- the attention: reduction to the bf16 V4 oracle, which is pinned separately.
  Every fp8 row value is a bf16 value, so the bf16 oracle on torch-dequantised
  rows and queries must give the same bits, with sink, empty ranges and rows
  outside their pool;
- a planted mistake (scales dropped) changes the result.
"""
from __future__ import annotations

import numpy as np
import torch

import oracle

H_SMALL = 3
NB = 448 // 32


def torch_dequant(nope: np.ndarray, rope: np.ndarray) -> np.ndarray:
    """V4 fp8 rows -> fp32 [..., 512] by torch's e4m3fn decode and the E8M0 bytes at 448.."""
    codes = np.ascontiguousarray(nope[..., :448])
    v = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy().astype(np.float64)
    e = np.repeat(nope[..., 448:448 + NB].astype(np.int32) - 127, 32, axis=-1)
    with np.errstate(over="ignore"):
        x = (v * np.ldexp(1.0, e)).astype(np.float32)
    return np.concatenate([x, oracle.bf16_to_f32(rope)], axis=-1)


def test_dequant_every_code_block_and_rope():
    rope = np.arange(64, dtype=np.uint16) + 0x3F00
    for e in (0, 1, 120, 127, 131, 200, 254):
        nope = np.full(512, 0xFF, np.uint8)
        nope[:448] = np.arange(448) % 256
        nope[448:448 + NB] = e
        got = oracle.dequant_rows_v4fp8(nope, rope)[0]
        want = torch_dequant(nope[None], rope[None])[0]
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(got), nan)
        assert np.array_equal(got[~nan], want[~nan]), f"E8M0 byte {e}"
    rng = np.random.default_rng(9)
    nope = np.zeros(512, np.uint8)
    nope[:448] = 0x38                                  # e4m3 1.0
    sc = rng.permutation(np.arange(120, 120 + NB)).astype(np.uint8)
    nope[448:448 + NB] = sc
    nope[448 + NB:] = rng.integers(0, 256, 512 - 448 - NB)   # pad: ignored
    got = oracle.dequant_rows_v4fp8(nope, rope)[0]
    assert np.array_equal(got[:448], np.ldexp(1.0, np.repeat(sc.astype(int) - 127, 32)).astype(np.float32))
    assert np.array_equal(got[448:], oracle.bf16_to_f32(rope))


def v4fp8_case(seed, N=10, total_pages=50, total_tokens=24, n_pre=6, window=4, bad=True):
    rng = np.random.default_rng(seed)
    qn, qr = oracle.v4fp8_rows(rng, N * H_SMALL)
    q = (qn.reshape(N, H_SMALL, 512), qr.reshape(N, H_SMALL, 64))
    ukv = oracle.v4fp8_rows(rng, total_pages)
    xkv = oracle.v4fp8_rows(rng, total_tokens)
    ipp, idp, ipe, ide = [0], [], [0], []
    for i in range(N):
        pre = rng.choice(total_pages, 0 if i == 3 else n_pre, replace=False).astype(np.int32)
        ext = np.arange(max(0, i + 1 - window), i + 1, dtype=np.int32) % total_tokens
        if i == 3:
            ext = ext[:0]                        # no rows at all
        if bad and i % 4 == 1:
            pre[0], pre[1] = -2, total_pages + 1     # outside the prefix pool: skipped
        idp += list(pre)
        ide += list(ext)
        ipp.append(len(idp))
        ipe.append(len(ide))
    sink = rng.normal(0.3, 1.0, H_SMALL).astype(np.float32)
    return q, ukv, xkv, sink, *(np.array(x, np.int32) for x in (ipp, idp, ipe, ide))


def test_v4fp8_oracle_equals_bf16_v4_oracle():
    q, ukv, xkv, sink, ipp, idp, ipe, ide = v4fp8_case(21)
    scale = 0.06
    for s in (sink, None):
        o, lse = oracle.mla_prefill_v4_fp8(*q, *ukv, *xkv, s, ipp, idp, ipe, ide, scale)
        q16 = oracle.bf16_bits(torch_dequant(*q))
        u16 = oracle.bf16_bits(torch_dequant(*ukv))
        x16 = oracle.bf16_bits(torch_dequant(*xkv))
        assert np.array_equal(oracle.bf16_to_f32(q16), torch_dequant(*q)), "values must be bf16-exact"
        o_ref, l_ref = oracle.mla_prefill_v4(q16, u16, x16, s, ipp, idp, ipe, ide, scale)
        assert np.array_equal(o, o_ref)
        assert np.array_equal(lse, l_ref)
    assert (o[3] == 0).all() and np.isinf(lse[3]).all()


def test_v4fp8_oracle_scale_matters():
    q, ukv, xkv, sink, ipp, idp, ipe, ide = v4fp8_case(22, bad=False)
    o, lse = oracle.mla_prefill_v4_fp8(*q, *ukv, *xkv, sink, ipp, idp, ipe, ide, 0.06)
    un = ukv[0].copy()
    un[:, 448:448 + NB] = 127
    o2, l2 = oracle.mla_prefill_v4_fp8(*q, un, ukv[1], *xkv, sink, ipp, idp, ipe, ide, 0.06)
    assert not np.array_equal(lse, l2)
