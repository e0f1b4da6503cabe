"""Pins the oracle's codecs (CPU only).

- e4m3 decode: all 256 codes against the OCP E4M3FN closed form
  (sign, 4-bit exponent with bias 7, 3-bit mantissa, subnormals, S.1111.111 = NaN),
  the format of float_to_fp8_e4m3 / fp8_e4m3_to_float, opus_attn/dsa_v32/common/defs.h:11-52.
- e4m3 encode: brute-force nearest of the 254 finite codes with ties to the even
  code, saturation to +-448 (defs.h:17) and NaN for Inf/NaN inputs (defs.h:16).
- bf16 rounding: against torch's float32 -> bfloat16 conversion (round to nearest even).
- 656-byte rows: byte layout, scale = amax/448, and the dequant round-trip bound.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle


def closed_form_e4m3(c: int) -> float:
    s = -1.0 if c & 0x80 else 1.0
    e = (c >> 3) & 0xF
    m = c & 7
    if e == 15 and m == 7:
        return float("nan")
    if e == 0:
        return s * m * 2.0 ** -9
    return s * (1.0 + m / 8.0) * 2.0 ** (e - 7)


def test_e4m3_decode_exhaustive():
    codes = np.arange(256, dtype=np.uint8)
    got = oracle.fp8_decode(codes)
    for c in range(256):
        want = closed_form_e4m3(c)
        if np.isnan(want):
            assert np.isnan(got[c]), c
        else:
            assert got[c] == np.float32(want), (c, got[c], want)
    # landmarks
    assert got[0x7E] == 448.0 and got[0xFE] == -448.0
    assert got[0x01] == 2.0 ** -9 and got[0x08] == 2.0 ** -6


def _brute_encode(x: np.ndarray) -> np.ndarray:
    finite = [c for c in range(256) if not np.isnan(closed_form_e4m3(c))]
    vals = np.array([closed_form_e4m3(c) for c in finite], np.float64)
    codes = np.array(finite, np.int64)
    out = np.empty(x.shape, np.uint8)
    for i, v in enumerate(x.astype(np.float64)):
        if np.isnan(v) or np.isinf(v):
            out[i] = 0x7F | (0x80 if np.signbit(v) else 0)
            continue
        if abs(v) >= 448.0:
            out[i] = 0x7E | (0x80 if v < 0 else 0)
            continue
        d = np.abs(vals - v)
        best = np.flatnonzero(d == d.min())
        # candidates: same value may appear twice (+0 / -0); prefer the sign of v
        cand = codes[best]
        if len(cand) > 1:
            same_sign = [c for c in cand if (c & 0x80) == (0x80 if np.signbit(v) else 0)]
            even = [c for c in same_sign if (c & 1) == 0]
            pick = even[0] if even else same_sign[0]
        else:
            pick = cand[0]
        out[i] = pick
    return out


def test_e4m3_encode_brute_force():
    rng = np.random.default_rng(1)
    grid = oracle.fp8_decode(np.arange(256, dtype=np.uint8))
    grid = grid[np.isfinite(grid)]
    mids = []
    g = np.unique(grid.astype(np.float64))
    mids = (g[1:] + g[:-1]) / 2                     # exact ties between neighbours
    x = np.concatenate([
        grid, mids, np.nextafter(mids.astype(np.float32), np.float32(np.inf)),
        np.nextafter(mids.astype(np.float32), np.float32(-np.inf)),
        rng.standard_normal(4000) * 50, rng.standard_normal(2000) * 1e-3,
        np.array([447.9, 448.0, 464.0, 480.0, 1e30, -1e30, 2.0 ** -10, 2.0 ** -11,
                  -2.0 ** -10, 1e-40, 0.0, -0.0]),
    ]).astype(np.float32)
    got = oracle.fp8_encode(x)
    want = _brute_encode(x)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, [(x[i], got[i], want[i]) for i in bad[:10]]


def test_e4m3_encode_specials():
    x = np.array([np.inf, -np.inf, np.nan, 500.0, -1e9], np.float32)
    assert list(oracle.fp8_encode(x)) == [0x7F, 0xFF, 0x7F, 0x7E, 0xFE]


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(2)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * 10,
        (rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32)).view(np.float32),
    ])
    x = x[np.isfinite(x)]
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = oracle.bf16_bits(x)
    assert np.array_equal(got, want)
    # ties: 1 + 2^-8 is halfway between bf16 neighbours 1 and 1 + 2^-7 -> even (1.0)
    assert oracle.bf16_bits(np.array([1.0 + 2.0 ** -8], np.float32))[0] == 0x3F80
    assert oracle.bf16_bits(np.array([1.0 + 3 * 2.0 ** -8], np.float32))[0] == 0x3F82


def test_row_656_layout_and_roundtrip():
    rng = np.random.default_rng(3)
    src = oracle.bf16_to_f32(oracle.normal_bf16(rng, (64, 576)))
    src[5, 128:256] = 0.0                      # all-zero group -> scale 0, codes 0
    # rows far outside N(0,1): a whole row times 2^15 (amax ~1e5) and one group with a
    # -1e5 entry (scale ~223, above the GPU fp16 path's limit of 128): the oracle's codec
    # and dequant hold the same bound there (the reference dequantises in fp32,
    # opus_attn/dsa_v32/common/host.cc:418-429)
    src[9] *= np.float32(2.0 ** 15)
    src[10, 3 * 128 + 9] = oracle.bf16_to_f32(oracle.bf16_bits(np.array([-1.0e5], np.float32)))[0]
    rows = oracle.quantize_rows_656(src)
    assert rows.shape == (64, 656)
    scales = rows[:, 512:528].copy().view(np.float32)
    amax = np.abs(src[:, :512]).reshape(64, 4, 128).max(axis=2)
    assert np.array_equal(scales, (amax / np.float32(448.0)).astype(np.float32))
    assert (rows[5, 128:256] == 0).all() and scales[5, 1] == 0.0
    # codes are e4m3(x / scale) and the group max maps to +-448
    codes = rows[:, :512]
    for r in range(0, 64, 7):
        for g in range(4):
            if scales[r, g] == 0:
                continue
            ref = oracle.fp8_encode((src[r, 128 * g:128 * g + 128] / scales[r, g]).astype(np.float32))
            assert np.array_equal(codes[r, 128 * g:128 * g + 128], ref)
            assert np.abs(oracle.fp8_decode(ref)).max() == 448.0
    # RoPE stored as bf16 bytes
    rope = rows[:, 528:656].copy().view(np.uint16)
    assert np.array_equal(rope, oracle.bf16_bits(src[:, 512:]))
    deq = oracle.dequant_rows_656(rows)
    assert np.array_equal(deq[:, 512:], src[:, 512:])
    # |x - dq(q(x))| <= half an e4m3 ulp of x/scale, times scale (normal range: 2^(e-4))
    # (ties such as x/scale = 10.5 sit exactly on the bound: evaluated in fp64 with slack)
    sc = scales.astype(np.float64)[:, :, None]
    x = src[:, :512].reshape(64, 4, 128).astype(np.float64) / np.maximum(sc, 1e-30)
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -6)))
    bound = (2.0 ** (e - 4)) * sc * (1 + 1e-5)
    err = np.abs(deq[:, :512].reshape(64, 4, 128).astype(np.float64)
                 - src[:, :512].reshape(64, 4, 128).astype(np.float64))
    assert (err <= bound + 1e-30).all()
    assert scales[10, 3] > 128.0 and np.abs(deq[10, 3 * 128 + 9] + 1.0e5) <= 1.0e5 * 2.0 ** -4


@pytest.mark.parametrize("v", [0.0, 1.0, -3.5, 448.0])
def test_scalar_entry_points(v):
    L = oracle.lib()
    c = L.oracle_fp8_e4m3_encode(v)
    assert L.oracle_fp8_e4m3_decode(c) == np.float32(v)
    assert L.oracle_f32_to_bf16(v) == oracle.bf16_bits(np.array([v], np.float32))[0]
