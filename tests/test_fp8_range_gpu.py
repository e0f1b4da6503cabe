"""The numeric range of the 656-byte fp8 path (DSA_KV_FP8_656), on the GPU.

That path computes K and V in fp16 (a row's value = fp16(code * 2^e) * fp16(mantissa),
scale = mantissa * 2^e) and Q's NoPE part in fp16.  Its contract (include/dsa_mla.h):
- any finite q: each head is scaled by a power of two into fp16's range, and the
  softmax scale by the inverse (exact), so |q| up to 1e5 and beyond keeps parity with
  the oracle's fp32 arithmetic (the reference dequantises in fp32,
  opus_attn/dsa_v32/common/host.cc:418-429);
- every attended row's four scales below 128 (group amax below 57,344): then every K / V
  value is a finite fp16 value and parity holds up to the limit;
- a query token that attends a row with a scale of 128 or more (or a negative or
  non-finite one) gets NaN O and LSE: a defined signal, never a silently wrong result.
  Tokens that do not attend such a row are unaffected.

Same bar as every parity test (tests/_cases.py).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from _cases import D_QK, DecodeCase, assert_parity, bf16_rows
from opfoundry_amd import dsa

pytestmark = pytest.mark.gpu


def t16(a: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(dev)


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def case_with_rows(seed, src_f32, B=4, kv_len=2048, topk=512, H=128, q_mult=None, sm_scale=None,
                   force=None):
    """Flat per-batch fp8 cache from fp32 rows src_f32 [B * kv_len, 576]; force = {(b, row in
    batch): [tokens that must attend it]} puts the row into those tokens' lists."""
    rng = np.random.default_rng(seed)
    q = oracle.normal_bf16(rng, (B, 1, H, D_QK))
    if q_mult is not None:
        qf = oracle.bf16_to_f32(q) * q_mult.reshape(1, 1, H, 1)
        q = oracle.bf16_bits(qf.astype(np.float32))
    kv = oracle.quantize_rows_656(src_f32)
    idx = np.full((B, 1, topk), -1, np.int32)
    for b in range(B):
        idx[b, 0] = oracle.distinct_indices(rng, kv_len, topk)
    for (b, r) in (force or {}):
        if r not in idx[b, 0]:
            idx[b, 0, 7] = r
    seq = np.full(B, kv_len, np.int32)
    c = DecodeCase(q, kv, idx, seq, None, 1, kv_len, False)
    if sm_scale is not None:
        c.sm_scale = sm_scale
    return c


def run(c, dev, num_splits=0):
    out, lse = dsa.mla_decode(t16(c.q, dev), torch.from_numpy(c.kv).to(dev),
                              torch.from_numpy(c.indices).to(dev), c.sm_scale,
                              seq_lens=torch.from_numpy(c.seq_lens).to(dev),
                              kv_batch_stride=c.kv_batch_stride, num_splits=num_splits)
    torch.cuda.synchronize()
    return bits(out), lse.cpu().numpy()


@pytest.mark.parametrize("num_splits", [1, 4])
def test_large_q_keeps_parity(dev, num_splits):
    """Heads with |q| up to ~1e5 (Q times 3e4 on a third of the heads, 300 on another third)
    and a softmax scale shrunk by 3e4 keep the scores a real mixture: the GPU result must
    match the oracle, which runs in fp32 on the same bf16 q."""
    rng = np.random.default_rng(5)
    B, kv_len = 4, 2048
    src = oracle.bf16_to_f32(bf16_rows(rng, B * kv_len))
    mult = np.ones(128, np.float32)
    mult[0::3] = 3.0e4
    mult[1::3] = 300.0
    c = case_with_rows(11, src, B=B, kv_len=kv_len, q_mult=mult, sm_scale=1.0 / np.sqrt(192.0) / 3.0e4)
    qa = np.abs(oracle.bf16_to_f32(c.q)).max()
    assert qa > 6.5e4, qa            # above fp16's largest value
    print(f"[case] large q: max|q| = {qa:.3e}, splits {num_splits}", flush=True)
    o_ref, l_ref = c.oracle()
    o, l = run(c, dev, num_splits)
    e = assert_parity(o, l, o_ref, l_ref, "large q")
    print(f"[case] large q: max|dO|={e[0]:.3e} max rel dLSE={e[1]:.3e}", flush=True)


def test_scale_limit(dev):
    """A group with amax 56,000 (scale 125, just below the limit of 128) keeps parity; a
    row with a 1e5-amax group (scale 223) makes exactly the tokens that attend it NaN."""
    rng = np.random.default_rng(6)
    B, kv_len = 4, 2048
    src = oracle.bf16_to_f32(bf16_rows(rng, B * kv_len))
    # batch 0, row 100: group 1 at amax 56,000 (in range); batch 2, row 200: group 3 at 1e5
    src[0 * kv_len + 100, 128 + 5] = 56000.0
    src[2 * kv_len + 200, 3 * 128 + 9] = -1.0e5
    c = case_with_rows(12, src, B=B, kv_len=kv_len, force={(0, 100): [0], (2, 200): [0]})
    sc = c.kv[:, 512:528].copy().view(np.float32)
    assert 120.0 < sc[100, 1] < 128.0 and sc[2 * kv_len + 200, 3] > 128.0
    o_ref, l_ref = c.oracle()
    for ns in (1, 4):
        print(f"[case] scale limit, splits {ns}", flush=True)
        o, l = run(c, dev, ns)
        bad = np.array([False, False, True, False])           # batch 2 attends the 1e5 group
        assert np.isnan(l[bad]).all()
        assert np.isnan(oracle.bf16_to_f32(o[bad])).all()
        e = assert_parity(o[~bad], l[~bad], o_ref[~bad], l_ref[~bad], "scale limit: in-range tokens")
        print(f"[case] scale limit: max|dO|={e[0]:.3e} max rel dLSE={e[1]:.3e}", flush=True)
