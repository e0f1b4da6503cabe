"""GPU parity of the MXFP8 split-stream decode entry (dsa_mla_decode_mxfp8).

The format is the reference's own "-dtype fp8" one:
- separate NoPE (fp8 e4m3fn), E8M0-scale and RoPE (bf16) streams for Q and KV;
- opus_attn/dsa_v32/common/host.cc:551-697, with inputs drawn as in
  init_fp8_mla_split (host.cc:207-237);
- CSR kv_indptr / kv_indices with count-based MTP causality (host.cc:481-482).

The kernel is checked against the CPU oracle (oracle.mla_decode_mxfp8, pinned
in tests/test_oracle_mxfp8.py) with the bar of every parity test:
- bf16 O max-abs <= 2e-2;
- LSE within 1e-3 * (1 + |LSE|).

Two more checks:
- MXFP8 values dequantise exactly to bf16, so the bf16 CSR entry on the
  dequantised rows is a second reference: the NoPE part of QK^T runs as
  scaled fp8 MFMAs (block dot products accumulated inside the MFMA, not
  bit-identical to fp32 sums), and the outputs agree with the bf16 entry's to
  the same bar;
- padded streams (non-dense strides) give the same results.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from _cases import SM_SCALE, assert_parity, lse_rel, o_max_abs
from opfoundry_amd import dsa

pytestmark = pytest.mark.gpu
H = 128


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def t16(a: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(dev)


def mx_case(seed, lens, s_q, total, bad=0, csr_shuffle=False):
    rng = np.random.default_rng(seed)
    B = len(lens)
    kv = oracle.mxfp8_rows(rng, total)
    qn, qs, qr = oracle.mxfp8_rows(rng, B * s_q * H)
    q = (qn.reshape(B * s_q, H, 512), qs.reshape(B * s_q, H, 16), qr.reshape(B * s_q, H, 64))
    indptr = np.zeros(B + 1, np.int32)
    indptr[1:] = np.cumsum(lens)
    if csr_shuffle:
        # init_kv_page_table (host.cc:239-262): a permutation of all rows
        indices = rng.permutation(total).astype(np.int32)[:indptr[-1]]
    else:
        indices = rng.integers(0, total, int(indptr[-1])).astype(np.int32)
    if bad:
        pos = rng.choice(indices.size, bad, replace=False)
        indices[pos] = np.where(np.arange(bad) % 2 == 0, -1 - pos, total + pos).astype(np.int32)
    return q, kv, indptr, indices


def dev_streams(q, kv, dev):
    (qn, qs, qr), (kn, ks, kr) = q, kv
    u8 = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    return (u8(qn), u8(qs), t16(qr, dev)), (u8(kn), u8(ks), t16(kr, dev))


def run_mx(qd, kvd, indptr, indices, s_q, dev, num_splits=0):
    ti = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    out, lse = dsa.mla_decode_mxfp8(*qd, *kvd, ti(indptr), ti(indices), SM_SCALE, s_q=s_q,
                                    num_splits=num_splits)
    torch.cuda.synchronize()
    return bits(out), lse.cpu().numpy()


def sub_csr(indptr, indices, batches):
    """The CSR lists of a subset of batches (for a sampled oracle run)."""
    ip, ix = [0], []
    for b in batches:
        ix += list(indices[indptr[b]:indptr[b + 1]])
        ip.append(len(ix))
    return np.array(ip, np.int32), np.array(ix, np.int32)


@pytest.mark.parametrize("num_splits", [0, 4])
def test_mxfp8_varlen_mtp(dev, num_splits):
    """Varlen lists (one longer than a workgroup's 2048 rows, one empty), s_q = 2, rows
    outside the cache mixed in."""
    lens = [700, 3000, 1, 0, 2048]
    print(f"[case] mxfp8 varlen mtp lens={lens} splits={num_splits}", flush=True)
    q, kv, indptr, indices = mx_case(51, lens, 2, 6000, bad=40)
    o_ref, l_ref = oracle.mla_decode_mxfp8(*q, *kv, indptr, indices, 2, SM_SCALE)
    qd, kvd = dev_streams(q, kv, dev)
    o, l = run_mx(qd, kvd, indptr, indices, 2, dev, num_splits)
    e = assert_parity(o, l, o_ref, l_ref, f"mxfp8 varlen mtp splits={num_splits}")
    print(f"[case] max|dO|={e[0]:.3e} max rel dLSE={e[1]:.3e}", flush=True)
    assert np.isinf(l[6:8]).all() and (o[6:8] == 0).all()      # batch 3: no rows
    assert np.isinf(l[4]).all() and not np.isinf(l[5]).any()   # batch 2: token 0 sees none


def test_mxfp8_reference_harness_shape(dev):
    """The reference's default fp8 case: H = 128, B = 128, s = 1024, s_q = 1, a shuffled
    permutation of all rows as the page table.  Every batch goes through the oracle."""
    print("[case] mxfp8 reference shape B=128 s=1024", flush=True)
    B, s = 128, 1024
    q, kv, indptr, indices = mx_case(52, [s] * B, 1, B * s, csr_shuffle=True)
    qd, kvd = dev_streams(q, kv, dev)
    o, l = run_mx(qd, kvd, indptr, indices, 1, dev)
    assert np.isfinite(l).all()
    pick = list(range(B))
    ip, ix = sub_csr(indptr, indices, pick)
    qs = tuple(x[pick] for x in q)
    o_ref, l_ref = oracle.mla_decode_mxfp8(*qs, *kv, ip, ix, 1, SM_SCALE)
    e = assert_parity(o[pick], l[pick], o_ref, l_ref, "mxfp8 reference shape")
    print(f"[case] {len(pick)} batches: max|dO|={e[0]:.3e} max rel dLSE={e[1]:.3e}", flush=True)


def test_mxfp8_matches_bf16_entry(dev):
    """The dequantised rows and queries are bf16 values; the bf16 CSR entry on them agrees with
    the MXFP8 entry's outputs to the parity bar (with 1 and 2 splits)."""
    print("[case] mxfp8 vs bf16 CSR entry", flush=True)
    lens = [1500, 900, 33]
    q, kv, indptr, indices = mx_case(53, lens, 1, 4096)
    qd, kvd = dev_streams(q, kv, dev)
    q16 = oracle.bf16_bits(oracle.dequant_rows_mxfp8(*(x.reshape(-1, x.shape[-1]) for x in q)))
    kv16 = oracle.bf16_bits(oracle.dequant_rows_mxfp8(*kv))
    for ns in (1, 2):
        o_mx, l_mx = run_mx(qd, kvd, indptr, indices, 1, dev, ns)
        out, lse = dsa.mla_decode_csr(t16(q16, dev).view(len(lens), H, 576), t16(kv16, dev),
                                      torch.from_numpy(indptr).to(dev), torch.from_numpy(indices).to(dev),
                                      SM_SCALE, s_q=1, num_splits=ns)
        torch.cuda.synchronize()
        e = assert_parity(o_mx, l_mx, bits(out), lse.cpu().numpy(), f"mxfp8 vs bf16 entry splits={ns}")
        print(f"[case] splits={ns}: max|dO|={e[0]:.3e} max rel dLSE={e[1]:.3e}", flush=True)


def test_mxfp8_padded_streams(dev):
    """Streams with padded strides (scale rows 32 bytes apart as in the reference's traits,
    RoPE rows 72 elements apart, Q heads 528 / 32 / 72 apart) give the same results."""
    print("[case] mxfp8 padded streams", flush=True)
    lens = [300, 1200]
    q, kv, indptr, indices = mx_case(54, lens, 1, 2048)
    qd, kvd = dev_streams(q, kv, dev)
    o0, l0 = run_mx(qd, kvd, indptr, indices, 1, dev)

    def pad(t, w):
        z = torch.zeros(*t.shape[:-1], w, dtype=t.dtype, device=dev)
        z[..., :t.shape[-1]] = t
        return z[..., :t.shape[-1]]

    qp = (pad(qd[0], 528), pad(qd[1], 32), pad(qd[2], 72))
    kvp = (pad(kvd[0], 528), pad(kvd[1], 32), pad(kvd[2], 72))
    o1, l1 = run_mx(qp, kvp, indptr, indices, 1, dev)
    assert (o1 == o0).all() and np.array_equal(l1, l0)
    o_ref, l_ref = oracle.mla_decode_mxfp8(*q, *kv, indptr, indices, 1, SM_SCALE)
    assert o_max_abs(o1, o_ref) <= 2e-2 and lse_rel(l1, l_ref) <= 1e-3
