"""GPU parity of the sparse-MLA decode / prefill / combine / cache-writer kernels
against the CPU oracle (through the C ABI of libdsa_mla.so).

Bar: bf16 O max-abs error <= 2e-2 on every element, LSE within 1e-3 * (1 + |LSE|)
(the reference's rtol = atol = 1e-3 check, host.cc:379-416),
index handling (-1 padding, seq_len and causal bounds, bad block-table
entries) exact - invalid entries are filtered identically by the oracle, and
every cache row the index list does not select is NaN-poisoned so a wrong
gather fails loudly.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from _cases import (D_QK, SM_SCALE, assert_parity, flat_case, fp8_rows, bf16_rows, lse_rel,
                    o_max_abs, paged_case, poison)
from opfoundry_amd import dsa

pytestmark = pytest.mark.gpu


def t16(a: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(dev)


def kv_tensor(kv: np.ndarray, dev) -> torch.Tensor:
    return t16(kv, dev) if kv.dtype == np.uint16 else torch.from_numpy(kv).to(dev)


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def run_decode(case, dev, num_splits=0):
    q = t16(case.q, dev)
    kv = kv_tensor(case.kv, dev)
    idx = torch.from_numpy(case.indices).to(dev)
    sl = torch.from_numpy(case.seq_lens).to(dev)
    bt = None if case.block_table is None else torch.from_numpy(case.block_table).to(dev)
    out, lse = dsa.mla_decode(q, kv, idx, case.sm_scale, seq_lens=sl, block_table=bt,
                              block_size=case.block_size, causal=case.causal,
                              num_splits=num_splits, kv_batch_stride=case.kv_batch_stride)
    torch.cuda.synchronize()
    return bits(out), lse.cpu().numpy()


def check(case, dev, what, num_splits=0):
    print(f"[case] {what} shape={case.shape} splits={num_splits}", flush=True)
    o_ref, l_ref = case.oracle()
    o, l = run_decode(case, dev, num_splits)
    e = assert_parity(o, l, o_ref, l_ref, what)
    print(f"[case] {what}: max|dO|={e[0]:.3e} max rel dLSE={e[1]:.3e}", flush=True)
    return o, l, o_ref, l_ref


# -------------------------------------------------------------------- decode

def test_c1_flat_bf16(dev):
    """BASELINE config 1 at full size: B=2, 8192 rows per batch, top-k 2048, last 256 = -1."""
    check(flat_case(), dev, "C1 flat bf16")


@pytest.mark.parametrize("num_splits", [1, 0, 3])
def test_paged_bf16(dev, num_splits):
    check(paged_case(seed=11, B=4, seq_len=4096, topk=2048), dev, "paged bf16", num_splits)


def test_paged_fp8_mtp_causal(dev):
    """fp8 656-B rows, s_q = 2 (MTP), causal: query t only sees positions <= L - 2 + t."""
    c = paged_case(seed=12, B=4, s_q=2, seq_len=3000, topk=1024, fp8=True, causal=True)
    check(c, dev, "paged fp8 mtp causal")


def test_fp8_flat_unsplit_and_split(dev):
    c = flat_case(seed=13, B=2, kv_len=4096, topk=2048, pad=100, fp8=True)
    check(c, dev, "flat fp8 unsplit", num_splits=1)
    check(c, dev, "flat fp8 split4", num_splits=4)


def test_varlen_padding(dev):
    """seq_lens drawn in [1, 3000]; top-k = min(2048, L) padded with -1 (config 4 style)."""
    c = paged_case(seed=14, B=6, seq_len=3000, topk=2048, varlen=True)
    check(c, dev, "varlen padded", num_splits=8)


@pytest.mark.parametrize("topk", [1, 5, 31, 33, 100])
def test_small_topk(dev, topk):
    c = paged_case(seed=15 + topk, B=3, seq_len=700, topk=topk)
    check(c, dev, f"topk={topk}")


@pytest.mark.parametrize("fp8", [False, True])
def test_reference_restart(dev, fp8):
    """The kernel's softmax keeps the first tile's maximum as a fixed reference; a later score
    more than 100 (bf16) / 15 (fp16 path) above it in log2 units makes the workgroup rerun its
    tiles against the exact maximum.  Token 0 gets an all-ones Q and two spike rows, in tiles 1
    and 2: 7.0 in dims 0..255 (score 1792) and in dims 256..510 (score 1785), about 200 log2
    units above the rest.  7.0 = 448 * 2^-6 is exact in bf16, fp16 and the fp8 row (scale
    amax / 448 = 2^-6), so the result is a plain 1 : e^-0.505 mixture of the two V halves."""
    c = paged_case(seed=41, B=2, seq_len=2048, topk=200, fp8=fp8)   # 7 tiles per token
    q = oracle.bf16_to_f32(c.q)
    q[0, 0] = 1.0
    c.q = oracle.bf16_bits(q)

    def row_of(j):
        return int(c.block_table[0][j // c.block_size]) * c.block_size + j % c.block_size

    ra, rb = row_of(int(c.indices[0, 0, 40])), row_of(int(c.indices[0, 0, 75]))
    spike = np.zeros((2, D_QK), np.float32)
    spike[0, :256] = 7.0
    spike[1, 256:511] = 7.0
    c.kv[[ra, rb]] = oracle.quantize_rows_656(spike) if fp8 else oracle.bf16_bits(spike)
    o, l, o_ref, l_ref = check(c, dev, f"reference restart fp8={fp8}")
    # the case does exercise the mixture: both V halves carry weight in token 0's output
    w = 7.0 * np.exp(-7 * SM_SCALE) / (1 + np.exp(-7 * SM_SCALE))
    of = oracle.bf16_to_f32(o).reshape(-1, 128, 512)[0]
    assert np.allclose(of[:, :256], 7.0 - w, atol=2e-2) and np.allclose(of[:, 256:511], w, atol=2e-2)


def test_all_invalid(dev):
    """No valid entry: O = 0 and LSE = +inf (host.cc:486-489)."""
    c = paged_case(seed=16, B=2, seq_len=512, topk=64)
    c.indices[:] = -1
    o, l, o_ref, l_ref = check(c, dev, "all invalid")
    assert (o == 0).all() and np.isposinf(l).all()
    c.indices[0, 0, :5] = [700, 512, -7, 100000, 513]  # all out of range for L = 512
    o, l, _, _ = check(c, dev, "out of range only")
    assert np.isposinf(l[0]).all()


def test_invalid_entries_are_filtered(dev):
    """-1 anywhere, j >= seq_len, j < -1 and causal violations give exactly the result of
    the list with those entries removed."""
    c = paged_case(seed=17, B=3, s_q=2, seq_len=1500, topk=512, causal=True, poison_unused=False)
    rng = np.random.default_rng(5)
    dirty = c.indices.copy()
    L = int(c.seq_lens[0])
    bad = rng.random(dirty.shape) < 0.2
    junk = rng.choice(np.array([-1, -5, L, L + 1000, L - 1, 2**30], np.int32), size=dirty.shape)
    dirty[bad] = junk[bad]
    c_dirty = paged_case(seed=17, B=3, s_q=2, seq_len=1500, topk=512, causal=True,
                         poison_unused=False)
    c_dirty.indices = dirty
    o_ref, l_ref = c_dirty.oracle()
    o0, l0 = run_decode(c_dirty, dev)
    assert_parity(o0, l0, o_ref, l_ref, "dirty list")
    o1, l1 = run_decode(c_dirty, dev, num_splits=1)
    assert_parity(o1, l1, o_ref, l_ref, "dirty list unsplit")
    # unsplit, the filtered list (valid entries only, order kept, -1 padded) must give the
    # same bits: the kernel compacts the valid entries, so both run the identical computation
    filt = np.full_like(dirty, -1)
    for b in range(dirty.shape[0]):
        for t in range(dirty.shape[1]):
            hi = min(L, L - 2 + t + 1)
            v = [j for j in dirty[b, t] if 0 <= j < hi]
            filt[b, t, :len(v)] = v
    c_dirty.indices = filt
    o2, l2 = run_decode(c_dirty, dev, num_splits=1)
    assert np.array_equal(o1, o2)
    assert np.array_equal(l1, l2)


def test_duplicates_and_bad_block_table(dev):
    c = paged_case(seed=18, B=2, seq_len=1024, topk=256, poison_unused=False)
    c.indices[:, :, 100:200] = c.indices[:, :, 0:100]          # duplicated positions
    c.block_table = c.block_table.copy()
    c.block_table[1, 3] = 10**6                                # outside the pool: invalid
    c.block_table[1, 4] = -3
    check(c, dev, "duplicates + bad block table")


def test_strided_q_and_out(dev):
    c = paged_case(seed=19, B=3, s_q=2, seq_len=800, topk=300)
    big = torch.zeros((3, 2, 128, D_QK + 64), dtype=torch.bfloat16, device=dev)
    big[..., :D_QK] = t16(c.q, dev)
    q = big[..., :D_QK]
    out_big = torch.full((3, 2, 128, 512 + 32), float("nan"), dtype=torch.bfloat16, device=dev)
    out = out_big[..., :512]
    lse = torch.empty((3, 2, 128), dtype=torch.float32, device=dev)
    dsa.mla_decode(q, t16(c.kv, dev), torch.from_numpy(c.indices).to(dev), SM_SCALE, out, lse,
                   seq_lens=torch.from_numpy(c.seq_lens).to(dev),
                   block_table=torch.from_numpy(c.block_table).to(dev), block_size=64,
                   num_splits=2)
    torch.cuda.synchronize()
    o_ref, l_ref = c.oracle()
    assert_parity(bits(out), lse.cpu().numpy(), o_ref, l_ref, "strided")
    assert torch.isnan(out_big[..., 512:].float()).all(), "kernel wrote outside the output view"


@pytest.mark.parametrize("fp8", [False, True])
def test_padded_cache_rows(dev, fp8):
    """Top-k form on a paged cache whose rows sit in a wider tensor (kv_stride_row = 640
    bf16 elements / 672 bytes, NaN-filled pad): same results as the dense rows, split and
    unsplit, for decode and for prefill."""
    c = paged_case(seed=20, B=3, s_q=2, seq_len=900, topk=400, fp8=fp8, causal=True)
    pad = 16 if fp8 else 64
    width = c.kv.shape[1]
    if fp8:
        big = np.full((c.kv.shape[0], width + pad), 0xFF, np.uint8)
        big[:, :width] = c.kv
        kv = torch.from_numpy(big).to(dev)[:, :width]
    else:
        big = np.full((c.kv.shape[0], width + pad), 0x7FC0, np.uint16)
        big[:, :width] = c.kv
        kv = t16(big, dev)[:, :width]
    assert kv.stride(0) == width + pad
    print(f"[case] padded cache rows fp8={fp8} stride={width + pad}", flush=True)
    o_ref, l_ref = c.oracle()
    for ns in (1, 3):
        out, lse = dsa.mla_decode(t16(c.q, dev), kv, torch.from_numpy(c.indices).to(dev), SM_SCALE,
                                  seq_lens=torch.from_numpy(c.seq_lens).to(dev),
                                  block_table=torch.from_numpy(c.block_table).to(dev),
                                  block_size=c.block_size, causal=True, num_splits=ns)
        torch.cuda.synchronize()
        assert_parity(bits(out), lse.cpu().numpy(), o_ref, l_ref, f"padded rows splits={ns}")
    # prefill over the same padded pool (flat indices = physical rows the decode lists name;
    # every other row is NaN-poisoned)
    rng = np.random.default_rng(22)
    N = 40
    qp = oracle.normal_bf16(rng, (N, 128, D_QK))
    good = np.flatnonzero(c.kv[:, 0] != (0xFF if fp8 else 0x7FC0))
    idx = np.stack([rng.choice(good, 300, replace=False) for _ in range(N)]).astype(np.int32)
    o_ref, l_ref = oracle.mla_prefill(qp, c.kv, idx, SM_SCALE)
    out, lse = dsa.mla_prefill(t16(qp, dev), kv, torch.from_numpy(idx).to(dev), SM_SCALE)
    torch.cuda.synchronize()
    assert_parity(bits(out), lse.cpu().numpy(), o_ref, l_ref, "padded rows prefill")


# ------------------------------------------------------------------ prefill

@pytest.mark.parametrize("fp8", [False, True])
def test_prefill_causal(dev, fp8):
    """Config 5 style at small size: query t attends min(topk, t+1) distinct positions <= t.
    Every query is checked, the short lists of the first queries included (one row for
    query 0: its LSE is a single score)."""
    rng = np.random.default_rng(21)
    N, H, topk = 300, 128, 256
    q = oracle.normal_bf16(rng, (N, H, D_QK))
    kv = fp8_rows(rng, N) if fp8 else bf16_rows(rng, N)
    idx = np.full((N, topk), -1, np.int32)
    for t in range(N):
        n = min(topk, t + 1)
        idx[t, :n] = oracle.distinct_indices(rng, t + 1, n)
    print(f"[case] prefill fp8={fp8} N={N} topk={topk}", flush=True)
    o_ref, l_ref = oracle.mla_prefill(q, kv, idx, SM_SCALE, causal=True)
    out, lse = dsa.mla_prefill(t16(q, dev), kv_tensor(kv, dev), torch.from_numpy(idx).to(dev),
                               SM_SCALE, causal=True)
    torch.cuda.synchronize()
    e = assert_parity(bits(out), lse.cpu().numpy(), o_ref, l_ref, "prefill")
    print(f"[case] prefill: max|dO|={e[0]:.3e} max rel dLSE={e[1]:.3e}", flush=True)


# ------------------------------------------------------- combine and writer

def test_combine_kernel(dev):
    rng = np.random.default_rng(31)
    S, rows, H = 5, 7, 128
    po = rng.standard_normal((S, rows, H, 512)).astype(np.float32)
    pl = (rng.standard_normal((S, rows, H)) * 3).astype(np.float32)
    pl[1, 2, :] = -np.finfo(np.float32).max      # an empty split
    pl[:, 4, 7] = -np.finfo(np.float32).max      # every split empty -> O = 0, LSE = +inf
    o_ref, l_ref = oracle.mla_combine(po, pl)
    out, lse = dsa.mla_combine(torch.from_numpy(po).to(dev), torch.from_numpy(pl).to(dev))
    torch.cuda.synchronize()
    assert_parity(bits(out), lse.cpu().numpy(), o_ref, l_ref, "combine")
    assert np.isposinf(lse.cpu().numpy()[4, 7]) and (bits(out)[4, 7] == 0).all()


def test_quantize_bit_exact(dev):
    rng = np.random.default_rng(41)
    n = 777
    src = oracle.bf16_to_f32(oracle.normal_bf16(rng, (n, D_QK)))
    src[3] *= 1e4
    src[4] *= 1e-30                                 # subnormal-heavy group
    src[5, :128] = 0.0                              # all-zero group -> scale 0
    src[6, 7] = 3.0e38
    src = oracle.bf16_to_f32(oracle.bf16_bits(src))
    ref = oracle.quantize_rows_656(src)
    got = dsa.quantize_kv_fp8(t16(oracle.bf16_bits(src), dev))
    torch.cuda.synchronize()
    got = got.cpu().numpy()
    assert np.array_equal(got, ref), f"{(got != ref).sum()} bytes differ"
    # scattered destinations (cache append through a slot mapping)
    dst = torch.zeros((2 * n, 656), dtype=torch.uint8, device=dev)
    rows = torch.from_numpy(rng.permutation(2 * n)[:n].astype(np.int64)).to(dev)
    dsa.quantize_kv_fp8(t16(oracle.bf16_bits(src), dev), dst, rows)
    torch.cuda.synchronize()
    assert np.array_equal(dst.cpu().numpy()[rows.cpu().numpy()], ref)
