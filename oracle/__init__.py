"""CPU oracle for the DSA sparse-MLA path - TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the checker (or the timed CPU baseline).  The
product (opfoundry_amd) never imports or calls it.

The arithmetic lives in oracle/dsa_oracle.c (built by oracle/Makefile into
oracle/_build/libdsa_oracle.so); this module is its ctypes front end plus the
seeded input generators the tests and the bench share.  Reference anchors for
each C function are in that file's header.  Pinning: every function here is
checked in tests/test_oracle_*.py against an independent statement of its
answer (closed forms, brute force, torch's bf16 rounding, identities) - no
function of the oracle is left "parity unpinned".
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

from opfoundry_amd.abi import (D_QK, D_V4, D_VO, V4_NOPE, DecodeArgs, KV_BF16, KV_FP8_656, MxArgs,
                               PrefillArgs, PrefillV4Args, PrefillV4Fp8Args)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libdsa_oracle.so")

_LIB = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32
        L.oracle_f32_to_bf16.restype = ctypes.c_uint16
        L.oracle_f32_to_bf16.argtypes = [ctypes.c_float]
        L.oracle_fp8_e4m3_encode.restype = ctypes.c_uint8
        L.oracle_fp8_e4m3_encode.argtypes = [ctypes.c_float]
        L.oracle_fp8_e4m3_decode.restype = ctypes.c_float
        L.oracle_fp8_e4m3_decode.argtypes = [ctypes.c_uint8]
        for n in ("oracle_fp8_encode_n", "oracle_fp8_decode_n", "oracle_bf16_round_n",
                  "oracle_quantize_rows_656", "oracle_dequant_rows_656"):
            getattr(L, n).argtypes = [vp, i64, vp] if "rows" in n else [vp, vp, i64]
            getattr(L, n).restype = None
        L.oracle_mla_decode.argtypes = [ctypes.POINTER(DecodeArgs), ctypes.c_int]
        L.oracle_mla_decode_partial.argtypes = [ctypes.POINTER(DecodeArgs), i32, i32, vp, vp,
                                                ctypes.c_int]
        L.oracle_mla_combine.argtypes = [vp, vp, i32, i64, i32, vp, vp]
        L.oracle_mla_combine.restype = None
        L.oracle_mla_prefill.argtypes = [ctypes.POINTER(PrefillArgs), ctypes.c_int]
        L.oracle_mla_prefill_v4.argtypes = [ctypes.POINTER(PrefillV4Args), ctypes.c_int]
        L.oracle_mla_decode_mxfp8.argtypes = [ctypes.POINTER(MxArgs), ctypes.c_int]
        L.oracle_dequant_row_mxfp8.argtypes = [vp, vp, vp, vp]
        L.oracle_dequant_row_mxfp8.restype = None
        L.oracle_mla_prefill_v4_fp8.argtypes = [ctypes.POINTER(PrefillV4Fp8Args), ctypes.c_int]
        L.oracle_dequant_row_v4fp8.argtypes = [vp, vp, vp]
        L.oracle_dequant_row_v4fp8.restype = None
        L.oracle_num_threads.argtypes = [ctypes.c_int]
        _LIB = L
    return _LIB


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


# ------------------------------------------------------------------ codecs

def bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns (uint16), round to nearest even."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().oracle_bf16_round_n(_p(x), _p(out), x.size)
    return out


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def fp8_encode(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint8)
    lib().oracle_fp8_encode_n(_p(x), _p(out), x.size)
    return out


def fp8_decode(c: np.ndarray) -> np.ndarray:
    c = np.ascontiguousarray(c, dtype=np.uint8)
    out = np.empty(c.shape, np.float32)
    lib().oracle_fp8_decode_n(_p(c), _p(out), c.size)
    return out


def quantize_rows_656(rows_f32: np.ndarray) -> np.ndarray:
    """[n, 576] fp32 (bf16-representable) -> [n, 656] uint8 cache rows."""
    r = np.ascontiguousarray(rows_f32, dtype=np.float32).reshape(-1, D_QK)
    out = np.empty((r.shape[0], 656), np.uint8)
    lib().oracle_quantize_rows_656(_p(r), r.shape[0], _p(out))
    return out


def dequant_rows_656(rows: np.ndarray) -> np.ndarray:
    r = np.ascontiguousarray(rows, dtype=np.uint8).reshape(-1, 656)
    out = np.empty((r.shape[0], D_QK), np.float32)
    lib().oracle_dequant_rows_656(_p(r), r.shape[0], _p(out))
    return out


# ------------------------------------------------------------- top-k selection

def order_keys(x: np.ndarray) -> np.ndarray:
    """uint32 keys that order fp32 scores as IEEE values, every NaN above +inf and -0 equal
    to +0 (the order of dsa_topk_indices, include/dsa_topk.h).  The reference has no top-k
    step: its kernels take the caller's lists (opus_attn/dsa_v4/README.md:185)."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    mag = b & np.uint32(0x7FFFFFFF)
    key = np.where(b >> np.uint32(31) != 0, ~b, b | np.uint32(0x80000000)).astype(np.uint32)
    key = np.where(mag == 0, np.uint32(0x80000000), key)
    return np.where(mag > np.uint32(0x7F800000), np.uint32(0xFFFFFFFF), key).astype(np.uint32)


def topk_indices(scores: np.ndarray, lengths, topk: int) -> np.ndarray:
    """Per row t, the topk positions of scores[t, :lengths[t]] with the highest keys (ties:
    lower position first), ascending, then -1 up to topk: int32 [T, topk].  These rows are
    the `indices` the decode path reads (-1 = padding)."""
    T, n_max = scores.shape
    out = np.full((T, topk), -1, np.int32)
    for t in range(T):
        n = n_max if lengths is None else int(min(max(int(lengths[t]), 0), n_max))
        key = order_keys(scores[t, :n]).astype(np.int64)
        order = np.lexsort((np.arange(n), -key))      # key descending, then position ascending
        sel = np.sort(order[:topk])
        out[t, :sel.size] = sel
    return out


def indexer_scores(q, weights, k_rows, seq_lens, *, block_table=None, block_size=1, k_batch_stride=0,
                   causal=False, n_cols=None):
    """The index scorer's contract (include/dsa_indexer.h; the reference has none - this is
    the DeepSeek-V3.2 lightning indexer's score), in float64: q bf16 bits [B, s_q, H_I, 128],
    weights f32 [B, s_q, H_I], k_rows bf16 bits [rows, 128].  Returns f64 [B, s_q, n_cols]:
    score[b, t, j] = sum_h w[b, t, h] * max(0, q[b, t, h] . k[row(b, j)]) for
    j < min(len(b, t), n_cols), -inf where the row lies outside the cache, NaN where no score
    is defined (j past the list).  Rows as dsa_mla_decode's top-k form."""
    qf = bf16_to_f32(np.asarray(q, np.uint16)).astype(np.float64)
    kf = bf16_to_f32(np.asarray(k_rows, np.uint16).reshape(-1, 128)).astype(np.float64)
    w = np.asarray(weights, np.float64)
    B, s_q, H_I, _ = qf.shape
    if n_cols is None:
        n_cols = int(np.max(seq_lens)) if B else 0
    out = np.full((B, s_q, n_cols), np.nan)
    for b in range(B):
        L = int(seq_lens[b])
        for t in range(s_q):
            n = min(max(L - (s_q - 1 - t) if causal else L, 0), n_cols)
            j = np.arange(n)
            if block_table is not None:
                phys = block_table[b][j // block_size].astype(np.int64) * block_size + j % block_size
            else:
                phys = b * k_batch_stride + j
            ok = (phys >= 0) & (phys < kf.shape[0])
            dots = qf[b, t] @ kf[np.where(ok, phys, 0)].T          # [H_I, n]
            s = (w[b, t][:, None] * np.maximum(dots, 0.0)).sum(0)
            out[b, t, :n] = np.where(ok, s, -np.inf)
    return out


# ------------------------------------------------------------- attention

def _decode_args(q, kv, fmt, indices, seq_lens, block_table, block_size, kv_batch_stride, causal,
                 sm_scale, out, lse):
    B, s_q, H, _ = q.shape
    a = DecodeArgs()
    a.q = _p(q)
    a.q_stride_b, a.q_stride_t, a.q_stride_h = s_q * H * D_QK, H * D_QK, D_QK
    a.kv_cache = _p(kv)
    a.kv_total_rows = kv.shape[0]
    a.kv_format = fmt
    a.block_size = block_size
    a.kv_batch_stride = kv_batch_stride
    # rows wider than the format's row are padded rows (the row stride is the array's width)
    width = D_QK if fmt == KV_BF16 else 656
    a.kv_stride_row = 0 if kv.shape[1] == width else kv.shape[1]
    a.block_table = _p(block_table)
    a.block_table_stride = 0 if block_table is None else block_table.shape[1]
    a.seq_lens = _p(seq_lens)
    a.indices = _p(indices)
    a.idx_stride_b, a.idx_stride_t = indices.shape[1] * indices.shape[2], indices.shape[2]
    a.out = _p(out)
    a.o_stride_b, a.o_stride_t, a.o_stride_h = s_q * H * D_VO, H * D_VO, D_VO
    a.lse = _p(lse)
    a.B, a.s_q, a.H, a.topk = B, s_q, H, indices.shape[2]
    a.num_splits = 1
    a.causal = 1 if causal else 0
    a.sm_scale = float(sm_scale)
    return a


def _prep(q, kv, indices, seq_lens, block_table):
    q = np.ascontiguousarray(q, dtype=np.uint16)
    kv = np.ascontiguousarray(kv)
    fmt = KV_BF16 if kv.dtype == np.uint16 else KV_FP8_656
    width = D_QK if fmt == KV_BF16 else 656
    # [..., width] dense rows, or [rows, stride] padded rows (stride > width)
    kv = kv.reshape(-1, width) if kv.shape[-1] == width else kv.reshape(-1, kv.shape[-1])
    indices = np.ascontiguousarray(indices, dtype=np.int32)
    seq_lens = np.ascontiguousarray(seq_lens, dtype=np.int32)
    if block_table is not None:
        block_table = np.ascontiguousarray(block_table, dtype=np.int32)
    return q, kv, fmt, indices, seq_lens, block_table


def mla_decode(q, kv, indices, seq_lens, sm_scale, *, block_table=None, block_size=1,
               kv_batch_stride=0, causal=False, num_threads=0):
    """Host oracle of dsa_mla_decode: q uint16(bf16) [B,s_q,H,576]; kv uint16 [rows,576]
    (bf16) or uint8 [rows,656] (fp8); returns (O uint16 bf16 [B,s_q,H,512], LSE f32)."""
    q, kv, fmt, indices, seq_lens, block_table = _prep(q, kv, indices, seq_lens, block_table)
    B, s_q, H, _ = q.shape
    out = np.zeros((B, s_q, H, D_VO), np.uint16)
    lse = np.zeros((B, s_q, H), np.float32)
    a = _decode_args(q, kv, fmt, indices, seq_lens, block_table, block_size, kv_batch_stride,
                     causal, sm_scale, out, lse)
    rc = lib().oracle_mla_decode(ctypes.byref(a), num_threads)
    assert rc == 0
    return out, lse


def mla_decode_partial(q, kv, indices, seq_lens, sm_scale, k_begin, k_end, *, block_table=None,
                       block_size=1, kv_batch_stride=0, causal=False, num_threads=0):
    """Split partial over top-k range [k_begin, k_end): fp32 O [B*s_q,H,512], LSE [B*s_q,H]."""
    q, kv, fmt, indices, seq_lens, block_table = _prep(q, kv, indices, seq_lens, block_table)
    B, s_q, H, _ = q.shape
    out = np.zeros((B, s_q, H, D_VO), np.uint16)
    po = np.zeros((B * s_q, H, D_VO), np.float32)
    pl = np.zeros((B * s_q, H), np.float32)
    a = _decode_args(q, kv, fmt, indices, seq_lens, block_table, block_size, kv_batch_stride,
                     causal, sm_scale, out, None)
    rc = lib().oracle_mla_decode_partial(ctypes.byref(a), k_begin, k_end, _p(po), _p(pl),
                                         num_threads)
    assert rc == 0
    return po, pl


def mla_combine(part_o: np.ndarray, part_lse: np.ndarray):
    """[S, rows, H, 512] + [S, rows, H] -> (bf16 bits [rows, H, 512], lse [rows, H])."""
    po = np.ascontiguousarray(part_o, dtype=np.float32)
    pl = np.ascontiguousarray(part_lse, dtype=np.float32)
    S, rows, H, _ = po.shape
    out = np.zeros((rows, H, D_VO), np.uint16)
    lse = np.zeros((rows, H), np.float32)
    lib().oracle_mla_combine(_p(po), _p(pl), S, rows, H, _p(out), _p(lse))
    return out, lse


def mla_prefill_v4(q, unified_kv, kv, attn_sink, indptr_prefix, indices_prefix, indptr_extend,
                   indices_extend, softmax_scale, *, num_threads=0):
    """Host oracle of dsa_mla_prefill_v4: q uint16 [N,H,512]; unified_kv / kv uint16 [rows,512];
    attn_sink float32 [H] or None; CSR lists int32.  Returns (O uint16 [N,H,512], LSE f32)."""
    q = np.ascontiguousarray(q, dtype=np.uint16)
    ukv = np.ascontiguousarray(unified_kv, dtype=np.uint16).reshape(-1, D_V4)
    xkv = np.ascontiguousarray(kv, dtype=np.uint16).reshape(-1, D_V4)
    sink = None if attn_sink is None else np.ascontiguousarray(attn_sink, dtype=np.float32)
    ipp, idp = (np.ascontiguousarray(x, dtype=np.int32) for x in (indptr_prefix, indices_prefix))
    ipe, ide = (np.ascontiguousarray(x, dtype=np.int32) for x in (indptr_extend, indices_extend))
    N, H, _ = q.shape
    out = np.zeros((N, H, D_V4), np.uint16)
    lse = np.zeros((N, H), np.float32)
    max_rows = int(max((ipp[1:] - ipp[:-1]).max(initial=0) + (ipe[1:] - ipe[:-1]).max(initial=0), 1))
    a = PrefillV4Args()
    a.q, a.unified_kv, a.kv, a.attn_sink, a.out, a.lse = _p(q), _p(ukv), _p(xkv), _p(sink), _p(out), _p(lse)
    a.kv_indptr_prefix, a.kv_indices_prefix = _p(ipp), _p(idp)
    a.kv_indptr_extend, a.kv_indices_extend = _p(ipe), _p(ide)
    a.N, a.H, a.D = N, H, D_V4
    a.total_pages, a.total_tokens = ukv.shape[0], xkv.shape[0]
    a.stride_qo_n, a.stride_qo_h = H * D_V4, D_V4
    a.stride_kv_page = D_V4
    a.max_rows = max_rows
    a.softmax_scale = float(softmax_scale)
    rc = lib().oracle_mla_prefill_v4(ctypes.byref(a), num_threads)
    assert rc == 0
    return out, lse


def dequant_rows_mxfp8(nope: np.ndarray, scale: np.ndarray, rope: np.ndarray) -> np.ndarray:
    """MXFP8 split-stream rows (uint8 [n,512], uint8 [n,16], uint16 [n,64]) -> fp32 [n,576]."""
    nope = np.ascontiguousarray(nope, dtype=np.uint8).reshape(-1, 512)
    scale = np.ascontiguousarray(scale, dtype=np.uint8).reshape(-1, 16)
    rope = np.ascontiguousarray(rope, dtype=np.uint16).reshape(-1, 64)
    out = np.zeros((nope.shape[0], D_QK), np.float32)
    for r in range(nope.shape[0]):
        lib().oracle_dequant_row_mxfp8(_p(nope[r]), _p(scale[r]), _p(rope[r]), _p(out[r]))
    return out


def mla_decode_mxfp8(q_nope, q_scale, q_rope, kv_nope, kv_scale, kv_rope, kv_indptr, kv_indices, s_q,
                     softmax_scale, *, num_threads=0):
    """Host oracle of dsa_mla_decode_mxfp8 (dense streams): q_* [B*s_q, H, 512 | 16 | 64]
    (uint8, uint8, uint16), kv_* [rows, 512 | 16 | 64], CSR lists int32.  Returns
    (O uint16 [B*s_q, H, 512], LSE f32 [B*s_q, H])."""
    qn = np.ascontiguousarray(q_nope, dtype=np.uint8)
    qs = np.ascontiguousarray(q_scale, dtype=np.uint8)
    qr = np.ascontiguousarray(q_rope, dtype=np.uint16)
    kn = np.ascontiguousarray(kv_nope, dtype=np.uint8).reshape(-1, 512)
    ks = np.ascontiguousarray(kv_scale, dtype=np.uint8).reshape(-1, 16)
    kr = np.ascontiguousarray(kv_rope, dtype=np.uint16).reshape(-1, 64)
    ip = np.ascontiguousarray(kv_indptr, dtype=np.int32)
    ix = np.ascontiguousarray(kv_indices, dtype=np.int32)
    if ix.size == 0:
        ix = np.zeros(1, np.int32)
    T, H, _ = qn.shape
    B = ip.size - 1
    assert T == B * s_q
    out = np.zeros((T, H, D_VO), np.uint16)
    lse = np.zeros((T, H), np.float32)
    a = MxArgs()
    a.q_nope, a.q_scale, a.q_rope = _p(qn), _p(qs), _p(qr)
    a.kv_nope, a.kv_scale, a.kv_rope = _p(kn), _p(ks), _p(kr)
    a.out, a.lse, a.kv_indptr, a.kv_indices = _p(out), _p(lse), _p(ip), _p(ix)
    a.B, a.s_q, a.H, a.total_tokens = B, s_q, H, kn.shape[0]
    a.stride_q_nope_b, a.stride_q_nope_h = H * 512, 512
    a.stride_q_scale_b, a.stride_q_scale_h = H * 16, 16
    a.stride_q_rope_b, a.stride_q_rope_h = H * 64, 64
    a.stride_o_b, a.stride_o_h = H * D_VO, D_VO
    a.stride_kv_nope_page, a.stride_kv_scale_page, a.stride_kv_rope_page = 512, 16, 64
    a.max_kv_len = int(max((ip[1:] - ip[:-1]).max(initial=0), 1))
    a.softmax_scale = float(softmax_scale)
    rc = lib().oracle_mla_decode_mxfp8(ctypes.byref(a), num_threads)
    assert rc == 0
    return out, lse


def dequant_rows_v4fp8(nope: np.ndarray, rope: np.ndarray) -> np.ndarray:
    """V4 fp8 rows (uint8 [n,512]: 448 codes, 14 E8M0, pad; uint16 [n,64] bf16) -> fp32 [n,512]."""
    nope = np.ascontiguousarray(nope, dtype=np.uint8).reshape(-1, 512)
    rope = np.ascontiguousarray(rope, dtype=np.uint16).reshape(-1, 64)
    out = np.zeros((nope.shape[0], D_V4), np.float32)
    for r in range(nope.shape[0]):
        lib().oracle_dequant_row_v4fp8(_p(nope[r]), _p(rope[r]), _p(out[r]))
    return out


def mla_prefill_v4_fp8(q_nope, q_rope, ukv_nope, ukv_rope, kv_nope, kv_rope, attn_sink, indptr_prefix,
                       indices_prefix, indptr_extend, indices_extend, softmax_scale, *, num_threads=0):
    """Host oracle of dsa_mla_prefill_v4_fp8 (dense streams): q_nope uint8 [N,H,512], q_rope uint16
    [N,H,64], pools uint8 [rows,512] + uint16 [rows,64]; returns (O uint16 [N,H,512], LSE f32)."""
    qn = np.ascontiguousarray(q_nope, dtype=np.uint8)
    qr = np.ascontiguousarray(q_rope, dtype=np.uint16)
    un = np.ascontiguousarray(ukv_nope, dtype=np.uint8).reshape(-1, 512)
    ur = np.ascontiguousarray(ukv_rope, dtype=np.uint16).reshape(-1, 64)
    xn = np.ascontiguousarray(kv_nope, dtype=np.uint8).reshape(-1, 512)
    xr = np.ascontiguousarray(kv_rope, dtype=np.uint16).reshape(-1, 64)
    sink = None if attn_sink is None else np.ascontiguousarray(attn_sink, dtype=np.float32)
    ipp, idp = (np.ascontiguousarray(x, dtype=np.int32) for x in (indptr_prefix, indices_prefix))
    ipe, ide = (np.ascontiguousarray(x, dtype=np.int32) for x in (indptr_extend, indices_extend))
    N, H, _ = qn.shape
    out = np.zeros((N, H, D_V4), np.uint16)
    lse = np.zeros((N, H), np.float32)
    a = PrefillV4Fp8Args()
    a.q_nope, a.q_rope = _p(qn), _p(qr)
    a.unified_kv_nope, a.unified_kv_rope, a.kv_nope, a.kv_rope = _p(un), _p(ur), _p(xn), _p(xr)
    a.attn_sink, a.out, a.lse = _p(sink), _p(out), _p(lse)
    a.kv_indptr_prefix, a.kv_indices_prefix = _p(ipp), _p(idp)
    a.kv_indptr_extend, a.kv_indices_extend = _p(ipe), _p(ide)
    a.N, a.H, a.total_pages, a.total_tokens = N, H, un.shape[0], xn.shape[0]
    a.stride_q_nope_n, a.stride_q_nope_h = H * 512, 512
    a.stride_q_rope_n, a.stride_q_rope_h = H * 64, 64
    a.stride_o_n, a.stride_o_h = H * D_V4, D_V4
    a.stride_kv_nope_page, a.stride_kv_rope_page = 512, 64
    a.max_rows = int(max((ipp[1:] - ipp[:-1]).max(initial=0) + (ipe[1:] - ipe[:-1]).max(initial=0), 1))
    a.softmax_scale = float(softmax_scale)
    rc = lib().oracle_mla_prefill_v4_fp8(ctypes.byref(a), num_threads)
    assert rc == 0
    return out, lse


def mla_prefill(q, kv, indices, sm_scale, *, causal=False, causal_offset=0, num_threads=0):
    """Host oracle of dsa_mla_prefill: q uint16 [N,H,576], kv uint16 [rows,576] or uint8
    [rows,656], indices int32 [N, topk]."""
    q = np.ascontiguousarray(q, dtype=np.uint16)
    kv = np.ascontiguousarray(kv)
    fmt = KV_BF16 if kv.dtype == np.uint16 else KV_FP8_656
    kv = kv.reshape(-1, D_QK if fmt == KV_BF16 else 656)
    indices = np.ascontiguousarray(indices, dtype=np.int32)
    N, H, _ = q.shape
    out = np.zeros((N, H, D_VO), np.uint16)
    lse = np.zeros((N, H), np.float32)
    a = PrefillArgs()
    a.q = _p(q)
    a.q_stride_n, a.q_stride_h = H * D_QK, D_QK
    a.kv = _p(kv)
    a.kv_rows = kv.shape[0]
    a.kv_format = fmt
    a.indices = _p(indices)
    a.idx_stride_n = indices.shape[1]
    a.out = _p(out)
    a.o_stride_n, a.o_stride_h = H * D_VO, D_VO
    a.lse = _p(lse)
    a.N, a.H, a.topk = N, H, indices.shape[1]
    a.causal = 1 if causal else 0
    a.causal_offset = causal_offset
    a.sm_scale = float(sm_scale)
    rc = lib().oracle_mla_prefill(ctypes.byref(a), num_threads)
    assert rc == 0
    return out, lse


def num_threads(requested: int = 0) -> int:
    return lib().oracle_num_threads(requested)


# ------------------------------------------------------------- generators

def normal_bf16(rng: np.random.Generator, shape) -> np.ndarray:
    """~N(0,1) rounded to bf16 (bit patterns)."""
    return bf16_bits(rng.standard_normal(shape, dtype=np.float32))


def mxfp8_rows(rng: np.random.Generator, n: int):
    """MXFP8 split-stream rows distributed as the reference harness's init_fp8_mla_split
    (opus_attn/dsa_v32/common/host.cc:207-237): per 32-value block an exponent e in
    [0, 3], scale byte e + 127, codes e4m3(N(0,1) * 2^-e); RoPE N(0,1) in bf16.
    Returns (nope uint8 [n,512], scale uint8 [n,16], rope uint16 [n,64])."""
    e = rng.integers(0, 4, size=(n, 16))
    x = rng.standard_normal((n, 16, 32), dtype=np.float32) * np.ldexp(1.0, -e)[:, :, None].astype(np.float32)
    nope = fp8_encode(x.reshape(n, 512))
    return nope, (e + 127).astype(np.uint8), normal_bf16(rng, (n, 64))


def v4fp8_rows(rng: np.random.Generator, n: int):
    """V4 fp8 rows drawn as init_fp8_dsa_split (opus_attn/dsa_v4/common/mla_v4_host.cc:208-240):
    14 blocks of 32 codes e4m3(N(0,1) * 2^-e), e in [0, 3], scale bytes e + 127 at 448..461,
    the rest of the 512-byte row 0xFF; RoPE N(0,1) bf16.  Returns (nope uint8 [n,512],
    rope uint16 [n,64])."""
    nb = V4_NOPE // 32
    e = rng.integers(0, 4, size=(n, nb))
    x = rng.standard_normal((n, nb, 32), dtype=np.float32) * np.ldexp(1.0, -e)[:, :, None].astype(np.float32)
    nope = np.full((n, 512), 0xFF, np.uint8)
    nope[:, :V4_NOPE] = fp8_encode(x.reshape(n, V4_NOPE))
    nope[:, V4_NOPE:V4_NOPE + nb] = (e + 127).astype(np.uint8)
    return nope, normal_bf16(rng, (n, 64))


def distinct_indices(rng: np.random.Generator, high: int, k: int) -> np.ndarray:
    """k distinct positions drawn uniformly from [0, high), scattered order (k <= high)."""
    return rng.choice(high, size=k, replace=False).astype(np.int32)
