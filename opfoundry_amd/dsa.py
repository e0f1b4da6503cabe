"""Torch-facing host API of the DSA sparse-MLA library.

These functions mirror the reference's launch API for the path - q, latent KV
cache, top-k index tensor, sm_scale, output and LSE
(``mla_decode_launch_pipeline``, opus_attn/dsa_v32/common/host.cc:114-138;
``mla_v4_prefill_launch``, opus_attn/dsa_v4/common/mla_v4_host.cc:28-47) -
and forward to the C ABI of libdsa_mla.so.  PyTorch only provides device
memory and the current stream; all compute happens in the HIP kernels.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch

from . import abi
from .abi import DecodeArgs, PrefillArgs, check, load_library


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream(stream) -> Optional[int]:
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream)


def kv_format_of(kv: torch.Tensor) -> Tuple[int, int, int]:
    """(kv_format, total_rows, row_stride) of a cache tensor: bf16 [..., 576] or uint8
    [..., 656] with a dense last dim.  Rows may be padded (a view of wider rows): row_stride
    is the element distance between rows, 0 when they are dense."""
    if kv.dtype == torch.bfloat16 and kv.shape[-1] == abi.D_QK:
        fmt, width = abi.KV_BF16, abi.D_QK
    elif kv.dtype == torch.uint8 and kv.shape[-1] == abi.FP8_ROW_BYTES:
        fmt, width = abi.KV_FP8_656, abi.FP8_ROW_BYTES
    else:
        raise ValueError(f"kv cache must be bf16 [..., 576] or uint8 [..., 656], got {kv.dtype} "
                         f"{tuple(kv.shape)}")
    if kv.stride(-1) != 1:
        raise ValueError("kv cache rows must have a dense last dim")
    rs = kv.stride(-2) if kv.dim() >= 2 else width
    expect = rs
    for d in range(kv.dim() - 2, -1, -1):
        if kv.shape[d] > 1 and kv.stride(d) != expect:
            raise ValueError("kv cache rows must be one uniform stride apart")
        expect *= kv.shape[d]
    return fmt, kv.numel() // width, (0 if rs == width else rs)


def _need(t: torch.Tensor, dtype, name: str):
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")


def _run_with_workspace(size_fn, run_fn, args, workspace, device, stream, where: str):
    """Size the call's workspace (size_fn), allocate one if the caller's is missing or too small,
    and launch (run_fn(args, ws_ptr, ws_bytes, stream))."""
    n = ctypes.c_size_t(0)
    check(size_fn(ctypes.byref(args), ctypes.byref(n)), where + "_workspace_size")
    if n.value and (workspace is None or workspace.numel() * workspace.element_size() < n.value):
        workspace = torch.empty(n.value, dtype=torch.uint8, device=device)
    check(run_fn(ctypes.byref(args), _ptr(workspace) if n.value else None, n.value, _stream(stream)), where)


def make_decode_args(q, kv_cache, indices, sm_scale, out, lse, *, seq_lens, block_table=None,
                     block_size=None, causal=False, num_splits=0, kv_batch_stride=0):
    B, s_q, H, D = q.shape
    if D != abi.D_QK or q.stride(3) != 1:
        raise ValueError("q must be [B, s_q, H, 576] with a dense last dim")
    if tuple(indices.shape[:2]) != (B, s_q) or indices.stride(2) != 1:
        raise ValueError("indices must be [B, s_q, topk] with a dense last dim")
    fmt, rows, row_stride = kv_format_of(kv_cache)
    if block_table is not None:
        if block_size is None:
            block_size = kv_cache.shape[-2] if kv_cache.dim() >= 3 else None
        if block_size is None:
            raise ValueError("block_size is required with a block table")
        bt_stride = block_table.stride(0)
    else:
        block_size = block_size or 1
        bt_stride = 0
    a = DecodeArgs()
    a.q = _ptr(q)
    a.q_stride_b, a.q_stride_t, a.q_stride_h = q.stride(0), q.stride(1), q.stride(2)
    a.kv_cache = _ptr(kv_cache)
    a.kv_total_rows = rows
    a.kv_format = fmt
    a.block_size = int(block_size)
    a.kv_batch_stride = int(kv_batch_stride)
    a.kv_stride_row = row_stride
    a.block_table = _ptr(block_table)
    a.block_table_stride = bt_stride
    a.seq_lens = _ptr(seq_lens)
    a.indices = _ptr(indices)
    a.idx_stride_b, a.idx_stride_t = indices.stride(0), indices.stride(1)
    a.out = _ptr(out)
    a.o_stride_b, a.o_stride_t, a.o_stride_h = out.stride(0), out.stride(1), out.stride(2)
    a.lse = _ptr(lse)
    a.B, a.s_q, a.H, a.topk = B, s_q, H, indices.shape[2]
    a.num_splits = int(num_splits)
    a.causal = 1 if causal else 0
    a.sm_scale = float(sm_scale)
    return a


def decode_workspace_size(args: DecodeArgs) -> int:
    n = ctypes.c_size_t(0)
    check(load_library().dsa_mla_decode_workspace_size(ctypes.byref(args), ctypes.byref(n)),
          "dsa_mla_decode_workspace_size")
    return n.value


def decode_num_splits(args: DecodeArgs) -> int:
    n = ctypes.c_int32(0)
    check(load_library().dsa_mla_decode_num_splits(ctypes.byref(args), ctypes.byref(n)),
          "dsa_mla_decode_num_splits")
    return n.value


def mla_decode(q: torch.Tensor, kv_cache: torch.Tensor, indices: torch.Tensor, sm_scale: float,
               out: Optional[torch.Tensor] = None, lse: Optional[torch.Tensor] = None, *,
               seq_lens: torch.Tensor, block_table: Optional[torch.Tensor] = None,
               block_size: Optional[int] = None, causal: bool = False, num_splits: int = 0,
               kv_batch_stride: int = 0, workspace: Optional[torch.Tensor] = None,
               stream=None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Sparse MLA decode over a (paged) latent cache; returns (out bf16, lse fp32).

    q [B, s_q, H, 576] bf16; kv_cache bf16 [..., 576] or uint8 [..., 656]
    (fp8 e4m3 + per-128 scales + bf16 RoPE); indices int32 [B, s_q, topk]
    with -1 padding; seq_lens int32 [B]; block_table int32 [B, max_blocks].
    """
    _need(q, torch.bfloat16, "q")
    _need(indices, torch.int32, "indices")
    _need(seq_lens, torch.int32, "seq_lens")
    if block_table is not None:
        _need(block_table, torch.int32, "block_table")
    B, s_q, H, _ = q.shape
    if out is None:
        out = torch.empty((B, s_q, H, abi.D_VO), dtype=torch.bfloat16, device=q.device)
    if lse is None:
        lse = torch.empty((B, s_q, H), dtype=torch.float32, device=q.device)
    a = make_decode_args(q, kv_cache, indices, sm_scale, out, lse, seq_lens=seq_lens,
                         block_table=block_table, block_size=block_size, causal=causal,
                         num_splits=num_splits, kv_batch_stride=kv_batch_stride)
    ws_bytes = decode_workspace_size(a)
    if ws_bytes and (workspace is None or workspace.numel() * workspace.element_size() < ws_bytes):
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
    check(load_library().dsa_mla_decode(ctypes.byref(a), _ptr(workspace) if ws_bytes else None,
                                        ws_bytes, _stream(stream)), "dsa_mla_decode")
    return out, lse


def make_decode_csr_args(q, kv, kv_indptr, kv_indices, sm_scale, out, lse, *, s_q=1,
                         max_kv_len=None, num_splits=0):
    """CSR-form arguments: q [B*s_q, H, 576], kv [total_tokens, row], kv_indptr int32 [B+1],
    kv_indices int32 (physical rows, page size 1)."""
    total_q, H, D = q.shape
    if D != abi.D_QK or q.stride(2) != 1:
        raise ValueError("q must be [B*s_q, H, 576] with a dense last dim")
    if total_q % s_q:
        raise ValueError("q rows must be B * s_q")
    fmt, rows, row_stride = kv_format_of(kv)
    B = kv_indptr.numel() - 1
    if B * s_q != total_q:
        raise ValueError("kv_indptr must have B + 1 entries with B * s_q == q.shape[0]")
    if max_kv_len is None:
        max_kv_len = int((kv_indptr[1:] - kv_indptr[:-1]).max()) if B > 0 else 0
    a = abi.CsrArgs()
    a.q, a.kv, a.out, a.lse = _ptr(q), _ptr(kv), _ptr(out), _ptr(lse)
    a.kv_indptr, a.kv_indices = _ptr(kv_indptr), _ptr(kv_indices)
    a.B, a.s_q, a.H, a.total_tokens = B, s_q, H, rows
    a.stride_q_b, a.stride_q_h = q.stride(0), q.stride(1)
    a.stride_o_b, a.stride_o_h = out.stride(0), out.stride(1)
    a.stride_kv_page = row_stride
    a.kv_format = fmt
    a.max_kv_len = int(max_kv_len)
    a.num_splits = int(num_splits)
    a.softmax_scale = float(sm_scale)
    return a


def mla_decode_csr(q: torch.Tensor, kv: torch.Tensor, kv_indptr: torch.Tensor,
                   kv_indices: torch.Tensor, sm_scale: float, out: Optional[torch.Tensor] = None,
                   lse: Optional[torch.Tensor] = None, *, s_q: int = 1,
                   max_kv_len: Optional[int] = None, num_splits: int = 0,
                   workspace: Optional[torch.Tensor] = None,
                   stream=None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Sparse MLA decode in the reference's CSR form (kv_indptr / kv_indices, page size 1,
    count-based MTP causality); returns (out bf16 [B*s_q, H, 512], lse fp32 [B*s_q, H])."""
    _need(q, torch.bfloat16, "q")
    _need(kv_indptr, torch.int32, "kv_indptr")
    _need(kv_indices, torch.int32, "kv_indices")
    total_q, H, _ = q.shape
    if out is None:
        out = torch.empty((total_q, H, abi.D_VO), dtype=torch.bfloat16, device=q.device)
    if lse is None:
        lse = torch.empty((total_q, H), dtype=torch.float32, device=q.device)
    a = make_decode_csr_args(q, kv, kv_indptr, kv_indices, sm_scale, out, lse, s_q=s_q,
                             max_kv_len=max_kv_len, num_splits=num_splits)
    lib = load_library()
    n = ctypes.c_size_t(0)
    check(lib.dsa_mla_decode_csr_workspace_size(ctypes.byref(a), ctypes.byref(n)),
          "dsa_mla_decode_csr_workspace_size")
    if n.value and (workspace is None or workspace.numel() * workspace.element_size() < n.value):
        workspace = torch.empty(n.value, dtype=torch.uint8, device=q.device)
    check(lib.dsa_mla_decode_csr(ctypes.byref(a), _ptr(workspace) if n.value else None, n.value,
                                 _stream(stream)), "dsa_mla_decode_csr")
    return out, lse


def csr_plan(kv_indptr: torch.Tensor, B: int, s_q: int, H: int, max_kv_len: int,
             workspace: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """Build the CSR work plan of kv_indptr into a workspace (allocated when None) and return
    it; decode calls with num_splits=abi.SPLITS_PLANNED and that workspace reuse the plan
    (dsa_mla_csr_plan)."""
    _need(kv_indptr, torch.int32, "kv_indptr")
    lib = load_library()
    a = abi.CsrArgs()
    a.B, a.s_q, a.H, a.max_kv_len, a.num_splits = B, s_q, H, max_kv_len, 0
    a.q = a.kv = a.out = a.kv_indptr = a.kv_indices = 16        # sizing only: any aligned non-null
    a.stride_q_b, a.stride_q_h, a.stride_o_b, a.stride_o_h = H * 576, 576, H * 512, 512
    a.kv_format = abi.KV_BF16
    n = ctypes.c_size_t(0)
    check(lib.dsa_mla_decode_csr_workspace_size(ctypes.byref(a), ctypes.byref(n)),
          "dsa_mla_decode_csr_workspace_size")
    if workspace is None or workspace.numel() * workspace.element_size() < n.value:
        workspace = torch.empty(max(n.value, 16), dtype=torch.uint8, device=kv_indptr.device)
    check(lib.dsa_mla_csr_plan(_ptr(kv_indptr), B, s_q, H, max_kv_len, _ptr(workspace),
                               workspace.numel() * workspace.element_size(), _stream(stream)),
          "dsa_mla_csr_plan")
    return workspace


def make_decode_mxfp8_args(q_nope, q_scale, q_rope, kv_nope, kv_scale, kv_rope, kv_indptr,
                           kv_indices, sm_scale, out, lse, *, s_q=1, max_kv_len=None, num_splits=0):
    """dsa_mla_decode_mxfp8_args for split-stream tensors: q_nope uint8 [T, H, 512], q_scale
    uint8 [T, H, 16], q_rope bf16 [T, H, 64] (T = B * s_q); kv_nope uint8 [rows, 512], kv_scale
    uint8 [rows, 16], kv_rope bf16 [rows, 64]; every last dim dense."""
    T, H, _ = q_nope.shape
    for t, n, w in ((q_nope, "q_nope", 512), (q_scale, "q_scale", 16), (q_rope, "q_rope", 64)):
        if t.dim() != 3 or t.shape[0] != T or t.shape[1] != H or t.shape[2] != w or t.stride(2) != 1:
            raise ValueError(f"{n} must be [T, H, {w}] with a dense last dim")
    rows = kv_nope.shape[0]
    for t, n, w in ((kv_nope, "kv_nope", 512), (kv_scale, "kv_scale", 16), (kv_rope, "kv_rope", 64)):
        if t.dim() != 2 or t.shape[0] != rows or t.shape[1] != w or t.stride(1) != 1:
            raise ValueError(f"{n} must be [rows, {w}] with a dense last dim")
    B = kv_indptr.numel() - 1
    if B < 0 or T != B * s_q:
        raise ValueError("q streams must hold B * s_q query rows (B = kv_indptr.numel() - 1)")
    if max_kv_len is None:
        max_kv_len = int((kv_indptr[1:] - kv_indptr[:-1]).max().item()) if B > 0 else 0
    a = abi.MxArgs()
    a.q_nope, a.q_scale, a.q_rope = _ptr(q_nope), _ptr(q_scale), _ptr(q_rope)
    a.kv_nope, a.kv_scale, a.kv_rope = _ptr(kv_nope), _ptr(kv_scale), _ptr(kv_rope)
    a.out, a.lse = _ptr(out), _ptr(lse)
    a.kv_indptr, a.kv_indices = _ptr(kv_indptr), _ptr(kv_indices)
    a.B, a.s_q, a.H, a.total_tokens = B, s_q, H, rows
    a.stride_q_nope_b, a.stride_q_nope_h = q_nope.stride(0), q_nope.stride(1)
    a.stride_q_scale_b, a.stride_q_scale_h = q_scale.stride(0), q_scale.stride(1)
    a.stride_q_rope_b, a.stride_q_rope_h = q_rope.stride(0), q_rope.stride(1)
    a.stride_o_b, a.stride_o_h = out.stride(0), out.stride(1)
    a.stride_kv_nope_page, a.stride_kv_scale_page = kv_nope.stride(0), kv_scale.stride(0)
    a.stride_kv_rope_page = kv_rope.stride(0)
    a.max_kv_len = max_kv_len
    a.num_splits = num_splits
    a.softmax_scale = float(sm_scale)
    return a


def mla_decode_mxfp8(q_nope: torch.Tensor, q_scale: torch.Tensor, q_rope: torch.Tensor,
                     kv_nope: torch.Tensor, kv_scale: torch.Tensor, kv_rope: torch.Tensor,
                     kv_indptr: torch.Tensor, kv_indices: torch.Tensor, sm_scale: float,
                     out: Optional[torch.Tensor] = None, lse: Optional[torch.Tensor] = None, *,
                     s_q: int = 1, max_kv_len: Optional[int] = None, num_splits: int = 0,
                     workspace: Optional[torch.Tensor] = None,
                     stream=None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Sparse MLA decode on MXFP8 split streams (the reference's -dtype fp8 format), CSR
    form; returns (out bf16 [B*s_q, H, 512], lse fp32 [B*s_q, H])."""
    for t, n in ((q_nope, "q_nope"), (q_scale, "q_scale"), (kv_nope, "kv_nope"), (kv_scale, "kv_scale")):
        _need(t, torch.uint8, n)
    _need(q_rope, torch.bfloat16, "q_rope")
    _need(kv_rope, torch.bfloat16, "kv_rope")
    _need(kv_indptr, torch.int32, "kv_indptr")
    _need(kv_indices, torch.int32, "kv_indices")
    T, H, _ = q_nope.shape
    if out is None:
        out = torch.empty((T, H, abi.D_VO), dtype=torch.bfloat16, device=q_nope.device)
    if lse is None:
        lse = torch.empty((T, H), dtype=torch.float32, device=q_nope.device)
    a = make_decode_mxfp8_args(q_nope, q_scale, q_rope, kv_nope, kv_scale, kv_rope, kv_indptr,
                               kv_indices, sm_scale, out, lse, s_q=s_q, max_kv_len=max_kv_len,
                               num_splits=num_splits)
    lib = load_library()
    n = ctypes.c_size_t(0)
    check(lib.dsa_mla_decode_mxfp8_workspace_size(ctypes.byref(a), ctypes.byref(n)),
          "dsa_mla_decode_mxfp8_workspace_size")
    if n.value and (workspace is None or workspace.numel() * workspace.element_size() < n.value):
        workspace = torch.empty(n.value, dtype=torch.uint8, device=q_nope.device)
    check(lib.dsa_mla_decode_mxfp8(ctypes.byref(a), _ptr(workspace) if n.value else None, n.value,
                                   _stream(stream)), "dsa_mla_decode_mxfp8")
    return out, lse


def mla_combine(partial_o: torch.Tensor, partial_lse: torch.Tensor,
                out: Optional[torch.Tensor] = None, lse: Optional[torch.Tensor] = None,
                stream=None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Merge split partials fp32 [S, rows, H, 512] + [S, rows, H] -> bf16 [rows, H, 512], lse."""
    _need(partial_o, torch.float32, "partial_o")
    _need(partial_lse, torch.float32, "partial_lse")
    S, rows, H, D = partial_o.shape
    if D != abi.D_VO or tuple(partial_lse.shape) != (S, rows, H):
        raise ValueError("partial_o must be [S, rows, H, 512] and partial_lse [S, rows, H]")
    if not (partial_o.is_contiguous() and partial_lse.is_contiguous()):
        raise ValueError("partials must be contiguous")
    if out is None:
        out = torch.empty((rows, H, D), dtype=torch.bfloat16, device=partial_o.device)
    if lse is None:
        lse = torch.empty((rows, H), dtype=torch.float32, device=partial_o.device)
    check(load_library().dsa_mla_combine(_ptr(partial_o), _ptr(partial_lse), S, rows, H, _ptr(out),
                                         out.stride(0), out.stride(1), _ptr(lse), _stream(stream)),
          "dsa_mla_combine")
    return out, lse


def make_prefill_args(q, kv, indices, sm_scale, out, lse, *, causal=False, causal_offset=0, num_splits=0):
    N, H, D = q.shape
    if D != abi.D_QK or q.stride(2) != 1:
        raise ValueError("q must be [N, H, 576] with a dense last dim")
    if indices.shape[0] != N or indices.stride(1) != 1:
        raise ValueError("indices must be [N, topk] with a dense last dim")
    fmt, rows, row_stride = kv_format_of(kv)
    a = PrefillArgs()
    a.q = _ptr(q)
    a.q_stride_n, a.q_stride_h = q.stride(0), q.stride(1)
    a.kv = _ptr(kv)
    a.kv_rows = rows
    a.kv_stride_row = row_stride
    a.kv_format = fmt
    a.indices = _ptr(indices)
    a.idx_stride_n = indices.stride(0)
    a.out = _ptr(out)
    a.o_stride_n, a.o_stride_h = out.stride(0), out.stride(1)
    a.lse = _ptr(lse)
    a.N, a.H, a.topk = N, H, indices.shape[1]
    a.causal = 1 if causal else 0
    a.causal_offset = int(causal_offset)
    a.sm_scale = float(sm_scale)
    a.num_splits = int(num_splits)
    return a


def prefill_workspace_size(args: PrefillArgs) -> int:
    n = ctypes.c_size_t(0)
    check(load_library().dsa_mla_prefill_workspace_size(ctypes.byref(args), ctypes.byref(n)),
          "dsa_mla_prefill_workspace_size")
    return n.value


def mla_prefill(q: torch.Tensor, kv: torch.Tensor, indices: torch.Tensor, sm_scale: float,
                out: Optional[torch.Tensor] = None, lse: Optional[torch.Tensor] = None, *,
                causal: bool = False, causal_offset: int = 0, num_splits: int = 0,
                workspace: Optional[torch.Tensor] = None,
                stream=None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Sparse MLA prefill: per-query top-k over one KV pool; returns (out bf16, lse fp32).
    num_splits: split-K over each query's list (0 = automatic, more than one only for few
    queries)."""
    _need(q, torch.bfloat16, "q")
    _need(indices, torch.int32, "indices")
    N, H, _ = q.shape
    if out is None:
        out = torch.empty((N, H, abi.D_VO), dtype=torch.bfloat16, device=q.device)
    if lse is None:
        lse = torch.empty((N, H), dtype=torch.float32, device=q.device)
    a = make_prefill_args(q, kv, indices, sm_scale, out, lse, causal=causal,
                          causal_offset=causal_offset, num_splits=num_splits)
    nbytes = prefill_workspace_size(a)
    if nbytes and (workspace is None or workspace.numel() * workspace.element_size() < nbytes):
        workspace = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
    check(load_library().dsa_mla_prefill(ctypes.byref(a), _ptr(workspace) if nbytes else None,
                                         nbytes, _stream(stream)), "dsa_mla_prefill")
    return out, lse


def mla_prefill_v4(q: torch.Tensor, unified_kv: torch.Tensor, kv: torch.Tensor,
                   attn_sink: Optional[torch.Tensor], kv_indptr_prefix: torch.Tensor,
                   kv_indices_prefix: torch.Tensor, kv_indptr_extend: torch.Tensor,
                   kv_indices_extend: torch.Tensor, softmax_scale: float,
                   out: Optional[torch.Tensor] = None, lse: Optional[torch.Tensor] = None, *,
                   max_rows: Optional[int] = None, num_splits: int = 0,
                   workspace: Optional[torch.Tensor] = None,
                   stream=None) -> Tuple[torch.Tensor, torch.Tensor]:
    """DeepSeek-V4 sparse prefill (opus_mla_v4_prefill_kargs form): q [N, H, 512] bf16, prefix
    rows from unified_kv [total_pages, 512], extend rows from kv [total_tokens, 512], per-head
    attn_sink fp32 [H] in the softmax denominator (or None); returns (out [N, H, 512], lse [N, H]).
    num_splits: split-K over each query's list (0 = automatic, more than one only for few
    queries); the split partials live in `workspace` (allocated here when missing)."""
    _need(q, torch.bfloat16, "q")
    for t, n in ((unified_kv, "unified_kv"), (kv, "kv")):
        _need(t, torch.bfloat16, n)
        if t.shape[-1] != abi.D_V4 or t.stride(-1) != 1:
            raise ValueError(f"{n} must be [rows, 512] bf16 with a dense last dim")
    for t, n in ((kv_indptr_prefix, "kv_indptr_prefix"), (kv_indices_prefix, "kv_indices_prefix"),
                 (kv_indptr_extend, "kv_indptr_extend"), (kv_indices_extend, "kv_indices_extend")):
        _need(t, torch.int32, n)
    if attn_sink is not None:
        _need(attn_sink, torch.float32, "attn_sink")
    N, H, D = q.shape
    if D != abi.D_V4 or q.stride(2) != 1:
        raise ValueError("q must be [N, H, 512] with a dense last dim")
    if out is None:
        out = torch.empty_like(q)
    if out.stride() != q.stride():
        raise ValueError("out must have q's strides (the reference shares stride_qo_n / stride_qo_h)")
    if lse is None:
        lse = torch.empty((N, H), dtype=torch.float32, device=q.device)
    if max_rows is None:
        max_rows = int(((kv_indptr_prefix[1:] - kv_indptr_prefix[:-1]) +
                        (kv_indptr_extend[1:] - kv_indptr_extend[:-1])).max()) if N else 0
    a = abi.PrefillV4Args()
    a.q, a.unified_kv, a.kv, a.attn_sink = _ptr(q), _ptr(unified_kv), _ptr(kv), _ptr(attn_sink)
    a.out, a.lse = _ptr(out), _ptr(lse)
    a.kv_indptr_prefix, a.kv_indices_prefix = _ptr(kv_indptr_prefix), _ptr(kv_indices_prefix)
    a.kv_indptr_extend, a.kv_indices_extend = _ptr(kv_indptr_extend), _ptr(kv_indices_extend)
    a.N, a.H, a.D = N, H, D
    a.total_pages, a.total_tokens = unified_kv.shape[0], kv.shape[0]
    a.stride_qo_n, a.stride_qo_h = q.stride(0), q.stride(1)
    a.stride_kv_page = unified_kv.stride(0)
    if kv.stride(0) != unified_kv.stride(0):
        raise ValueError("unified_kv and kv must share the row stride (stride_kv_page)")
    a.max_rows = int(max_rows)
    a.softmax_scale = float(softmax_scale)
    a.num_splits = int(num_splits)
    lib = load_library()
    _run_with_workspace(lib.dsa_mla_prefill_v4_workspace_size, lib.dsa_mla_prefill_v4, a, workspace,
                        q.device, stream, "dsa_mla_prefill_v4")
    return out, lse


def quantize_kv_fp8(src: torch.Tensor, dst: Optional[torch.Tensor] = None,
                    dst_rows: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """Write bf16 latent rows [n, 576] into 656-byte fp8 cache rows (uint8 [rows, 656])."""
    _need(src, torch.bfloat16, "src")
    if src.shape[-1] != abi.D_QK or src.stride(-1) != 1:
        raise ValueError("src must be [n, 576] bf16 with a dense last dim")
    src2 = src.reshape(-1, abi.D_QK)
    n = src2.shape[0]
    if dst is None:
        dst = torch.empty((n, abi.FP8_ROW_BYTES), dtype=torch.uint8, device=src.device)
    _need(dst, torch.uint8, "dst")
    if dst_rows is not None:
        _need(dst_rows, torch.int64, "dst_rows")
    check(load_library().dsa_kv_quantize_fp8(_ptr(src2), src2.stride(0), n, _ptr(dst),
                                             dst.numel() // abi.FP8_ROW_BYTES, _ptr(dst_rows),
                                             _stream(stream)), "dsa_kv_quantize_fp8")
    return dst


def topk_indices(scores: torch.Tensor, topk: int, lengths: Optional[torch.Tensor] = None,
                 out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """Per query token, the `topk` positions of its fp32 index-score row [T, n] with the
    highest scores, ascending, -1 padded: int32 [T, topk], the `indices` rows mla_decode takes
    (one token per row; reshape to [B, s_q, topk]).  lengths (int32 [T]) limits row t to its
    first lengths[t] positions.  NaN ranks above +inf, -0 equals +0, and ties at the threshold
    go to the lower positions (dsa_topk_indices in include/dsa_topk.h)."""
    _need(scores, torch.float32, "scores")
    if scores.dim() != 2 or scores.stride(1) != 1:
        raise ValueError("scores must be [T, n] fp32 with a dense last dim")
    T, n = scores.shape
    stride = scores.stride(0) if T > 1 else ((n + 3) // 4) * 4
    # rows are read in 16-byte pieces up to n rounded up to 4: that much must lie in storage
    need = (T - 1) * stride + ((n + 3) // 4) * 4 if T else 0
    have = scores.untyped_storage().nbytes() // 4 - scores.storage_offset()
    if T and (stride % 4 or need > have):
        raise ValueError("scores rows must have a stride that is a multiple of 4 and be readable "
                         "up to n rounded up to a multiple of 4")
    if lengths is not None:
        _need(lengths, torch.int32, "lengths")
        if lengths.numel() != T or not lengths.is_contiguous():
            raise ValueError("lengths must be a contiguous int32 [T]")
    if out is None:
        out = torch.empty((T, topk), dtype=torch.int32, device=scores.device)
    _need(out, torch.int32, "out")
    if out.dim() != 2 or out.shape[0] != T or out.shape[1] < topk or out.stride(1) != 1:
        raise ValueError("out must be int32 [T, >= topk] with a dense last dim")
    check(load_library().dsa_topk_indices(_ptr(scores), stride, _ptr(lengths), T, n, int(topk),
                                          _ptr(out), out.stride(0), _stream(stream)), "dsa_topk_indices")
    return out


def mla_prefill_v4_fp8(q_nope: torch.Tensor, q_rope: torch.Tensor, unified_kv_nope: torch.Tensor,
                       unified_kv_rope: torch.Tensor, kv_nope: torch.Tensor, kv_rope: torch.Tensor,
                       attn_sink: Optional[torch.Tensor], kv_indptr_prefix: torch.Tensor,
                       kv_indices_prefix: torch.Tensor, kv_indptr_extend: torch.Tensor,
                       kv_indices_extend: torch.Tensor, softmax_scale: float,
                       out: Optional[torch.Tensor] = None, lse: Optional[torch.Tensor] = None, *,
                       max_rows: Optional[int] = None, num_splits: int = 0,
                       workspace: Optional[torch.Tensor] = None,
                       stream=None) -> Tuple[torch.Tensor, torch.Tensor]:
    """DeepSeek-V4 sparse prefill on fp8 rows (opus_mla_v4_prefill_fp8_kargs form): every row and
    Q head is a 512-byte NoPE stream row (448 e4m3 codes, 14 E8M0 scales, pad; uint8) plus 64 bf16
    RoPE values; q_* [N, H, 512 | 64], pools [rows, 512 | 64].  Returns (out bf16 [N, H, 512],
    lse fp32 [N, H])."""
    for t, n in ((q_nope, "q_nope"), (unified_kv_nope, "unified_kv_nope"), (kv_nope, "kv_nope")):
        _need(t, torch.uint8, n)
        if t.shape[-1] != 512 or t.stride(-1) != 1:
            raise ValueError(f"{n} must have 512-byte rows with a dense last dim")
    for t, n in ((q_rope, "q_rope"), (unified_kv_rope, "unified_kv_rope"), (kv_rope, "kv_rope")):
        _need(t, torch.bfloat16, n)
        if t.shape[-1] != 64 or t.stride(-1) != 1:
            raise ValueError(f"{n} must have 64 bf16 values per row with a dense last dim")
    for t, n in ((kv_indptr_prefix, "kv_indptr_prefix"), (kv_indices_prefix, "kv_indices_prefix"),
                 (kv_indptr_extend, "kv_indptr_extend"), (kv_indices_extend, "kv_indices_extend")):
        _need(t, torch.int32, n)
    if attn_sink is not None:
        _need(attn_sink, torch.float32, "attn_sink")
    N, H, _ = q_nope.shape
    if tuple(q_rope.shape[:2]) != (N, H):
        raise ValueError("q_nope and q_rope must cover the same [N, H]")
    if unified_kv_nope.shape[0] != unified_kv_rope.shape[0] or kv_nope.shape[0] != kv_rope.shape[0]:
        raise ValueError("each pool's nope and rope streams must have the same row count")
    if unified_kv_nope.stride(0) != kv_nope.stride(0) or unified_kv_rope.stride(0) != kv_rope.stride(0):
        raise ValueError("both pools must share the row strides (stride_kv_nope_page / _rope_page)")
    if out is None:
        out = torch.empty((N, H, abi.D_V4), dtype=torch.bfloat16, device=q_nope.device)
    if lse is None:
        lse = torch.empty((N, H), dtype=torch.float32, device=q_nope.device)
    if max_rows is None:
        max_rows = int(((kv_indptr_prefix[1:] - kv_indptr_prefix[:-1]) +
                        (kv_indptr_extend[1:] - kv_indptr_extend[:-1])).max()) if N else 0
    a = abi.PrefillV4Fp8Args()
    a.q_nope, a.q_rope = _ptr(q_nope), _ptr(q_rope)
    a.unified_kv_nope, a.unified_kv_rope = _ptr(unified_kv_nope), _ptr(unified_kv_rope)
    a.kv_nope, a.kv_rope = _ptr(kv_nope), _ptr(kv_rope)
    a.attn_sink, a.out, a.lse = _ptr(attn_sink), _ptr(out), _ptr(lse)
    a.kv_indptr_prefix, a.kv_indices_prefix = _ptr(kv_indptr_prefix), _ptr(kv_indices_prefix)
    a.kv_indptr_extend, a.kv_indices_extend = _ptr(kv_indptr_extend), _ptr(kv_indices_extend)
    a.N, a.H = N, H
    a.total_pages, a.total_tokens = unified_kv_nope.shape[0], kv_nope.shape[0]
    a.stride_q_nope_n, a.stride_q_nope_h = q_nope.stride(0), q_nope.stride(1)
    a.stride_q_rope_n, a.stride_q_rope_h = q_rope.stride(0), q_rope.stride(1)
    a.stride_o_n, a.stride_o_h = out.stride(0), out.stride(1)
    a.stride_kv_nope_page, a.stride_kv_rope_page = unified_kv_nope.stride(0), unified_kv_rope.stride(0)
    a.max_rows = int(max_rows)
    a.softmax_scale = float(softmax_scale)
    a.num_splits = int(num_splits)
    lib = load_library()
    _run_with_workspace(lib.dsa_mla_prefill_v4_fp8_workspace_size, lib.dsa_mla_prefill_v4_fp8, a, workspace,
                        q_nope.device, stream, "dsa_mla_prefill_v4_fp8")
    return out, lse


def indexer_scores(q: torch.Tensor, weights: torch.Tensor, k_cache: torch.Tensor, seq_lens: torch.Tensor,
                   *, block_table: Optional[torch.Tensor] = None, block_size: Optional[int] = None,
                   causal: bool = False, n_cols: Optional[int] = None, k_batch_stride: int = 0,
                   scores: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """DSA index scores (dsa_indexer_scores): q bf16 [B, s_q, H_I, 128], weights fp32
    [B, s_q, H_I], k_cache bf16 [rows, 128] (or [blocks, block_size, 128]), seq_lens int32 [B].
    Returns fp32 [B, s_q, n_cols]: score[b, t, j] = sum_h w * relu(q . k_j) for j < len(b, t)
    (-inf where k_j's row lies outside the cache); other entries are left as allocated (NaN
    here)."""
    _need(q, torch.bfloat16, "q")
    _need(weights, torch.float32, "weights")
    _need(k_cache, torch.bfloat16, "k_cache")
    _need(seq_lens, torch.int32, "seq_lens")
    B, s_q, H_I, D = q.shape
    if D != 128 or q.stride(3) != 1:
        raise ValueError("q must be [B, s_q, H_I, 128] with a dense last dim")
    if not weights.is_contiguous() or tuple(weights.shape) != (B, s_q, H_I):
        raise ValueError("weights must be dense [B, s_q, H_I]")
    kc = k_cache.reshape(-1, 128) if k_cache.is_contiguous() else k_cache
    if kc.dim() != 2 or kc.shape[1] != 128 or kc.stride(1) != 1:
        raise ValueError("k_cache must be [rows, 128] (or [blocks, block_size, 128]) with a dense last dim")
    if n_cols is None:
        n_cols = int(seq_lens.max().item()) if B else 0
    if scores is None:
        scores = torch.full((B, s_q, max(n_cols, 1)), float("nan"), dtype=torch.float32, device=q.device)
    a = abi.IndexerArgs()
    a.q = _ptr(q)
    a.q_stride_b, a.q_stride_t, a.q_stride_h = q.stride(0), q.stride(1), q.stride(2)
    a.weights = _ptr(weights)
    a.k_cache = _ptr(kc)
    a.k_total_rows = kc.shape[0]
    a.k_stride_row = kc.stride(0)
    if block_table is not None:
        _need(block_table, torch.int32, "block_table")
        if block_size is None:
            block_size = k_cache.shape[-2] if k_cache.dim() >= 3 else None
        if block_size is None:
            raise ValueError("block_size is required with a block table")
        a.block_table = _ptr(block_table)
        a.block_table_stride = block_table.stride(0)
        a.block_size = int(block_size)
    a.k_batch_stride = int(k_batch_stride)
    a.seq_lens = _ptr(seq_lens)
    a.scores = _ptr(scores)
    a.score_stride = scores.stride(1) if scores.dim() == 3 else scores.stride(0)
    a.B, a.s_q, a.H_I, a.n_cols, a.causal = B, s_q, H_I, n_cols, 1 if causal else 0
    check(load_library().dsa_indexer_scores(ctypes.byref(a), _stream(stream)), "dsa_indexer_scores")
    return scores
