"""ctypes mirror of include/dsa_mla.h and the loader of libdsa_mla.so.

The library is the product: every call in :mod:`opfoundry_amd.dsa` goes
through it.  There is no CPU fallback - if the shared object is missing the
loader raises, so a GPU run can never silently compute elsewhere.
"""
from __future__ import annotations

import ctypes
import os

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "_build", "libdsa_mla.so")

D_QK, D_NOPE, D_ROPE, D_VO = 576, 512, 64, 512
FP8_ROW_BYTES, BF16_ROW_BYTES = 656, 1152
MAX_SPLITS = 64
SPLITS_PLANNED = -1               # DSA_MLA_SPLITS_PLANNED: CSR plan already in the workspace
MAX_LIST = 2 ** 31 - 1 - 2048      # DSA_MLA_MAX_LIST: longest top-k / max_kv_len / max_rows

KV_BF16 = 0
KV_FP8_656 = 1
KV_BF16_D512 = 2
KV_MXFP8 = 3
KV_MXFP8_V4 = 4
V4_NOPE = 448
D_V4 = 512

DSA_OK = 0
ERRORS = {
    -1: "DSA_ERR_NULL_POINTER",
    -2: "DSA_ERR_BAD_SHAPE",
    -3: "DSA_ERR_UNSUPPORTED",
    -4: "DSA_ERR_BAD_FORMAT",
    -5: "DSA_ERR_WORKSPACE",
    -6: "DSA_ERR_BAD_SPLITS",
    -7: "DSA_ERR_BAD_STRIDE",
    -8: "DSA_ERR_HIP",
    -9: "DSA_ERR_SCRATCH_LIMIT",
}
NOALLOC_SCRATCH_BYTES = 16 << 20

# Every symbol include/*.h declares (dsa_mla.h, then dsa_topk.h), in declaration order.
EXPORTED_SYMBOLS = (
    "dsa_mla_decode_workspace_size",
    "dsa_mla_decode_num_splits",
    "dsa_mla_decode",
    "dsa_mla_decode_noalloc",
    "dsa_mla_decode_csr_workspace_size",
    "dsa_mla_decode_csr",
    "dsa_mla_csr_plan",
    "dsa_mla_decode_mxfp8_workspace_size",
    "dsa_mla_decode_mxfp8",
    "dsa_mla_combine",
    "dsa_mla_prefill_workspace_size",
    "dsa_mla_prefill",
    "dsa_mla_prefill_v4_workspace_size",
    "dsa_mla_prefill_v4",
    "dsa_mla_prefill_v4_fp8_workspace_size",
    "dsa_mla_prefill_v4_fp8",
    "dsa_kv_quantize_fp8",
    "dsa_topk_indices",
    "dsa_indexer_scores",
    "dsa_mla_strerror",
    "dsa_mla_abi_version",
)

ABI_VERSION = 8

_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_vp = ctypes.c_void_p


class DecodeArgs(ctypes.Structure):
    """dsa_mla_decode_args (include/dsa_mla.h)."""

    _fields_ = [
        ("q", _vp), ("q_stride_b", _i64), ("q_stride_t", _i64), ("q_stride_h", _i64),
        ("kv_cache", _vp), ("kv_total_rows", _i64), ("kv_format", _i32), ("block_size", _i32),
        ("kv_batch_stride", _i64), ("kv_stride_row", _i64),
        ("block_table", _vp), ("block_table_stride", _i64),
        ("seq_lens", _vp),
        ("indices", _vp), ("idx_stride_b", _i64), ("idx_stride_t", _i64),
        ("out", _vp), ("o_stride_b", _i64), ("o_stride_t", _i64), ("o_stride_h", _i64),
        ("lse", _vp),
        ("B", _i32), ("s_q", _i32), ("H", _i32), ("topk", _i32),
        ("num_splits", _i32), ("causal", _i32), ("sm_scale", ctypes.c_float),
    ]


class CsrArgs(ctypes.Structure):
    """dsa_mla_decode_csr_args (include/dsa_mla.h): the reference's opus_mla_decode_kargs fields."""

    _fields_ = [
        ("q", _vp), ("kv", _vp), ("out", _vp), ("lse", _vp),
        ("kv_indptr", _vp), ("kv_indices", _vp),
        ("B", _i32), ("s_q", _i32), ("H", _i32), ("total_tokens", _i32),
        ("stride_q_b", _i32), ("stride_q_h", _i32), ("stride_o_b", _i32), ("stride_o_h", _i32),
        ("stride_kv_page", _i32),
        ("kv_format", _i32), ("max_kv_len", _i32), ("num_splits", _i32),
        ("softmax_scale", ctypes.c_float),
    ]


class MxArgs(ctypes.Structure):
    """dsa_mla_decode_mxfp8_args (include/dsa_mla.h): the reference's opus_mla_decode_mxfp8_kargs fields."""

    _fields_ = [
        ("q_nope", _vp), ("q_scale", _vp), ("q_rope", _vp),
        ("kv_nope", _vp), ("kv_scale", _vp), ("kv_rope", _vp),
        ("out", _vp), ("lse", _vp),
        ("kv_indptr", _vp), ("kv_indices", _vp),
        ("B", _i32), ("s_q", _i32), ("H", _i32), ("total_tokens", _i32),
        ("stride_q_nope_b", _i32), ("stride_q_nope_h", _i32),
        ("stride_q_scale_b", _i32), ("stride_q_scale_h", _i32),
        ("stride_q_rope_b", _i32), ("stride_q_rope_h", _i32),
        ("stride_o_b", _i32), ("stride_o_h", _i32),
        ("stride_kv_nope_page", _i32), ("stride_kv_scale_page", _i32), ("stride_kv_rope_page", _i32),
        ("max_kv_len", _i32), ("num_splits", _i32),
        ("softmax_scale", ctypes.c_float),
    ]


class PrefillArgs(ctypes.Structure):
    """dsa_mla_prefill_args (include/dsa_mla.h)."""

    _fields_ = [
        ("q", _vp), ("q_stride_n", _i64), ("q_stride_h", _i64),
        ("kv", _vp), ("kv_rows", _i64), ("kv_stride_row", _i64), ("kv_format", _i32),
        ("indices", _vp), ("idx_stride_n", _i64),
        ("out", _vp), ("o_stride_n", _i64), ("o_stride_h", _i64),
        ("lse", _vp),
        ("N", _i32), ("H", _i32), ("topk", _i32), ("causal", _i32),
        ("causal_offset", _i64), ("sm_scale", ctypes.c_float), ("num_splits", _i32),
    ]


class PrefillV4Args(ctypes.Structure):
    """dsa_mla_prefill_v4_args (include/dsa_mla.h): the reference's opus_mla_v4_prefill_kargs."""

    _fields_ = [
        ("q", _vp), ("unified_kv", _vp), ("kv", _vp), ("attn_sink", _vp), ("out", _vp), ("lse", _vp),
        ("kv_indptr_prefix", _vp), ("kv_indices_prefix", _vp),
        ("kv_indptr_extend", _vp), ("kv_indices_extend", _vp),
        ("N", _i32), ("H", _i32), ("D", _i32), ("total_pages", _i32), ("total_tokens", _i32),
        ("stride_qo_n", _i32), ("stride_qo_h", _i32), ("stride_kv_page", _i32), ("max_rows", _i32),
        ("softmax_scale", ctypes.c_float), ("num_splits", _i32),
    ]


class PrefillV4Fp8Args(ctypes.Structure):
    """dsa_mla_prefill_v4_fp8_args (include/dsa_mla.h): the fields of opus_mla_v4_prefill_fp8_kargs."""

    _fields_ = [
        ("q_nope", _vp), ("q_rope", _vp),
        ("unified_kv_nope", _vp), ("unified_kv_rope", _vp),
        ("kv_nope", _vp), ("kv_rope", _vp),
        ("attn_sink", _vp), ("out", _vp), ("lse", _vp),
        ("kv_indptr_prefix", _vp), ("kv_indices_prefix", _vp),
        ("kv_indptr_extend", _vp), ("kv_indices_extend", _vp),
        ("N", _i32), ("H", _i32), ("total_pages", _i32), ("total_tokens", _i32),
        ("stride_q_nope_n", _i32), ("stride_q_nope_h", _i32),
        ("stride_q_rope_n", _i32), ("stride_q_rope_h", _i32),
        ("stride_o_n", _i32), ("stride_o_h", _i32),
        ("stride_kv_nope_page", _i32), ("stride_kv_rope_page", _i32),
        ("max_rows", _i32), ("softmax_scale", ctypes.c_float), ("num_splits", _i32),
    ]


class IndexerArgs(ctypes.Structure):
    """dsa_indexer_args (include/dsa_indexer.h)."""

    _fields_ = [
        ("q", _vp), ("q_stride_b", _i64), ("q_stride_t", _i64), ("q_stride_h", _i64),
        ("weights", _vp),
        ("k_cache", _vp), ("k_total_rows", _i64), ("k_stride_row", _i64),
        ("block_table", _vp), ("block_table_stride", _i64), ("block_size", _i32),
        ("k_batch_stride", _i64),
        ("seq_lens", _vp),
        ("scores", _vp), ("score_stride", _i64),
        ("B", _i32), ("s_q", _i32), ("H_I", _i32), ("n_cols", _i32), ("causal", _i32),
    ]


class DsaError(RuntimeError):
    def __init__(self, code: int, where: str):
        self.code = code
        super().__init__(f"{where} failed: {ERRORS.get(code, code)} ({_strerror(code)})")


_LIB = None


def bind_torch_hip_runtime() -> None:
    """Import torch (when installed) before a HIP library of this package is loaded.

    PyTorch-ROCm ships its own libamdhip64 with the soname libamdhip64.so.7, which is also
    the soname the library links against.  Loaded after torch, the library's dependency
    resolves to torch's copy: one HIP runtime in the process.  Loaded first, it pulls in
    /opt/rocm's runtime, torch later loads its own, and the library's launches on torch's
    memory and streams then fail (DSA_ERR_HIP).  A process without torch has one runtime
    either way."""
    try:
        import torch  # noqa: F401
    except ImportError:
        pass


def load_library(path: str | None = None) -> ctypes.CDLL:
    """Load libdsa_mla.so (built by opfoundry_amd.build); raise if it is absent."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = path or LIB_PATH
    if not os.path.exists(p):
        raise RuntimeError(
            f"libdsa_mla.so not found at {p}: build it with `python -m opfoundry_amd.build` "
            "(there is no CPU fallback)")
    bind_torch_hip_runtime()
    lib = ctypes.CDLL(p)
    sz = ctypes.POINTER(ctypes.c_size_t)
    lib.dsa_mla_decode_workspace_size.argtypes = [ctypes.POINTER(DecodeArgs), sz]
    lib.dsa_mla_decode_num_splits.argtypes = [ctypes.POINTER(DecodeArgs), ctypes.POINTER(_i32)]
    lib.dsa_mla_decode.argtypes = [ctypes.POINTER(DecodeArgs), _vp, ctypes.c_size_t, _vp]
    lib.dsa_mla_decode_noalloc.argtypes = [ctypes.POINTER(DecodeArgs), _vp]
    lib.dsa_mla_decode_csr_workspace_size.argtypes = [ctypes.POINTER(CsrArgs), sz]
    lib.dsa_mla_decode_csr.argtypes = [ctypes.POINTER(CsrArgs), _vp, ctypes.c_size_t, _vp]
    lib.dsa_mla_csr_plan.argtypes = [_vp, _i32, _i32, _i32, _i32, _vp, ctypes.c_size_t, _vp]
    lib.dsa_indexer_scores.argtypes = [ctypes.POINTER(IndexerArgs), _vp]
    lib.dsa_mla_decode_mxfp8_workspace_size.argtypes = [ctypes.POINTER(MxArgs), sz]
    lib.dsa_mla_decode_mxfp8.argtypes = [ctypes.POINTER(MxArgs), _vp, ctypes.c_size_t, _vp]
    lib.dsa_mla_combine.argtypes = [_vp, _vp, _i32, _i32, _i32, _vp, _i64, _i64, _vp, _vp]
    lib.dsa_mla_prefill_workspace_size.argtypes = [ctypes.POINTER(PrefillArgs), sz]
    lib.dsa_mla_prefill.argtypes = [ctypes.POINTER(PrefillArgs), _vp, ctypes.c_size_t, _vp]
    lib.dsa_mla_prefill_v4_workspace_size.argtypes = [ctypes.POINTER(PrefillV4Args), sz]
    lib.dsa_mla_prefill_v4.argtypes = [ctypes.POINTER(PrefillV4Args), _vp, ctypes.c_size_t, _vp]
    lib.dsa_mla_prefill_v4_fp8_workspace_size.argtypes = [ctypes.POINTER(PrefillV4Fp8Args), sz]
    lib.dsa_mla_prefill_v4_fp8.argtypes = [ctypes.POINTER(PrefillV4Fp8Args), _vp, ctypes.c_size_t, _vp]
    lib.dsa_kv_quantize_fp8.argtypes = [_vp, _i64, _i64, _vp, _i64, _vp, _vp]
    lib.dsa_topk_indices.argtypes = [_vp, _i64, _vp, _i32, _i32, _i32, _vp, _i64, _vp]
    lib.dsa_mla_strerror.argtypes = [ctypes.c_int]
    lib.dsa_mla_strerror.restype = ctypes.c_char_p
    lib.dsa_mla_abi_version.argtypes = []
    for name in EXPORTED_SYMBOLS:
        if name not in ("dsa_mla_strerror",):
            getattr(lib, name).restype = ctypes.c_int
    if lib.dsa_mla_abi_version() != ABI_VERSION:
        raise RuntimeError("libdsa_mla.so ABI version mismatch; rebuild it")
    if path is None:
        _LIB = lib
    return lib


def _strerror(code: int) -> str:
    try:
        return load_library().dsa_mla_strerror(code).decode()
    except Exception:  # the library itself may be what is missing
        return ERRORS.get(code, "unknown")


def check(code: int, where: str) -> None:
    if code != DSA_OK:
        raise DsaError(code, where)
