"""ctypes binding of libfa4cp.so, the gfx950 HIP library behind fa4_ring (include/fa4cp.h).

The library is built in-tree next to this file.  There is no fallback: if it is missing
or fails to load, every device entry point raises RuntimeError, as the reference does
when FlashAttention-4 is not importable (fa4_ring/fa4_backend.py:83-87).
"""

from __future__ import annotations

import ctypes
import os
from typing import Optional

import torch

LIB_NAME = "libfa4cp.so"
# FA4CP_LIB selects another build of the library (the in-tree one by default)
LIB_PATH = os.environ.get("FA4CP_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)
ABI_VERSION = 8

# element types (FA4CP_*)
BF16, FP16, E4M3, FP32 = 0, 1, 2, 3
# per-sequence row selections (FA4CP_SEL_*)
SEL_ALL, SEL_FRONT_HALF, SEL_BACK_HALF = 0, 1, 2

_DTYPE_CODE = {
    torch.bfloat16: BF16,
    torch.float16: FP16,
    torch.float8_e4m3fn: E4M3,
    torch.float32: FP32,
}


class AttnArgs(ctypes.Structure):
    """Mirror of fa4cp_attn_args."""

    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("lse", ctypes.c_void_p),
        ("q_row_stride", ctypes.c_int64),
        ("q_head_stride", ctypes.c_int64),
        ("k_row_stride", ctypes.c_int64),
        ("k_head_stride", ctypes.c_int64),
        ("v_row_stride", ctypes.c_int64),
        ("v_head_stride", ctypes.c_int64),
        ("o_row_stride", ctypes.c_int64),
        ("o_head_stride", ctypes.c_int64),
        ("lse_row_stride", ctypes.c_int64),
        ("cu_q", ctypes.c_void_p),
        ("cu_k", ctypes.c_void_p),
        ("nseq", ctypes.c_int32),
        ("max_seqlen_q", ctypes.c_int32),
        ("max_seqlen_k", ctypes.c_int32),
        ("total_q", ctypes.c_int32),
        ("total_k", ctypes.c_int32),
        ("h_q", ctypes.c_int32),
        ("h_kv", ctypes.c_int32),
        ("d", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("causal", ctypes.c_int32),
        ("q_sel", ctypes.c_int32),
        ("k_sel", ctypes.c_int32),
        ("softmax_scale", ctypes.c_float),
        ("q_descale", ctypes.c_void_p),
        ("k_descale", ctypes.c_void_p),
        ("v_descale", ctypes.c_void_p),
        ("v_t", ctypes.c_void_p),
        ("vt_d_stride", ctypes.c_int64),
    ]


class TransposeArgs(ctypes.Structure):
    """Mirror of fa4cp_transpose_args."""

    _fields_ = [
        ("v", ctypes.c_void_p),
        ("v_row_stride", ctypes.c_int64),
        ("v_head_stride", ctypes.c_int64),
        ("cu_k", ctypes.c_void_p),
        ("nseq", ctypes.c_int32),
        ("total_k", ctypes.c_int32),
        ("max_seqlen_k", ctypes.c_int32),
        ("k_sel", ctypes.c_int32),
        ("h_kv", ctypes.c_int32),
        ("d", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("v_t", ctypes.c_void_p),
        ("vt_d_stride", ctypes.c_int64),
    ]


class QuantArgs(ctypes.Structure):
    """Mirror of fa4cp_quant_args."""

    _fields_ = [
        ("x", ctypes.c_void_p),
        ("rows", ctypes.c_int64),
        ("h", ctypes.c_int32),
        ("d", ctypes.c_int32),
        ("row_stride", ctypes.c_int64),
        ("head_stride", ctypes.c_int64),
        ("dtype", ctypes.c_int32),
        ("heads_per_scale", ctypes.c_int32),
        ("amax", ctypes.c_void_p),
        ("descale", ctypes.c_void_p),
        ("y", ctypes.c_void_p),
    ]


MAX_CP = 16  # FA4CP_MAX_CP


class SweepArgs(ctypes.Structure):
    """Mirror of fa4cp_sweep_args."""

    _fields_ = [
        ("q", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("lse", ctypes.c_void_p),
        ("q_row_stride", ctypes.c_int64),
        ("q_head_stride", ctypes.c_int64),
        ("o_row_stride", ctypes.c_int64),
        ("o_head_stride", ctypes.c_int64),
        ("lse_row_stride", ctypes.c_int64),
        ("k", ctypes.c_void_p * MAX_CP),
        ("v_t", ctypes.c_void_p * MAX_CP),
        ("k_row_stride", ctypes.c_int64),
        ("k_head_stride", ctypes.c_int64),
        ("vt_d_stride", ctypes.c_int64),
        ("cu", ctypes.c_void_p),
        ("nseq", ctypes.c_int32),
        ("max_seqlen", ctypes.c_int32),
        ("total", ctypes.c_int32),
        ("h_q", ctypes.c_int32),
        ("h_kv", ctypes.c_int32),
        ("d", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("cp_rank", ctypes.c_int32),
        ("cp_size", ctypes.c_int32),
        ("softmax_scale", ctypes.c_float),
        ("q_descale", ctypes.c_void_p),
        ("k_descale", ctypes.c_void_p),
        ("v_descale", ctypes.c_void_p),
    ]


class SweepKPages(ctypes.Structure):
    """Mirror of fa4cp_sweep_kpages."""

    _fields_ = [
        ("page_table", ctypes.c_void_p * MAX_CP),
        ("pt_stride", ctypes.c_int64),
        ("page_size", ctypes.c_int32),
        ("num_pages", ctypes.c_int32),
    ]


class SweepBwdArgs(ctypes.Structure):
    """Mirror of fa4cp_sweep_bwd_args."""

    _fields_ = [
        ("q", ctypes.c_void_p),
        ("dout", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("lse", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_int64),
        ("dq", ctypes.c_void_p),
        ("q_row_stride", ctypes.c_int64),
        ("q_head_stride", ctypes.c_int64),
        ("do_row_stride", ctypes.c_int64),
        ("do_head_stride", ctypes.c_int64),
        ("o_row_stride", ctypes.c_int64),
        ("o_head_stride", ctypes.c_int64),
        ("lse_row_stride", ctypes.c_int64),
        ("k", ctypes.c_void_p * MAX_CP),
        ("v", ctypes.c_void_p * MAX_CP),
        ("dk", ctypes.c_void_p * MAX_CP),
        ("dv", ctypes.c_void_p * MAX_CP),
        ("k_row_stride", ctypes.c_int64),
        ("k_head_stride", ctypes.c_int64),
        ("v_row_stride", ctypes.c_int64),
        ("v_head_stride", ctypes.c_int64),
        ("cu", ctypes.c_void_p),
        ("nseq", ctypes.c_int32),
        ("max_seqlen", ctypes.c_int32),
        ("total", ctypes.c_int32),
        ("h_q", ctypes.c_int32),
        ("h_kv", ctypes.c_int32),
        ("d", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("cp_rank", ctypes.c_int32),
        ("cp_size", ctypes.c_int32),
        ("softmax_scale", ctypes.c_float),
        ("accumulate", ctypes.c_int32),
    ]


class PagedArgs(ctypes.Structure):
    """Mirror of fa4cp_paged_args."""
    _fields_ = [
        ("cu", ctypes.c_void_p),
        ("nseq", ctypes.c_int32),
        ("max_seqlen", ctypes.c_int32),
        ("total", ctypes.c_int32),
        ("h_kv", ctypes.c_int32),
        ("d", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("page_size", ctypes.c_int32),
        ("num_pages", ctypes.c_int32),
        ("cache_row_stride", ctypes.c_int64),
        ("cache_head_stride", ctypes.c_int64),
        ("pt_stride", ctypes.c_int64),
    ]


# exported symbol -> (restype, argtypes)
SIGNATURES = {
    "fa4cp_gather_kv_pages": (
        ctypes.c_int,
        [ctypes.POINTER(PagedArgs), ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_void_p),
         ctypes.POINTER(ctypes.c_void_p), ctypes.c_int64, ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p],
    ),
    "fa4cp_transpose_v_paged_many": (
        ctypes.c_int,
        [ctypes.POINTER(PagedArgs), ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_void_p),
         ctypes.POINTER(ctypes.c_void_p), ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p],
    ),
    "fa4cp_attn_fwd": (ctypes.c_int, [ctypes.POINTER(AttnArgs), ctypes.c_void_p]),
    "fa4cp_merge_state_inplace": (
        ctypes.c_int,
        [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
         ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p, ctypes.c_int32,
         ctypes.c_int32, ctypes.c_void_p],
    ),
    "fa4cp_merge_state": (
        ctypes.c_int,
        [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
         ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p, ctypes.c_int32,
         ctypes.c_int32, ctypes.c_void_p],
    ),
    "fa4cp_merge_states_list": (
        ctypes.c_int,
        [ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_void_p), ctypes.c_int32, ctypes.c_void_p,
         ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p],
    ),
    "fa4cp_merge_states": (
        ctypes.c_int,
        [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
         ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p],
    ),
    "fa4cp_zigzag_shard": (
        ctypes.c_int,
        [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int32,
         ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p],
    ),
    "fa4cp_zigzag_unshard": (
        ctypes.c_int,
        [ctypes.POINTER(ctypes.c_void_p), ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
         ctypes.c_int32, ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p],
    ),
    "fa4cp_transpose_v": (ctypes.c_int, [ctypes.POINTER(TransposeArgs), ctypes.c_void_p]),
    "fa4cp_vt_min_d_stride": (ctypes.c_int64, [ctypes.c_int32, ctypes.c_int32]),
    "fa4cp_transpose_v_many": (
        ctypes.c_int,
        [ctypes.POINTER(TransposeArgs), ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_void_p),
         ctypes.c_int32, ctypes.c_void_p],
    ),
    "fa4cp_ring_sweep_fwd": (ctypes.c_int, [ctypes.POINTER(SweepArgs), ctypes.c_void_p]),
    "fa4cp_ring_sweep_fwd_paged": (
        ctypes.c_int, [ctypes.POINTER(SweepArgs), ctypes.POINTER(SweepKPages), ctypes.c_void_p]),
    "fa4cp_ring_sweep_bwd": (ctypes.c_int, [ctypes.POINTER(SweepBwdArgs), ctypes.c_void_p]),
    "fa4cp_ring_sweep_bwd_workspace_bytes": (ctypes.c_int64, [ctypes.POINTER(SweepBwdArgs)]),
    "fa4cp_quantize_e4m3": (ctypes.c_int, [ctypes.POINTER(QuantArgs), ctypes.c_void_p]),
    "fa4cp_quantize_e4m3_noalloc": (ctypes.c_int, [ctypes.POINTER(QuantArgs), ctypes.c_void_p]),
    "fa4cp_last_error": (ctypes.c_char_p, []),
    "fa4cp_abi_version": (ctypes.c_int, []),
}

_lib: Optional[ctypes.CDLL] = None
_load_error: Optional[str] = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Loads the HIP library (once) and declares every entry point's signature."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        _load_error = (f"{path} is not built; run `python -c 'import __graft_entry__ as g; "
                       f"g.build()'` in the repository root")
        raise RuntimeError(f"fa4_ring HIP library unavailable: {_load_error}")
    try:
        lib = ctypes.CDLL(path)
    except OSError as e:  # pragma: no cover - depends on the runtime install
        _load_error = str(e)
        raise RuntimeError(f"fa4_ring HIP library failed to load: {e}") from e
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    ver = lib.fa4cp_abi_version()
    if ver != ABI_VERSION:
        raise RuntimeError(f"{path}: ABI version {ver}, expected {ABI_VERSION}; rebuild it")
    _lib = lib
    return lib


def available() -> bool:
    try:
        load()
        return True
    except RuntimeError:
        return False


def check(rc: int, what: str) -> None:
    """Raises RuntimeError with the library's message when an entry point failed."""
    if rc != 0:
        msg = _lib.fa4cp_last_error().decode() if _lib is not None else ""
        raise RuntimeError(f"{what} failed (status {rc}): {msg}")


def dtype_code(dt: torch.dtype) -> int:
    if dt not in _DTYPE_CODE:
        raise AssertionError(f"unsupported dtype {dt}")
    return _DTYPE_CODE[dt]


def stream_handle(device: torch.device) -> int:
    """hipStream_t of torch's current stream on `device` (kernels are queued there)."""
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()
