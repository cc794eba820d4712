"""ctypes binding of ``libvoiceagent_attn.so`` (the C ABI in include/voiceagent_attn.h).

This module only marshals arguments: tensors become device pointers and
element strides, the HIP stream is torch's current stream, and a non-zero
status becomes :class:`NativeError` carrying ``va_last_error()``.  There is no
fallback: if the library is missing, :func:`lib` raises.
"""

from __future__ import annotations

import ctypes
from ctypes import c_float, c_int32, c_int64, c_size_t, c_uint32, c_void_p
from pathlib import Path

import torch

from voiceagent_amd.build import LIB_PATH

VA_OK = 0
VA_BF16, VA_F16, VA_F32 = 0, 1, 2
VA_I32, VA_I64 = 0, 1
VA_LENS_PER_SEQ, VA_LENS_CUMULATIVE = 0, 1
VA_KV_NATIVE, VA_KV_FP8_E4M3 = 0, 1
ABI_VERSION = 6  # VA_ATTN_ABI_VERSION of the header these structs mirror
DECODE_NOALLOC_SCRATCH_BYTES = 4 << 20  # VA_DECODE_NOALLOC_SCRATCH_BYTES
VA_SPLIT_EXACT = -1  # split_tokens: automatic split, max_seq_len exact

DTYPE_CODES = {torch.bfloat16: VA_BF16, torch.float16: VA_F16, torch.float32: VA_F32}
INDEX_CODES = {torch.int32: VA_I32, torch.int64: VA_I64}


class NativeError(RuntimeError):
    """A C-ABI entry point returned a non-zero status."""

    def __init__(self, name: str, status: int, message: str):
        super().__init__(f"{name} failed with status {status}: {message}")
        self.status = status


class KvPool(ctypes.Structure):
    _fields_ = [
        ("k", c_void_p),
        ("v", c_void_p),
        ("stride_block", c_int64),
        ("stride_slot", c_int64),
        ("stride_head", c_int64),
        ("block_size", c_int32),
        ("num_blocks", c_int32),
        ("kv_format", c_int32),
        ("k_scale", c_float),
        ("v_scale", c_float),
    ]


class StoreArgs(ctypes.Structure):
    _fields_ = [
        ("struct_size", c_uint32),
        ("dtype", c_int32),
        ("key", c_void_p),
        ("value", c_void_p),
        ("key_stride_tok", c_int64),
        ("key_stride_head", c_int64),
        ("value_stride_tok", c_int64),
        ("value_stride_head", c_int64),
        ("pool", KvPool),
        ("slot_mapping", c_void_p),
        ("slot_dtype", c_int32),
        ("num_tokens", c_int32),
        ("num_kv_heads", c_int32),
        ("head_dim", c_int32),
    ]


class QkPrologue(ctypes.Structure):
    _fields_ = [
        ("q_norm_weight", c_void_p),
        ("k_norm_weight", c_void_p),
        ("weight_dtype", c_int32),
        ("eps", c_float),
        ("cos_sin_cache", c_void_p),
        ("cos_sin_stride", c_int64),
        ("max_position", c_int32),
        ("positions_dtype", c_int32),
        ("positions", c_void_p),
    ]


class QkNormRopeArgs(ctypes.Structure):
    _fields_ = [
        ("struct_size", c_uint32),
        ("dtype", c_int32),
        ("q", c_void_p),
        ("q_stride_tok", c_int64),
        ("q_stride_head", c_int64),
        ("k", c_void_p),
        ("k_stride_tok", c_int64),
        ("k_stride_head", c_int64),
        ("q_out", c_void_p),
        ("q_out_stride_tok", c_int64),
        ("q_out_stride_head", c_int64),
        ("k_out", c_void_p),
        ("k_out_stride_tok", c_int64),
        ("k_out_stride_head", c_int64),
        ("num_tokens", c_int32),
        ("num_heads", c_int32),
        ("num_kv_heads", c_int32),
        ("head_dim", c_int32),
        ("prologue", QkPrologue),
    ]


class DecodeArgs(ctypes.Structure):
    _fields_ = [
        ("struct_size", c_uint32),
        ("dtype", c_int32),
        ("q", c_void_p),
        ("q_stride_seq", c_int64),
        ("q_stride_head", c_int64),
        ("out", c_void_p),
        ("out_stride_seq", c_int64),
        ("out_stride_head", c_int64),
        ("pool", KvPool),
        ("block_tables", c_void_p),
        ("table_dtype", c_int32),
        ("table_stride_seq", c_int64),
        ("table_width", c_int32),
        ("lens", c_void_p),
        ("lens_dtype", c_int32),
        ("lens_kind", c_int32),
        ("valid_mask", c_void_p),
        ("valid_stride_seq", c_int64),
        ("valid_len", c_int32),
        ("new_k", c_void_p),
        ("new_k_stride_seq", c_int64),
        ("new_k_stride_head", c_int64),
        ("new_v", c_void_p),
        ("new_v_stride_seq", c_int64),
        ("new_v_stride_head", c_int64),
        ("new_slots", c_void_p),
        ("new_slots_dtype", c_int32),
        ("num_seqs", c_int32),
        ("num_heads", c_int32),
        ("num_kv_heads", c_int32),
        ("head_dim", c_int32),
        ("max_seq_len", c_int32),
        ("split_tokens", c_int32),
        ("scale", c_float),
        ("workspace", c_void_p),
        ("workspace_bytes", c_size_t),
        ("prologue", ctypes.POINTER(QkPrologue)),
        ("key_limit", c_int32),
        ("table_read_width", c_int32),
    ]


class VarlenArgs(ctypes.Structure):
    _fields_ = [
        ("struct_size", c_uint32),
        ("dtype", c_int32),
        ("q", c_void_p),
        ("q_stride_tok", c_int64),
        ("q_stride_head", c_int64),
        ("k", c_void_p),
        ("k_stride_tok", c_int64),
        ("k_stride_head", c_int64),
        ("v", c_void_p),
        ("v_stride_tok", c_int64),
        ("v_stride_head", c_int64),
        ("out", c_void_p),
        ("out_stride_tok", c_int64),
        ("out_stride_head", c_int64),
        ("cu_seqlens_q", c_void_p),
        ("cu_seqlens_k", c_void_p),
        ("num_seqs", c_int32),
        ("total_q", c_int32),
        ("num_heads", c_int32),
        ("num_kv_heads", c_int32),
        ("head_dim", c_int32),
        ("max_seqlen_q", c_int32),
        ("max_seqlen_k", c_int32),
        ("causal", c_int32),
        ("scale", c_float),
        ("pool", KvPool),
        ("block_tables", c_void_p),
        ("table_dtype", c_int32),
        ("table_stride_seq", c_int64),
        ("table_width", c_int32),
        ("slot_mapping", c_void_p),
        ("slot_dtype", c_int32),
        ("workspace", c_void_p),
        ("workspace_bytes", c_size_t),
        ("prologue", ctypes.POINTER(QkPrologue)),
    ]


# Every function include/voiceagent_attn.h declares, with its ctypes signature.
SIGNATURES = {
    "va_store_kvcache": (c_int32, [ctypes.POINTER(StoreArgs), c_void_p]),
    "va_paged_decode_workspace_bytes": (c_size_t, [ctypes.POINTER(DecodeArgs)]),
    "va_paged_decode": (c_int32, [ctypes.POINTER(DecodeArgs), c_void_p]),
    "va_paged_decode_noalloc": (c_int32, [ctypes.POINTER(DecodeArgs), c_void_p]),
    "va_varlen_attention": (c_int32, [ctypes.POINTER(VarlenArgs), c_void_p]),
    "va_varlen_workspace_bytes": (c_size_t, [ctypes.POINTER(VarlenArgs)]),
    "va_qk_norm_rope": (c_int32, [ctypes.POINTER(QkNormRopeArgs), c_void_p]),
    "va_last_error": (ctypes.c_char_p, []),
    "va_abi_version": (c_int32, []),
}

_LIB: ctypes.CDLL | None = None


def library_path() -> Path:
    return LIB_PATH


def lib() -> ctypes.CDLL:
    """Load the native library (once).  Raises if it has not been built."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build the HIP kernels first "
                "(python -c 'import __graft_entry__ as g; g.build()')"
            )
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        if handle.va_abi_version() != ABI_VERSION:
            raise RuntimeError(f"libvoiceagent_attn ABI version {handle.va_abi_version()} != "
                               f"{ABI_VERSION} (rebuild the library)")
        _LIB = handle
    return _LIB


def last_error() -> str:
    msg = lib().va_last_error()
    return msg.decode() if msg else ""


def check(name: str, status: int) -> None:
    if status != VA_OK:
        raise NativeError(name, status, last_error())


def new_args(cls):
    args = cls()
    args.struct_size = ctypes.sizeof(cls)
    return args


def current_stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def call(name: str, args, device: torch.device) -> None:
    """Launch `name` on the current stream of `device`, with `device` made the
    current HIP device for the call (the library plans launches for, and
    launches on, the current device)."""
    fn = getattr(lib(), name)
    with torch.cuda.device(device):
        check(name, fn(ctypes.byref(args), current_stream(device)))
