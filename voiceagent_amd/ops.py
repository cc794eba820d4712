"""Tensor-level entry points over the C ABI.

Each function validates shapes, dtypes, devices and strides on the host
(shape metadata only: no device synchronisation), fills the argument struct
and launches on torch's current stream.  The HIP library is the only compute
path: CPU tensors or a missing library raise.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

import torch

from voiceagent_amd import _native as N

# split_tokens for a max_seq_len that is the batch's exact longest context
# (an eager step's): the automatic split with fixed partitions at any length
# (va_paged_decode, VA_SPLIT_EXACT).
SPLIT_EXACT = N.VA_SPLIT_EXACT
LAYOUT_NHD = "nhd"  # [num_blocks, block_size, Hkv, D]  (engine, model_runner.py:116-131)
LAYOUT_HND = "hnd"  # [pages, Hkv, page_size, D]        (TTS, qwen_tts_outer_paged_cache.py:116-119)
# An FP8 KV pool holds OCP e4m3 codes (torch.float8_e4m3fn); an element's
# value is code * k_scale (keys) or code * v_scale (values).
FP8_KV_DTYPE = torch.float8_e4m3fn


class AttentionArgumentError(ValueError):
    """Host-side contract violation detected before launch."""


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise AttentionArgumentError(msg)


def _check_gpu(*tensors: torch.Tensor | None) -> torch.device:
    device = None
    for t in tensors:
        if t is None:
            continue
        _require(t.is_cuda, "attention kernels need GPU tensors (there is no CPU path)")
        if device is None:
            device = t.device
        _require(t.device == device, "all tensors must be on the same device")
    return device


def _dtype_code(t: torch.Tensor) -> int:
    _require(t.dtype in N.DTYPE_CODES, f"unsupported dtype {t.dtype}")
    return N.DTYPE_CODES[t.dtype]


def _index_code(t: torch.Tensor, what: str) -> int:
    _require(t.dtype in N.INDEX_CODES, f"{what} must be int32 or int64, got {t.dtype}")
    return N.INDEX_CODES[t.dtype]


def _rows(t: torch.Tensor, what: str) -> None:
    _require(t.stride(-1) == 1, f"{what}: the last dimension must be contiguous")


def _pool_matches(pool: torch.Tensor, dtype: torch.dtype) -> bool:
    """A pool of `dtype` itself, or an FP8 pool for 16-bit data."""
    return pool.dtype == dtype or (pool.dtype == FP8_KV_DTYPE and
                                   dtype in (torch.bfloat16, torch.float16))


def kv_pool(k_cache: torch.Tensor, v_cache: torch.Tensor, layout: str = LAYOUT_NHD,
            k_scale: float = 1.0, v_scale: float = 1.0) -> N.KvPool:
    """Describe a paged K/V pool pair (4-D, NHD or HND) for the C ABI; an
    FP8 (float8_e4m3fn) pool carries its k_scale / v_scale."""
    _require(k_cache.dim() == 4, "KV pool must be 4-D")
    _require(
        v_cache.shape == k_cache.shape and v_cache.stride() == k_cache.stride(),
        "key and value pools must have identical shapes and strides",
    )
    _require(v_cache.dtype == k_cache.dtype, "key and value pools must share a dtype")
    _rows(k_cache, "KV pool")
    pool = N.KvPool()
    pool.k = k_cache.data_ptr()
    pool.v = v_cache.data_ptr()
    if layout == LAYOUT_NHD:
        nb, bs, _, _ = k_cache.shape
        pool.stride_block, pool.stride_slot, pool.stride_head = (
            k_cache.stride(0),
            k_cache.stride(1),
            k_cache.stride(2),
        )
    elif layout == LAYOUT_HND:
        nb, _, bs, _ = k_cache.shape
        pool.stride_block, pool.stride_slot, pool.stride_head = (
            k_cache.stride(0),
            k_cache.stride(2),
            k_cache.stride(1),
        )
    else:
        raise AttentionArgumentError(f"unknown pool layout {layout!r}")
    pool.block_size = int(bs)
    pool.num_blocks = int(nb)
    if k_cache.dtype == FP8_KV_DTYPE:
        _require(k_scale > 0 and v_scale > 0, "FP8 pool scales must be positive")
        pool.kv_format = N.VA_KV_FP8_E4M3
        pool.k_scale = float(k_scale)
        pool.v_scale = float(v_scale)
    else:
        pool.kv_format = N.VA_KV_NATIVE
        pool.k_scale = pool.v_scale = 1.0
    return pool


def pool_heads(k_cache: torch.Tensor, layout: str) -> tuple[int, int]:
    """(num_kv_heads, head_dim) of a pool."""
    if layout == LAYOUT_NHD:
        return int(k_cache.shape[2]), int(k_cache.shape[3])
    return int(k_cache.shape[1]), int(k_cache.shape[3])


# --------------------------------------------------------------------- store
def store_kvcache(
    key: torch.Tensor,
    value: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    layout: str = LAYOUT_NHD,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
) -> None:
    """Write key[i] / value[i] ([N, Hkv, D]) to pool slot slot_mapping[i]; -1 skips.
    An FP8 pool receives e4m3 codes of key / k_scale and value / v_scale."""
    fast = _FAST if _FAST_LOADED else _fast_calls()
    if fast is not None and layout in (LAYOUT_NHD, LAYOUT_HND):
        index = key.get_device()
        if index >= 0 and index == torch.cuda.current_device():
            rc = fast.store_kvcache(key, value, k_cache, v_cache, slot_mapping,
                                    layout == LAYOUT_HND, float(k_scale), float(v_scale), index,
                                    _raw_stream(index))
            if rc == 0:
                return
            if _FAST_NOT_TAKEN < rc < 0:
                N.check("va_store_kvcache", rc)
    device = _check_gpu(key, value, k_cache, v_cache, slot_mapping)
    _require(key.dim() == 3 and value.shape == key.shape, "key/value must be [N, Hkv, D]")
    _rows(key, "key")
    _rows(value, "value")
    hkv, d = pool_heads(k_cache, layout)
    _require(key.shape[1] == hkv and key.shape[2] == d, "key/value heads must match the pool")
    _require(key.dtype == value.dtype and _pool_matches(k_cache, key.dtype),
             "key/value/pool dtypes must match (or the pool be FP8 for 16-bit rows)")
    _require(slot_mapping.dim() == 1 and slot_mapping.numel() == key.shape[0],
             "slot_mapping must have one entry per token")
    _require(slot_mapping.is_contiguous(), "slot_mapping must be contiguous")
    args = N.new_args(N.StoreArgs)
    args.dtype = _dtype_code(key)
    args.key = key.data_ptr()
    args.value = value.data_ptr()
    args.key_stride_tok, args.key_stride_head = key.stride(0), key.stride(1)
    args.value_stride_tok, args.value_stride_head = value.stride(0), value.stride(1)
    args.pool = kv_pool(k_cache, v_cache, layout, k_scale, v_scale)
    args.slot_mapping = slot_mapping.data_ptr()
    args.slot_dtype = _index_code(slot_mapping, "slot_mapping")
    args.num_tokens = int(key.shape[0])
    args.num_kv_heads = hkv
    args.head_dim = d
    N.call("va_store_kvcache", args, device)


# ---------------------------------------------------------- q/k prologue
@dataclass(frozen=True)
class QKPrologue:
    """Qwen3's per-head q/k prologue (qwen_asr_vllm/models/qwen3.py:42-48):
    RMSNorm with ``q_norm_weight`` / ``k_norm_weight`` and ``eps``
    (layers/layernorm.py:19-25), then the half-split rotary embedding read from
    the fp32 ``cos_sin_cache`` ([max_position, D] or the reference's
    [max_position, 1, D] buffer) at ``positions`` (layers/rotary_embedding.py:9-32)."""

    q_norm_weight: torch.Tensor
    k_norm_weight: torch.Tensor
    eps: float
    cos_sin_cache: torch.Tensor
    positions: torch.Tensor


def _prologue_struct(pro: QKPrologue, head_dim: int, n_positions: int) -> N.QkPrologue:
    for name, w in (("q_norm_weight", pro.q_norm_weight), ("k_norm_weight", pro.k_norm_weight)):
        _require(w.dim() == 1 and w.numel() == head_dim and w.is_contiguous(),
                 f"{name} must be a contiguous [head_dim] vector")
    _require(pro.q_norm_weight.dtype == pro.k_norm_weight.dtype,
             "q_norm_weight and k_norm_weight must share a dtype")
    cs = pro.cos_sin_cache
    if cs.dim() == 3:
        _require(cs.shape[1] == 1, "cos_sin_cache must be [max_position, (1,) head_dim]")
        cs = cs[:, 0]
    _require(cs.dim() == 2 and cs.shape[1] == head_dim and cs.dtype == torch.float32
             and cs.stride(-1) == 1,
             "cos_sin_cache must be an fp32 [max_position, head_dim] table (cos | sin)")
    pos = pro.positions
    _require(pos.dim() == 1 and pos.numel() >= n_positions and pos.is_contiguous(),
             f"positions must be a contiguous vector of at least {n_positions} entries")
    st = N.QkPrologue()
    st.q_norm_weight = pro.q_norm_weight.data_ptr()
    st.k_norm_weight = pro.k_norm_weight.data_ptr()
    st.weight_dtype = _dtype_code(pro.q_norm_weight)
    st.eps = float(pro.eps)
    st.cos_sin_cache = cs.data_ptr()
    st.cos_sin_stride = cs.stride(0)
    st.max_position = int(cs.shape[0])
    st.positions_dtype = _index_code(pos, "positions")
    st.positions = pos.data_ptr()
    return st


def qk_norm_rope(
    q: torch.Tensor | None,
    k: torch.Tensor,
    prologue: QKPrologue,
    *,
    q_out: torch.Tensor | None = None,
    k_out: torch.Tensor | None = None,
) -> tuple[torch.Tensor | None, torch.Tensor]:
    """Apply the Qwen3 q/k prologue to q [T, Hq, D] and k [T, Hkv, D] (one
    position per token).  Outputs are allocated contiguous when not given and
    may be q / k themselves (in place).  ``q`` None: the keys alone (a
    prefill whose varlen launch applies the query prologue itself); the
    first result is then None."""
    if q is None:
        return None, _k_norm_rope(k, prologue, k_out)
    fast = _FAST if _FAST_LOADED else _fast_calls()
    if fast is not None:
        index = q.get_device()
        if index >= 0 and index == torch.cuda.current_device():
            if q_out is None:
                q_out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
            if k_out is None:
                k_out = torch.empty(k.shape, dtype=k.dtype, device=k.device)
            rc = fast.qk_norm_rope(q, k, q_out, k_out, prologue.q_norm_weight,
                                   prologue.k_norm_weight, float(prologue.eps),
                                   prologue.cos_sin_cache, prologue.positions, index,
                                   _raw_stream(index))
            if rc == 0:
                return q_out, k_out
            if _FAST_NOT_TAKEN < rc < 0:
                N.check("va_qk_norm_rope", rc)
    device = _check_gpu(q, k, q_out, k_out, prologue.q_norm_weight, prologue.k_norm_weight,
                        prologue.cos_sin_cache, prologue.positions)
    _require(q.dim() == 3 and k.dim() == 3 and q.shape[0] == k.shape[0] and
             q.shape[2] == k.shape[2], "q must be [T, Hq, D] and k [T, Hkv, D]")
    _require(q.dtype == k.dtype, "q and k must share a dtype")
    _rows(q, "q")
    _rows(k, "k")
    T, hq, d = (int(x) for x in q.shape)
    hkv = int(k.shape[1])
    if q_out is None:
        q_out = torch.empty(q.shape, dtype=q.dtype, device=device)
    if k_out is None:
        k_out = torch.empty(k.shape, dtype=k.dtype, device=device)
    _require(q_out.shape == q.shape and q_out.dtype == q.dtype, "q_out must match q")
    _require(k_out.shape == k.shape and k_out.dtype == k.dtype, "k_out must match k")
    _rows(q_out, "q_out")
    _rows(k_out, "k_out")
    args = N.new_args(N.QkNormRopeArgs)
    args.dtype = _dtype_code(q)
    args.q, args.q_stride_tok, args.q_stride_head = q.data_ptr(), q.stride(0), q.stride(1)
    args.k, args.k_stride_tok, args.k_stride_head = k.data_ptr(), k.stride(0), k.stride(1)
    args.q_out = q_out.data_ptr()
    args.q_out_stride_tok, args.q_out_stride_head = q_out.stride(0), q_out.stride(1)
    args.k_out = k_out.data_ptr()
    args.k_out_stride_tok, args.k_out_stride_head = k_out.stride(0), k_out.stride(1)
    args.num_tokens, args.num_heads, args.num_kv_heads, args.head_dim = T, hq, hkv, d
    args.prologue = _prologue_struct(prologue, d, T)
    N.call("va_qk_norm_rope", args, device)
    return q_out, k_out


def _k_norm_rope(k: torch.Tensor, prologue: QKPrologue,
                 k_out: torch.Tensor | None) -> torch.Tensor:
    """The key side of qk_norm_rope alone (num_heads = 0 in the C ABI)."""
    device = _check_gpu(k, k_out, prologue.k_norm_weight, prologue.cos_sin_cache,
                        prologue.positions)
    _require(k.dim() == 3, "k must be [T, Hkv, D]")
    _rows(k, "k")
    T, hkv, d = (int(x) for x in k.shape)
    if k_out is None:
        k_out = torch.empty(k.shape, dtype=k.dtype, device=device)
    _require(k_out.shape == k.shape and k_out.dtype == k.dtype, "k_out must match k")
    _rows(k_out, "k_out")
    args = N.new_args(N.QkNormRopeArgs)
    args.dtype = _dtype_code(k)
    args.k, args.k_stride_tok, args.k_stride_head = k.data_ptr(), k.stride(0), k.stride(1)
    args.k_out = k_out.data_ptr()
    args.k_out_stride_tok, args.k_out_stride_head = k_out.stride(0), k_out.stride(1)
    args.num_tokens, args.num_heads, args.num_kv_heads, args.head_dim = T, 0, hkv, d
    args.prologue = _prologue_struct(prologue, d, T)
    N.call("va_qk_norm_rope", args, device)
    return k_out


# -------------------------------------------------------------------- decode
_WORKSPACES: dict[tuple[int, int], torch.Tensor] = {}
# Workspaces replaced by a larger one.  They are never freed: a HIP graph
# captured while one was current keeps its address, and memory returned to
# torch's allocator (a graph's private pool included) could be handed to
# another tensor that the graph's replays would then overwrite.
_RETIRED: list[torch.Tensor] = []
_CUS: dict[int, int] = {}  # compute units per device index


def _device_index(device: torch.device) -> int:
    return device.index if device.index is not None else torch.cuda.current_device()


def _raw_stream(index: int) -> int:
    """Handle of torch's current stream on device `index`."""
    return torch._C._cuda_getCurrentRawStream(index)


class _current:
    """Make device `index` current for the block (the library plans launches
    for, and launches on, the current device); a no-op when it already is."""

    __slots__ = ("index", "prev")

    def __init__(self, index: int):
        self.index = index
        self.prev = -1

    def __enter__(self):
        cur = torch._C._cuda_getDevice()
        if cur != self.index:
            self.prev = cur
            torch._C._cuda_setDevice(self.index)
        return self

    def __exit__(self, *exc):
        if self.prev >= 0:
            torch._C._cuda_setDevice(self.prev)
        return False


_DECODE_ARGS_SIZE = ctypes.sizeof(N.DecodeArgs)
_VARLEN_ARGS_SIZE = ctypes.sizeof(N.VarlenArgs)

# Host fast path (csrc/host/fast_calls.cpp, the ``_fast_calls`` module next
# to the library): the same checks and the same C-ABI call in C++, for the
# common paged_decode / varlen_attention / store_kvcache / qk_norm_rope calls.  It launches nothing for a
# call it does not take, and the Python path below then runs (and raises the
# error for a bad argument), so results and errors are the same either way.
_FAST_NOT_TAKEN = -1000
_FAST = None
_FAST_LOADED = False


def _fast_calls():
    """The fast-path module with the library's entry points handed to it, or
    None when it is not built or does not load."""
    global _FAST, _FAST_LOADED
    if not _FAST_LOADED:
        _FAST_LOADED = True
        from voiceagent_amd.build import FAST_MODULE, FAST_PATH

        if FAST_PATH.exists():
            import importlib.util

            try:
                spec = importlib.util.spec_from_file_location(FAST_MODULE, FAST_PATH)
                mod = importlib.util.module_from_spec(spec)
                spec.loader.exec_module(mod)
            except ImportError:
                return None
            lib = N.lib()

            def addr(fn):
                return ctypes.cast(fn, ctypes.c_void_p).value

            mod.set_entries(addr(lib.va_paged_decode), addr(lib.va_paged_decode_workspace_bytes),
                            addr(lib.va_varlen_attention), addr(lib.va_store_kvcache),
                            addr(lib.va_qk_norm_rope))
            _FAST = mod
    return _FAST
_POOLS: dict[tuple, N.KvPool] = {}  # pool descriptions by tensor identity and geometry


def _pool_struct(k_cache, v_cache, layout, k_scale, v_scale) -> N.KvPool:
    """kv_pool(...), cached: engine pools live for the whole run, and the
    description depends only on the key's fields."""
    key = (k_cache.data_ptr(), v_cache.data_ptr(), k_cache.shape, k_cache.stride(),
           v_cache.shape, v_cache.stride(), k_cache.dtype, v_cache.dtype, layout,
           float(k_scale), float(v_scale))
    pool = _POOLS.get(key)
    if pool is None:
        pool = kv_pool(k_cache, v_cache, layout, k_scale, v_scale)
        if len(_POOLS) >= 1024:
            _POOLS.clear()
        _POOLS[key] = pool
    return pool


def decode_workspace_bound(device: torch.device, num_heads: int, num_kv_heads: int,
                           head_dim: int) -> int:
    """Bytes that covers every automatic split (split_tokens = 0) of a decode
    with these heads on `device`, whatever the batch and lengths: the split
    gives at most one partition per compute unit over all (sequence, kv head)
    pairs, each holding (m, l) and head_dim floats per query head of the
    group, with the (m, l) block rounded to 256 bytes."""
    index = _device_index(device)
    cus = _CUS.get(index)
    if cus is None:
        cus = _CUS[index] = torch.cuda.get_device_properties(index).multi_processor_count
    group = max(1, num_heads // max(1, num_kv_heads))
    return (cus * group * 2 * 4 + 255) // 256 * 256 + cus * group * head_dim * 4


def decode_workspace(device: torch.device, nbytes: int, floor: int = 0,
                     stream: torch.cuda.Stream | None = None, kind: str = "decode"
                     ) -> torch.Tensor | None:
    """Partial-result workspace of the decode launches on `stream` (torch's
    current stream of `device` by default): no initialisation needed.  One
    per stream: launches on one stream are ordered, while decodes on two
    streams (an ASR engine and a TTS talker, say) may run at once and must not
    share their partials.  The first allocation takes at least `floor` bytes;
    a later, larger need allocates anew (doubling) and retires, without
    freeing, the old buffer."""
    if nbytes == 0:
        return None
    if stream is None:
        stream = torch.cuda.current_stream(device)
    key = (_device_index(device), stream.cuda_stream)
    if kind != "decode":
        key = key + (kind,)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        size = max(nbytes, floor if ws is None else 2 * ws.numel())
        if ws is not None:
            _RETIRED.append(ws)
        ws = torch.empty(size, dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


# Stream of the last no_alloc decode per device (their scratch buffer is
# shared by every stream of a GPU).
_NOALLOC_STREAM: dict[int, torch.cuda.Stream] = {}


def _order_noalloc(index: int) -> None:
    """Order a no_alloc decode after the previous one on its GPU when they
    run on different streams: the current stream waits (on the GPU) for the
    other.  Skipped under graph capture, where a wait on work outside the
    capture is not allowed."""
    cur = torch.cuda.current_stream(index)
    prev = _NOALLOC_STREAM.get(index)
    if (prev is not None and prev.cuda_stream != cur.cuda_stream
            and not torch.cuda.is_current_stream_capturing()):
        cur.wait_stream(prev)
    _NOALLOC_STREAM[index] = cur


def reserve_decode_workspace(device: torch.device, num_heads: int, num_kv_heads: int,
                             head_dim: int, stream: torch.cuda.Stream | None = None) -> None:
    """Allocate the decode workspace of `stream` (torch's current stream by
    default) up front, at the size every automatic split needs, e.g. before
    HIP graph capture.  ``torch.cuda.graph`` captures on a stream of its own
    unless it is given one: pass that stream here to reserve for it."""
    device = torch.device(device)
    bound = decode_workspace_bound(device, num_heads, num_kv_heads, head_dim)
    decode_workspace(device, bound, floor=bound, stream=stream)


def paged_decode(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    lens: torch.Tensor,
    *,
    max_seq_len: int,
    scale: float,
    lens_cumulative: bool = False,
    layout: str = LAYOUT_NHD,
    valid_mask: torch.Tensor | None = None,
    new_k: torch.Tensor | None = None,
    new_v: torch.Tensor | None = None,
    new_slots: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    split_tokens: int = 0,
    prologue: QKPrologue | None = None,
    key_limit: int = 0,
    table_read_width: int = 0,
    no_alloc: bool = False,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
) -> torch.Tensor:
    """One-token paged GQA attention.

    q: [B, Hq, D]; out: [B, Hq, D] (allocated if None); lens: per-sequence
    context lengths [B], or cu_seqlens_k [B + 1] with ``lens_cumulative``.
    ``new_k``/``new_v`` ([B, Hkv, D]) are written at position len-1 (or at
    ``new_slots[b]``) and used for that position in the same launch.  With a
    ``prologue``, q and new_k are raw projections, normalised and rotated at
    ``prologue.positions[b]`` inside the launch.  ``key_limit`` (> 0) leaves
    tokens at or past it unattended and ``table_read_width`` (> 0) makes the
    attention read block 0 for table columns at or past it (the TTS kernel's
    kernel_seq_len / kernel_page_count bounds); the current row is written at
    len - 1 either way.  ``no_alloc`` launches va_paged_decode_noalloc, which
    keeps the split partials in the library's own scratch buffer instead of a
    workspace; ``out`` must then be given, so that nothing is allocated.  That
    buffer is one per GPU, shared by every stream: no_alloc calls on two
    streams would race on it, so a no_alloc call issued on another stream than
    the previous one on its GPU first makes its stream wait for that stream
    (on the GPU, outside graph capture; under capture the caller must order
    them).
    An FP8 (float8_e4m3fn) pool is read as code * k_scale / v_scale, and the
    current row is stored into it quantised.  ``split_tokens``: 0 splits
    contexts automatically; ``SPLIT_EXACT`` does too, for a ``max_seq_len``
    that is the batch's exact longest context (partitions fixed from it); a
    positive value fixes the partition size.
    """
    fast = _FAST if _FAST_LOADED else _fast_calls()
    if fast is not None and not no_alloc and layout in (LAYOUT_NHD, LAYOUT_HND):
        index = q.get_device()
        if index >= 0 and index == torch.cuda.current_device():
            if out is None:
                out = torch.empty_like(q)
            stream = _raw_stream(index)
            pro = prologue
            rc = fast.paged_decode(
                q, k_cache, v_cache, block_tables, lens, out, new_k, new_v, new_slots,
                valid_mask, None if pro is None else pro.q_norm_weight,
                None if pro is None else pro.k_norm_weight,
                0.0 if pro is None else float(pro.eps),
                None if pro is None else pro.cos_sin_cache,
                None if pro is None else pro.positions, _WORKSPACES.get((index, stream)),
                lens_cumulative, layout == LAYOUT_HND,
                int(max_seq_len), float(scale), int(split_tokens), int(key_limit),
                int(table_read_width), float(k_scale), float(v_scale), index, stream)
            if rc == 0:
                return out
            if _FAST_NOT_TAKEN < rc < 0:
                N.check("va_paged_decode", rc)
            # Not taken, or a workspace is needed first: the path below.
    device = _check_gpu(q, k_cache, v_cache, block_tables, lens, valid_mask, new_k, new_v,
                        new_slots, out)
    if prologue is not None:
        _check_gpu(q, prologue.q_norm_weight, prologue.k_norm_weight, prologue.cos_sin_cache,
                   prologue.positions)
    _require(not no_alloc or out is not None, "no_alloc needs the output tensor (out=...)")
    _require(q.dim() == 3, "q must be [num_seqs, num_heads, head_dim]")
    qs = q.stride()
    _require(qs[2] == 1, "q: the last dimension must be contiguous")
    B, hq, d = q.shape
    hkv, pd = pool_heads(k_cache, layout)
    _require(pd == d, f"head_dim mismatch: q {d}, pool {pd}")
    _require(hq % hkv == 0, "num_heads must be a multiple of num_kv_heads")
    _require(_pool_matches(k_cache, q.dtype),
             "q and the KV pool must share a dtype (or the pool be FP8 for 16-bit q)")
    bts = block_tables.stride()
    _require(block_tables.dim() == 2 and block_tables.shape[0] >= B,
             "block_tables must be [num_seqs, width]")
    _require(bts[1] == 1, "block_tables rows must be contiguous")
    expect = B + 1 if lens_cumulative else B
    _require(lens.dim() == 1 and lens.numel() >= expect and lens.is_contiguous(),
             f"lens must be a contiguous vector of at least {expect} entries")
    if out is None:
        out = torch.empty_like(q)
    os_ = out.stride()
    _require(out.shape == q.shape and out.dtype == q.dtype, "out must match q")
    _require(os_[2] == 1, "out: the last dimension must be contiguous")
    _require(key_limit >= 0 and table_read_width >= 0,
             "key_limit and table_read_width must be non-negative")
    fields = dict(
        struct_size=_DECODE_ARGS_SIZE, dtype=_dtype_code(q), q=q.data_ptr(),
        q_stride_seq=qs[0], q_stride_head=qs[1], out=out.data_ptr(), out_stride_seq=os_[0],
        out_stride_head=os_[1], pool=_pool_struct(k_cache, v_cache, layout, k_scale, v_scale),
        block_tables=block_tables.data_ptr(),
        table_dtype=_index_code(block_tables, "block_tables"), table_stride_seq=bts[0],
        table_width=block_tables.shape[1], lens=lens.data_ptr(),
        lens_dtype=_index_code(lens, "lens"),
        lens_kind=N.VA_LENS_CUMULATIVE if lens_cumulative else N.VA_LENS_PER_SEQ,
        num_seqs=B, num_heads=hq, num_kv_heads=hkv, head_dim=d, max_seq_len=int(max_seq_len),
        split_tokens=int(split_tokens), scale=float(scale), key_limit=int(key_limit),
        table_read_width=int(table_read_width))
    if valid_mask is not None:
        _require(valid_mask.dim() == 2 and valid_mask.shape[0] >= B and
                 valid_mask.dtype == torch.bool and valid_mask.stride(-1) == 1,
                 "key_valid_mask must be a [num_seqs, max_seq] bool tensor")
        fields.update(valid_mask=valid_mask.data_ptr(), valid_stride_seq=valid_mask.stride(0),
                      valid_len=valid_mask.shape[1])
    _require((new_k is None) == (new_v is None), "new_k and new_v must be given together")
    if new_k is not None:
        nks, nvs = new_k.stride(), new_v.stride()
        _require(new_k.shape == (B, hkv, d) and new_v.shape == new_k.shape,
                 "new_k/new_v must be [num_seqs, num_kv_heads, head_dim]")
        _require(new_k.dtype == new_v.dtype == q.dtype, "new_k/new_v must match q's dtype")
        _require(nks[2] == 1 and nvs[2] == 1, "new_k/new_v: the last dimension must be contiguous")
        fields.update(new_k=new_k.data_ptr(), new_k_stride_seq=nks[0], new_k_stride_head=nks[1],
                      new_v=new_v.data_ptr(), new_v_stride_seq=nvs[0], new_v_stride_head=nvs[1])
    if new_slots is not None:
        _require(new_k is not None, "new_slots requires new_k/new_v")
        _require(new_slots.dim() == 1 and new_slots.numel() >= B and new_slots.is_contiguous(),
                 "new_slots must be a contiguous [num_seqs] vector")
        fields.update(new_slots=new_slots.data_ptr(),
                      new_slots_dtype=_index_code(new_slots, "new_slots"))
    pro_struct = None
    if prologue is not None:
        pro_struct = _prologue_struct(prologue, d, B)  # kept alive through the call
        fields["prologue"] = ctypes.pointer(pro_struct)
    args = N.DecodeArgs(**fields)
    lib = N.lib()
    index = _device_index(device)
    with _current(index):  # the split plan depends on the device's CU count
        if no_alloc:
            _order_noalloc(index)
            N.check("va_paged_decode_noalloc",
                    lib.va_paged_decode_noalloc(ctypes.byref(args), _raw_stream(index)))
            return out
        nbytes = lib.va_paged_decode_workspace_bytes(ctypes.byref(args))
        if nbytes:
            ws = decode_workspace(device, nbytes, floor=decode_workspace_bound(device, hq, hkv, d))
            args.workspace = ws.data_ptr()
            args.workspace_bytes = ws.numel()
        N.check("va_paged_decode", lib.va_paged_decode(ctypes.byref(args), _raw_stream(index)))
    return out


# -------------------------------------------------------------------- varlen
def varlen_attention(
    q: torch.Tensor,
    k: torch.Tensor | None,
    v: torch.Tensor | None,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    max_seqlen_q: int,
    max_seqlen_k: int,
    *,
    scale: float,
    causal: bool,
    k_cache: torch.Tensor | None = None,
    v_cache: torch.Tensor | None = None,
    block_tables: torch.Tensor | None = None,
    slot_mapping: torch.Tensor | None = None,
    layout: str = LAYOUT_NHD,
    out: torch.Tensor | None = None,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
    prologue: QKPrologue | None = None,
) -> torch.Tensor:
    """Packed variable-length attention (flash_attn_varlen_func semantics).

    Causal attention is bottom-right aligned: query i of a sequence with
    (q_len, k_len) sees keys j <= k_len - q_len + i.  With a pool, keys
    j < k_len - q_len are read through ``block_tables``; the others from
    ``k``/``v`` rows aligned with the queries (all from the pool if ``k`` is
    None).  ``slot_mapping`` fuses store_kvcache of k/v into the same launch.
    ``max_seqlen_q`` must be at least every q_len, as for flash-attn: it sizes
    the launch, and query rows past it are not computed.  ``max_seqlen_k`` is
    not read: key ranges come from ``cu_seqlens_k``.  An FP8 pool
    (float8_e4m3fn codes, values code * k_scale / v_scale) is converted tile
    by tile inside the kernel (no workspace); its new rows are stored
    quantised after the attention.  With a ``prologue`` (causal, head_dim
    128, a 16-bit pool or none), q holds the raw query projections and the
    launch normalises and rotates them at ``prologue.positions`` (one per
    query token); k and the pool must hold processed keys.
    """
    fast = _FAST if _FAST_LOADED else _fast_calls()
    if (fast is not None and prologue is None and layout in (LAYOUT_NHD, LAYOUT_HND) and
            (k_cache is None or k_cache.dtype != FP8_KV_DTYPE)):
        index = q.get_device()
        if index >= 0 and index == torch.cuda.current_device():
            if out is None:
                out = torch.empty_like(q)
            rc = fast.varlen_attention(
                q, k, v, cu_seqlens_q, cu_seqlens_k, int(max_seqlen_q), int(max_seqlen_k),
                float(scale), bool(causal), k_cache, v_cache, block_tables, slot_mapping, out,
                layout == LAYOUT_HND, index, _raw_stream(index))
            if rc == 0:
                return out
            if _FAST_NOT_TAKEN < rc < 0:
                N.check("va_varlen_attention", rc)
    device = _check_gpu(q, k, v, cu_seqlens_q, cu_seqlens_k, k_cache, v_cache, block_tables,
                        slot_mapping, out)
    _require(q.dim() == 3, "q must be [total_q, num_heads, head_dim]")
    qs = q.stride()
    _require(qs[2] == 1, "q: the last dimension must be contiguous")
    total_q, hq, d = q.shape
    _require(cu_seqlens_q.dtype == torch.int32 and cu_seqlens_k.dtype == torch.int32,
             "cu_seqlens must be int32")
    _require(cu_seqlens_q.dim() == 1 and cu_seqlens_q.numel() >= 2 and
             cu_seqlens_k.numel() == cu_seqlens_q.numel(), "cu_seqlens must be [num_seqs + 1]")
    _require(cu_seqlens_q.is_contiguous() and cu_seqlens_k.is_contiguous(),
             "cu_seqlens must be contiguous")
    num_seqs = cu_seqlens_q.numel() - 1
    fields = {}
    if k_cache is not None:
        _require(v_cache is not None and block_tables is not None,
                 "a KV pool needs v_cache and block_tables")
        hkv, pd = pool_heads(k_cache, layout)
        _require(pd == d, "pool head_dim must match q")
        _require(_pool_matches(k_cache, q.dtype),
                 "pool dtype must match q (or the pool be FP8 for 16-bit q)")
        bts = block_tables.stride()
        _require(block_tables.dim() == 2 and block_tables.shape[0] >= num_seqs and bts[1] == 1,
                 "block_tables must be [num_seqs, width]")
        fields.update(pool=_pool_struct(k_cache, v_cache, layout, k_scale, v_scale),
                      block_tables=block_tables.data_ptr(),
                      table_dtype=_index_code(block_tables, "block_tables"),
                      table_stride_seq=bts[0], table_width=block_tables.shape[1])
    else:
        _require(k is not None and v is not None, "k and v are required without a KV pool")
        hkv = k.shape[1]
    if k is not None:
        _require(v is not None and k.dim() == 3 and v.shape == k.shape,
                 "k/v must be [tokens, num_kv_heads, head_dim]")
        _require(k.shape[1] == hkv and k.shape[2] == d, "k/v heads must match")
        _require(k.dtype == v.dtype == q.dtype, "q/k/v dtypes must match")
        ks, vs = k.stride(), v.stride()
        _require(ks[2] == 1 and vs[2] == 1, "k/v: the last dimension must be contiguous")
        fields.update(k=k.data_ptr(), k_stride_tok=ks[0], k_stride_head=ks[1], v=v.data_ptr(),
                      v_stride_tok=vs[0], v_stride_head=vs[1])
    _require(hq % hkv == 0, "num_heads must be a multiple of num_kv_heads")
    if slot_mapping is not None:
        _require(k_cache is not None and k is not None, "slot_mapping needs a pool and k/v")
        _require(slot_mapping.dim() == 1 and slot_mapping.numel() == total_q and
                 slot_mapping.is_contiguous(), "slot_mapping must have one entry per query")
        fields.update(slot_mapping=slot_mapping.data_ptr(),
                      slot_dtype=_index_code(slot_mapping, "slot_mapping"))
    pro_struct = None
    if prologue is not None:
        _check_gpu(q, prologue.q_norm_weight, prologue.cos_sin_cache, prologue.positions)
        pro_struct = _prologue_struct(prologue, d, total_q)  # kept alive through the call
        fields["prologue"] = ctypes.pointer(pro_struct)
    if out is None:
        out = torch.empty_like(q)
    os_ = out.stride()
    _require(out.shape == q.shape and out.dtype == q.dtype, "out must match q")
    _require(os_[2] == 1, "out: the last dimension must be contiguous")
    args = N.VarlenArgs(
        struct_size=_VARLEN_ARGS_SIZE, dtype=_dtype_code(q), q=q.data_ptr(), q_stride_tok=qs[0],
        q_stride_head=qs[1], out=out.data_ptr(), out_stride_tok=os_[0], out_stride_head=os_[1],
        cu_seqlens_q=cu_seqlens_q.data_ptr(), cu_seqlens_k=cu_seqlens_k.data_ptr(),
        num_seqs=num_seqs, total_q=total_q, num_heads=hq, num_kv_heads=hkv, head_dim=d,
        max_seqlen_q=int(max_seqlen_q), max_seqlen_k=int(max_seqlen_k),
        causal=1 if causal else 0, scale=float(scale), **fields)
    lib = N.lib()
    index = _device_index(device)
    with _current(index):
        N.check("va_varlen_attention",
                lib.va_varlen_attention(ctypes.byref(args), _raw_stream(index)))
    return out


def default_scale(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)
