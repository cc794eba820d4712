// Host fast path of ops.paged_decode, ops.varlen_attention, ops.store_kvcache
// and ops.qk_norm_rope.
//
// The Python wrappers validate every argument and fill a ctypes struct on
// each call, about 10 us of host time, which an eager engine step pays once
// per layer.  This module takes the same tensors through pybind11, makes the
// same checks on them, fills the same argument structs and calls the same
// entry points of libvoiceagent_attn.so (their addresses come from ops.py,
// so nothing here links the library or any GPU runtime).
//
// Only the common calls are taken, and only with arguments that pass every
// check the Python wrapper makes.  Anything else returns kNotTaken without
// touching the GPU; the wrapper then runs its own path, which raises the
// wrapper's error for a bad argument.  A status from the library is returned
// as is (negative VA_ERR_*), and a decode that needs a workspace larger than
// the one given returns the bytes it needs, launching nothing.
#include <torch/extension.h>

#include <cstdint>
#include <limits>

#include "voiceagent_attn.h"

namespace {

using DecodeFn = int (*)(const va_decode_args*, void*);
using DecodeWsFn = size_t (*)(const va_decode_args*);
using VarlenFn = int (*)(const va_varlen_args*, void*);
using StoreFn = int (*)(const va_store_args*, void*);
using RopeFn = int (*)(const va_qk_norm_rope_args*, void*);

DecodeFn g_decode = nullptr;
DecodeWsFn g_decode_ws = nullptr;
VarlenFn g_varlen = nullptr;
StoreFn g_store = nullptr;
RopeFn g_rope = nullptr;

constexpr int64_t kNotTaken = -1000;

int dtype_code(c10::ScalarType t) {
  switch (t) {
    case at::kBFloat16: return VA_BF16;
    case at::kHalf: return VA_F16;
    case at::kFloat: return VA_F32;
    default: return -1;
  }
}

int index_code(c10::ScalarType t) {
  switch (t) {
    case at::kInt: return VA_I32;
    case at::kLong: return VA_I64;
    default: return -1;
  }
}

bool fits_i32(int64_t x) {
  return x >= std::numeric_limits<int32_t>::min() && x <= std::numeric_limits<int32_t>::max();
}

// A dense GPU tensor on `device`.
bool on(const at::Tensor& t, int64_t device) {
  return t.defined() && t.layout() == at::kStrided && t.is_cuda() && t.get_device() == device;
}

// The pool description of kv_pool(): 4-D NHD [blocks, block_size, Hkv, D] or
// HND [blocks, Hkv, block_size, D], k and v alike, rows contiguous; an FP8
// pool with positive scales.  False when any of that fails.
bool fill_pool(const at::Tensor& kc, const at::Tensor& vc, bool hnd, double k_scale,
               double v_scale, va_kv_pool* pool) {
  if (kc.dim() != 4 || vc.sizes() != kc.sizes() || vc.strides() != kc.strides() ||
      vc.scalar_type() != kc.scalar_type() || kc.stride(3) != 1)
    return false;
  pool->k = kc.data_ptr();
  pool->v = vc.data_ptr();
  pool->stride_block = kc.stride(0);
  pool->stride_slot = hnd ? kc.stride(2) : kc.stride(1);
  pool->stride_head = hnd ? kc.stride(1) : kc.stride(2);
  const int64_t bs = hnd ? kc.size(2) : kc.size(1);
  if (!fits_i32(bs) || !fits_i32(kc.size(0))) return false;
  pool->block_size = (int32_t)bs;
  pool->num_blocks = (int32_t)kc.size(0);
  if (kc.scalar_type() == at::kFloat8_e4m3fn) {
    if (!(k_scale > 0.0) || !(v_scale > 0.0)) return false;
    pool->kv_format = VA_KV_FP8_E4M3;
    pool->k_scale = (float)k_scale;
    pool->v_scale = (float)v_scale;
  } else {
    pool->kv_format = VA_KV_NATIVE;
    pool->k_scale = pool->v_scale = 1.0f;
  }
  return true;
}

// q's dtype for the pool: the pool's own, or FP8 codes for 16-bit q.
bool pool_matches(const at::Tensor& pool, c10::ScalarType dt) {
  return pool.scalar_type() == dt ||
         (pool.scalar_type() == at::kFloat8_e4m3fn && (dt == at::kBFloat16 || dt == at::kHalf));
}

// A contiguous index vector of at least n entries.
bool index_vector(const at::Tensor& t, int64_t n) {
  return t.dim() == 1 && t.numel() >= n && t.is_contiguous() && index_code(t.scalar_type()) >= 0;
}

void set_entries(int64_t decode, int64_t decode_ws, int64_t varlen, int64_t store,
                 int64_t rope) {
  g_decode = reinterpret_cast<DecodeFn>(static_cast<intptr_t>(decode));
  g_decode_ws = reinterpret_cast<DecodeWsFn>(static_cast<intptr_t>(decode_ws));
  g_varlen = reinterpret_cast<VarlenFn>(static_cast<intptr_t>(varlen));
  g_store = reinterpret_cast<StoreFn>(static_cast<intptr_t>(store));
  g_rope = reinterpret_cast<RopeFn>(static_cast<intptr_t>(rope));
}

// The prologue description of _prologue_struct(): [head_dim] weights of one
// dtype, contiguous; an fp32 [max_position, (1,) head_dim] cos | sin table
// with contiguous rows; at least n contiguous positions.
bool fill_prologue(const at::Tensor& qw, const at::Tensor& kw, double eps, const at::Tensor& cs,
                   const at::Tensor& pos, int64_t d, int64_t n, int64_t device,
                   va_qk_prologue* pro) {
  if (!on(qw, device) || !on(kw, device) || !on(cs, device) || !on(pos, device)) return false;
  for (const at::Tensor* w : {&qw, &kw})
    if (w->dim() != 1 || w->numel() != d || !w->is_contiguous()) return false;
  if (qw.scalar_type() != kw.scalar_type() || dtype_code(qw.scalar_type()) < 0) return false;
  if (cs.dim() == 3 && cs.size(1) != 1) return false;
  if ((cs.dim() != 2 && cs.dim() != 3) || cs.size(cs.dim() - 1) != d ||
      cs.scalar_type() != at::kFloat || cs.stride(cs.dim() - 1) != 1 || !fits_i32(cs.size(0)))
    return false;
  if (!index_vector(pos, n)) return false;
  pro->q_norm_weight = qw.data_ptr();
  pro->k_norm_weight = kw.data_ptr();
  pro->weight_dtype = dtype_code(qw.scalar_type());
  pro->eps = (float)eps;
  pro->cos_sin_cache = static_cast<const float*>(cs.data_ptr());
  pro->cos_sin_stride = cs.stride(0);
  pro->max_position = (int32_t)cs.size(0);
  pro->positions_dtype = index_code(pos.scalar_type());
  pro->positions = pos.data_ptr();
  return true;
}

// ops.paged_decode without no_alloc (layout_hnd picks the pool layout; the
// prologue is given by its four tensors and eps, all or none).  0: launched;
// > 0: workspace bytes needed, nothing launched; VA_ERR_*: the library's
// status; kNotTaken: nothing done.
int64_t paged_decode(const at::Tensor& q, const at::Tensor& kc, const at::Tensor& vc,
                     const at::Tensor& tables, const at::Tensor& lens, const at::Tensor& out,
                     const c10::optional<at::Tensor>& new_k,
                     const c10::optional<at::Tensor>& new_v,
                     const c10::optional<at::Tensor>& new_slots,
                     const c10::optional<at::Tensor>& valid_mask,
                     const c10::optional<at::Tensor>& pro_q_w,
                     const c10::optional<at::Tensor>& pro_k_w, double pro_eps,
                     const c10::optional<at::Tensor>& pro_cos_sin,
                     const c10::optional<at::Tensor>& pro_positions,
                     const c10::optional<at::Tensor>& workspace, bool cumulative, bool layout_hnd,
                     int64_t max_seq_len, double scale, int64_t split_tokens, int64_t key_limit,
                     int64_t table_read_width, double k_scale, double v_scale, int64_t device,
                     int64_t stream) {
  if (g_decode == nullptr || g_decode_ws == nullptr) return kNotTaken;
  if (!on(q, device) || !on(kc, device) || !on(vc, device) || !on(tables, device) ||
      !on(lens, device) || !on(out, device))
    return kNotTaken;
  if (q.dim() != 3 || q.stride(2) != 1) return kNotTaken;
  const int64_t B = q.size(0), hq = q.size(1), d = q.size(2);
  if (kc.dim() != 4) return kNotTaken;
  const int64_t hkv = layout_hnd ? kc.size(1) : kc.size(2);
  if (kc.size(3) != d || hkv <= 0 || hq % hkv != 0) return kNotTaken;
  if (!pool_matches(kc, q.scalar_type())) return kNotTaken;
  const int dt = dtype_code(q.scalar_type());
  if (dt < 0) return kNotTaken;
  if (tables.dim() != 2 || tables.size(0) < B || tables.stride(1) != 1 ||
      index_code(tables.scalar_type()) < 0)
    return kNotTaken;
  if (!index_vector(lens, cumulative ? B + 1 : B)) return kNotTaken;
  if (out.sizes() != q.sizes() || out.scalar_type() != q.scalar_type() || out.stride(2) != 1)
    return kNotTaken;
  if (key_limit < 0 || table_read_width < 0) return kNotTaken;
  if (new_k.has_value() != new_v.has_value()) return kNotTaken;
  if (!fits_i32(B) || !fits_i32(hq) || !fits_i32(d) || !fits_i32(max_seq_len) ||
      !fits_i32(split_tokens) || !fits_i32(key_limit) || !fits_i32(table_read_width) ||
      !fits_i32(tables.size(1)))
    return kNotTaken;

  va_decode_args a{};
  a.struct_size = sizeof(a);
  a.dtype = dt;
  a.q = q.data_ptr();
  a.q_stride_seq = q.stride(0);
  a.q_stride_head = q.stride(1);
  a.out = out.data_ptr();
  a.out_stride_seq = out.stride(0);
  a.out_stride_head = out.stride(1);
  if (!fill_pool(kc, vc, layout_hnd, k_scale, v_scale, &a.pool)) return kNotTaken;
  a.block_tables = tables.data_ptr();
  a.table_dtype = index_code(tables.scalar_type());
  a.table_stride_seq = tables.stride(0);
  a.table_width = (int32_t)tables.size(1);
  a.lens = lens.data_ptr();
  a.lens_dtype = index_code(lens.scalar_type());
  a.lens_kind = cumulative ? VA_LENS_CUMULATIVE : VA_LENS_PER_SEQ;
  if (new_k.has_value()) {
    const at::Tensor& nk = *new_k;
    const at::Tensor& nv = *new_v;
    if (!on(nk, device) || !on(nv, device) || nk.dim() != 3 || nk.size(0) != B ||
        nk.size(1) != hkv || nk.size(2) != d || nv.sizes() != nk.sizes() ||
        nk.scalar_type() != q.scalar_type() || nv.scalar_type() != q.scalar_type() ||
        nk.stride(2) != 1 || nv.stride(2) != 1)
      return kNotTaken;
    a.new_k = nk.data_ptr();
    a.new_k_stride_seq = nk.stride(0);
    a.new_k_stride_head = nk.stride(1);
    a.new_v = nv.data_ptr();
    a.new_v_stride_seq = nv.stride(0);
    a.new_v_stride_head = nv.stride(1);
  }
  if (new_slots.has_value()) {
    const at::Tensor& ns = *new_slots;
    if (!new_k.has_value() || !on(ns, device) || !index_vector(ns, B)) return kNotTaken;
    a.new_slots = ns.data_ptr();
    a.new_slots_dtype = index_code(ns.scalar_type());
  }
  if (valid_mask.has_value()) {
    const at::Tensor& vm = *valid_mask;
    if (!on(vm, device) || vm.dim() != 2 || vm.size(0) < B || vm.scalar_type() != at::kBool ||
        vm.stride(1) != 1 || !fits_i32(vm.size(1)))
      return kNotTaken;
    a.valid_mask = static_cast<const uint8_t*>(vm.data_ptr());
    a.valid_stride_seq = vm.stride(0);
    a.valid_len = (int32_t)vm.size(1);
  }
  va_qk_prologue pro{};
  if (pro_q_w.has_value()) {
    if (!pro_k_w.has_value() || !pro_cos_sin.has_value() || !pro_positions.has_value() ||
        !fill_prologue(*pro_q_w, *pro_k_w, pro_eps, *pro_cos_sin, *pro_positions, d, B, device,
                       &pro))
      return kNotTaken;
    a.prologue = &pro;
  }
  a.num_seqs = (int32_t)B;
  a.num_heads = (int32_t)hq;
  a.num_kv_heads = (int32_t)hkv;
  a.head_dim = (int32_t)d;
  a.max_seq_len = (int32_t)max_seq_len;
  a.split_tokens = (int32_t)split_tokens;
  a.scale = (float)scale;
  a.key_limit = (int32_t)key_limit;
  a.table_read_width = (int32_t)table_read_width;

  const size_t need = g_decode_ws(&a);
  if (need > 0) {
    if (!workspace.has_value()) return (int64_t)need;
    const at::Tensor& ws = *workspace;
    if (!on(ws, device) || (size_t)ws.numel() * ws.element_size() < need || !ws.is_contiguous())
      return (int64_t)need;
    a.workspace = ws.data_ptr();
    a.workspace_bytes = (size_t)ws.numel() * ws.element_size();
  }
  return g_decode(&a, reinterpret_cast<void*>(static_cast<intptr_t>(stream)));
}

// ops.varlen_attention over a 16-bit pool or none (an FP8 pool needs a
// workspace: not taken).  0: launched; VA_ERR_*: the library's status;
// kNotTaken: nothing done.
int64_t varlen_attention(const at::Tensor& q, const c10::optional<at::Tensor>& k,
                         const c10::optional<at::Tensor>& v, const at::Tensor& cu_q,
                         const at::Tensor& cu_k, int64_t max_seqlen_q, int64_t max_seqlen_k,
                         double scale, bool causal, const c10::optional<at::Tensor>& k_cache,
                         const c10::optional<at::Tensor>& v_cache,
                         const c10::optional<at::Tensor>& tables,
                         const c10::optional<at::Tensor>& slot_mapping, const at::Tensor& out,
                         bool layout_hnd, int64_t device, int64_t stream) {
  if (g_varlen == nullptr) return kNotTaken;
  if (!on(q, device) || !on(cu_q, device) || !on(cu_k, device) || !on(out, device))
    return kNotTaken;
  if (q.dim() != 3 || q.stride(2) != 1) return kNotTaken;
  const int64_t total_q = q.size(0), hq = q.size(1), d = q.size(2);
  const int dt = dtype_code(q.scalar_type());
  if (dt < 0) return kNotTaken;
  if (cu_q.scalar_type() != at::kInt || cu_k.scalar_type() != at::kInt || cu_q.dim() != 1 ||
      cu_q.numel() < 2 || cu_k.numel() != cu_q.numel() || !cu_q.is_contiguous() ||
      !cu_k.is_contiguous())
    return kNotTaken;
  const int64_t num_seqs = cu_q.numel() - 1;

  va_varlen_args a{};
  a.struct_size = sizeof(a);
  int64_t hkv = 0;
  if (k_cache.has_value()) {
    const at::Tensor& kc = *k_cache;
    if (!v_cache.has_value() || !tables.has_value() || !on(kc, device) ||
        !on(*v_cache, device) || !on(*tables, device))
      return kNotTaken;
    if (kc.dim() != 4) return kNotTaken;
    hkv = layout_hnd ? kc.size(1) : kc.size(2);
    if (kc.size(3) != d || kc.scalar_type() != q.scalar_type()) return kNotTaken;
    const at::Tensor& t = *tables;
    if (t.dim() != 2 || t.size(0) < num_seqs || t.stride(1) != 1 ||
        index_code(t.scalar_type()) < 0 || !fits_i32(t.size(1)))
      return kNotTaken;
    if (!fill_pool(kc, *v_cache, layout_hnd, 1.0, 1.0, &a.pool)) return kNotTaken;
    a.block_tables = t.data_ptr();
    a.table_dtype = index_code(t.scalar_type());
    a.table_stride_seq = t.stride(0);
    a.table_width = (int32_t)t.size(1);
  } else {
    if (!k.has_value() || !v.has_value() || k->dim() != 3) return kNotTaken;
    hkv = k->size(1);
  }
  if (k.has_value()) {
    if (!v.has_value()) return kNotTaken;
    const at::Tensor& kk = *k;
    const at::Tensor& vv = *v;
    if (!on(kk, device) || !on(vv, device) || kk.dim() != 3 || vv.sizes() != kk.sizes() ||
        kk.size(1) != hkv || kk.size(2) != d || kk.scalar_type() != q.scalar_type() ||
        vv.scalar_type() != q.scalar_type() || kk.stride(2) != 1 || vv.stride(2) != 1)
      return kNotTaken;
    a.k = kk.data_ptr();
    a.k_stride_tok = kk.stride(0);
    a.k_stride_head = kk.stride(1);
    a.v = vv.data_ptr();
    a.v_stride_tok = vv.stride(0);
    a.v_stride_head = vv.stride(1);
  } else if (v.has_value()) {
    return kNotTaken;
  }
  if (hkv <= 0 || hq % hkv != 0) return kNotTaken;
  if (slot_mapping.has_value()) {
    const at::Tensor& sm = *slot_mapping;
    if (!k_cache.has_value() || !k.has_value() || !on(sm, device) || sm.dim() != 1 ||
        sm.numel() != total_q || !sm.is_contiguous() || index_code(sm.scalar_type()) < 0)
      return kNotTaken;
    a.slot_mapping = sm.data_ptr();
    a.slot_dtype = index_code(sm.scalar_type());
  }
  if (out.sizes() != q.sizes() || out.scalar_type() != q.scalar_type() || out.stride(2) != 1)
    return kNotTaken;
  if (!fits_i32(num_seqs) || !fits_i32(total_q) || !fits_i32(hq) || !fits_i32(d) ||
      !fits_i32(max_seqlen_q) || !fits_i32(max_seqlen_k))
    return kNotTaken;
  a.dtype = dt;
  a.q = q.data_ptr();
  a.q_stride_tok = q.stride(0);
  a.q_stride_head = q.stride(1);
  a.out = out.data_ptr();
  a.out_stride_tok = out.stride(0);
  a.out_stride_head = out.stride(1);
  a.cu_seqlens_q = static_cast<const int32_t*>(cu_q.data_ptr());
  a.cu_seqlens_k = static_cast<const int32_t*>(cu_k.data_ptr());
  a.num_seqs = (int32_t)num_seqs;
  a.total_q = (int32_t)total_q;
  a.num_heads = (int32_t)hq;
  a.num_kv_heads = (int32_t)hkv;
  a.head_dim = (int32_t)d;
  a.max_seqlen_q = (int32_t)max_seqlen_q;
  a.max_seqlen_k = (int32_t)max_seqlen_k;
  a.causal = causal ? 1 : 0;
  a.scale = (float)scale;
  return g_varlen(&a, reinterpret_cast<void*>(static_cast<intptr_t>(stream)));
}

// ops.store_kvcache.  0: launched; VA_ERR_*: the library's status;
// kNotTaken: nothing done.
int64_t store_kvcache(const at::Tensor& key, const at::Tensor& value, const at::Tensor& kc,
                      const at::Tensor& vc, const at::Tensor& slots, bool layout_hnd,
                      double k_scale, double v_scale, int64_t device, int64_t stream) {
  if (g_store == nullptr) return kNotTaken;
  if (!on(key, device) || !on(value, device) || !on(kc, device) || !on(vc, device) ||
      !on(slots, device))
    return kNotTaken;
  if (key.dim() != 3 || value.sizes() != key.sizes() || key.stride(2) != 1 ||
      value.stride(2) != 1 || kc.dim() != 4)
    return kNotTaken;
  const int64_t hkv = layout_hnd ? kc.size(1) : kc.size(2);
  if (key.size(1) != hkv || key.size(2) != kc.size(3)) return kNotTaken;
  if (key.scalar_type() != value.scalar_type() || !pool_matches(kc, key.scalar_type()) ||
      dtype_code(key.scalar_type()) < 0)
    return kNotTaken;
  if (slots.dim() != 1 || slots.numel() != key.size(0) || !slots.is_contiguous() ||
      index_code(slots.scalar_type()) < 0 ||
      !fits_i32(key.size(0)) || !fits_i32(hkv) || !fits_i32(key.size(2)))
    return kNotTaken;
  va_store_args a{};
  a.struct_size = sizeof(a);
  if (!fill_pool(kc, vc, layout_hnd, k_scale, v_scale, &a.pool)) return kNotTaken;
  a.dtype = dtype_code(key.scalar_type());
  a.key = key.data_ptr();
  a.value = value.data_ptr();
  a.key_stride_tok = key.stride(0);
  a.key_stride_head = key.stride(1);
  a.value_stride_tok = value.stride(0);
  a.value_stride_head = value.stride(1);
  a.slot_mapping = slots.data_ptr();
  a.slot_dtype = index_code(slots.scalar_type());
  a.num_tokens = (int32_t)key.size(0);
  a.num_kv_heads = (int32_t)hkv;
  a.head_dim = (int32_t)key.size(2);
  return g_store(&a, reinterpret_cast<void*>(static_cast<intptr_t>(stream)));
}

// ops.qk_norm_rope with both outputs given.  0: launched; VA_ERR_*: the
// library's status; kNotTaken: nothing done.
int64_t qk_norm_rope(const at::Tensor& q, const at::Tensor& k, const at::Tensor& q_out,
                     const at::Tensor& k_out, const at::Tensor& q_w, const at::Tensor& k_w,
                     double eps, const at::Tensor& cos_sin, const at::Tensor& positions,
                     int64_t device, int64_t stream) {
  if (g_rope == nullptr) return kNotTaken;
  if (!on(q, device) || !on(k, device) || !on(q_out, device) || !on(k_out, device))
    return kNotTaken;
  if (q.dim() != 3 || k.dim() != 3 || q.size(0) != k.size(0) || q.size(2) != k.size(2) ||
      q.scalar_type() != k.scalar_type() || q.stride(2) != 1 || k.stride(2) != 1)
    return kNotTaken;
  if (q_out.sizes() != q.sizes() || q_out.scalar_type() != q.scalar_type() ||
      k_out.sizes() != k.sizes() || k_out.scalar_type() != k.scalar_type() ||
      q_out.stride(2) != 1 || k_out.stride(2) != 1 || dtype_code(q.scalar_type()) < 0)
    return kNotTaken;
  const int64_t T = q.size(0), hq = q.size(1), hkv = k.size(1), d = q.size(2);
  if (!fits_i32(T) || !fits_i32(hq) || !fits_i32(hkv) || !fits_i32(d)) return kNotTaken;
  va_qk_norm_rope_args a{};
  a.struct_size = sizeof(a);
  if (!fill_prologue(q_w, k_w, eps, cos_sin, positions, d, T, device, &a.prologue))
    return kNotTaken;
  a.dtype = dtype_code(q.scalar_type());
  a.q = q.data_ptr();
  a.q_stride_tok = q.stride(0);
  a.q_stride_head = q.stride(1);
  a.k = k.data_ptr();
  a.k_stride_tok = k.stride(0);
  a.k_stride_head = k.stride(1);
  a.q_out = q_out.data_ptr();
  a.q_out_stride_tok = q_out.stride(0);
  a.q_out_stride_head = q_out.stride(1);
  a.k_out = k_out.data_ptr();
  a.k_out_stride_tok = k_out.stride(0);
  a.k_out_stride_head = k_out.stride(1);
  a.num_tokens = (int32_t)T;
  a.num_heads = (int32_t)hq;
  a.num_kv_heads = (int32_t)hkv;
  a.head_dim = (int32_t)d;
  return g_rope(&a, reinterpret_cast<void*>(static_cast<intptr_t>(stream)));
}

}  // namespace

PYBIND11_MODULE(_fast_calls, m) {
  m.doc() = "Host fast path of the ops wrappers";
  m.attr("NOT_TAKEN") = kNotTaken;
  m.def("set_entries", &set_entries);
  m.def("paged_decode", &paged_decode);
  m.def("varlen_attention", &varlen_attention);
  m.def("store_kvcache", &store_kvcache);
  m.def("qk_norm_rope", &qk_norm_rope);
}
