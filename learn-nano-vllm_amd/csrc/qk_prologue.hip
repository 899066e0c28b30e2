// Fused attention prologue of a Qwen3 decoder layer for gfx950: per-head
// RMSNorm of q and k, rotary embedding of q and k, and the KV-store scatter of
// the rotated k and the raw v, in one pass over the packed qkv projection.
//
// Semantics (nanovllm/models/qwen3.py:79-86 then attention.py:62-63):
//   q, k, v = qkv.split([Hq*D, Hkv*D, Hkv*D], -1), viewed [T, H, D]
//   q = RMSNorm(q) ; k = RMSNorm(k)                  (layernorm.py:16-26)
//       x.float(); x *= rsqrt(mean(x^2) + eps); x = T(x) * weight (T)
//   q, k = rope(positions, q, k)                     (rotary_embedding.py:6-14, 37-48)
//       x1, x2 = halves of x.float(); cos, sin = halves of cos_sin_cache[pos]
//       y1 = x1*cos - x2*sin ; y2 = x2*cos + x1*sin ; T(cat(y1, y2))
// with T the model's element type, bf16 or f16 (model_runner.py:29).
//   k_cache[slot] = k ; v_cache[slot] = v  for slot != -1  (attention.py:10-30)
// Every f32 product and sum is rounded on its own (no fused multiply-add), as
// the reference's separate tensor operations do.
//
// Data movement: the reference reads qkv, writes the normed q and k, reads
// them back for the rotation, writes the rotated q and k, then the store reads
// k and v again and writes the caches.  Here each head row (D = 128 bf16 =
// 256 B) is read once and written once to each destination.
//
// Lane mapping: a row group of 16 lanes owns one head row of one token, 8
// elements (16 B) per lane.  The row's sum of squares is a 16-lane DPP
// reduction; the rotation partner of element i (i +- D/2) sits in lane
// j ^ 8 of the same row group and is fetched with one DPP row rotation by 8.
// A workgroup owns one token (Hq + 2*Hkv rows, 8 KiB contiguous for Qwen3),
// measured ~10 % faster than 16-row workgroups over the flattened row space,
// which read the position, slot and cos/sin row once per row group.
#include "qk_math.h"

namespace {

using nvk_qk::kHD;
using nvk_qk::kLanesPerRow;
// Row groups per workgroup (256 threads): Qwen3's 32 head rows take two per
// row group.  Measured on the 4288-token layer (interleaved A/B, same outputs):
// 32 groups (one row each) 16.3 us, 16 groups 15.6 us, 8 groups 16.6 us; two
// tokens per 1024-thread workgroup 19.3 us.
constexpr int kMaxGroups = 16;
// Steps of up to kSmallTokens tokens (decode steps) are latency bound: one row
// group per head row (up to kMaxRowGroups, 512 threads), each loading only the
// norm weight and cos/sin its row needs.  Measured (interleaved A/B, same
// outputs): 64 tokens 3.16 -> 2.96 us, 512 tokens 4.65 -> 4.08 us against two
// rows per group; at 4288 tokens one row per group takes 17.6 us.
constexpr int kMaxRowGroups = 32;
constexpr int64_t kSmallTokens = 512;

struct PrologueArgs {
  const uint16_t* qkv;
  int64_t qkv_row_stride;
  int64_t n_tokens;
  const int64_t* positions;
  const uint16_t* q_weight;
  const uint16_t* k_weight;
  float eps;
  const float* cos_sin;
  int64_t cos_sin_stride;
  int64_t max_position;
  int num_q_heads, num_kv_heads;
  uint16_t* q_out;
  int64_t q_out_stride_tok, q_out_stride_head;
  uint16_t* k_out;  // may be null
  int64_t k_out_stride_tok, k_out_stride_head;
  uint16_t* k_cache;  // null: no store
  uint16_t* v_cache;
  const int32_t* slot_mapping;
  int64_t cache_slots;
};

// The qkv rows are read once and every output row (q, k, cache rows) written
// once per step: non-temporal 16-byte accesses.  Measured on one layer of the
// mixed step (4288 tokens, inputs cycling through more than the Infinity
// Cache): 19.3 us cached, 17.7 us non-temporal; non-temporal loads or cache
// stores alone change nothing.  The cos/sin rows are shared by the tokens of a
// position and stay cached.
__device__ __forceinline__ nvk_u32x4 load_nt(const uint16_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const nvk_u32x4*>(p));
}
__device__ __forceinline__ void store_nt(uint16_t* p, nvk_u32x4 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<nvk_u32x4*>(p));
}


// Head rows of a row group whose loads are issued together, before any of
// their arithmetic.
constexpr int kRowsPerPass = 2;

// One head row r of token t (uniform per 16-lane row group), its 16 bytes
// `raw` already loaded; wq / wk: the lane's 8 norm weights of q / k, cs: its
// cos and sin at the token's position.
template <bool F16>
__device__ __forceinline__ void prologue_row(const PrologueArgs& a, int64_t t, int r, int j,
                                             int32_t slot, nvk_u32x4 raw, nvk_u32x4 wq,
                                             nvk_u32x4 wk, const nvk_u32x4 (&cs)[4]) {
#pragma clang fp contract(off)
  const bool is_q = r < a.num_q_heads;
  const bool is_k = !is_q && r < a.num_q_heads + a.num_kv_heads;

  const int64_t row_elems = (int64_t)a.num_kv_heads * kHD;

  if (!is_q && !is_k) {  // v row: a plain copy into the cache
    if (slot >= 0) {
      const int kvh = r - a.num_q_heads - a.num_kv_heads;
      store_nt(a.v_cache + (int64_t)slot * row_elems + kvh * kHD + 8 * j, raw);
    }
    return;
  }

  const nvk_u32x4 outw = nvk_qk::norm_rope8_cs<F16>(raw, is_q ? wq : wk, a.eps, cs, j);
  if (is_q) {
    store_nt(a.q_out + t * a.q_out_stride_tok + (int64_t)r * a.q_out_stride_head + 8 * j, outw);
    return;
  }
  const int kvh = r - a.num_q_heads;
  if (a.k_out != nullptr)
    store_nt(a.k_out + t * a.k_out_stride_tok + (int64_t)kvh * a.k_out_stride_head + 8 * j, outw);
  if (slot >= 0)
    store_nt(a.k_cache + (int64_t)slot * row_elems + kvh * kHD + 8 * j, outw);
}


// One workgroup per token: the token's position and slot are workgroup-uniform
// (scalar loads), its cos/sin row is read by every row group from the same
// 512 bytes (L1 hits after the first).  Row group g of the workgroup takes
// rows g, g + groups, ...; the loads of kRowsPerPass of them, of the norm
// weights and of the lane's cos/sin all leave before the first wait (left to
// itself the compiler issues a row's load only after the previous row's
// arithmetic and stores: two round trips for Qwen3's two rows per group).
template <bool F16>
__global__ __launch_bounds__(16 * kMaxRowGroups) void qk_prologue_kernel(PrologueArgs a) {
  const int64_t t = blockIdx.x;
  const int j = threadIdx.x & (kLanesPerRow - 1);
  const int groups = blockDim.x / kLanesPerRow;
  const int R = a.num_q_heads + 2 * a.num_kv_heads;
  int64_t pos = a.positions[t];
  pos = pos < 0 ? 0 : (pos >= a.max_position ? a.max_position - 1 : pos);
  int32_t slot = a.slot_mapping != nullptr ? a.slot_mapping[t] : -1;
  if ((int64_t)slot >= a.cache_slots) slot = -1;
  const float* c = a.cos_sin + pos * a.cos_sin_stride + 8 * (j & 7);
  auto load_cs = [&](nvk_u32x4 (&cs)[4]) {
    cs[0] = *reinterpret_cast<const nvk_u32x4*>(c);
    cs[1] = *reinterpret_cast<const nvk_u32x4*>(c + 4);
    cs[2] = *reinterpret_cast<const nvk_u32x4*>(c + kHD / 2);
    cs[3] = *reinterpret_cast<const nvk_u32x4*>(c + kHD / 2 + 4);
  };
  const uint16_t* row0 = a.qkv + t * a.qkv_row_stride + 8 * j;
  const int g = threadIdx.x / kLanesPerRow;
  if (groups >= R) {  // one row per row group (small steps): only the loads it needs
    if (g >= R) return;
    const nvk_u32x4 raw = load_nt(row0 + (int64_t)g * kHD);
    const bool is_q = g < a.num_q_heads, is_k = !is_q && g < a.num_q_heads + a.num_kv_heads;
    nvk_u32x4 w = {0u, 0u, 0u, 0u}, cs[4] = {};
    if (is_q || is_k) {
      w = *reinterpret_cast<const nvk_u32x4*>((is_q ? a.q_weight : a.k_weight) + 8 * j);
      load_cs(cs);
    }
    prologue_row<F16>(a, t, g, j, slot, raw, w, w, cs);
    return;
  }
  nvk_u32x4 cs[4];
  load_cs(cs);
  const nvk_u32x4 wq = *reinterpret_cast<const nvk_u32x4*>(a.q_weight + 8 * j);
  const nvk_u32x4 wk = *reinterpret_cast<const nvk_u32x4*>(a.k_weight + 8 * j);
  auto pass = [&](int r0) {
    nvk_u32x4 raw[kRowsPerPass];
#pragma unroll
    for (int i = 0; i < kRowsPerPass; ++i) {
      const int r = r0 + i * groups;  // a row past R loads row r0 (< R) unused
      raw[i] = load_nt(row0 + (int64_t)(r < R ? r : r0) * kHD);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < kRowsPerPass; ++i) {
      const int r = r0 + i * groups;
      if (r < R) prologue_row<F16>(a, t, r, j, slot, raw[i], wq, wk, cs);
    }
  };
  if (R <= kRowsPerPass * groups) {  // one pass (Qwen3: 32 rows, 16 groups): no loop
    pass(g);
  } else {
    for (int r0 = g; r0 < R; r0 += kRowsPerPass * groups) pass(r0);
  }
}

}  // namespace

extern "C" int nvk_qk_norm_rope_store(
    const void* qkv, int64_t qkv_row_stride, int64_t n_tokens, const int64_t* positions,
    const void* q_norm_weight, const void* k_norm_weight, float eps, const float* cos_sin_cache,
    int64_t cos_sin_row_stride, int64_t max_position, int32_t num_q_heads, int32_t num_kv_heads,
    int32_t head_dim, void* q_out, int64_t q_out_stride_tok, int64_t q_out_stride_head, void* k_out,
    int64_t k_out_stride_tok, int64_t k_out_stride_head, void* k_cache, void* v_cache,
    const int32_t* slot_mapping, int64_t cache_slots, int32_t dtype, void* stream) {
  if (n_tokens < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || !(eps >= 0.f)) return NVK_EINVAL;
  if ((dtype != NVK_DTYPE_BF16 && dtype != NVK_DTYPE_F16) || head_dim != kHD)
    return NVK_EUNSUPPORTED;
  if (n_tokens == 0) return NVK_OK;
  if (!qkv || !positions || !q_norm_weight || !k_norm_weight || !cos_sin_cache || !q_out)
    return NVK_EINVAL;
  if (max_position <= 0 || cos_sin_row_stride < head_dim) return NVK_EINVAL;
  const int64_t R = (int64_t)num_q_heads + 2 * num_kv_heads;
  if (qkv_row_stride < R * head_dim) return NVK_EINVAL;
  if (q_out_stride_head < head_dim || q_out_stride_tok < (int64_t)num_q_heads * q_out_stride_head)
    return NVK_EINVAL;
  if (k_out && (k_out_stride_head < head_dim ||
                k_out_stride_tok < (int64_t)num_kv_heads * k_out_stride_head))
    return NVK_EINVAL;
  const bool store = slot_mapping != nullptr;
  if (store && (!k_cache || !v_cache || cache_slots < 0)) return NVK_EINVAL;
  // 16-byte vector access of every row and of the cos/sin rows.
  if (((uintptr_t)qkv | (uintptr_t)q_out | (uintptr_t)k_out | (uintptr_t)q_norm_weight |
       (uintptr_t)k_norm_weight | (uintptr_t)cos_sin_cache | (uintptr_t)k_cache |
       (uintptr_t)v_cache) % 16)
    return NVK_EALIGN;
  if ((qkv_row_stride % 8) || (q_out_stride_tok % 8) || (q_out_stride_head % 8) ||
      (k_out && ((k_out_stride_tok % 8) || (k_out_stride_head % 8))) || (cos_sin_row_stride % 4))
    return NVK_EALIGN;
  if (n_tokens > INT32_MAX || R > 65535) return NVK_EINVAL;
  const int max_groups = n_tokens <= kSmallTokens ? kMaxRowGroups : kMaxGroups;
  const int groups = R < max_groups ? (int)R : max_groups;

  PrologueArgs a;
  a.qkv = static_cast<const uint16_t*>(qkv);
  a.qkv_row_stride = qkv_row_stride;
  a.n_tokens = n_tokens;
  a.positions = positions;
  a.q_weight = static_cast<const uint16_t*>(q_norm_weight);
  a.k_weight = static_cast<const uint16_t*>(k_norm_weight);
  a.eps = eps;
  a.cos_sin = cos_sin_cache;
  a.cos_sin_stride = cos_sin_row_stride;
  a.max_position = max_position;
  a.num_q_heads = num_q_heads;
  a.num_kv_heads = num_kv_heads;
  a.q_out = static_cast<uint16_t*>(q_out);
  a.q_out_stride_tok = q_out_stride_tok;
  a.q_out_stride_head = q_out_stride_head;
  a.k_out = static_cast<uint16_t*>(k_out);
  a.k_out_stride_tok = k_out_stride_tok;
  a.k_out_stride_head = k_out_stride_head;
  a.k_cache = store ? static_cast<uint16_t*>(k_cache) : nullptr;
  a.v_cache = store ? static_cast<uint16_t*>(v_cache) : nullptr;
  a.slot_mapping = store ? slot_mapping : nullptr;
  a.cache_slots = cache_slots;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (dtype == NVK_DTYPE_F16)
    hipLaunchKernelGGL(qk_prologue_kernel<true>, dim3((unsigned)n_tokens),
                       dim3(groups * kLanesPerRow), 0, st, a);
  else
    hipLaunchKernelGGL(qk_prologue_kernel<false>, dim3((unsigned)n_tokens),
                       dim3(groups * kLanesPerRow), 0, st, a);
  return nvk_launch_status();
}
