// KV-store scatter: the slot_mapping copy of new key/value rows into the
// paged cache.  Same semantics as store_kvcache_kernel
// (nanovllm/layers/attention.py:10-30): slot -1 skips the token, otherwise
// the token's K row and V row are copied to row `slot` of the flat cache.
//
// Mapping (MI355X): the work is a pure HBM copy of 2 * row_bytes per valid
// token.  One thread owns one VEC-byte chunk at the same offset of the K row
// and of the V row of U tokens (U = 1, 2, 4 or 8), so each thread has 2U
// independent loads in flight before its 2U stores; a 256-thread workgroup
// covers U * 256/chunks_per_row whole tokens.  U is the smallest that keeps
// the grid within about one round of two workgroups per CU (512 on the 256
// CUs of an MI355X): the 4096-token layer step runs 512 workgroups of 4
// tokens per thread.  The rows are loaded whatever their slot, so that no
// load waits for the slot's (a token whose slot is -1 is read and not
// written).  Every input row is read once and every cache row written once
// per step, so loads and stores are non-temporal.
// Measured on the 4096-token step with inputs and caches cycling through more
// than the 256 MB Infinity Cache (interleaved A/B, same process, bit-identical
// caches): rows loaded after the slot, 1024 workgroups of 2 tokens per thread
// 8.24 us; rows loaded with the slot: 1024 x 2 tokens 7.40 us, 2048 x 1
// 7.81 us, 683 x 3 7.56 us, 512 x 4 6.33 us, 342 x 6 7.67 us, 256 x 8 6.57 us.
// (Earlier, rows after the slot: cached loads and stores 9.05 us against
// 7.96 us non-temporal.)
#include "nvk_common.h"

namespace {

constexpr int kStoreWGs = 640;  // 512 workgroup slots (256 CUs x 2) + 25 %

// Non-temporal 2-, 4- and 16-byte accesses.  Stores go through a by-value
// copy: indexing the destination with the element of a private array directly
// lets the compiler promote the whole array to LDS (16 KiB per workgroup for
// 16-byte chunks), which halves occupancy.
template <typename T>
__device__ __forceinline__ void store_chunk(T v, T* p) {
  if constexpr (sizeof(T) == 16)
    __builtin_nontemporal_store(__builtin_bit_cast(nvk_u32x4, v), reinterpret_cast<nvk_u32x4*>(p));
  else
    __builtin_nontemporal_store(v, p);
}
template <typename T>
__device__ __forceinline__ T load_chunk(const T* p) {
  if constexpr (sizeof(T) == 16)
    return __builtin_bit_cast(T, __builtin_nontemporal_load(reinterpret_cast<const nvk_u32x4*>(p)));
  else
    return __builtin_nontemporal_load(p);
}

template <typename VecT, int U>
__global__ __launch_bounds__(256) void kv_store_rows_kernel(
    const char* __restrict__ key, int64_t key_stride_bytes,
    const char* __restrict__ value, int64_t value_stride_bytes,
    char* __restrict__ k_cache, char* __restrict__ v_cache,
    const int32_t* __restrict__ slot_mapping, int64_t n_tokens,
    int64_t row_bytes, int chunk_shift, int64_t cache_slots) {
  // chunk_shift = log2(chunks_per_row); a pass covers 256 >> chunk_shift tokens
  // and a workgroup U passes.
  const int tid = threadIdx.x;
  const int per_pass = 256 >> chunk_shift;
  const int chunk = tid & ((1 << chunk_shift) - 1);
  VecT kx[U], vx[U];
  int32_t sl[U];
  int64_t tk[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    tk[u] = ((int64_t)blockIdx.x * U + u) * per_pass + (tid >> chunk_shift);
    sl[u] = tk[u] < n_tokens ? slot_mapping[tk[u]] : -1;
    if (tk[u] < n_tokens) {  // whatever the slot: the loads do not wait for it
      kx[u] = load_chunk(reinterpret_cast<const VecT*>(key + tk[u] * key_stride_bytes) + chunk);
      vx[u] = load_chunk(reinterpret_cast<const VecT*>(value + tk[u] * value_stride_bytes) + chunk);
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (sl[u] >= 0 && (int64_t)sl[u] < cache_slots) {
      const int64_t dst = (int64_t)sl[u] * row_bytes;
      store_chunk(kx[u], reinterpret_cast<VecT*>(k_cache + dst) + chunk);
      store_chunk(vx[u], reinterpret_cast<VecT*>(v_cache + dst) + chunk);
    }
  }
}

// Any row size: one workgroup per token, threads stride over the row's chunks.
template <typename VecT>
__global__ __launch_bounds__(256) void kv_store_generic_kernel(
    const char* __restrict__ key, int64_t key_stride_bytes,
    const char* __restrict__ value, int64_t value_stride_bytes,
    char* __restrict__ k_cache, char* __restrict__ v_cache,
    const int32_t* __restrict__ slot_mapping, int64_t n_tokens,
    int64_t row_bytes, int64_t cache_slots) {
  const int64_t token = blockIdx.x;
  if (token >= n_tokens) return;
  const int32_t slot = slot_mapping[token];
  if (slot < 0 || (int64_t)slot >= cache_slots) return;
  const int64_t nchunks = row_bytes / (int64_t)sizeof(VecT);
  const VecT* ks = reinterpret_cast<const VecT*>(key + token * key_stride_bytes);
  const VecT* vs = reinterpret_cast<const VecT*>(value + token * value_stride_bytes);
  VecT* kd = reinterpret_cast<VecT*>(k_cache + (int64_t)slot * row_bytes);
  VecT* vd = reinterpret_cast<VecT*>(v_cache + (int64_t)slot * row_bytes);
  for (int64_t c = threadIdx.x; c < nchunks; c += blockDim.x) {
    const VecT kx = ks[c];
    const VecT vx = vs[c];
    kd[c] = kx;
    vd[c] = vx;
  }
}

inline bool aligned_to(const void* p, int64_t a) { return ((uintptr_t)p % (uintptr_t)a) == 0; }

template <typename VecT>
int launch_kv_store(const char* key, int64_t ksb, const char* value, int64_t vsb, char* kc,
                    char* vc, const int32_t* slots, int64_t n_tokens, int64_t row_bytes,
                    int64_t cache_slots, hipStream_t stream) {
  const int64_t cpr = row_bytes / (int64_t)sizeof(VecT);
  const int shift = nvk_log2_exact((int)(cpr <= 256 ? cpr : 0));
  if (shift >= 0) {
    const int64_t per_pass = 256 >> shift;
    auto grid_of = [&](int u) { return (n_tokens + per_pass * u - 1) / (per_pass * u); };
    auto launch = [&](auto kernel, int u) {
      hipLaunchKernelGGL(kernel, dim3((unsigned)grid_of(u)), dim3(256), 0, stream, key, ksb, value,
                         vsb, kc, vc, slots, n_tokens, row_bytes, shift, cache_slots);
    };
    if (grid_of(1) <= kStoreWGs) launch(kv_store_rows_kernel<VecT, 1>, 1);
    else if (grid_of(2) <= kStoreWGs) launch(kv_store_rows_kernel<VecT, 2>, 2);
    else if (grid_of(4) <= kStoreWGs) launch(kv_store_rows_kernel<VecT, 4>, 4);
    else launch(kv_store_rows_kernel<VecT, 8>, 8);
  } else {
    hipLaunchKernelGGL(kv_store_generic_kernel<VecT>, dim3((unsigned)n_tokens), dim3(256), 0,
                       stream, key, ksb, value, vsb, kc, vc, slots, n_tokens, row_bytes,
                       cache_slots);
  }
  return nvk_launch_status();
}

}  // namespace

extern "C" int nvk_kv_store(const void* key, int64_t key_row_stride, const void* value,
                            int64_t value_row_stride, void* k_cache, void* v_cache,
                            const int32_t* slot_mapping, int64_t n_tokens, int32_t row_elems,
                            int32_t elem_bytes, int64_t cache_slots, void* stream) {
  if (n_tokens < 0 || row_elems <= 0 || cache_slots < 0) return NVK_EINVAL;
  if (elem_bytes != 2 && elem_bytes != 4) return NVK_EUNSUPPORTED;
  if (n_tokens == 0) return NVK_OK;
  if (!key || !value || !k_cache || !v_cache || !slot_mapping) return NVK_EINVAL;
  if (key_row_stride < row_elems || value_row_stride < row_elems) return NVK_EINVAL;
  if (n_tokens > (int64_t)INT32_MAX) return NVK_EINVAL;
  if (!aligned_to(slot_mapping, 4)) return NVK_EALIGN;

  const int64_t row_bytes = (int64_t)row_elems * elem_bytes;
  const int64_t ksb = key_row_stride * elem_bytes;
  const int64_t vsb = value_row_stride * elem_bytes;
  auto fits = [&](int64_t a) {
    return row_bytes % a == 0 && ksb % a == 0 && vsb % a == 0 && aligned_to(key, a) &&
           aligned_to(value, a) && aligned_to(k_cache, a) && aligned_to(v_cache, a);
  };
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const char* kp = static_cast<const char*>(key);
  const char* vp = static_cast<const char*>(value);
  char* kcp = static_cast<char*>(k_cache);
  char* vcp = static_cast<char*>(v_cache);
  if (fits(16))
    return launch_kv_store<uint4>(kp, ksb, vp, vsb, kcp, vcp, slot_mapping, n_tokens, row_bytes,
                                  cache_slots, s);
  if (fits(4))
    return launch_kv_store<uint32_t>(kp, ksb, vp, vsb, kcp, vcp, slot_mapping, n_tokens,
                                     row_bytes, cache_slots, s);
  if (fits(2))
    return launch_kv_store<uint16_t>(kp, ksb, vp, vsb, kcp, vcp, slot_mapping, n_tokens,
                                     row_bytes, cache_slots, s);
  return NVK_EALIGN;
}

extern "C" const char* nvk_strerror(int code) {
  switch (code) {
    case NVK_OK: return "ok";
    case NVK_EINVAL: return "nvk: invalid argument (null pointer, negative size or inconsistent shape)";
    case NVK_EUNSUPPORTED: return "nvk: unsupported head_dim / group size / dtype";
    case NVK_EALIGN: return "nvk: pointer or stride misaligned for the element type";
    case NVK_EWORKSPACE: return "nvk: workspace missing or too small";
    case NVK_ESCRATCH:
      return "nvk: these sizes need more than the static scratch of the no-allocation entry "
             "point (NVK_NOALLOC_SCRATCH_BYTES); use the entry point with a workspace";
    default: break;
  }
  if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
  return "nvk: unknown error";
}

extern "C" const char* nvk_build_target(void) { return "gfx950"; }
