// LM-head last-token gather and temperature sampler for gfx950.
//
// Gather (nanovllm/layers/embed_head.py:56-60): in a prefill step the LM head
// only needs the hidden state of each sequence's last new token,
//   out[b] = x[cu_seqlens_q[b+1] - 1],
// one 16-byte chunk of the row per thread.
//
// Sampler (nanovllm/layers/sampler.py:7-12):
//   probs = softmax(logits.float() / temperature[b]);
//   token = argmax_i probs_i / max(E_i, 1e-10),  E_i ~ Exp(1) i.i.d.
// This is the exponential race: the winner is distributed as probs.  The
// softmax normaliser is one positive constant per row and exp is monotone, so
//   argmax_i probs_i / E_i = argmax_i (logits_i / T - log E_i),
// which needs no max or sum pass: one read of the logits row.  The noise is
// either the caller's (E, float32 [B][V]: used as given, for reproducing a
// reference draw) or drawn in the kernel from Philox4x32-10 (Salmon, Moraes,
// Dror, Shaw, "Parallel random numbers: as easy as 1, 2, 3", SC'11) keyed by
// (seed) and counted by (offset, row, element / 4), E = -log(u) with u in
// (0, 1].  Ties go to the smallest index.
//
// Work split: a row is cut into chunks of 8192 elements, one 256-thread
// workgroup each (8 elements per thread per pass, 4 passes), so even a
// 64-row step fills the GPU; each workgroup leaves its (score, index) winner
// in the workspace and a second kernel (one wave per row) picks the row's
// winner.  The Philox draw (quarter-rate 32x32->64 multiplies) and the two
// log2 per element, not the logits read, bound the kernel.
#include "nvk_common.h"

namespace {

constexpr float kMinNoise = 1e-10f;  // clamp_min_(1e-10), sampler.py:11

// ---- Philox4x32-10 (constants from the SC'11 paper) -------------------------
struct U4 {
  uint32_t x, y, z, w;
};

// hi(p1) ^ c.y ^ k0 and hi(p0) ^ c.w ^ k1 as one three-input v_bitop3_b32 each
// (truth table 0x96 = a ^ b ^ c); the 32x32->64 products are v_mad_u64_u32.
__device__ __forceinline__ U4 philox_round(U4 c, uint32_t k0, uint32_t k1) {
  const uint64_t p0 = (uint64_t)0xD2511F53u * c.x;
  const uint64_t p1 = (uint64_t)0xCD9E8D57u * c.z;
  return U4{(uint32_t)__builtin_amdgcn_bitop3_b32((uint32_t)(p1 >> 32), c.y, k0, 0x96),
            (uint32_t)p1,
            (uint32_t)__builtin_amdgcn_bitop3_b32((uint32_t)(p0 >> 32), c.w, k1, 0x96),
            (uint32_t)p0};
}

__device__ __forceinline__ U4 philox10(U4 c, uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    c = philox_round(c, k0, k1);
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return c;
}

struct SampleArgs {
  const void* logits;
  int64_t row_stride;
  int vocab, chunks;
  int vec_ok;  // bf16 rows 16-byte aligned: 16-byte loads
  const float* temperatures;
  const float* noise;  // null: Philox
  int64_t noise_stride;
  uint64_t seed, offset;
  float* part_score;  // [batch][chunks]
  int* part_index;
  int64_t* tokens;
};

constexpr int kPartThreads = 256;
constexpr int kIters = 4;
constexpr int kChunk = kPartThreads * 8 * kIters;  // elements of a row per workgroup

// (s, i) beats (bs, bi): larger score, the smaller index on a tie.
__device__ __forceinline__ bool better(float s, int i, float bs, int bi) {
  return s > bs || (s == bs && i < bi);
}

template <typename T>
__device__ __forceinline__ void load8(const SampleArgs& a, int row, int base, bool full, float* l) {
  if constexpr (sizeof(T) == 2) {
    const uint16_t* p = static_cast<const uint16_t*>(a.logits) + (int64_t)row * a.row_stride + base;
    if (full && a.vec_ok) {
      const nvk_u32x4 w = *reinterpret_cast<const nvk_u32x4*>(p);
      const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        l[2 * i] = nvk_bf16lo_to_f32(ww[i]);
        l[2 * i + 1] = nvk_bf16hi_to_f32(ww[i]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        l[i] = (full || base + i < a.vocab) ? __uint_as_float((uint32_t)p[i] << 16) : -INFINITY;
    }
  } else {
    const float* p = static_cast<const float*>(a.logits) + (int64_t)row * a.row_stride + base;
#pragma unroll
    for (int i = 0; i < 8; ++i) l[i] = (full || base + i < a.vocab) ? p[i] : -INFINITY;
  }
}

// Scores of one row chunk in log2 units: logits * log2(e) / T - log2(E)
// (the base change and the constant log2(ln 2) of E = -ln u = -log2(u) ln 2
// are common to every element of the row and do not move the maximiser).
template <typename T, bool NOISE>
__global__ __launch_bounds__(kPartThreads) void sample_partial_kernel(SampleArgs a) {
  const int c = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
  const float scale = NVK_LOG2E / a.temperatures[row];
  const uint32_t k0 = (uint32_t)a.seed, k1 = (uint32_t)(a.seed >> 32);
  float best = -INFINITY;
  int best_i = 0x7fffffff;
#pragma unroll
  for (int it = 0; it < kIters; ++it) {
    const int base = c * kChunk + (it * kPartThreads + tid) * 8;
    if (base >= a.vocab) break;
    const bool full = base + 8 <= a.vocab;
    float l[8];
    load8<T>(a, row, base, full, l);
    float le[8];  // log2 of the noise
    if constexpr (NOISE) {
      const float* q = a.noise + (int64_t)row * a.noise_stride + base;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float e = (full || base + i < a.vocab) ? q[i] : 1.0f;
        le[i] = __builtin_amdgcn_logf(fmaxf(e, kMinNoise));
      }
    } else {
      const uint64_t ctr = a.offset + (uint64_t)(base >> 2);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const U4 r = philox10(U4{(uint32_t)(ctr + h), (uint32_t)((ctr + h) >> 32), (uint32_t)row, 0u},
                              k0, k1);
        const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          // u = (bits + 1) 2^-32 in (0, 1]; E / ln 2 = -log2(u), clamped like E >= 1e-10
          const float u = ((float)w[j] + 1.0f) * 2.3283064365386963e-10f;
          const float e2 = fmaxf(-__builtin_amdgcn_logf(u), kMinNoise * 1.4426950408889634f);
          le[4 * h + j] = __builtin_amdgcn_logf(e2);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float sc = l[i] * scale - le[i];
      // a thread visits its indices in increasing order: strictly greater wins
      if (sc > best && (full || base + i < a.vocab)) {
        best = sc;
        best_i = base + i;
      }
    }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const float os = __shfl_xor(best, m);
    const int oi = __shfl_xor(best_i, m);
    if (better(os, oi, best, best_i)) {
      best = os;
      best_i = oi;
    }
  }
  __shared__ float s_best[kPartThreads / 64];
  __shared__ int s_idx[kPartThreads / 64];
  if ((tid & 63) == 0) {
    s_best[tid >> 6] = best;
    s_idx[tid >> 6] = best_i;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < kPartThreads / 64; ++w)
      if (better(s_best[w], s_idx[w], best, best_i)) {
        best = s_best[w];
        best_i = s_idx[w];
      }
    a.part_score[(int64_t)row * a.chunks + c] = best;
    a.part_index[(int64_t)row * a.chunks + c] = best_i;
  }
}

// One wave per row: the best of the row's chunk winners.
__global__ __launch_bounds__(256) void sample_final_kernel(SampleArgs a, int batch) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= batch) return;
  float best = -INFINITY;
  int best_i = 0x7fffffff;
  for (int c = lane; c < a.chunks; c += 64) {
    const float s = a.part_score[(int64_t)row * a.chunks + c];
    const int i = a.part_index[(int64_t)row * a.chunks + c];
    if (better(s, i, best, best_i)) {
      best = s;
      best_i = i;
    }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const float os = __shfl_xor(best, m);
    const int oi = __shfl_xor(best_i, m);
    if (better(os, oi, best, best_i)) {
      best = os;
      best_i = oi;
    }
  }
  // every score NaN (NaN logits): token 0
  if (lane == 0) a.tokens[row] = best_i == 0x7fffffff ? 0 : best_i;
}

struct GatherArgs {
  const uint16_t* x;
  int64_t x_row_stride;
  const int32_t* cu_seqlens_q;
  int batch, row_chunks;  // 16-byte chunks per row
  uint16_t* out;
  int64_t out_row_stride;
};

__global__ __launch_bounds__(256) void gather_last_kernel(GatherArgs a) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= (int64_t)a.batch * a.row_chunks) return;
  const int b = (int)(e / a.row_chunks), c = (int)(e - (int64_t)b * a.row_chunks);
  const int src = a.cu_seqlens_q[b + 1] - 1;
  if (src < 0) return;  // empty sequence: its row is left as it was
  *reinterpret_cast<nvk_u32x4*>(a.out + (int64_t)b * a.out_row_stride + 8 * c) =
      *reinterpret_cast<const nvk_u32x4*>(a.x + (int64_t)src * a.x_row_stride + 8 * c);
}

}  // namespace

extern "C" size_t nvk_sample_workspace_size(int32_t batch, int32_t vocab) {
  if (batch <= 0 || vocab <= 0) return 0;
  const size_t chunks = ((size_t)vocab + kChunk - 1) / kChunk;
  return (size_t)batch * chunks * 8;
}

extern "C" int nvk_sample(const void* logits, int64_t row_stride, int32_t batch, int32_t vocab,
                          int32_t dtype, const float* temperatures, const float* noise,
                          int64_t noise_row_stride, uint64_t seed, uint64_t offset,
                          int64_t* tokens, void* workspace, size_t workspace_bytes,
                          void* stream) {
  if (batch < 0 || vocab <= 0 || row_stride < vocab) return NVK_EINVAL;
  if (dtype != NVK_DTYPE_BF16 && dtype != NVK_DTYPE_F32) return NVK_EUNSUPPORTED;
  if (batch == 0) return NVK_OK;
  if (batch > 65535) return NVK_EUNSUPPORTED;
  if (!logits || !temperatures || !tokens) return NVK_EINVAL;
  if (noise && noise_row_stride < vocab) return NVK_EINVAL;
  const size_t need = nvk_sample_workspace_size(batch, vocab);
  if (!workspace || workspace_bytes < need) return NVK_EWORKSPACE;
  if ((uintptr_t)workspace % 16) return NVK_EALIGN;
  SampleArgs a;
  a.logits = logits;
  a.row_stride = row_stride;
  a.vocab = vocab;
  a.chunks = (vocab + kChunk - 1) / kChunk;
  a.vec_ok = ((uintptr_t)logits % 16) == 0 && (row_stride % 8) == 0;
  a.temperatures = temperatures;
  a.noise = noise;
  a.noise_stride = noise_row_stride;
  a.seed = seed;
  a.offset = offset;
  a.part_score = static_cast<float*>(workspace);
  a.part_index = reinterpret_cast<int*>(static_cast<char*>(workspace) + need / 2);
  a.tokens = tokens;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid(a.chunks, batch);
  const bool bf16 = dtype == NVK_DTYPE_BF16;
  if (bf16 && noise)
    hipLaunchKernelGGL((sample_partial_kernel<uint16_t, true>), grid, dim3(kPartThreads), 0, s, a);
  else if (bf16)
    hipLaunchKernelGGL((sample_partial_kernel<uint16_t, false>), grid, dim3(kPartThreads), 0, s, a);
  else if (noise)
    hipLaunchKernelGGL((sample_partial_kernel<float, true>), grid, dim3(kPartThreads), 0, s, a);
  else
    hipLaunchKernelGGL((sample_partial_kernel<float, false>), grid, dim3(kPartThreads), 0, s, a);
  int st = nvk_launch_status();
  if (st != NVK_OK) return st;
  hipLaunchKernelGGL(sample_final_kernel, dim3((batch + 3) / 4), dim3(256), 0, s, a, batch);
  return nvk_launch_status();
}

extern "C" int nvk_gather_last_tokens(const void* x, int64_t x_row_stride,
                                      const int32_t* cu_seqlens_q, int32_t batch, int32_t hidden,
                                      int32_t dtype, void* out, int64_t out_row_stride,
                                      void* stream) {
  if (batch < 0 || hidden <= 0 || x_row_stride < hidden || out_row_stride < hidden)
    return NVK_EINVAL;
  if (dtype != NVK_DTYPE_BF16) return NVK_EUNSUPPORTED;
  if (batch == 0) return NVK_OK;
  if (!x || !cu_seqlens_q || !out) return NVK_EINVAL;
  if (((uintptr_t)x | (uintptr_t)out) % 16 || (hidden % 8) || (x_row_stride % 8) ||
      (out_row_stride % 8))
    return NVK_EALIGN;
  GatherArgs a;
  a.x = static_cast<const uint16_t*>(x);
  a.x_row_stride = x_row_stride;
  a.cu_seqlens_q = cu_seqlens_q;
  a.batch = batch;
  a.row_chunks = hidden / 8;
  a.out = static_cast<uint16_t*>(out);
  a.out_row_stride = out_row_stride;
  const int64_t n = (int64_t)batch * a.row_chunks;
  hipLaunchKernelGGL(gather_last_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), a);
  return nvk_launch_status();
}
