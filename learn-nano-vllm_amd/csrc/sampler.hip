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
// log2 per element, not the logits read, bound the kernel.  So for large
// steps (batch x vocab >= 2^24) without the caller's noise, the draw is an
// inverse-CDF one instead (two uniforms per row; see sample_mass_kernel).
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

constexpr int64_t kCdfMinElements = int64_t{1} << 24;  // batch x vocab for the inverse-CDF path
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

// log2 of the exponential noise E of elements base .. base+7 of a row: from
// the caller's draw e[0..7] (NOISE), or from Philox at counter (offset +
// base/4 + h, row) for h = 0, 1.
template <bool NOISE>
__device__ __forceinline__ void noise_log2(const SampleArgs& a, int row, int base, const float* e,
                                           float* le) {
  if constexpr (NOISE) {
#pragma unroll
    for (int i = 0; i < 8; ++i) le[i] = __builtin_amdgcn_logf(fmaxf(e[i], kMinNoise));
  } else {
    const uint32_t k0 = (uint32_t)a.seed, k1 = (uint32_t)(a.seed >> 32);
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
}

// Scores of one row chunk in log2 units: logits * log2(e) / T - log2(E)
// (the base change and the constant log2(ln 2) of E = -ln u = -log2(u) ln 2
// are common to every element of the row and do not move the maximiser).
template <typename T, bool NOISE>
__global__ __launch_bounds__(kPartThreads) void sample_partial_kernel(SampleArgs a) {
  const int c = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
  const float scale = NVK_LOG2E / a.temperatures[row];
  float best = -INFINITY;
  int best_i = 0x7fffffff;
  if (sizeof(T) == 2 && a.vec_ok && (int64_t)(c + 1) * kChunk <= a.vocab) {
    // a whole chunk of bf16: its logits (and the caller's noise) are all
    // loaded before the first wait, so the loads overlap the Philox draw
    const int64_t off = (int64_t)c * kChunk + tid * 8;
    const uint16_t* p = static_cast<const uint16_t*>(a.logits) + (int64_t)row * a.row_stride + off;
    nvk_u32x4 w[kIters];
#pragma unroll
    for (int it = 0; it < kIters; ++it)
      w[it] = *reinterpret_cast<const nvk_u32x4*>(p + it * kPartThreads * 8);
    float nz[NOISE ? kIters : 1][8];
    if constexpr (NOISE) {
      const float* q = a.noise + (int64_t)row * a.noise_stride + off;
#pragma unroll
      for (int it = 0; it < kIters; ++it)
#pragma unroll
        for (int i = 0; i < 8; ++i) nz[it][i] = q[it * kPartThreads * 8 + i];
    }
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
      const int base = c * kChunk + (it * kPartThreads + tid) * 8;
      float le[8];
      noise_log2<NOISE>(a, row, base, nz[NOISE ? it : 0], le);
      const uint32_t ww[4] = {w[it].x, w[it].y, w[it].z, w[it].w};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float l = (i & 1) ? nvk_bf16hi_to_f32(ww[i >> 1]) : nvk_bf16lo_to_f32(ww[i >> 1]);
        const float sc = l * scale - le[i];
        // a thread visits its indices in increasing order: strictly greater wins
        if (sc > best) {
          best = sc;
          best_i = base + i;
        }
      }
    }
  } else {
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
      const int base = c * kChunk + (it * kPartThreads + tid) * 8;
      if (base >= a.vocab) break;
      const bool full = base + 8 <= a.vocab;
      float l[8];
      load8<T>(a, row, base, full, l);
      float e[8];
      if constexpr (NOISE) {
        const float* q = a.noise + (int64_t)row * a.noise_stride + base;
#pragma unroll
        for (int i = 0; i < 8; ++i) e[i] = (full || base + i < a.vocab) ? q[i] : 1.0f;
      }
      float le[8];
      noise_log2<NOISE>(a, row, base, e, le);
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

// ---- the kernel's own randomness: inverse-CDF sampling ----------------------
// Without the caller's noise the token is drawn by inverse transform over the
// row's softmax, with two uniforms per row instead of one exponential per
// element (the Philox draw per element, not the logits read, bounded the
// race): the mass kernel reduces every chunk of the row to its maximum M_c of
// x_i = logits_i * log2(e) / T and S_c = sum_i 2^(x_i - M_c); the pick kernel
// draws (u1, u2) from Philox4x32-10 keyed by (seed) at counter (offset, row),
// selects chunk c with probability S_c 2^(M_c - M) / sum, then the first index
// of that chunk whose running sum of 2^(x_i - M_c) reaches u2 S_c.  A token is
// drawn with probability p_i up to float32 rounding of the running sums (a
// token with less than ~2^-24 of its chunk's mass is not drawn).  Rows with no
// finite score give token 0, as in the race.

// x of one element (non-finite logits: -inf, no mass)
__device__ __forceinline__ float mass_x(float l, float scale) {
  const float x = l * scale;
  return (x == x && x != INFINITY) ? x : -INFINITY;
}

__device__ __forceinline__ float block_max256(float v, float* red) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m));
  const int tid = threadIdx.x;
  __syncthreads();
  if ((tid & 63) == 0) red[tid >> 6] = v;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}
__device__ __forceinline__ float block_sum256(float v, float* red) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
  const int tid = threadIdx.x;
  __syncthreads();
  if ((tid & 63) == 0) red[tid >> 6] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}
// Exclusive prefix of v over the 256 threads (in thread order); *total = sum.
__device__ __forceinline__ float block_excl256(float v, float* red, float* total) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  float x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  __syncthreads();
  if (lane == 63) red[w] = x;
  __syncthreads();
  float before = 0.f;
  for (int i = 0; i < w; ++i) before += red[i];
  *total = (red[0] + red[1]) + (red[2] + red[3]);
  return before + x - v;
}

template <typename T>
__global__ __launch_bounds__(kPartThreads) void sample_mass_kernel(SampleArgs a) {
  static_assert(kPartThreads == 256, "block reductions assume 256 threads");
  const int c = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
  __shared__ float red[4];
  const float scale = NVK_LOG2E / a.temperatures[row];
  float x[kIters][8];
  float mx = -INFINITY;
  if (sizeof(T) == 2 && a.vec_ok && (int64_t)(c + 1) * kChunk <= a.vocab) {
    // a whole chunk of bf16: the kIters 16-byte loads all leave before the
    // first wait (the loop below waits for each in turn)
    const uint16_t* p = static_cast<const uint16_t*>(a.logits) + (int64_t)row * a.row_stride +
                        c * kChunk + tid * 8;
    nvk_u32x4 w[kIters];
#pragma unroll
    for (int it = 0; it < kIters; ++it)
      w[it] = *reinterpret_cast<const nvk_u32x4*>(p + it * kPartThreads * 8);
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
      const uint32_t ww[4] = {w[it].x, w[it].y, w[it].z, w[it].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        x[it][2 * i] = mass_x(nvk_bf16lo_to_f32(ww[i]), scale);
        x[it][2 * i + 1] = mass_x(nvk_bf16hi_to_f32(ww[i]), scale);
        mx = fmaxf(mx, fmaxf(x[it][2 * i], x[it][2 * i + 1]));
      }
    }
  } else {
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
      const int base = c * kChunk + (it * kPartThreads + tid) * 8;
      float l[8];
      if (base < a.vocab) {
        load8<T>(a, row, base, base + 8 <= a.vocab, l);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) l[i] = -INFINITY;
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        x[it][i] = mass_x(l[i], scale);
        mx = fmaxf(mx, x[it][i]);
      }
    }
  }
  const float M = block_max256(mx, red);
  float sum = 0.f;
  if (M != -INFINITY) {
#pragma unroll
    for (int it = 0; it < kIters; ++it)
#pragma unroll
      for (int i = 0; i < 8; ++i) sum += exp2f(x[it][i] - M);
  }
  const float S = block_sum256(sum, red);
  if (tid == 0) {
    a.part_score[(int64_t)row * a.chunks + c] = M;
    reinterpret_cast<float*>(a.part_index)[(int64_t)row * a.chunks + c] = S;
  }
}

template <typename T>
__global__ __launch_bounds__(256) void sample_pick_kernel(SampleArgs a) {
  const int row = blockIdx.x, tid = threadIdx.x;
  __shared__ float red[4];
  const float* pm = a.part_score + (int64_t)row * a.chunks;
  const float* ps = reinterpret_cast<const float*>(a.part_index) + (int64_t)row * a.chunks;
  float m = -INFINITY;
  for (int c = tid; c < a.chunks; c += 256) m = fmaxf(m, pm[c]);
  const float Mg = block_max256(m, red);
  if (Mg == -INFINITY) {  // no finite score in the row
    if (tid == 0) a.tokens[row] = 0;
    return;
  }
  auto weight = [&](int c) { return c < a.chunks && pm[c] != -INFINITY ? ps[c] * exp2f(pm[c] - Mg) : 0.f; };
  float wsum = 0.f;
  for (int c = tid; c < a.chunks; c += 256) wsum += weight(c);
  const float W = block_sum256(wsum, red);
  // two uniforms in (0, 1] for this row and call
  const U4 r = philox10(U4{(uint32_t)a.offset, (uint32_t)(a.offset >> 32), (uint32_t)row, 1u},
                        (uint32_t)a.seed, (uint32_t)(a.seed >> 32));
  const float u1 = ((float)r.x + 1.0f) * 2.3283064365386963e-10f;
  const float u2 = ((float)r.y + 1.0f) * 2.3283064365386963e-10f;
  // chunk: the first whose running weight reaches u1 W (rounding: the last with weight)
  const float t1 = u1 * W;
  float run = 0.f;
  int pick = a.chunks, last_pos = -1;
  for (int base = 0; base < a.chunks; base += 256) {
    const int c = base + tid;
    const float wc = weight(c);
    float tot;
    const float ex = block_excl256(wc, red, &tot);
    const int hit = (wc > 0.f && run + ex + wc >= t1) ? c : a.chunks;
    const int lp = wc > 0.f ? c : -1;
    // smallest hit and largest positive chunk over the block
    int h = hit, l = lp;
#pragma unroll
    for (int mm = 32; mm >= 1; mm >>= 1) {
      h = min(h, __shfl_xor(h, mm));
      l = max(l, __shfl_xor(l, mm));
    }
    __shared__ int s_h[4], s_l[4];
    __syncthreads();
    if ((tid & 63) == 0) { s_h[tid >> 6] = h; s_l[tid >> 6] = l; }
    __syncthreads();
    pick = min(pick, min(min(s_h[0], s_h[1]), min(s_h[2], s_h[3])));
    last_pos = max(last_pos, max(max(s_l[0], s_l[1]), max(s_l[2], s_l[3])));
    run += tot;
  }
  if (pick >= a.chunks) pick = last_pos;
  // element: the first of the chunk whose running mass reaches u2 S_c
  const float Mc = pm[pick];
  const float t2 = u2 * ps[pick];
  const float scale = NVK_LOG2E / a.temperatures[row];
  float e[32];  // the thread's 32 elements, in index order
  float tsum = 0.f;
  const int first = pick * kChunk + 32 * tid;
  if (sizeof(T) == 2 && a.vec_ok && first + 32 <= a.vocab) {
    // 64 bf16 bytes: the four 16-byte loads leave before the first wait
    const uint16_t* p = static_cast<const uint16_t*>(a.logits) + (int64_t)row * a.row_stride + first;
    nvk_u32x4 w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j] = *reinterpret_cast<const nvk_u32x4*>(p + 8 * j);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t ww[4] = {w[j].x, w[j].y, w[j].z, w[j].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        e[8 * j + 2 * i] = exp2f(mass_x(nvk_bf16lo_to_f32(ww[i]), scale) - Mc);
        e[8 * j + 2 * i + 1] = exp2f(mass_x(nvk_bf16hi_to_f32(ww[i]), scale) - Mc);
        tsum += e[8 * j + 2 * i];
        tsum += e[8 * j + 2 * i + 1];
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int base = first + 8 * j;
      float l[8];
      if (base < a.vocab) {
        load8<T>(a, row, base, base + 8 <= a.vocab, l);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) l[i] = -INFINITY;
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        e[8 * j + i] = exp2f(mass_x(l[i], scale) - Mc);
        tsum += e[8 * j + i];
      }
    }
  }
  float tot;
  const float ex = block_excl256(tsum, red, &tot);
  int found = a.vocab, lastpos = -1;
  for (int i = 31; i >= 0; --i)
    if (e[i] > 0.f) { lastpos = first + i; break; }
  if (tsum > 0.f && ex < t2 && t2 <= ex + tsum) {  // the target falls in this thread's run
    float cum = ex;
    found = lastpos;  // if rounding keeps the running sum below the target
    for (int i = 0; i < 32; ++i) {
      cum += e[i];
      if (e[i] > 0.f && cum >= t2) { found = first + i; break; }
    }
  }
  int fnd = found, lst = lastpos;
#pragma unroll
  for (int mm = 32; mm >= 1; mm >>= 1) {
    fnd = min(fnd, __shfl_xor(fnd, mm));
    lst = max(lst, __shfl_xor(lst, mm));
  }
  __shared__ int s_f[4], s_ls[4];
  __syncthreads();
  if ((tid & 63) == 0) { s_f[tid >> 6] = fnd; s_ls[tid >> 6] = lst; }
  __syncthreads();
  if (tid == 0) {
    int tok = min(min(s_f[0], s_f[1]), min(s_f[2], s_f[3]));
    if (tok >= a.vocab) tok = max(max(s_ls[0], s_ls[1]), max(s_ls[2], s_ls[3]));
    a.tokens[row] = tok < 0 ? 0 : tok;
  }
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
  // The kernel's own randomness: the exponential race for small steps (one
  // pass, its Philox draws per element cheap enough), inverse-CDF over the
  // chunk masses for large ones (two draws per row; its pick kernel adds a
  // fixed ~8 us).  Measured on MI355X, vocab 151936: B = 64 race 14.8 us,
  // inverse-CDF 16.8 us; B = 512 race 58.5 us, inverse-CDF 45.4 us.
  if (!noise && (int64_t)batch * vocab >= kCdfMinElements) {
    if (bf16) hipLaunchKernelGGL((sample_mass_kernel<uint16_t>), grid, dim3(kPartThreads), 0, s, a);
    else hipLaunchKernelGGL((sample_mass_kernel<float>), grid, dim3(kPartThreads), 0, s, a);
    int st = nvk_launch_status();
    if (st != NVK_OK) return st;
    if (bf16) hipLaunchKernelGGL((sample_pick_kernel<uint16_t>), dim3(batch), dim3(256), 0, s, a);
    else hipLaunchKernelGGL((sample_pick_kernel<float>), dim3(batch), dim3(256), 0, s, a);
    return nvk_launch_status();
  }
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
