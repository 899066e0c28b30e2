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
// This is the exponential race: the winner is distributed as probs.
// * With the caller's noise (E, float32 [B][V]: used as given, for
//   reproducing a reference draw) the race itself is evaluated: the softmax
//   normaliser is one positive constant per row and exp is monotone, so
//     argmax_i probs_i / E_i = argmax_i (logits_i / T - log E_i),
//   which needs no max or sum pass: one read of the logits and the noise.
//   Ties go to the smallest index.  A row is cut into chunks of 8192
//   elements, one 256-thread workgroup each (8 elements per thread per pass,
//   4 passes), so even a 64-row step fills the GPU; each workgroup leaves its
//   (score, index) winner in the workspace and a second kernel (one wave per
//   row) picks the row's winner.
// * Without it the kernel draws from the same distribution by inverse
//   transform (sample_draw_kernel): uniforms from Philox4x32-10 (Salmon,
//   Moraes, Dror, Shaw, "Parallel random numbers: as easy as 1, 2, 3", SC'11)
//   keyed by (seed), two per 2048 logits and one per row, instead of one
//   exponential per element (whose Philox draw and logarithms, not the
//   logits read, bounded the race).
#include "nvk_common.h"

namespace {

constexpr float kMinNoise = 1e-10f;  // clamp_min_(1e-10), sampler.py:11

// Philox4x32-10 counter and output block (the rounds: row_uniforms)
struct U4 {
  uint32_t x, y, z, w;
};

struct SampleArgs {
  const void* logits;
  int64_t row_stride;
  int vocab, chunks;
  int vec_ok;  // bf16 rows 16-byte aligned: 16-byte loads
  const float* temperatures;
  const float* noise;  // null: the kernel's own draw (Philox)
  int64_t noise_stride;
  uint64_t seed, offset;
  // per workgroup chunk [batch][chunks] (race) or wave chunk [batch][4 chunks] (draw):
  float* part_score;  // the best score, or M_w
  int* part_index;    // the best index, or S_w (float bits)
  int* part_token;    // the wave chunk's drawn token (draw only)
  int64_t* tokens;
};

constexpr int kPartThreads = 256;
constexpr int kIters = 4;
constexpr int kChunk = kPartThreads * 8 * kIters;  // elements of a row per workgroup

// (s, i) beats (bs, bi): larger score, the smaller index on a tie.
__device__ __forceinline__ bool better(float s, int i, float bs, int bi) {
  return s > bs || (s == bs && i < bi);
}

// Logits of T = uint16_t (bf16, or f16 when F16) or float.
template <typename T, bool F16>
__device__ __forceinline__ void load8(const SampleArgs& a, int row, int base, bool full, float* l) {
  if constexpr (sizeof(T) == 2) {
    const uint16_t* p = static_cast<const uint16_t*>(a.logits) + (int64_t)row * a.row_stride + base;
    if (full && a.vec_ok) {
      const nvk_u32x4 w = *reinterpret_cast<const nvk_u32x4*>(p);
      const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        l[2 * i] = NvkElt<F16>::lo(ww[i]);
        l[2 * i + 1] = NvkElt<F16>::hi(ww[i]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        l[i] = (full || base + i < a.vocab) ? NvkElt<F16>::lo((uint32_t)p[i]) : -INFINITY;
    }
  } else {
    const float* p = static_cast<const float*>(a.logits) + (int64_t)row * a.row_stride + base;
#pragma unroll
    for (int i = 0; i < 8; ++i) l[i] = (full || base + i < a.vocab) ? p[i] : -INFINITY;
  }
}

// Race scores of one row chunk in log2 units: logits * log2(e) / T - log2(E),
// E = max(noise, 1e-10) (the base change does not move the maximiser).
template <typename T, bool F16>
__global__ __launch_bounds__(kPartThreads) void sample_partial_kernel(SampleArgs a) {
  const int c = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
  const float scale = NVK_LOG2E / a.temperatures[row];
  float best = -INFINITY;
  int best_i = 0x7fffffff;
  if (sizeof(T) == 2 && a.vec_ok && (int64_t)(c + 1) * kChunk <= a.vocab) {
    // a whole chunk of bf16: its logits and noise are all loaded before the
    // first wait
    const int64_t off = (int64_t)c * kChunk + tid * 8;
    const uint16_t* p = static_cast<const uint16_t*>(a.logits) + (int64_t)row * a.row_stride + off;
    nvk_u32x4 w[kIters];
#pragma unroll
    for (int it = 0; it < kIters; ++it)
      w[it] = *reinterpret_cast<const nvk_u32x4*>(p + it * kPartThreads * 8);
    float nz[kIters][8];
    const float* q = a.noise + (int64_t)row * a.noise_stride + off;
#pragma unroll
    for (int it = 0; it < kIters; ++it)
#pragma unroll
      for (int i = 0; i < 8; ++i) nz[it][i] = q[it * kPartThreads * 8 + i];
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
      const int base = c * kChunk + (it * kPartThreads + tid) * 8;
      const uint32_t ww[4] = {w[it].x, w[it].y, w[it].z, w[it].w};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float l = (i & 1) ? NvkElt<F16>::hi(ww[i >> 1]) : NvkElt<F16>::lo(ww[i >> 1]);
        const float sc = l * scale - __builtin_amdgcn_logf(fmaxf(nz[it][i], kMinNoise));
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
      load8<T, F16>(a, row, base, full, l);
      const float* q = a.noise + (int64_t)row * a.noise_stride + base;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float e = (full || base + i < a.vocab) ? q[i] : 1.0f;
        const float sc = l[i] * scale - __builtin_amdgcn_logf(fmaxf(e, kMinNoise));
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
// row's softmax instead of by the race (whose Philox draw per element, not the
// logits read, bounds it).  One read of the logits.  The draw kernel cuts a
// row into wave chunks of 2048 elements (each wave of a 256-thread workgroup
// takes every fourth run of 512 elements of the workgroup's 8192); a wave
// reduces its chunk to the maximum M_w of x_i = logits_i * log2(e) / T and
// S_w = sum_i 2^(x_i - M_w), and draws the chunk's own token in two steps
// with two uniforms (u1, u2) from Philox4x32-10 at counter (offset, row,
// 2 + wave chunk): the lane whose running share of S_w first reaches u1 S_w,
// then the first of that lane's 32 elements whose running sum reaches u2 times
// the lane's sum.  The choose kernel draws u from Philox at (offset, row, 1),
// selects wave chunk w with probability S_w 2^(M_w - M) / sum and returns its
// token.  Each step's choice is independent of the others and proportional to
// the mass it selects, so token i is drawn with probability
//   S_w 2^(M_w - M) / sum * s_lane / S_w * 2^(x_i - M_w) / s_lane = p_i
// up to float32 rounding of the running sums (a token with less than ~2^-24
// of its lane's mass is not drawn).  Which order the sums walk does not change
// the distribution.  Non-finite logits carry no mass; rows with no finite
// score give token 0, as in the race.

// x of one element (non-finite logits: -inf, no mass)
__device__ __forceinline__ float mass_x(float l, float scale) {
  const float x = l * scale;
  return (x == x && x != INFINITY) ? x : -INFINITY;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m));
  return v;
}
// Inclusive prefix of v over the 64 lanes of a wave (in lane order).
__device__ __forceinline__ float wave_incl(float v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float y = __shfl_up(v, o);
    if (lane >= o) v += y;
  }
  return v;
}

// two uniforms in (0, 1] from Philox4x32-10 at counter (offset, row, word),
// for a counter the same in every lane: plain xors, so that the rounds run on
// the scalar unit (v_bitop3_b32 has no scalar form)
__device__ __forceinline__ void row_uniforms(const SampleArgs& a, uint32_t row, uint32_t word,
                                             float* u1, float* u2) {
  U4 r{(uint32_t)a.offset, (uint32_t)(a.offset >> 32), row, word};
  uint32_t k0 = (uint32_t)a.seed, k1 = (uint32_t)(a.seed >> 32);
#pragma unroll
  for (int i = 0; i < 10; ++i) {
    const uint64_t p0 = (uint64_t)0xD2511F53u * r.x;
    const uint64_t p1 = (uint64_t)0xCD9E8D57u * r.z;
    r = U4{(uint32_t)(p1 >> 32) ^ r.y ^ k0, (uint32_t)p1, (uint32_t)(p0 >> 32) ^ r.w ^ k1,
           (uint32_t)p0};
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  *u1 = ((float)r.x + 1.0f) * 2.3283064365386963e-10f;
  *u2 = ((float)r.y + 1.0f) * 2.3283064365386963e-10f;
}

// Index of the first of cum[0..31] (non-decreasing) that reaches t, for
// 0 < t <= cum[31]: five halvings, each a compare and selects.
__device__ __forceinline__ int first_reaching(const float (&cum)[32], float t) {
  float h16[16], h8[8], h4[4], h2[2];
  bool b = cum[15] < t;
  int idx = b ? 16 : 0;
#pragma unroll
  for (int j = 0; j < 16; ++j) h16[j] = b ? cum[16 + j] : cum[j];
  b = h16[7] < t;
  idx += b ? 8 : 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) h8[j] = b ? h16[8 + j] : h16[j];
  b = h8[3] < t;
  idx += b ? 4 : 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) h4[j] = b ? h8[4 + j] : h8[j];
  b = h4[1] < t;
  idx += b ? 2 : 0;
  h2[0] = b ? h4[2] : h4[0];
  h2[1] = b ? h4[3] : h4[1];
  return idx + (h2[0] < t ? 1 : 0);
}

template <typename T, bool F16>
__global__ __launch_bounds__(kPartThreads) void sample_draw_kernel(SampleArgs a) {
  const int c = blockIdx.x, row = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const float scale = NVK_LOG2E / a.temperatures[row];
  // element k = 8 it + i of the lane: c kChunk + (it kPartThreads + tid) 8 + i
  float l[32];
  const int first = c * kChunk + tid * 8;
  if (sizeof(T) == 2 && a.vec_ok && (int64_t)(c + 1) * kChunk <= a.vocab) {
    // a whole chunk of bf16: the kIters 16-byte loads all leave before the first wait
    const uint16_t* p = static_cast<const uint16_t*>(a.logits) + (int64_t)row * a.row_stride + first;
    nvk_u32x4 w[kIters];
#pragma unroll
    for (int it = 0; it < kIters; ++it)
      w[it] = *reinterpret_cast<const nvk_u32x4*>(p + it * kPartThreads * 8);
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
      const uint32_t ww[4] = {w[it].x, w[it].y, w[it].z, w[it].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        l[8 * it + 2 * i] = NvkElt<F16>::lo(ww[i]);
        l[8 * it + 2 * i + 1] = NvkElt<F16>::hi(ww[i]);
      }
    }
  } else {
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
      const int base = first + it * kPartThreads * 8;
      if (base < a.vocab) {
        load8<T, F16>(a, row, base, base + 8 <= a.vocab, &l[8 * it]);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) l[8 * it + i] = -INFINITY;
      }
    }
  }
  // The wave's maximum and running sums, from the raw logits (the scale is
  // positive).  A NaN logit leaves a NaN sum and a +inf one an infinite
  // maximum: then the wave takes the path that gives them no mass.
  float mx = l[0];
#pragma unroll
  for (int k = 1; k < 32; k += 2) mx = fmaxf(mx, fmaxf(l[k], k + 1 < 32 ? l[k + 1] : l[k]));
  float M = wave_max(mx) * scale;
  float cum[32];
  float run = 0.f;
#pragma unroll
  for (int k = 0; k < 32; ++k) {
    run += __builtin_amdgcn_exp2f(fmaf(l[k], scale, -M));
    cum[k] = run;
  }
  if (__builtin_amdgcn_readfirstlane(__ballot(!(run == run)) != 0) ||
      !(M > -INFINITY && M < INFINITY)) {
#pragma unroll
    for (int k = 0; k < 32; ++k) l[k] = mass_x(l[k], scale);
    mx = l[0];
#pragma unroll
    for (int k = 1; k < 32; ++k) mx = fmaxf(mx, l[k]);
    M = wave_max(mx);
    run = 0.f;
#pragma unroll
    for (int k = 0; k < 32; ++k) {
      run += M != -INFINITY ? __builtin_amdgcn_exp2f(l[k] - M) : 0.f;
      cum[k] = run;
    }
  }
  // the lane, then the element of the lane
  const float incl = wave_incl(run);
  const float total = __shfl(incl, 63);
  float u1, u2;
  row_uniforms(a, (uint32_t)row, 2u + (uint32_t)(c * (kPartThreads / 64) + wave), &u1, &u2);
  const uint64_t pos = __ballot(run > 0.f);
  const uint64_t hit = __ballot(run > 0.f && incl >= u1 * total);
  // rounding can leave every running share below the target: the last lane with mass
  const int pick = hit ? __builtin_ctzll(hit) : (pos ? 63 - __builtin_clzll(pos) : 0);
  const int k = first_reaching(cum, fmaxf(u2 * run, 1.401298464e-45f));
  const int tok = first + (k >> 3) * (kPartThreads * 8) + (k & 7);
  const int tok_pick = __shfl(tok, pick);
  if (lane == 0) {
    const int64_t slot = (int64_t)row * (a.chunks * (kPartThreads / 64)) + c * (kPartThreads / 64) + wave;
    a.part_score[slot] = pos ? M : -INFINITY;
    reinterpret_cast<float*>(a.part_index)[slot] = total;
    a.part_token[slot] = pos ? tok_pick : -1;
  }
}

// One wave per row: wave chunk w with probability S_w 2^(M_w - M) / sum, then
// its drawn token.
__global__ __launch_bounds__(256) void sample_choose_kernel(SampleArgs a, int batch) {
  constexpr int kCached = 2;  // entries per lane held in registers (rows of up to 128 wave chunks)
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= batch) return;
  const int n = a.chunks * (kPartThreads / 64);
  const int64_t r0 = (int64_t)row * n;
  const float* pm = a.part_score + r0;
  const float* ps = reinterpret_cast<const float*>(a.part_index) + r0;
  const int* pt = a.part_token + r0;
  float m[kCached], sm[kCached];
  int tk[kCached];
#pragma unroll
  for (int j = 0; j < kCached; ++j) {
    const int e = 64 * j + lane;
    m[j] = e < n ? pm[e] : -INFINITY;
    sm[j] = e < n ? ps[e] : 0.f;
    tk[j] = e < n ? pt[e] : -1;
  }
  float mg = fmaxf(m[0], m[1]);
  for (int e = 64 * kCached + lane; e < n; e += 64) mg = fmaxf(mg, pm[e]);
  mg = wave_max(mg);
  if (mg == -INFINITY) {  // no finite score in the row
    if (lane == 0) a.tokens[row] = 0;
    return;
  }
  auto weight = [&](float mc, float sc) { return mc != -INFINITY ? sc * exp2f(mc - mg) : 0.f; };
  float w[kCached], incl[kCached];
  float total = 0.f;
#pragma unroll
  for (int j = 0; j < kCached; ++j) {
    w[j] = weight(m[j], sm[j]);
    incl[j] = wave_incl(w[j]);
    total += __shfl(incl[j], 63);
  }
  for (int base = 64 * kCached; base < n; base += 64) {
    const int e = base + lane;
    total += __shfl(wave_incl(e < n ? weight(pm[e], ps[e]) : 0.f), 63);
  }
  float u, unused;
  row_uniforms(a, (uint32_t)row, 1u, &u, &unused);
  const float t = u * total;
  // the first entry whose running weight reaches t (rounding: the last with weight)
  int tok = -1, last = -1;
  float run = 0.f;
#pragma unroll
  for (int j = 0; j < kCached; ++j) {
    const uint64_t pos = __ballot(w[j] > 0.f);
    const uint64_t hit = __ballot(w[j] > 0.f && run + incl[j] >= t);
    if (pos) last = __shfl(tk[j], 63 - __builtin_clzll(pos));
    if (tok < 0 && hit) tok = __shfl(tk[j], __builtin_ctzll(hit));
    run += __shfl(incl[j], 63);
  }
  for (int base = 64 * kCached; tok < 0 && base < n; base += 64) {
    const int e = base + lane;
    const float we = e < n ? weight(pm[e], ps[e]) : 0.f;
    const float ie = wave_incl(we);
    const uint64_t pos = __ballot(we > 0.f);
    const uint64_t hit = __ballot(we > 0.f && run + ie >= t);
    const int te = e < n ? pt[e] : -1;
    if (pos) last = __shfl(te, 63 - __builtin_clzll(pos));
    if (hit) tok = __shfl(te, __builtin_ctzll(hit));
    run += __shfl(ie, 63);
  }
  if (tok < 0) tok = last;
  if (lane == 0) a.tokens[row] = tok < 0 ? 0 : tok;
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
  return (size_t)batch * chunks * (kPartThreads / 64) * 12;
}

extern "C" int nvk_sample(const void* logits, int64_t row_stride, int32_t batch, int32_t vocab,
                          int32_t dtype, const float* temperatures, const float* noise,
                          int64_t noise_row_stride, uint64_t seed, uint64_t offset,
                          int64_t* tokens, void* workspace, size_t workspace_bytes,
                          void* stream) {
  if (batch < 0 || vocab <= 0 || row_stride < vocab) return NVK_EINVAL;
  if (dtype != NVK_DTYPE_BF16 && dtype != NVK_DTYPE_F16 && dtype != NVK_DTYPE_F32)
    return NVK_EUNSUPPORTED;
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
  const size_t slots = (size_t)batch * a.chunks * (kPartThreads / 64);
  a.part_score = static_cast<float*>(workspace);
  a.part_index = reinterpret_cast<int*>(static_cast<char*>(workspace) + 4 * slots);
  a.part_token = reinterpret_cast<int*>(static_cast<char*>(workspace) + 8 * slots);
  a.tokens = tokens;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid(a.chunks, batch);
  // The kernel's own randomness: inverse CDF (one read of the logits, one
  // exp2 per element, two uniforms per 2048 elements and one per row).
  if (!noise) {
    if (dtype == NVK_DTYPE_BF16)
      hipLaunchKernelGGL((sample_draw_kernel<uint16_t, false>), grid, dim3(kPartThreads), 0, s, a);
    else if (dtype == NVK_DTYPE_F16)
      hipLaunchKernelGGL((sample_draw_kernel<uint16_t, true>), grid, dim3(kPartThreads), 0, s, a);
    else
      hipLaunchKernelGGL((sample_draw_kernel<float, false>), grid, dim3(kPartThreads), 0, s, a);
    int st = nvk_launch_status();
    if (st != NVK_OK) return st;
    hipLaunchKernelGGL(sample_choose_kernel, dim3((batch + 3) / 4), dim3(256), 0, s, a, batch);
    return nvk_launch_status();
  }
  // The caller's noise: the race.
  if (dtype == NVK_DTYPE_BF16)
    hipLaunchKernelGGL((sample_partial_kernel<uint16_t, false>), grid, dim3(kPartThreads), 0, s, a);
  else if (dtype == NVK_DTYPE_F16)
    hipLaunchKernelGGL((sample_partial_kernel<uint16_t, true>), grid, dim3(kPartThreads), 0, s, a);
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
  if (dtype != NVK_DTYPE_BF16 && dtype != NVK_DTYPE_F16) return NVK_EUNSUPPORTED;  // 16-bit rows
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
