// Paged GQA decode attention (one query token per sequence) for gfx950.
//
// Semantics: flash_attn_with_kvcache(q[B,1,Hq,D], k_cache, v_cache,
// cache_seqlens=context_lens, block_table, softmax_scale, causal=True) as
// called at nanovllm/layers/attention.py:72-74: every query attends to the
// first context_lens[b] cached keys of its sequence (causal is a no-op for a
// single query row); q head h reads kv head h / (Hq/Hkv).
//
// Decomposition (split-K, "flash decoding"):
//   grid = (splits, Hkv, B), split = SPLIT consecutive key positions
//   (256 = one page at the reference's block size).  A workgroup owns one
//   (sequence, kv head, split) and all G = Hq/Hkv query heads of that kv
//   head, so each K/V byte is read from HBM once per step.  Its 4 waves each
//   stream 64 keys: the K row of a key (HD bf16 = 256 B for HD=128) is spread
//   over HD/8 lanes with one 16-byte load each, so one load instruction covers
//   64/(HD/8) whole rows and a wave keeps 2*64*HD*2 bytes (32 KiB) in flight.
//   q.k is v_dot2_f32_bf16 on bf16 pairs followed by a DPP butterfly over the
//   HD/8 lanes of the row; P.V packs two keys' probabilities as a bf16 pair and
//   uses v_dot2_f32_bf16 against the two keys' V values (f32 accumulation).
//   The online-softmax state (m, l, o) is merged across the 4 waves in LDS,
//   then either written as the final bf16 row (single split) or as an f32
//   partial that a second kernel combines.
#include "nvk_common.h"

namespace {

constexpr int kWaves = 4;
constexpr int kTile = 64;                  // keys per wave per tile
constexpr int kSplit = kWaves * kTile;     // keys per workgroup (one split)

struct DecodeArgs {
  const uint16_t* q;
  int64_t q_stride_tok, q_stride_head;
  const uint16_t* k_cache;
  const uint16_t* v_cache;
  const int32_t* block_tables;
  int64_t bt_stride;
  const int32_t* context_lens;
  int batch, num_q_heads, num_kv_heads;
  int block_size, bs_shift, max_blocks, num_blocks;
  float scale_log2;  // softmax_scale * log2(e)
  uint16_t* out;
  int64_t out_stride_tok, out_stride_head;
  float* ws_o;   // [B][Hq][S][HD]
  float* ws_ml;  // [B][Hq][S][2]
  int max_splits;
};

__device__ __forceinline__ int clamp_ctx(const DecodeArgs& a, int b) {
  int ctx = a.context_lens[b];
  const int64_t cap = (int64_t)a.max_blocks * a.block_size;
  if (ctx < 0) ctx = 0;
  if ((int64_t)ctx > cap) ctx = (int)cap;
  return ctx;
}

template <int HD>
__device__ __forceinline__ float group_sum_row(float x) {
  return nvk_group_sum<HD / 8>(x);
}

// max over the lanes that share the same position within a row (all lanes
// whose index differs by a multiple of HD/8).
template <int HD>
__device__ __forceinline__ float cross_group_max(float x) {
  if constexpr (HD == 64) x = fmaxf(x, nvk_dpp<0x128>(x));  // row_ror:8
  x = fmaxf(x, nvk_xor_lane<16>(x));
  x = fmaxf(x, nvk_xor_lane<32>(x));
  return x;
}
template <int HD>
__device__ __forceinline__ float cross_group_sum(float x) {
  if constexpr (HD == 64) x += nvk_dpp<0x128>(x);
  x += nvk_xor_lane<16>(x);
  x += nvk_xor_lane<32>(x);
  return x;
}

template <int HD, int G>
__global__ __launch_bounds__(256) void paged_decode_kernel(DecodeArgs a) {
  constexpr int LPR = HD / 8;          // lanes per K/V row
  constexpr int RPL = 64 / LPR;        // rows per load instruction
  constexpr int LOADS = kTile / RPL;   // load instructions per tile
  static_assert(LOADS % 2 == 0, "P.V pairs keys");

  const int split = blockIdx.x;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int j = lane % LPR;  // 16-byte chunk of the row: d in [8j, 8j+8)
  const int g = lane / LPR;  // row within a load instruction

  const int ctx = clamp_ctx(a, b);
  const int nsplit = (ctx + kSplit - 1) / kSplit;

  __shared__ float s_m[kWaves][G];
  __shared__ float s_l[kWaves][G];
  __shared__ float s_o[kWaves][G][HD];

  if (ctx == 0) {
    // padded graph row: defined zero output (model_runner.py:204-211).
    if (split == 0) {
      for (int e = tid; e < G * HD; e += 256) {
        const int h = e / HD, d = e % HD;
        a.out[(int64_t)b * a.out_stride_tok + (int64_t)(kvh * G + h) * a.out_stride_head + d] = 0;
      }
    }
    return;
  }
  if (split >= nsplit) return;

  // ---- query fragment: q[b, kvh*G + h, 8j : 8j+8] as 4 bf16x2 words -------
  uint32_t qw[G][4];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const uint16_t* qp = a.q + (int64_t)b * a.q_stride_tok + (int64_t)(kvh * G + h) * a.q_stride_head + 8 * j;
    const nvk_u32x4 v = *reinterpret_cast<const nvk_u32x4*>(qp);
    qw[h][0] = v.x; qw[h][1] = v.y; qw[h][2] = v.z; qw[h][3] = v.w;
  }

  const int32_t* bt_row = a.block_tables + (int64_t)b * a.bt_stride;
  const int64_t row_elems = (int64_t)a.num_kv_heads * HD;
  const int64_t head_off = (int64_t)kvh * HD + 8 * j;
  const int tile_base = split * kSplit + wave * kTile;
  const bool one_page = (a.block_size % kTile) == 0;

  float m_run[G], l_run[G], o_run[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m_run[h] = -INFINITY;
    l_run[h] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) o_run[h][e] = 0.f;
  }

  if (tile_base < ctx) {
    // ---- issue all K and V loads of the tile ---------------------------------
    int64_t tile_row0 = -1;
    if (one_page) tile_row0 = nvk_paged_row(bt_row, tile_base, a.block_size, a.bs_shift, a.num_blocks);
    nvk_u32x4 kr[LOADS], vr[LOADS];
    bool valid[LOADS];
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int pos = tile_base + i * RPL + g;
      int64_t row;
      if (one_page) row = tile_row0 < 0 ? -1 : tile_row0 + i * RPL + g;
      else row = pos < ctx ? nvk_paged_row(bt_row, pos, a.block_size, a.bs_shift, a.num_blocks) : -1;
      valid[i] = (pos < ctx) && (row >= 0);
      kr[i] = nvk_u32x4{0, 0, 0, 0};
      if (valid[i]) kr[i] = *reinterpret_cast<const nvk_u32x4*>(a.k_cache + row * row_elems + head_off);
    }
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int pos = tile_base + i * RPL + g;
      int64_t row;
      if (one_page) row = tile_row0 < 0 ? -1 : tile_row0 + i * RPL + g;
      else row = pos < ctx ? nvk_paged_row(bt_row, pos, a.block_size, a.bs_shift, a.num_blocks) : -1;
      vr[i] = nvk_u32x4{0, 0, 0, 0};
      if (valid[i]) vr[i] = *reinterpret_cast<const nvk_u32x4*>(a.v_cache + row * row_elems + head_off);
    }

    // ---- scores s[h][i] (already in log2 units) --------------------------------
    float s[G][LOADS];
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
#pragma unroll
      for (int h = 0; h < G; ++h) {
        float acc = nvk_dot2_bf16(qw[h][0], kr[i].x, 0.f);
        acc = nvk_dot2_bf16(qw[h][1], kr[i].y, acc);
        acc = nvk_dot2_bf16(qw[h][2], kr[i].z, acc);
        acc = nvk_dot2_bf16(qw[h][3], kr[i].w, acc);
        acc = group_sum_row<HD>(acc);
        s[h][i] = valid[i] ? acc * a.scale_log2 : -INFINITY;
      }
    }

    // ---- online softmax over the tile ------------------------------------------
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float mt = s[h][0];
#pragma unroll
      for (int i = 1; i < LOADS; ++i) mt = fmaxf(mt, s[h][i]);
      mt = cross_group_max<HD>(mt);
      m_run[h] = mt;  // first (and only) tile of this wave
      const float moff = (mt == -INFINITY) ? 0.f : mt;
      float lsum = 0.f;
#pragma unroll
      for (int i = 0; i < LOADS; ++i) {
        s[h][i] = nvk_fast_exp2(s[h][i] - moff);
        lsum += s[h][i];
      }
      l_run[h] = lsum;
    }

    // ---- P.V with bf16-pair dot products ---------------------------------------
#pragma unroll
    for (int i = 0; i < LOADS; i += 2) {
      uint32_t pk[G];
#pragma unroll
      for (int h = 0; h < G; ++h) pk[h] = nvk_pack_bf16x2(s[h][i], s[h][i + 1]);
      const uint32_t va[4] = {vr[i].x, vr[i].y, vr[i].z, vr[i].w};
      const uint32_t vb[4] = {vr[i + 1].x, vr[i + 1].y, vr[i + 1].z, vr[i + 1].w};
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t even = __builtin_amdgcn_perm(vb[w], va[w], 0x05040100u);  // (va.lo, vb.lo)
        const uint32_t odd = __builtin_amdgcn_perm(vb[w], va[w], 0x07060302u);   // (va.hi, vb.hi)
#pragma unroll
        for (int h = 0; h < G; ++h) {
          o_run[h][2 * w] = nvk_dot2_bf16(pk[h], even, o_run[h][2 * w]);
          o_run[h][2 * w + 1] = nvk_dot2_bf16(pk[h], odd, o_run[h][2 * w + 1]);
        }
      }
    }

    // ---- reduce the row groups of the wave ------------------------------------
#pragma unroll
    for (int h = 0; h < G; ++h) {
      l_run[h] = cross_group_sum<HD>(l_run[h]);
#pragma unroll
      for (int e = 0; e < 8; ++e) o_run[h][e] = cross_group_sum<HD>(o_run[h][e]);
    }
  }

  // ---- merge the 4 waves in LDS -----------------------------------------------
  if (g == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
#pragma unroll
      for (int e = 0; e < 8; ++e) s_o[wave][h][8 * j + e] = o_run[h][e];
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      s_m[wave][h] = m_run[h];
      s_l[wave][h] = l_run[h];
    }
  }
  __syncthreads();

  const int q_head0 = kvh * G;
  for (int e = tid; e < G * HD; e += 256) {
    const int h = e / HD, d = e % HD;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_m[w][h]);
    float L = 0.f, O = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float wt = nvk_fast_exp2(s_m[w][h] - M);  // exp2(-inf) = 0 for empty waves
        L += s_l[w][h] * wt;
        O += s_o[w][h][d] * wt;
      }
    }
    if (nsplit == 1) {
      const float r = L > 0.f ? O / L : 0.f;
      a.out[(int64_t)b * a.out_stride_tok + (int64_t)(q_head0 + h) * a.out_stride_head + d] =
          __builtin_bit_cast(uint16_t, (__bf16)r);
    } else {
      const int64_t part = ((int64_t)b * a.num_q_heads + q_head0 + h) * a.max_splits + split;
      a.ws_o[part * HD + d] = O;
      if (d == 0) {
        a.ws_ml[2 * part] = M;
        a.ws_ml[2 * part + 1] = L;
      }
    }
  }
}

// Combines the split partials of sequences with more than one split.
// grid = (Hq, B), block = HD threads (one output element each).
template <int HD>
__global__ __launch_bounds__(HD) void paged_decode_combine_kernel(DecodeArgs a) {
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int d = threadIdx.x;
  const int ctx = clamp_ctx(a, b);
  const int nsplit = (ctx + kSplit - 1) / kSplit;
  if (nsplit <= 1) return;
  const int64_t part0 = ((int64_t)b * a.num_q_heads + h) * a.max_splits;
  float M = -INFINITY;
  for (int s = 0; s < nsplit; ++s) M = fmaxf(M, a.ws_ml[2 * (part0 + s)]);
  float L = 0.f, O = 0.f;
  if (M != -INFINITY) {
    for (int s = 0; s < nsplit; ++s) {
      const float wt = nvk_fast_exp2(a.ws_ml[2 * (part0 + s)] - M);
      L += a.ws_ml[2 * (part0 + s) + 1] * wt;
      O += a.ws_o[(part0 + s) * HD + d] * wt;
    }
  }
  const float r = L > 0.f ? O / L : 0.f;
  a.out[(int64_t)b * a.out_stride_tok + (int64_t)h * a.out_stride_head + d] =
      __builtin_bit_cast(uint16_t, (__bf16)r);
}

int decode_max_splits(int block_size, int max_blocks) {
  const int64_t cap = (int64_t)block_size * max_blocks;
  return (int)((cap + kSplit - 1) / kSplit);
}

template <int HD, int G>
int launch_decode(const DecodeArgs& a, hipStream_t stream) {
  dim3 grid(a.max_splits, a.num_kv_heads, a.batch);
  hipLaunchKernelGGL((paged_decode_kernel<HD, G>), grid, dim3(256), 0, stream, a);
  int st = nvk_launch_status();
  if (st != NVK_OK) return st;
  if (a.max_splits > 1) {
    hipLaunchKernelGGL((paged_decode_combine_kernel<HD>), dim3(a.num_q_heads, a.batch), dim3(HD), 0,
                       stream, a);
    st = nvk_launch_status();
  }
  return st;
}

template <int HD>
int dispatch_group(const DecodeArgs& a, int G, hipStream_t s) {
  switch (G) {
    case 1: return launch_decode<HD, 1>(a, s);
    case 2: return launch_decode<HD, 2>(a, s);
    case 4: return launch_decode<HD, 4>(a, s);
    case 8: return launch_decode<HD, 8>(a, s);
    default: return NVK_EUNSUPPORTED;
  }
}

}  // namespace

extern "C" size_t nvk_paged_decode_workspace_size(int32_t batch, int32_t num_q_heads,
                                                  int32_t head_dim, int32_t block_size,
                                                  int32_t max_blocks) {
  if (batch <= 0 || num_q_heads <= 0 || head_dim <= 0 || block_size <= 0 || max_blocks <= 0)
    return 0;
  const int S = decode_max_splits(block_size, max_blocks);
  if (S <= 1) return 0;
  const size_t parts = (size_t)batch * num_q_heads * S;
  return parts * (size_t)head_dim * sizeof(float) + parts * 2 * sizeof(float);
}

extern "C" int nvk_paged_decode(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                                const void* k_cache, const void* v_cache,
                                const int32_t* block_tables, int64_t bt_stride,
                                const int32_t* context_lens, int32_t batch, int32_t num_q_heads,
                                int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                int32_t max_blocks, int32_t num_blocks, float scale, void* out,
                                int64_t out_stride_tok, int64_t out_stride_head, void* workspace,
                                size_t workspace_bytes, int32_t dtype, void* stream) {
  if (batch < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || block_size <= 0 || max_blocks <= 0 ||
      num_blocks < 0)
    return NVK_EINVAL;
  if (!(scale > 0.f)) return NVK_EINVAL;
  if (dtype != NVK_DTYPE_BF16) return NVK_EUNSUPPORTED;
  if (num_q_heads % num_kv_heads) return NVK_EINVAL;
  if (head_dim != 64 && head_dim != 128) return NVK_EUNSUPPORTED;
  if (batch == 0) return NVK_OK;
  if (!q || !k_cache || !v_cache || !block_tables || !context_lens || !out) return NVK_EINVAL;
  if (bt_stride < max_blocks) return NVK_EINVAL;
  // 16-byte vector access of q / K / V rows.
  if (((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache) % 16) return NVK_EALIGN;
  if ((q_stride_tok % 8) || (q_stride_head % 8) || ((uintptr_t)out % 2)) return NVK_EALIGN;
  if (batch > 65535) return NVK_EINVAL;
  const size_t need =
      nvk_paged_decode_workspace_size(batch, num_q_heads, head_dim, block_size, max_blocks);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) return NVK_EWORKSPACE;
  if (need > 0 && ((uintptr_t)workspace % 16)) return NVK_EALIGN;

  DecodeArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.q_stride_tok = q_stride_tok;
  a.q_stride_head = q_stride_head;
  a.k_cache = static_cast<const uint16_t*>(k_cache);
  a.v_cache = static_cast<const uint16_t*>(v_cache);
  a.block_tables = block_tables;
  a.bt_stride = bt_stride;
  a.context_lens = context_lens;
  a.batch = batch;
  a.num_q_heads = num_q_heads;
  a.num_kv_heads = num_kv_heads;
  a.block_size = block_size;
  a.bs_shift = nvk_log2_exact(block_size);
  a.max_blocks = max_blocks;
  a.num_blocks = num_blocks;
  a.scale_log2 = scale * NVK_LOG2E;
  a.out = static_cast<uint16_t*>(out);
  a.out_stride_tok = out_stride_tok;
  a.out_stride_head = out_stride_head;
  a.max_splits = decode_max_splits(block_size, max_blocks);
  const size_t parts = (size_t)batch * num_q_heads * a.max_splits;
  a.ws_o = need ? static_cast<float*>(workspace) : nullptr;
  a.ws_ml = need ? static_cast<float*>(workspace) + parts * head_dim : nullptr;
  const int G = num_q_heads / num_kv_heads;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (head_dim == 128) return dispatch_group<128>(a, G, s);
  return dispatch_group<64>(a, G, s);
}
