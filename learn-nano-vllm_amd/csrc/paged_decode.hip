// Paged GQA decode attention (one query token per sequence) for gfx950.
//
// Semantics: flash_attn_with_kvcache(q[B,1,Hq,D], k_cache, v_cache,
// cache_seqlens=context_lens, block_table, softmax_scale, causal=True) as
// called at nanovllm/layers/attention.py:72-74: every query attends to the
// first context_lens[b] cached keys of its sequence (causal is a no-op for a
// single query row); q head h reads kv head h / (Hq/Hkv).
//
// The step is a pure HBM stream (2 FLOP per byte), so the design is about
// keeping the memory system busy with useful bytes only.
//
// Lane mapping.  A token's K (or V) row in the cache is Hkv*HD contiguous
// bf16 (2 KiB for Qwen3-0.6B).  A wave's 16-byte-per-lane load instruction
// covers 1 KiB = 64/(HD/8) head rows: HPI consecutive kv heads of the same
// token times 64/(HD/8)/HPI tokens.  The mapping supports any power-of-two
// HPI; the library uses HPI = 1 (4 tokens x one head's 256 B for HD = 128, see
// decode_hpi).  Each group of HD/8 lanes ("row group") sees one kv head and
// keeps the online-softmax state (m, l, o) of the G query heads that read it;
// row groups of the same head are merged when a group of work ends.  q.k is
// v_dot2_f32_bf16 on bf16 pairs plus a DPP butterfly over the row group; P.V
// packs two keys' probabilities as bf16x2 and applies v_dot2_f32_bf16 against
// the two keys' V values, f32 accumulation.
//
// Work split: balanced stream-K.  A group is (sequence b, block of HPI kv
// heads); its keys are cut into chunks of TC = 8 * (tokens per instruction)
// tokens, i.e. 8 load instructions of K and 8 of V (16 KiB per wave).  Groups
// are ordered b-major, head block next, and the T chunks of the step are cut
// into equal contiguous ranges, one per wave of a persistent grid of at most
// 512 workgroups x 4 waves (static, so the launch can be captured in a graph;
// when T is small only T/2 waves take part).  Every wave streams the same
// number of bytes whatever the mix of context lengths.  Measured on MI355X, a
// wave that issues one chunk, waits and computes it, with 8 waves per CU,
// streams this access pattern at the rate of a plain read probe; deeper
// per-wave prefetch or more waves only add cache pressure.  K/V loads are
// non-temporal (read once).  The page of a chunk comes through a scalar load
// when a page holds whole chunks.
//
// Finishing: a group that ends inside a wave's range is normalised in
// registers and written as bf16.  A group cut between waves leaves one
// partial (o, m, l) record per wave and head; every wave also writes the
// group's descriptor (its first and last wave), so a small combine kernel
// merges the cut groups after two dependent reads and writes the zero rows of
// empty contexts.  Steps with few groups and long contexts (a group cut into
// up to 256 parts) use a combine whose 16 waves fold interleaved slices of the
// parts and merge them through LDS.  (Merging inside the main kernel needs cross-XCD release /
// acquire fences per part; on MI355X those cost far more than the combine.)
#include <mutex>

#include "nvk_common.h"
#include "qk_math.h"

namespace {

constexpr int kLoads = 8;          // load instructions per tensor per chunk
constexpr int kWavesPerWG = 4;
constexpr int kMaxWGs = 512;       // 256 CUs x 2 workgroups (8 waves per CU)
constexpr int kMaxBatch = 2048;    // sequences per call (LDS prefix table)
// A wave streams at least this many chunks.  Measured on MI355X: 2 against 8
// takes a 4-sequence decode from 30 to 17 us and a 16-sequence one from 34 to
// 27 us (more waves share a small step), and changes nothing from 64 up.
constexpr int kMinChunks = 2;
#ifndef NVK_DECODE_SLICE_MIN_WAVES
#define NVK_DECODE_SLICE_MIN_WAVES 32
#endif
constexpr int kSliceMinWaves = NVK_DECODE_SLICE_MIN_WAVES;

typedef __attribute__((address_space(4))) const int32_t nvk_const_i32;
typedef __attribute__((address_space(4))) const int64_t nvk_const_i64;

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
  int32_t* ws_desc;  // [batch][Hkv/HPI] x 2: first and last wave of the group, -1 if empty
  float* ws_rec;     // [P][2][HPI][G][HD+4] partial records
  int n_waves;       // P: waves of the grid
  int hpi;           // kv heads per load instruction
  int tc;            // tokens per chunk
  // Fused prologue (nvk_paged_decode_prologue, head_dim 128): q and the new
  // token's k and v come from the packed qkv row of each sequence (RMSNorm +
  // rotary embedding of q and k at positions[b]); the new k and v are stored
  // at slot_mapping[b] and used from registers for key context_lens[b] - 1.
  const uint16_t* qkv;
  int64_t qkv_row_stride;
  const int64_t* positions;
  const uint16_t* q_weight;
  const uint16_t* k_weight;
  float eps;
  const float* cos_sin;
  int64_t cos_sin_stride, max_position;
  const int32_t* slot_mapping;
  int64_t cache_slots;
  uint16_t* k_store;  // the caches, written at the slots
  uint16_t* v_store;
  bool f16;           // elements are f16 (else bf16)
};

// context_lens and block_tables are read-only for the whole launch: read them
// through the constant address space so wave-uniform reads become scalar loads.
__device__ __forceinline__ int clamp_ctx(const DecodeArgs& a, int b) {
  int ctx = ((nvk_const_i32*)a.context_lens)[b];
  const int64_t cap = (int64_t)a.max_blocks * a.block_size;
  if (ctx < 0) ctx = 0;
  if ((int64_t)ctx > cap) ctx = (int)cap;
  return ctx;
}

// Waves that take part for T chunks: at most P, and few enough that each
// range holds kMinChunks chunks (bounds how finely a context is split).
__device__ __forceinline__ int64_t active_waves(int64_t T, int64_t P) {
  int64_t p = T / kMinChunks;
  if (p > P) p = P;
  return p < 1 ? 1 : p;
}
// first chunk of wave w's range
__device__ __forceinline__ int64_t range_begin(int64_t w, int64_t T, int64_t P) { return w * T / P; }
// wave whose range holds chunk c
__device__ __forceinline__ int64_t chunk_owner(int64_t c, int64_t T, int64_t P) {
  return ((c + 1) * P - 1) / T;
}

__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

__device__ __forceinline__ float xor_lane(float x, int mask) {
  const int lane = __lane_id();
  return __int_as_float(__builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, __float_as_int(x)));
}

// Exclusive prefix of chunks per sequence into s_cs[0..B] and the clamped
// context lengths into s_ctx[0..B); returns the total.
__device__ int chunk_prefix(const DecodeArgs& a, int* s_cs, int* s_ctx, int* s_wsum) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int B = a.batch;
  const int per = (B + 255) / 256;
  const int b0 = tid * per;
  int local = 0;
  for (int i = 0; i < per; ++i) {
    const int b = b0 + i;
    if (b < B) {
      const int ctx = clamp_ctx(a, b);
      s_ctx[b] = ctx;
      local += (ctx + a.tc - 1) / a.tc;
    }
  }
  const int x = nvk_wave_scan_add(local);  // inclusive over the wave
  if (lane == 63) s_wsum[wave] = x;
  __syncthreads();
  int base = 0;
  for (int w = 0; w < wave; ++w) base += s_wsum[w];
  int run = base + x - local;
  for (int i = 0; i < per; ++i) {
    const int b = b0 + i;
    if (b < B) {
      s_cs[b] = run;
      run += (s_ctx[b] + a.tc - 1) / a.tc;
    }
  }
  const int total = s_wsum[0] + s_wsum[1] + s_wsum[2] + s_wsum[3];
  if (tid == 0) s_cs[B] = total;
  __syncthreads();
  return total;
}

// Loads of one chunk held by one lane.
template <int HD, int G>
struct ChunkBuf {
  static constexpr int LPR = HD / 8;   // lanes per head row
  nvk_u32x4 k[kLoads], v[kLoads];
  uint32_t q[G][4];
};

// Position of a wave in its range (all fields wave-uniform).
struct ChunkPos {
  int b, blk, k, n;  // sequence, kv-head block, chunk index in the group, chunks in the group
};

__device__ __forceinline__ void advance(ChunkPos& p, const int* s_cs, int n_blk) {
  if (++p.k == p.n) {
    p.k = 0;
    if (++p.blk == n_blk) {
      p.blk = 0;
      int b = p.b + 1;
      while (s_cs[b + 1] == s_cs[b]) ++b;  // skip empty contexts (a next chunk exists)
      p.b = b;
      p.n = s_cs[b + 1] - s_cs[b];
    }
  }
  p.b = uniform(p.b); p.blk = uniform(p.blk); p.k = uniform(p.k); p.n = uniform(p.n);
}

// This lane's place in a load instruction.
struct LaneRole {
  int j;    // 16-byte chunk of the head row: d in [8j, 8j+8)
  int hh;   // kv head within the block
  int tt;   // token within the instruction
};

// Issues the loads of chunk p.  Every lane issues the same load instructions
// whatever the data (no branches).  A row that does not exist (past the
// context, or a page id outside the pool) reads this lane's q row instead: it
// is finite, and its probability is masked to exactly 0 by the scores.
template <int HD, int G, bool ALIGNED, bool FUSED>
__device__ __forceinline__ void load_chunk(const DecodeArgs& a, const ChunkPos& p, int ctx,
                                           const LaneRole& r, int tpi, ChunkBuf<HD, G>& buf) {
  const int64_t row_elems = (int64_t)a.num_kv_heads * HD;
  const int kvh = p.blk * a.hpi + r.hh;
  const int64_t head_off = (int64_t)kvh * HD + 8 * r.j;
  const int base = p.k * a.tc;  // < ctx: p is a chunk of the group
  // the q row (fused: the raw q row of the packed qkv row) doubles as the
  // finite source of rows that do not exist
  const uint16_t* q0 =
      FUSED ? a.qkv + (int64_t)p.b * a.qkv_row_stride + (int64_t)(kvh * G) * HD + 8 * r.j
            : a.q + (int64_t)p.b * a.q_stride_tok + (int64_t)(kvh * G) * a.q_stride_head + 8 * r.j;
  if constexpr (!FUSED) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const nvk_u32x4 v = *reinterpret_cast<const nvk_u32x4*>(q0 + h * a.q_stride_head);
      buf.q[h][0] = v.x; buf.q[h][1] = v.y; buf.q[h][2] = v.z; buf.q[h][3] = v.w;
    }
  }
  const int64_t bt_off = (int64_t)p.b * a.bt_stride;
  if constexpr (ALIGNED) {
    // the whole chunk lies in one page: one scalar table read
    const int logical = a.bs_shift >= 0 ? (base >> a.bs_shift) : base / a.block_size;
    const int page = ((nvk_const_i32*)a.block_tables)[bt_off + logical];
    const bool page_ok = page >= 0 && page < a.num_blocks;
    const int64_t row0 = (int64_t)page * a.block_size + (base - logical * a.block_size);
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int t = i * tpi + r.tt;
      const bool ok = page_ok && base + t < ctx;
      const int64_t off = (row0 + t) * row_elems + head_off;
      const uint16_t* kp = ok ? a.k_cache + off : q0;
      const uint16_t* vp = ok ? a.v_cache + off : q0;
      buf.k[i] = __builtin_nontemporal_load(reinterpret_cast<const nvk_u32x4*>(kp));
      buf.v[i] = __builtin_nontemporal_load(reinterpret_cast<const nvk_u32x4*>(vp));
    }
  } else {
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int pos = base + i * tpi + r.tt;
      const int lpos = pos < ctx ? pos : ctx - 1;  // keeps the table read inside the row
      const int64_t row = nvk_paged_row(a.block_tables + bt_off, lpos, a.block_size, a.bs_shift,
                                        a.num_blocks);
      const bool ok = pos < ctx && row >= 0;
      const int64_t off = row * row_elems + head_off;
      const uint16_t* kp = ok ? a.k_cache + off : q0;
      const uint16_t* vp = ok ? a.v_cache + off : q0;
      buf.k[i] = __builtin_nontemporal_load(reinterpret_cast<const nvk_u32x4*>(kp));
      buf.v[i] = __builtin_nontemporal_load(reinterpret_cast<const nvk_u32x4*>(vp));
    }
  }
}

// Fused prologue, head_dim 128 (16 lanes per head row, lane j = r.j).  Its
// loads are issued before the chunk's K/V loads and its arithmetic runs after
// them, so that its round trip overlaps the chunk's (loads complete in issue
// order for the wait counter, so the arithmetic waits for its own loads only).
// The computed q goes to the wave's LDS slice sq[h * 16 + j] and is read back
// for every chunk, as the plain kernel reads q from memory; the new token's k
// and v replace the cache rows read for key ctx - 1.
template <int G>
struct FusedIn {
  nvk_u32x4 q[G], qw;        // raw q rows of the G heads, q norm weight
  nvk_u32x4 k, kw, v;        // the new token's raw k row, k norm weight, v row
  nvk_u32x4 cs[4];           // cos (2) and sin (2) of the lane's 8 dims
};
template <int HD, int G>
__device__ __forceinline__ void fused_load(const DecodeArgs& a, int b, int64_t pos, int kvh,
                                           bool need_q, bool need_new, const LaneRole& r,
                                           FusedIn<G>& in) {
  pos = pos < 0 ? 0 : (pos >= a.max_position ? a.max_position - 1 : pos);
  const float* c = a.cos_sin + pos * a.cos_sin_stride + 8 * (r.j & 7);
  in.cs[0] = *reinterpret_cast<const nvk_u32x4*>(c);
  in.cs[1] = *reinterpret_cast<const nvk_u32x4*>(c + 4);
  in.cs[2] = *reinterpret_cast<const nvk_u32x4*>(c + nvk_qk::kHD / 2);
  in.cs[3] = *reinterpret_cast<const nvk_u32x4*>(c + nvk_qk::kHD / 2 + 4);
  const uint16_t* row = a.qkv + (int64_t)b * a.qkv_row_stride + 8 * r.j;
  if (need_q) {
#pragma unroll
    for (int h = 0; h < G; ++h)
      in.q[h] = *reinterpret_cast<const nvk_u32x4*>(row + (int64_t)(kvh * G + h) * HD);
    in.qw = *reinterpret_cast<const nvk_u32x4*>(a.q_weight + 8 * r.j);
  }
  if (need_new) {
    in.k = *reinterpret_cast<const nvk_u32x4*>(row + (int64_t)(a.num_q_heads + kvh) * HD);
    in.v = *reinterpret_cast<const nvk_u32x4*>(
        row + (int64_t)(a.num_q_heads + a.num_kv_heads + kvh) * HD);
    in.kw = *reinterpret_cast<const nvk_u32x4*>(a.k_weight + 8 * r.j);
  }
}
template <int HD, int G, bool F16>
__device__ __forceinline__ void fused_apply(const DecodeArgs& a, const FusedIn<G>& in, int b,
                                            int kvh, int slot, bool need_q, bool need_new, int base,
                                            int ctx, int tpi, const LaneRole& r, nvk_u32x4* sq,
                                            ChunkBuf<HD, G>& buf) {
  if (need_q) {
#pragma unroll
    for (int h = 0; h < G; ++h)
      sq[h * nvk_qk::kLanesPerRow + r.j] =
          nvk_qk::norm_rope8_cs<F16>(in.q[h], in.qw, a.eps, in.cs, r.j);
  }
  if (need_new) {
    const nvk_u32x4 kn = nvk_qk::norm_rope8_cs<F16>(in.k, in.kw, a.eps, in.cs, r.j);
    const int rel = ctx - 1 - base;
    const int i_new = rel / tpi, tt_new = rel % tpi;
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      if (i == i_new && r.tt == tt_new) {
        buf.k[i] = kn;
        buf.v[i] = in.v;
      }
    }
    // row group 0 stores the new token's k and v at its slot
    if (r.tt == 0 && slot >= 0 && (int64_t)slot < a.cache_slots) {
      const int64_t off = (int64_t)slot * a.num_kv_heads * HD + (int64_t)kvh * HD + 8 * r.j;
      __builtin_nontemporal_store(kn, reinterpret_cast<nvk_u32x4*>(a.k_store + off));
      __builtin_nontemporal_store(in.v, reinterpret_cast<nvk_u32x4*>(a.v_store + off));
    }
  }
}

// Online-softmax state of one lane's row group for the G heads.
template <int G>
struct SoftmaxState {
  float m[G], l[G], o[G][8];
  __device__ __forceinline__ void reset() {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      m[h] = -INFINITY;
      l[h] = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[h][e] = 0.f;
    }
  }
};

template <int HD, int G, bool F16>
__device__ __forceinline__ void compute_chunk(const DecodeArgs& a, const ChunkBuf<HD, G>& buf,
                                              int base, int ctx, int tpi, const LaneRole& r,
                                              SoftmaxState<G>& st) {
  using CB = ChunkBuf<HD, G>;
  using E = NvkElt<F16>;
  float s[G][kLoads];
#pragma unroll
  for (int i = 0; i < kLoads; ++i) {
    const bool ok = base + i * tpi + r.tt < ctx;
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float acc = E::dot2(buf.q[h][0], buf.k[i].x, 0.f);
      acc = E::dot2(buf.q[h][1], buf.k[i].y, acc);
      acc = E::dot2(buf.q[h][2], buf.k[i].z, acc);
      acc = E::dot2(buf.q[h][3], buf.k[i].w, acc);
      acc = nvk_group_sum<CB::LPR>(acc);
      s[h][i] = ok ? acc * a.scale_log2 : -INFINITY;
    }
  }
#pragma unroll
  for (int h = 0; h < G; ++h) {
    float mt = s[h][0];
#pragma unroll
    for (int i = 1; i < kLoads; ++i) mt = fmaxf(mt, s[h][i]);
    const float m_new = fmaxf(st.m[h], mt);
    const float moff = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = nvk_fast_exp2(st.m[h] - moff);
    st.m[h] = m_new;
    float psum = 0.f;
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      s[h][i] = nvk_fast_exp2(s[h][i] - moff);
      psum += s[h][i];
    }
    st.l[h] = st.l[h] * alpha + psum;
#pragma unroll
    for (int e = 0; e < 8; ++e) st.o[h][e] *= alpha;
  }
#pragma unroll
  for (int i = 0; i < kLoads; i += 2) {
    uint32_t pk[G];
#pragma unroll
    for (int h = 0; h < G; ++h) pk[h] = E::pack2(s[h][i], s[h][i + 1]);
    const uint32_t va[4] = {buf.v[i].x, buf.v[i].y, buf.v[i].z, buf.v[i].w};
    const uint32_t vb[4] = {buf.v[i + 1].x, buf.v[i + 1].y, buf.v[i + 1].z, buf.v[i + 1].w};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint32_t even = __builtin_amdgcn_perm(vb[w], va[w], 0x05040100u);  // (va.lo, vb.lo)
      const uint32_t odd = __builtin_amdgcn_perm(vb[w], va[w], 0x07060302u);   // (va.hi, vb.hi)
#pragma unroll
      for (int h = 0; h < G; ++h) {
        st.o[h][2 * w] = E::dot2(pk[h], even, st.o[h][2 * w]);
        st.o[h][2 * w + 1] = E::dot2(pk[h], odd, st.o[h][2 * w + 1]);
      }
    }
  }
}

// x combined (max or sum) with lane l ^ S, for S in {8, 16, 32}, by VALU
// exchanges (a DPP row rotation by 8, v_permlane16_swap, v_permlane32_swap)
// instead of an LDS round trip.  Both lanes of a pair get op(even, odd):
// the same value as op(x, x of lane l ^ S), op being commutative.
template <int S, bool MAX>
__device__ __forceinline__ float pair_op(float x) {
  float a, b;
  if constexpr (S == 8) {
    a = x;
    b = nvk_dpp<NVK_DPP_ROW_ROR8>(x);  // row_ror:8: lane l ^ 8 of the 16-lane row
  } else {
    const auto r = S == 16 ? __builtin_amdgcn_permlane16_swap(__float_as_uint(x),
                                                                __float_as_uint(x), false, false)
                           : __builtin_amdgcn_permlane32_swap(__float_as_uint(x),
                                                                __float_as_uint(x), false, false);
    a = __uint_as_float(r[0]);
    b = __uint_as_float(r[1]);
  }
  return MAX ? fmaxf(a, b) : a + b;
}
// op over the row groups LPR, 2 LPR, ... apart (HPI = 1: all of a wave's
// row groups hold the same kv head)
template <int LPR, bool MAX>
__device__ __forceinline__ float rows_op(float x) {
  if constexpr (LPR <= 8) x = pair_op<8, MAX>(x);
  if constexpr (LPR <= 16) x = pair_op<16, MAX>(x);
  return pair_op<32, MAX>(x);
}

// Merges the row groups that hold the same kv head (they differ by multiples
// of `stride` lanes; `tpi` of them).  Afterwards the lanes with tt == 0 hold
// the head's state.  One kv head per load instruction (the library's choice,
// decode_hpi): VALU lane exchanges; otherwise LDS permutes.
template <int G, int LPR>
__device__ __forceinline__ void merge_same_head(SoftmaxState<G>& st, int tpi, int stride) {
  if (stride == LPR && stride * tpi == 64) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float M = rows_op<LPR, true>(st.m[h]);
      const float w = (M == -INFINITY) ? 0.f : nvk_fast_exp2(st.m[h] - M);
      st.l[h] = rows_op<LPR, false>(st.l[h] * w);
      st.m[h] = M;
#pragma unroll
      for (int e = 0; e < 8; ++e) st.o[h][e] = rows_op<LPR, false>(st.o[h][e] * w);
    }
    return;
  }
#pragma unroll
  for (int h = 0; h < G; ++h) {
    float M = st.m[h];
    for (int s = stride; s < stride * tpi; s <<= 1) M = fmaxf(M, xor_lane(M, s));
    const float w = (M == -INFINITY) ? 0.f : nvk_fast_exp2(st.m[h] - M);
    float l = st.l[h] * w;
    for (int s = stride; s < stride * tpi; s <<= 1) l += xor_lane(l, s);
    st.m[h] = M;
    st.l[h] = l;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float o = st.o[h][e] * w;
      for (int s = stride; s < stride * tpi; s <<= 1) o += xor_lane(o, s);
      st.o[h][e] = o;
    }
  }
}

template <bool F16>
__device__ __forceinline__ void store_x8(uint16_t* p, const float* v, float scale) {
  using E = NvkElt<F16>;
  nvk_u32x4 w;
  w.x = E::pack2(v[0] * scale, v[1] * scale);
  w.y = E::pack2(v[2] * scale, v[3] * scale);
  w.z = E::pack2(v[4] * scale, v[5] * scale);
  w.w = E::pack2(v[6] * scale, v[7] * scale);
  *reinterpret_cast<nvk_u32x4*>(p) = w;
}

template <int HD, int G, bool ALIGNED, bool FUSED, bool F16>
__global__ __launch_bounds__(256) void paged_decode_kernel(DecodeArgs a) {
  using CB = ChunkBuf<HD, G>;
  constexpr int RPI = 64 / CB::LPR;           // head rows per load instruction
  constexpr int REC_HEAD = G * (HD + 4);      // floats per head in a record
  __shared__ int s_cs[kMaxBatch + 1];
  // context lengths, read once per workgroup: a wave that moves to another
  // sequence finds its length here instead of in a dependent global load
  __shared__ int s_ctx[kMaxBatch];
  __shared__ int s_wsum[kWavesPerWG];
  __shared__ nvk_u32x4 s_q[FUSED ? kWavesPerWG * G * nvk_qk::kLanesPerRow : 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int hpi = a.hpi;
  const int tpi = RPI / hpi;
  LaneRole role;
  role.j = lane % CB::LPR;
  const int g = lane / CB::LPR;
  role.hh = g % hpi;
  role.tt = g / hpi;
  const int n_blk = a.num_kv_heads / hpi;

  const int S = chunk_prefix(a, s_cs, s_ctx, s_wsum);
  if (blockIdx.x == 0) {  // empty contexts: no wave visits them
    for (int e = tid; e < a.batch * n_blk; e += 256) {
      const int b = e / n_blk;
      if (s_cs[b + 1] == s_cs[b]) *reinterpret_cast<int2*>(a.ws_desc + 2 * e) = make_int2(-1, -1);
    }
  }
  const int64_t T = (int64_t)n_blk * S;
  const int64_t P = active_waves(T, a.n_waves);
  // the wave index is wave-uniform; say so, so that the range bookkeeping and
  // the page-table reads stay scalar
  const int64_t w = (int64_t)blockIdx.x * kWavesPerWG + uniform(tid >> 6);
  if (w >= P) return;
  const int64_t c0 = range_begin(w, T, P), c1 = range_begin(w + 1, T, P);
  if (c0 >= c1) return;

  // locate chunk c0: last b with n_blk*s_cs[b] <= c0
  ChunkPos cur;
  cur.b = nvk_last_le(s_cs, a.batch, n_blk, c0, lane);
  cur.n = uniform(s_cs[cur.b + 1] - s_cs[cur.b]);
  const int r = (int)(c0 - (int64_t)n_blk * s_cs[cur.b]);
  cur.blk = uniform(r / cur.n);
  cur.k = uniform(r % cur.n);
  bool started_here = cur.k == 0;
  int ctx = uniform(s_ctx[cur.b]);
  // fused: the new token's position (a scalar read beside the context length)
  int64_t pos = FUSED ? ((nvk_const_i64*)a.positions)[cur.b] : 0;
  int slot = FUSED ? ((nvk_const_i32*)a.slot_mapping)[cur.b] : -1;

  SoftmaxState<G> st;
  st.reset();
  CB buf;
  for (int64_t c = c0;; ++c) {
    if constexpr (FUSED) {
      const bool need_q = c == c0 || cur.k == 0;
      const bool need_new = cur.k == cur.n - 1;
      const int kvh = cur.blk * hpi + role.hh;
      nvk_u32x4* sq = s_q + (tid >> 6) * G * nvk_qk::kLanesPerRow;
      FusedIn<G> in;
      if (need_q || need_new) fused_load<HD, G>(a, cur.b, pos, kvh, need_q, need_new, role, in);
      load_chunk<HD, G, ALIGNED, FUSED>(a, cur, ctx, role, tpi, buf);
      if (need_q || need_new)
        fused_apply<HD, G, F16>(a, in, cur.b, kvh, slot, need_q, need_new, cur.k * a.tc, ctx, tpi, role, sq,
                           buf);
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const nvk_u32x4 v = sq[h * nvk_qk::kLanesPerRow + role.j];
        buf.q[h][0] = v.x; buf.q[h][1] = v.y; buf.q[h][2] = v.z; buf.q[h][3] = v.w;
      }
    } else {
      load_chunk<HD, G, ALIGNED, FUSED>(a, cur, ctx, role, tpi, buf);
    }
    compute_chunk<HD, G, F16>(a, buf, cur.k * a.tc, ctx, tpi, role, st);
    const bool last = c + 1 == c1;
    const bool group_end = cur.k == cur.n - 1;
    if (group_end || last) {
      if (tpi > 1) merge_same_head<G, CB::LPR>(st, tpi, hpi * CB::LPR);
      const int kvh = cur.blk * hpi + role.hh;
      const bool whole = group_end && started_here;
      if (role.tt == 0) {
        if (whole) {
#pragma unroll
          for (int h = 0; h < G; ++h) {
            const float inv = st.l[h] > 0.f ? 1.f / st.l[h] : 0.f;
            store_x8<F16>(a.out + (int64_t)cur.b * a.out_stride_tok +
                             (int64_t)(kvh * G + h) * a.out_stride_head + 8 * role.j,
                         st.o[h], inv);
          }
        } else {
          float* rec = a.ws_rec + ((w * 2 + (started_here ? 0 : 1)) * hpi + role.hh) * REC_HEAD;
#pragma unroll
          for (int h = 0; h < G; ++h) {
            float* ro = rec + h * (HD + 4);
            *reinterpret_cast<nvk_f32x4*>(ro + 8 * role.j) =
                nvk_f32x4{st.o[h][0], st.o[h][1], st.o[h][2], st.o[h][3]};
            *reinterpret_cast<nvk_f32x4*>(ro + 8 * role.j + 4) =
                nvk_f32x4{st.o[h][4], st.o[h][5], st.o[h][6], st.o[h][7]};
            if (role.j == 0) {
              ro[HD] = st.m[h];
              ro[HD + 1] = st.l[h];
            }
          }
        }
      }
      if (lane == 0) {  // group descriptor: first and last wave of the group
        const int64_t gfirst = (int64_t)n_blk * s_cs[cur.b] + (int64_t)cur.blk * cur.n;
        const int p1 = (int)chunk_owner(gfirst, T, P);
        const int p2 = (int)chunk_owner(gfirst + cur.n - 1, T, P);
        *reinterpret_cast<int2*>(a.ws_desc + 2 * (cur.b * n_blk + cur.blk)) = make_int2(p1, p2);
      }
      st.reset();
      started_here = true;
    }
    if (last) return;
    const int b_prev = cur.b;
    advance(cur, s_cs, n_blk);
    if (cur.b != b_prev) {
      ctx = uniform(s_ctx[cur.b]);
      if constexpr (FUSED) {
        pos = ((nvk_const_i64*)a.positions)[cur.b];
        slot = ((nvk_const_i32*)a.slot_mapping)[cur.b];
      }
    }
  }
}

// Merges the partial records of groups cut between waves and writes the zero
// output of empty contexts.
// Merge of one output element over the parts of a cut group: wave p1's head
// record (slot 0) and the continuation records (slot 1) of waves p1+1 .. p2
// (every active wave's range holds at least kMinChunks chunks, so each of
// them wrote one).  A slice s of S folds parts p1+s, p1+s+S, ...; kBatch
// parts are fetched per round trip (3 kBatch loads in flight), then folded
// into (M, L, O).  rec0: the record of wave 0, slot 0, for this thread's kv
// head and q head.
template <int kBatch, int HD, int G>
__device__ __forceinline__ void fold_parts(const DecodeArgs& a, const float* rec0, int p1, int p2,
                                           int s, int S, int d, float& M, float& L, float& O) {
  constexpr int REC_HEAD = G * (HD + 4);
  for (int base = p1 + s; base <= p2; base += kBatch * S) {
    float mv[kBatch], lv[kBatch], ov[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int p = base + u * S;
      const bool ok = p <= p2;
      const int pr = ok ? p : p1;
      const float* rec = rec0 + ((int64_t)pr * 2 + (pr == p1 ? 0 : 1)) * a.hpi * REC_HEAD;
      mv[u] = rec[HD];
      lv[u] = rec[HD + 1];
      ov[u] = rec[d];
      if (!ok) mv[u] = -INFINITY;
    }
    // All 3 kBatch loads of the batch are issued before the fold starts (one
    // round trip per batch): without the fence the compiler interleaves the
    // running max with the loads and waits for each part in turn.
    __builtin_amdgcn_sched_barrier(0);
    float mb = M;
#pragma unroll
    for (int u = 0; u < kBatch; ++u) mb = fmaxf(mb, mv[u]);
    const float mref = mb == -INFINITY ? 0.f : mb;  // no part so far: every weight 0
    const float r = nvk_fast_exp2(M - mref);        // 0 while M is still -inf
    L *= r;
    O *= r;
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const float wt = nvk_fast_exp2(mv[u] - mref);
      L += lv[u] * wt;
      O += ov[u] * wt;
    }
    M = mb;
  }
}

// grid = (Hkv, B), block = G*HD threads, one per output element of the
// (sequence, kv head).
template <int HD, int G, bool F16>
__global__ __launch_bounds__(G * HD) void paged_decode_combine_kernel(DecodeArgs a) {
  constexpr int REC_HEAD = G * (HD + 4);  // floats per kv head in a record
  const int kvh = blockIdx.x, b = blockIdx.y;
  const int h = threadIdx.x / HD, d = threadIdx.x % HD;
  const int n_blk = a.num_kv_heads / a.hpi;
  const int hh = kvh % a.hpi;
  const int2 desc = *reinterpret_cast<const int2*>(a.ws_desc + 2 * (b * n_blk + kvh / a.hpi));
  uint16_t* op = a.out + (int64_t)b * a.out_stride_tok + (int64_t)(kvh * G + h) * a.out_stride_head + d;
  if (desc.x < 0) {  // empty context (padded graph row): defined zero output
    *op = 0;
    return;
  }
  const int p1 = desc.x, p2 = desc.y;
  if (p1 == p2) return;  // finished inside one wave
  const float* rec0 = a.ws_rec + hh * REC_HEAD + h * (HD + 4);
  float M = -INFINITY, L = 0.f, O = 0.f;
  // records fetched per round trip: the smallest batch that holds every part
  // (32 for groups cut into more; uniform over the workgroup)
  const int parts = p2 - p1 + 1;
  if (parts <= 4)
    fold_parts<4, HD, G>(a, rec0, p1, p2, 0, 1, d, M, L, O);
  else if (parts <= 8)
    fold_parts<8, HD, G>(a, rec0, p1, p2, 0, 1, d, M, L, O);
  else if (parts <= 16)
    fold_parts<16, HD, G>(a, rec0, p1, p2, 0, 1, d, M, L, O);
  else
    fold_parts<32, HD, G>(a, rec0, p1, p2, 0, 1, d, M, L, O);
  *op = NvkElt<F16>::one(L > 0.f ? O / L : 0.f);
}

// Combine of steps whose groups are cut into many parts (few sequences, long
// contexts: a 1-sequence step over 16 K keys cuts each group into 256).
// grid = (Hkv * G*HD/64, B), block = kSlices waves; a workgroup owns 64
// consecutive output elements of one (sequence, kv head), wave s folds parts
// p1+s, p1+s+kSlices, ... (so a thread waits for 1/kSlices of the round
// trips), and wave 0 merges the waves' (M, L, O) through LDS.
constexpr int kSlices = 16;
template <int HD, int G, bool F16>
__global__ __launch_bounds__(64 * kSlices) void paged_decode_combine_sliced_kernel(DecodeArgs a) {
  constexpr int REC_HEAD = G * (HD + 4);
  constexpr int EB = G * HD / 64;  // workgroups per (sequence, kv head)
  const int kvh = blockIdx.x / EB, b = blockIdx.y;
  const int lane = threadIdx.x & 63, s = threadIdx.x >> 6;
  const int e = (blockIdx.x % EB) * 64 + lane;
  const int h = e / HD, d = e % HD;
  const int n_blk = a.num_kv_heads / a.hpi;
  const int hh = kvh % a.hpi;
  const int2 desc = *reinterpret_cast<const int2*>(a.ws_desc + 2 * (b * n_blk + kvh / a.hpi));
  uint16_t* op = a.out + (int64_t)b * a.out_stride_tok + (int64_t)(kvh * G + h) * a.out_stride_head + d;
  if (desc.x < 0) {  // empty context (padded graph row): defined zero output
    if (s == 0) *op = 0;
    return;
  }
  const int p1 = desc.x, p2 = desc.y;
  if (p1 == p2) return;  // finished inside one wave (uniform over the workgroup)
  const float* rec0 = a.ws_rec + hh * REC_HEAD + h * (HD + 4);
  float M = -INFINITY, L = 0.f, O = 0.f;
  const int per_slice = (p2 - p1 + kSlices) / kSlices;  // ceil(parts / kSlices)
  if (per_slice <= 4)
    fold_parts<4, HD, G>(a, rec0, p1, p2, s, kSlices, d, M, L, O);
  else if (per_slice <= 8)
    fold_parts<8, HD, G>(a, rec0, p1, p2, s, kSlices, d, M, L, O);
  else if (per_slice <= 16)
    fold_parts<16, HD, G>(a, rec0, p1, p2, s, kSlices, d, M, L, O);
  else
    fold_parts<32, HD, G>(a, rec0, p1, p2, s, kSlices, d, M, L, O);
  __shared__ float sm[kSlices][64], sl[kSlices][64], so[kSlices][64];
  sm[s][lane] = M;
  sl[s][lane] = L;
  so[s][lane] = O;
  __syncthreads();
  if (s != 0) return;
  float mx = sm[0][lane];
#pragma unroll
  for (int i = 1; i < kSlices; ++i) mx = fmaxf(mx, sm[i][lane]);
  const float mref = mx == -INFINITY ? 0.f : mx;
  L = 0.f;
  O = 0.f;
#pragma unroll
  for (int i = 0; i < kSlices; ++i) {
    const float wt = nvk_fast_exp2(sm[i][lane] - mref);
    L += sl[i][lane] * wt;
    O += so[i][lane] * wt;
  }
  *op = NvkElt<F16>::one(L > 0.f ? O / L : 0.f);
}

// kv heads per load instruction.  One: a group is then one (sequence, kv
// head), so a context is cut into fewer parts and the combine pass reads them
// in a single round trip.  Measured on MI355X (Qwen3 decode step), reading 4
// heads per instruction (1 KiB contiguous) streams no faster than 1 head
// (4 x 256 B), and quadruples the parts per cut group; 2 heads (each wave's
// range mixing two heads' rows) took B = 64 from 55.2 to 56.9 us and was
// slower at every batch from 1 to 512.
int decode_hpi(int num_kv_heads, int head_dim) {
  (void)num_kv_heads;
  (void)head_dim;
  return 1;
}

int decode_tc(int num_kv_heads, int head_dim) {
  const int rpi = 64 / (head_dim / 8);
  return kLoads * (rpi / decode_hpi(num_kv_heads, head_dim));
}

// Waves of the persistent grid for these static sizes.
int decode_waves(int batch, int num_kv_heads, int head_dim, int block_size, int max_blocks) {
  const int tc = decode_tc(num_kv_heads, head_dim);
  const int64_t max_chunks_seq = ((int64_t)block_size * max_blocks + tc - 1) / tc;
  const int64_t t_max = max_chunks_seq * batch * (num_kv_heads / decode_hpi(num_kv_heads, head_dim));
  int64_t wgs = (t_max / kMinChunks + kWavesPerWG - 1) / kWavesPerWG;
  if (wgs > kMaxWGs) wgs = kMaxWGs;
  if (wgs < 1) wgs = 1;
  return (int)wgs * kWavesPerWG;
}

size_t decode_ws_bytes(int batch, int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                       int max_blocks) {
  const int G = num_q_heads / num_kv_heads;
  const size_t P = decode_waves(batch, num_kv_heads, head_dim, block_size, max_blocks);
  const size_t hpi = decode_hpi(num_kv_heads, head_dim);
  const size_t desc = ((size_t)batch * (num_kv_heads / hpi) * 8 + 255) / 256 * 256;
  return desc + P * 2 * hpi * G * (head_dim + 4) * sizeof(float);
}

template <int HD, int G, bool FUSED, bool F16>
int launch_decode(const DecodeArgs& a, bool aligned, hipStream_t stream) {
  const dim3 grid(a.n_waves / kWavesPerWG);
  if (aligned)
    hipLaunchKernelGGL((paged_decode_kernel<HD, G, true, FUSED, F16>), grid, dim3(256), 0, stream,
                       a);
  else
    hipLaunchKernelGGL((paged_decode_kernel<HD, G, false, FUSED, F16>), grid, dim3(256), 0,
                       stream, a);
  int st = nvk_launch_status();
  if (st != NVK_OK) return st;
  // Steps with at least NVK_DECODE_SLICE_MIN_WAVES waves per group cut
  // their groups into many parts: the sliced combine folds them.
  const int64_t groups = (int64_t)a.batch * (a.num_kv_heads / a.hpi);
  if (a.n_waves >= (int64_t)kSliceMinWaves * groups)
    hipLaunchKernelGGL((paged_decode_combine_sliced_kernel<HD, G, F16>),
                       dim3(a.num_kv_heads * (G * HD / 64), a.batch), dim3(64 * kSlices), 0,
                       stream, a);
  else
    hipLaunchKernelGGL((paged_decode_combine_kernel<HD, G, F16>), dim3(a.num_kv_heads, a.batch),
                       dim3(G * HD), 0, stream, a);
  return nvk_launch_status();
}

template <int HD, bool FUSED = false, bool F16 = false>
int dispatch_group(const DecodeArgs& a, int G, bool aligned, hipStream_t s) {
  switch (G) {
    case 1: return launch_decode<HD, 1, FUSED, F16>(a, aligned, s);
    case 2: return launch_decode<HD, 2, FUSED, F16>(a, aligned, s);
    case 4: return launch_decode<HD, 4, FUSED, F16>(a, aligned, s);
    case 8: return launch_decode<HD, 8, FUSED, F16>(a, aligned, s);
    default: return NVK_EUNSUPPORTED;
  }
}

// Checks the arguments of a plain decode call (everything but the workspace)
// and fills `a`; returns NVK_OK, or the error code, before anything is
// launched.  *need = workspace bytes the call uses.
int decode_setup(const void* q, int64_t q_stride_tok, int64_t q_stride_head, const void* k_cache,
                 const void* v_cache, const int32_t* block_tables, int64_t bt_stride,
                 const int32_t* context_lens, int32_t batch, int32_t num_q_heads,
                 int32_t num_kv_heads, int32_t head_dim, int32_t block_size, int32_t max_blocks,
                 int32_t num_blocks, float scale, void* out, int64_t out_stride_tok,
                 int64_t out_stride_head, int32_t dtype, DecodeArgs& a, size_t* need) {
  *need = 0;
  if (batch < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || block_size <= 0 || max_blocks <= 0 ||
      num_blocks < 0)
    return NVK_EINVAL;
  if (!(scale > 0.f)) return NVK_EINVAL;
  if (dtype != NVK_DTYPE_BF16 && dtype != NVK_DTYPE_F16) return NVK_EUNSUPPORTED;
  if (num_q_heads % num_kv_heads) return NVK_EINVAL;
  if (head_dim != 64 && head_dim != 128) return NVK_EUNSUPPORTED;
  const int G = num_q_heads / num_kv_heads;
  if (G != 1 && G != 2 && G != 4 && G != 8) return NVK_EUNSUPPORTED;
  if (batch == 0) return NVK_OK;
  if (batch > kMaxBatch || num_kv_heads > 65535) return NVK_EUNSUPPORTED;
  if (!q || !k_cache || !v_cache || !block_tables || !context_lens || !out) return NVK_EINVAL;
  if (bt_stride < max_blocks) return NVK_EINVAL;
  if ((int64_t)block_size * max_blocks > INT32_MAX) return NVK_EINVAL;
  const int tc = decode_tc(num_kv_heads, head_dim);
  // chunk counts are 32-bit: batch * chunks per sequence * head blocks must fit
  if ((int64_t)batch * num_kv_heads * (((int64_t)block_size * max_blocks + tc - 1) / tc) >
      INT32_MAX)
    return NVK_EINVAL;
  // 16-byte vector access of q / K / V rows and of the output rows.
  if (((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)out) % 16)
    return NVK_EALIGN;
  if ((q_stride_tok % 8) || (q_stride_head % 8) || (out_stride_tok % 8) || (out_stride_head % 8))
    return NVK_EALIGN;
  *need = decode_ws_bytes(batch, num_q_heads, num_kv_heads, head_dim, block_size, max_blocks);

  a = DecodeArgs{};
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
  a.hpi = decode_hpi(num_kv_heads, head_dim);
  a.tc = tc;
  a.n_waves = decode_waves(batch, num_kv_heads, head_dim, block_size, max_blocks);
  a.f16 = dtype == NVK_DTYPE_F16;
  return NVK_OK;
}

// Points the descriptors and records of `a` into `workspace` and launches.
int decode_run(DecodeArgs& a, int head_dim, void* workspace, hipStream_t s) {
  const size_t desc = ((size_t)a.batch * (a.num_kv_heads / a.hpi) * 8 + 255) / 256 * 256;
  a.ws_desc = static_cast<int32_t*>(workspace);
  a.ws_rec = reinterpret_cast<float*>(static_cast<char*>(workspace) + desc);
  const bool aligned = (a.block_size % a.tc) == 0;
  const int G = a.num_q_heads / a.num_kv_heads;
  if (a.f16) {
    if (head_dim == 128) return dispatch_group<128, false, true>(a, G, aligned, s);
    return dispatch_group<64, false, true>(a, G, aligned, s);
  }
  if (head_dim == 128) return dispatch_group<128>(a, G, aligned, s);
  return dispatch_group<64>(a, G, aligned, s);
}

// Scratch of nvk_paged_decode_noalloc: one copy per GPU (the code object's
// device globals are instantiated on every device it is loaded on), held
// until the process ends.  Host code must not use the name `scratch` as a
// device address: its per-device address comes from hipGetSymbolAddress.
constexpr size_t kScratchBytes = NVK_NOALLOC_SCRATCH_BYTES;
__device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices];

// Device address of the current device's scratch, looked up once per device
// with that device current.
int scratch_of_current_device(int* dev_out, void** ptr) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return NVK_EUNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (p == nullptr || (uintptr_t)p % 256) return NVK_EALIGN;
    g_scratch_ptr[dev] = p;
  }
  *dev_out = dev;
  *ptr = g_scratch_ptr[dev];
  return NVK_OK;
}

// The scratch of the device `stream` belongs to, which must be the current one.
int scratch_for_stream(hipStream_t stream, void** ptr) {
  int dev = -1;
  const int st = scratch_of_current_device(&dev, ptr);
  if (st != NVK_OK) return st;
  if (stream != nullptr) {
    int sdev = -1;
    const hipError_t e = hipStreamGetDevice(stream, &sdev);
    if (e != hipSuccess) return (int)e;
    if (sdev != dev) return NVK_EINVAL;
  }
  return NVK_OK;
}

}  // namespace

extern "C" size_t nvk_paged_decode_workspace_size(int32_t batch, int32_t num_q_heads,
                                                  int32_t num_kv_heads, int32_t head_dim,
                                                  int32_t block_size, int32_t max_blocks) {
  if (batch <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || block_size <= 0 ||
      max_blocks <= 0 || num_q_heads % num_kv_heads || (head_dim != 64 && head_dim != 128))
    return 0;
  return decode_ws_bytes(batch, num_q_heads, num_kv_heads, head_dim, block_size, max_blocks);
}

extern "C" int nvk_paged_decode(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                                const void* k_cache, const void* v_cache,
                                const int32_t* block_tables, int64_t bt_stride,
                                const int32_t* context_lens, int32_t batch, int32_t num_q_heads,
                                int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                int32_t max_blocks, int32_t num_blocks, float scale, void* out,
                                int64_t out_stride_tok, int64_t out_stride_head, void* workspace,
                                size_t workspace_bytes, int32_t dtype, void* stream) {
  DecodeArgs a;
  size_t need = 0;
  const int st = decode_setup(q, q_stride_tok, q_stride_head, k_cache, v_cache, block_tables,
                              bt_stride, context_lens, batch, num_q_heads, num_kv_heads,
                              head_dim, block_size, max_blocks, num_blocks, scale, out,
                              out_stride_tok, out_stride_head, dtype, a, &need);
  if (st != NVK_OK || batch == 0) return st;
  if (workspace == nullptr || workspace_bytes < need) return NVK_EWORKSPACE;
  if ((uintptr_t)workspace % 256) return NVK_EALIGN;
  return decode_run(a, head_dim, workspace, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int nvk_paged_decode_noalloc(const void* q, int64_t q_stride_tok,
                                        int64_t q_stride_head, const void* k_cache,
                                        const void* v_cache, const int32_t* block_tables,
                                        int64_t bt_stride, const int32_t* context_lens,
                                        int32_t batch, int32_t num_q_heads,
                                        int32_t num_kv_heads, int32_t head_dim,
                                        int32_t block_size, int32_t max_blocks,
                                        int32_t num_blocks, float scale, void* out,
                                        int64_t out_stride_tok, int64_t out_stride_head,
                                        int32_t dtype, void* stream) {
  DecodeArgs a;
  size_t need = 0;
  const int st = decode_setup(q, q_stride_tok, q_stride_head, k_cache, v_cache, block_tables,
                              bt_stride, context_lens, batch, num_q_heads, num_kv_heads,
                              head_dim, block_size, max_blocks, num_blocks, scale, out,
                              out_stride_tok, out_stride_head, dtype, a, &need);
  if (st != NVK_OK || batch == 0) return st;
  if (need > kScratchBytes) return NVK_ESCRATCH;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  void* ws = nullptr;
  const int sst = scratch_for_stream(s, &ws);
  if (sst != NVK_OK) return sst;
  // Every descriptor and record the kernels read is written earlier in the
  // same call, so the scratch needs no clearing between calls.
  return decode_run(a, head_dim, ws, s);
}

extern "C" int nvk_paged_decode_noalloc_init(void) {
  int dev = -1;
  void* p = nullptr;
  return scratch_of_current_device(&dev, &p);
}

extern "C" int nvk_paged_decode_prologue(
    const void* qkv, int64_t qkv_row_stride, const int64_t* positions, const void* q_norm_weight,
    const void* k_norm_weight, float eps, const float* cos_sin_cache, int64_t cos_sin_row_stride,
    int64_t max_position, void* k_cache, void* v_cache, const int32_t* slot_mapping,
    int64_t cache_slots, const int32_t* block_tables, int64_t bt_stride,
    const int32_t* context_lens, int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
    int32_t head_dim, int32_t block_size, int32_t max_blocks, int32_t num_blocks, float scale,
    void* out, int64_t out_stride_tok, int64_t out_stride_head, void* workspace,
    size_t workspace_bytes, int32_t dtype, void* stream) {
  if (batch < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || block_size <= 0 || max_blocks <= 0 ||
      num_blocks < 0 || cache_slots < 0 || !(eps >= 0.f))
    return NVK_EINVAL;
  if (!(scale > 0.f)) return NVK_EINVAL;
  if ((dtype != NVK_DTYPE_BF16 && dtype != NVK_DTYPE_F16) || head_dim != nvk_qk::kHD)
    return NVK_EUNSUPPORTED;
  if (num_q_heads % num_kv_heads) return NVK_EINVAL;
  const int G = num_q_heads / num_kv_heads;
  if (G != 1 && G != 2 && G != 4 && G != 8) return NVK_EUNSUPPORTED;
  if (batch == 0) return NVK_OK;
  if (batch > kMaxBatch || num_kv_heads > 65535) return NVK_EUNSUPPORTED;
  if (!qkv || !positions || !q_norm_weight || !k_norm_weight || !cos_sin_cache || !k_cache ||
      !v_cache || !slot_mapping || !block_tables || !context_lens || !out)
    return NVK_EINVAL;
  if (bt_stride < max_blocks) return NVK_EINVAL;
  if ((int64_t)block_size * max_blocks > INT32_MAX) return NVK_EINVAL;
  if (max_position <= 0 || cos_sin_row_stride < head_dim) return NVK_EINVAL;
  if (qkv_row_stride < ((int64_t)num_q_heads + 2 * num_kv_heads) * head_dim) return NVK_EINVAL;
  const int tc = decode_tc(num_kv_heads, head_dim);
  if ((int64_t)batch * num_kv_heads * (((int64_t)block_size * max_blocks + tc - 1) / tc) >
      INT32_MAX)
    return NVK_EINVAL;
  if (((uintptr_t)qkv | (uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)out |
       (uintptr_t)q_norm_weight | (uintptr_t)k_norm_weight | (uintptr_t)cos_sin_cache) % 16)
    return NVK_EALIGN;
  if ((qkv_row_stride % 8) || (out_stride_tok % 8) || (out_stride_head % 8) ||
      (cos_sin_row_stride % 4))
    return NVK_EALIGN;
  const size_t need =
      decode_ws_bytes(batch, num_q_heads, num_kv_heads, head_dim, block_size, max_blocks);
  if (workspace == nullptr || workspace_bytes < need) return NVK_EWORKSPACE;
  if ((uintptr_t)workspace % 256) return NVK_EALIGN;

  DecodeArgs a = {};
  a.q = nullptr;
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
  a.hpi = decode_hpi(num_kv_heads, head_dim);
  a.tc = tc;
  a.n_waves = decode_waves(batch, num_kv_heads, head_dim, block_size, max_blocks);
  const size_t desc = ((size_t)batch * (num_kv_heads / a.hpi) * 8 + 255) / 256 * 256;
  a.ws_desc = static_cast<int32_t*>(workspace);
  a.ws_rec = reinterpret_cast<float*>(static_cast<char*>(workspace) + desc);
  a.qkv = static_cast<const uint16_t*>(qkv);
  a.qkv_row_stride = qkv_row_stride;
  a.positions = positions;
  a.q_weight = static_cast<const uint16_t*>(q_norm_weight);
  a.k_weight = static_cast<const uint16_t*>(k_norm_weight);
  a.eps = eps;
  a.cos_sin = cos_sin_cache;
  a.cos_sin_stride = cos_sin_row_stride;
  a.max_position = max_position;
  a.slot_mapping = slot_mapping;
  a.cache_slots = cache_slots;
  a.k_store = static_cast<uint16_t*>(k_cache);
  a.v_store = static_cast<uint16_t*>(v_cache);
  const bool aligned = (block_size % tc) == 0;
  a.f16 = dtype == NVK_DTYPE_F16;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (a.f16) return dispatch_group<128, true, true>(a, G, aligned, s);
  return dispatch_group<128, true>(a, G, aligned, s);
}
