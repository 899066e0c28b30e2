// Varlen causal prefill attention (new tokens over cached prefix + themselves)
// on gfx950 bf16 MFMA.
//
// Semantics: flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k,
// max_seqlen_q, max_seqlen_k, softmax_scale, causal=True, block_table) as
// called at nanovllm/layers/attention.py:64-70.  Query row i of a sequence
// with Lq queries and Lk keys sees key j iff j <= i + Lk - Lq (bottom-right
// aligned causal mask).  With block_table the keys are read from the paged
// cache (prefix-cache hit or a later chunk); without it from the dense k / v
// of the step.
//
// Tiling (MI355X):
//   * A workgroup = 4 waves owns one (sequence, kv head, query tile).  The
//     tile has 128 rows = (128/G) query tokens x the G query heads that share
//     the kv head, so every K/V tile staged in LDS feeds all G heads.  Row r
//     is token r/G, head r%G.
//   * Per 64-key tile: K is staged row-major in LDS ([key][d], padded), V is
//     staged transposed ([d][key], padded) with keys permuted inside each
//     group of 16 (bits 2 and 3 swapped).
//   * S^T = K Q^T uses v_mfma_f32_32x32x16_bf16 with K (from LDS) as the A
//     operand and the wave's Q fragment (registers, loaded once) as B.  In the
//     32x32 accumulator each lane then holds 32 keys of ONE query row, so the
//     row max / sum of the online softmax need one cross-lane step (lane^32).
//   * O^T = V^T P^T uses the same MFMA with V^T (from LDS) as A and the
//     probabilities as B straight from the S^T accumulators: the key order in
//     which a lane holds its 8 probabilities per 16-key step is exactly the
//     permuted order of the V^T tile, so P never leaves the registers.
//   * Global loads of the next key tile are issued before the MFMAs of the
//     current one (register staging); the grid runs the query tiles nearest
//     the end of each sequence (the ones with most keys) first.
#include "nvk_common.h"

namespace {

constexpr int HD = 128;
constexpr int kWaves = 4;
constexpr int kRows = 128;       // query rows per workgroup
constexpr int kKeys = 64;        // keys per tile
constexpr int kKPad = HD + 8;    // sK row stride (elements)
constexpr int kVPad = kKeys + 8; // sVt row stride (elements)

struct PrefillArgs {
  const uint16_t* q;
  int64_t q_stride_tok, q_stride_head, total_q;
  const uint16_t* k;
  const uint16_t* v;
  int64_t k_stride_tok, v_stride_tok, kv_stride_head, total_k;
  const int32_t* cu_q;
  const int32_t* cu_k;
  int batch;
  const int32_t* block_tables;  // null: dense k / v
  int64_t bt_stride;
  int max_blocks, block_size, bs_shift, num_blocks;
  int num_q_heads, num_kv_heads;
  float scale_log2;
  uint16_t* out;
  int64_t out_stride_tok, out_stride_head;
  int n_qtiles;
};

// How a workgroup finds its keys.
enum KvMode {
  kDense = 0,         // k / v rows of the step, key j of sequence s = row cu_k[s] + j
  kPagedAligned = 1,  // paged, block_size a multiple of 64: a key tile lies in one page
  kPagedAny = 2,      // paged, any other block size
};

// Raw buffer resource over [base, base + bytes): a load at an offset >= bytes
// returns zeros and touches no memory.  dword3 0x00020000 = 32-bit data
// format, the gfx9 setting for untyped buffer loads.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const uint16_t* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

template <int G, int MODE>
__global__ __launch_bounds__(256, 2) void varlen_prefill_kernel(PrefillArgs a) {
  constexpr int TQ = kRows / G;  // query tokens per workgroup

  const int kvh = blockIdx.x;
  const int s = blockIdx.y;
  const int qt = blockIdx.z;  // 0 = the tile that ends at the last query token
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int half = lane >> 5;  // 0/1: which 8-wide k slice this lane feeds
  const int l32 = lane & 31;

  const int q_row0 = a.cu_q[s];
  const int Lq = a.cu_q[s + 1] - q_row0;
  const int k_row0 = a.cu_k[s];
  const int Lk = a.cu_k[s + 1] - k_row0;
  const int q0 = Lq - (qt + 1) * TQ;  // first token of the tile (may be < 0)
  if (Lq <= 0 || q0 + TQ <= 0) return;

  int Lk_eff = Lk;
  if (MODE != kDense) {
    const int64_t cap = (int64_t)a.max_blocks * a.block_size;
    if ((int64_t)Lk_eff > cap) Lk_eff = (int)cap;
  } else {
    const int64_t cap = a.total_k - k_row0;  // rows past the end of k / v are absent
    if ((int64_t)Lk_eff > cap) Lk_eff = cap > 0 ? (int)cap : 0;
  }
  const int diag = Lk - Lq;                    // row i sees keys j <= i + diag
  int n_keys = (q0 + TQ - 1) + diag + 1;       // keys visible to the last row
  if (n_keys > Lk_eff) n_keys = Lk_eff;
  const int t_first = q0 < 0 ? 0 : q0;
  const int unmasked_keys = t_first + diag + 1;  // keys visible to every valid row

  __shared__ __attribute__((aligned(16))) uint16_t sK[kKeys * kKPad];
  __shared__ __attribute__((aligned(16))) uint16_t sVt[HD * kVPad];

  const int32_t* bt_row = MODE != kDense ? a.block_tables + (int64_t)s * a.bt_stride : nullptr;

  // ---- this lane's query row and its Q fragment (B operand of S^T) --------
  const int row = wave * 32 + l32;
  const int tok = q0 + row / G;
  const int head = kvh * G + row % G;
  const bool row_valid = tok >= 0 && tok < Lq;
  nvk_bf16x8 qf[HD / 16];
  {
    const int64_t qrow = (int64_t)q_row0 + tok;
    const bool ok = row_valid && qrow < a.total_q;
    const uint16_t* qp = a.q + qrow * a.q_stride_tok + (int64_t)head * a.q_stride_head + 8 * half;
#pragma unroll
    for (int ks = 0; ks < HD / 16; ++ks) {
      nvk_u32x4 w = {0, 0, 0, 0};
      if (ok) w = *reinterpret_cast<const nvk_u32x4*>(qp + 16 * ks);
      qf[ks] = __builtin_bit_cast(nvk_bf16x8, w);
    }
  }
  const int row_limit = tok + diag;  // last visible key of this row

  // ---- loader roles ----------------------------------------------------------
  // K: chunk c = tid + 256*i -> key (tid>>4) + 16 i, d chunk (tid & 15).
  // V: keys 4*(tid&15) .. +3, d chunk (tid >> 4).
  const int k_key0 = tid >> 4;
  const int k_dc = tid & 15;
  const int v_kg = tid & 15;
  const int v_dc = tid >> 4;
  const int v_kg_perm = (v_kg & ~3) | ((v_kg & 1) << 1) | ((v_kg & 2) >> 1);

  nvk_u32x4 kst[4], vst[4];
  // Dense and aligned-paged tiles: the tile's keys are consecutive rows of one
  // buffer, so each tile gets one buffer resource sized to its valid rows; a
  // key past the end (or on an invalid page) falls outside it and loads zeros.
  // The page id of the next tile is fetched one tile ahead, so no load waits
  // on the block table.
  const uint32_t k_row_bytes =
      MODE == kDense ? (uint32_t)a.k_stride_tok * 2u : (uint32_t)a.num_kv_heads * HD * 2u;
  const uint32_t v_row_bytes =
      MODE == kDense ? (uint32_t)a.v_stride_tok * 2u : (uint32_t)a.num_kv_heads * HD * 2u;
  const int last_page = n_keys > 0 ? (n_keys - 1) / a.block_size : 0;
  auto fetch_page = [&](int kt) -> int {
    int logical = a.bs_shift >= 0 ? (kt * kKeys) >> a.bs_shift : (kt * kKeys) / a.block_size;
    logical = logical < last_page ? logical : last_page;
    asm volatile("" : "+v"(logical));  // keep the table read a vector load
    return bt_row[logical];
  };
  int page_next = 0;
  if (MODE == kPagedAligned && n_keys > 0) page_next = fetch_page(0);

  // kPagedAny: per-key page lookup; a missing key reads the sequence's first q
  // row (finite), its score is masked to -inf and its probability is 0.
  const uint16_t* dummy = a.q + (int64_t)q_row0 * a.q_stride_tok;
  const int64_t paged_row_elems = (int64_t)a.num_kv_heads * HD;

  auto load_tile = [&](int kt) {
    const int base = kt * kKeys;
    if constexpr (MODE == kPagedAny) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int pos = base + k_key0 + 16 * i;
        const int64_t r = pos < n_keys ? nvk_paged_row(bt_row, pos, a.block_size, a.bs_shift,
                                                       a.num_blocks) : -1;
        const uint16_t* p = r >= 0 ? a.k + r * paged_row_elems + kvh * HD + 8 * k_dc : dummy;
        kst[i] = *reinterpret_cast<const nvk_u32x4*>(p);
      }
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int pos = base + 4 * v_kg + jj;
        const int64_t r = pos < n_keys ? nvk_paged_row(bt_row, pos, a.block_size, a.bs_shift,
                                                       a.num_blocks) : -1;
        const uint16_t* p = r >= 0 ? a.v + r * paged_row_elems + kvh * HD + 8 * v_dc : dummy;
        vst[jj] = *reinterpret_cast<const nvk_u32x4*>(p);
      }
    } else {
      const int rem = n_keys - base < kKeys ? n_keys - base : kKeys;  // valid rows, > 0
      const uint16_t* kb;
      const uint16_t* vb;
      uint32_t k_bytes = (uint32_t)rem * k_row_bytes;
      uint32_t v_bytes = (uint32_t)rem * v_row_bytes;
      if constexpr (MODE == kDense) {
        kb = a.k + (int64_t)(k_row0 + base) * a.k_stride_tok + (int64_t)kvh * a.kv_stride_head;
        vb = a.v + (int64_t)(k_row0 + base) * a.v_stride_tok + (int64_t)kvh * a.kv_stride_head;
      } else {
        const int page = __builtin_amdgcn_readfirstlane(page_next);
        if (kt + 1 < (n_keys + kKeys - 1) / kKeys) page_next = fetch_page(kt + 1);
        const int logical = a.bs_shift >= 0 ? base >> a.bs_shift : base / a.block_size;
        const int64_t row = (int64_t)page * a.block_size + (base - logical * a.block_size);
        const bool ok = (uint32_t)page < (uint32_t)a.num_blocks;
        kb = ok ? a.k + row * paged_row_elems + kvh * HD : a.k;
        vb = ok ? a.v + row * paged_row_elems + kvh * HD : a.v;
        k_bytes = ok ? k_bytes : 0u;
        v_bytes = ok ? v_bytes : 0u;
      }
      const __amdgpu_buffer_rsrc_t rk = tile_rsrc(kb, k_bytes);
      const __amdgpu_buffer_rsrc_t rv = tile_rsrc(vb, v_bytes);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        kst[i] = __builtin_bit_cast(nvk_u32x4, __builtin_amdgcn_raw_buffer_load_b128(
            rk, (k_key0 + 16 * i) * k_row_bytes + 16 * k_dc, 0, 0));
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
        vst[jj] = __builtin_bit_cast(nvk_u32x4, __builtin_amdgcn_raw_buffer_load_b128(
            rv, (4 * v_kg + jj) * v_row_bytes + 16 * v_dc, 0, 0));
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<nvk_u32x4*>(&sK[(k_key0 + 16 * i) * kKPad + 8 * k_dc]) = kst[i];
    const uint32_t r0[4] = {vst[0].x, vst[0].y, vst[0].z, vst[0].w};
    const uint32_t r1[4] = {vst[1].x, vst[1].y, vst[1].z, vst[1].w};
    const uint32_t r2[4] = {vst[2].x, vst[2].y, vst[2].z, vst[2].w};
    const uint32_t r3[4] = {vst[3].x, vst[3].y, vst[3].z, vst[3].w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
      nvk_u32x2 w;
      w.x = __builtin_amdgcn_perm(r1[e >> 1], r0[e >> 1], sel);
      w.y = __builtin_amdgcn_perm(r3[e >> 1], r2[e >> 1], sel);
      *reinterpret_cast<nvk_u32x2*>(&sVt[(8 * v_dc + e) * kVPad + 4 * v_kg_perm]) = w;
    }
  };

  nvk_f32x16 acc_o[HD / 32];
#pragma unroll
  for (int db = 0; db < HD / 32; ++db) acc_o[db] = nvk_f32x16{};
  float m_run = -INFINITY;  // running max, log2 units (already scaled)
  float l_run = 0.f;        // this lane's share of the row sum

  const int n_tiles = n_keys > 0 ? (n_keys + kKeys - 1) / kKeys : 0;
  if (n_tiles > 0) load_tile(0);

  for (int kt = 0; kt < n_tiles; ++kt) {
    store_tile();
    __syncthreads();
    if (kt + 1 < n_tiles) load_tile(kt + 1);

    // ---- S^T = K Q^T : two 32-key blocks ------------------------------------
    nvk_f32x16 acc_s[2];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      acc_s[mb] = nvk_f32x16{};
      const uint16_t* kp = &sK[(32 * mb + l32) * kKPad + 8 * half];
#pragma unroll
      for (int ks = 0; ks < HD / 16; ++ks) {
        const nvk_bf16x8 kf = *reinterpret_cast<const nvk_bf16x8*>(kp + 16 * ks);
        acc_s[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[ks], acc_s[mb], 0, 0, 0);
      }
    }

    // ---- mask (only tiles that cross the diagonal or the end of the keys) ---
    const int kbase = kt * kKeys;
    if (kbase + kKeys > unmasked_keys || kbase + kKeys > n_keys || !row_valid) {
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = kbase + 32 * mb + 8 * (i >> 2) + 4 * half + (i & 3);
          const bool vis = row_valid && key <= row_limit && key < n_keys;
          acc_s[mb][i] = vis ? acc_s[mb][i] : -INFINITY;
        }
      }
    }

    // ---- online softmax (row = l32, keys split across lane halves) ----------
    float mt = -INFINITY;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
      for (int i = 0; i < 16; ++i) mt = fmaxf(mt, acc_s[mb][i]);
    }
    mt = fmaxf(mt, nvk_xor_lane<32>(mt)) * a.scale_log2;
    const float m_new = fmaxf(m_run, mt);
    const float moff = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = nvk_fast_exp2(m_run - moff);
    m_run = m_new;
    float psum = 0.f;
    nvk_bf16x8 pf[4];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float p0 = nvk_fast_exp2(fmaf(acc_s[mb][8 * sub + 2 * e], a.scale_log2, -moff));
          const float p1 = nvk_fast_exp2(fmaf(acc_s[mb][8 * sub + 2 * e + 1], a.scale_log2, -moff));
          psum += p0 + p1;
          w[e] = nvk_pack_bf16x2(p0, p1);
        }
        pf[2 * mb + sub] = __builtin_bit_cast(nvk_bf16x8, nvk_u32x4{w[0], w[1], w[2], w[3]});
      }
    }
    l_run = l_run * alpha + psum;
#pragma unroll
    for (int db = 0; db < HD / 32; ++db) acc_o[db] *= alpha;

    // ---- O^T += V^T P^T ------------------------------------------------------
#pragma unroll
    for (int db = 0; db < HD / 32; ++db) {
      const uint16_t* vp = &sVt[(32 * db + l32) * kVPad + 8 * half];
#pragma unroll
      for (int ks = 0; ks < kKeys / 16; ++ks) {
        const nvk_bf16x8 vf = *reinterpret_cast<const nvk_bf16x8*>(vp + 16 * ks);
        acc_o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf[ks], acc_o[db], 0, 0, 0);
      }
    }
    __syncthreads();
  }

  // ---- epilogue: normalise and store the row -----------------------------------
  if (!row_valid) return;
  const float l_tot = l_run + nvk_xor_lane<32>(l_run);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  uint16_t* op = a.out + ((int64_t)q_row0 + tok) * a.out_stride_tok + (int64_t)head * a.out_stride_head;
#pragma unroll
  for (int db = 0; db < HD / 32; ++db) {
#pragma unroll
    for (int grp = 0; grp < 4; ++grp) {
      const int d = 32 * db + 8 * grp + 4 * half;
      nvk_u32x2 w;
      w.x = nvk_pack_bf16x2(acc_o[db][4 * grp] * inv, acc_o[db][4 * grp + 1] * inv);
      w.y = nvk_pack_bf16x2(acc_o[db][4 * grp + 2] * inv, acc_o[db][4 * grp + 3] * inv);
      *reinterpret_cast<nvk_u32x2*>(op + d) = w;
    }
  }
}

template <int G>
int launch_prefill(const PrefillArgs& a, hipStream_t stream) {
  dim3 grid(a.num_kv_heads, a.batch, a.n_qtiles);
  if (!a.block_tables)
    hipLaunchKernelGGL((varlen_prefill_kernel<G, kDense>), grid, dim3(256), 0, stream, a);
  else if (a.block_size % kKeys == 0)
    hipLaunchKernelGGL((varlen_prefill_kernel<G, kPagedAligned>), grid, dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((varlen_prefill_kernel<G, kPagedAny>), grid, dim3(256), 0, stream, a);
  return nvk_launch_status();
}

}  // namespace

extern "C" int nvk_varlen_prefill(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                                  int64_t total_q, const void* k, const void* v,
                                  int64_t k_stride_tok, int64_t v_stride_tok,
                                  int64_t kv_stride_head, int64_t total_k,
                                  const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                  int32_t batch, int32_t max_seqlen_q,
                                  const int32_t* block_tables, int64_t bt_stride,
                                  int32_t max_blocks, int32_t block_size, int32_t num_blocks,
                                  int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                  float scale, void* out, int64_t out_stride_tok,
                                  int64_t out_stride_head, int32_t dtype, void* stream) {
  if (batch < 0 || max_seqlen_q < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || total_q < 0 ||
      total_k < 0)
    return NVK_EINVAL;
  if (!(scale > 0.f)) return NVK_EINVAL;  // the row max is taken before scaling
  if (dtype != NVK_DTYPE_BF16) return NVK_EUNSUPPORTED;
  if (head_dim != HD) return NVK_EUNSUPPORTED;
  if (num_q_heads % num_kv_heads) return NVK_EINVAL;
  const int G = num_q_heads / num_kv_heads;
  if (G != 1 && G != 2 && G != 4 && G != 8) return NVK_EUNSUPPORTED;
  if (batch == 0 || max_seqlen_q == 0) return NVK_OK;
  if (!q || !k || !v || !cu_seqlens_q || !cu_seqlens_k || !out) return NVK_EINVAL;
  if (block_tables) {
    if (block_size <= 0 || max_blocks <= 0 || num_blocks < 0 || bt_stride < max_blocks)
      return NVK_EINVAL;
    // a key tile's byte offsets are 32-bit: 64 rows of num_kv_heads*head_dim
    if ((int64_t)num_kv_heads * HD >= (1 << 23)) return NVK_EINVAL;
  } else {
    if (k_stride_tok % 8 || v_stride_tok % 8 || kv_stride_head % 8) return NVK_EALIGN;
    if (k_stride_tok < HD || v_stride_tok < HD || k_stride_tok >= (1 << 23) ||
        v_stride_tok >= (1 << 23) || kv_stride_head < 0)
      return NVK_EINVAL;
  }
  if (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v) % 16) return NVK_EALIGN;
  if ((q_stride_tok % 8) || (q_stride_head % 8)) return NVK_EALIGN;
  if (((uintptr_t)out % 8) || (out_stride_tok % 4) || (out_stride_head % 4)) return NVK_EALIGN;
  if (batch > 65535) return NVK_EINVAL;

  PrefillArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.q_stride_tok = q_stride_tok;
  a.q_stride_head = q_stride_head;
  a.total_q = total_q;
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.k_stride_tok = k_stride_tok;
  a.v_stride_tok = v_stride_tok;
  a.kv_stride_head = kv_stride_head;
  a.total_k = total_k;
  a.cu_q = cu_seqlens_q;
  a.cu_k = cu_seqlens_k;
  a.batch = batch;
  a.block_tables = block_tables;
  a.bt_stride = bt_stride;
  a.max_blocks = max_blocks;
  a.block_size = block_size;
  a.bs_shift = block_tables ? nvk_log2_exact(block_size) : -1;
  a.num_blocks = num_blocks;
  a.num_q_heads = num_q_heads;
  a.num_kv_heads = num_kv_heads;
  a.scale_log2 = scale * NVK_LOG2E;
  a.out = static_cast<uint16_t*>(out);
  a.out_stride_tok = out_stride_tok;
  a.out_stride_head = out_stride_head;
  const int TQ = kRows / G;
  a.n_qtiles = (max_seqlen_q + TQ - 1) / TQ;
  if (a.n_qtiles > 65535) return NVK_EINVAL;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (G) {
    case 1: return launch_prefill<1>(a, s);
    case 2: return launch_prefill<2>(a, s);
    case 4: return launch_prefill<4>(a, s);
    default: return launch_prefill<8>(a, s);
  }
}
