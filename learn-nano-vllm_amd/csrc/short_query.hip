// Paged attention for short query ranges on gfx950 bf16 MFMA: every sequence
// has at most 16 rows of (query token x query head) per kv head, e.g. the
// verification step of speculative decoding (6 queries x 2 heads).  Same
// semantics as the prefill kernel (flash_attn_varlen_func with block_table,
// bottom-right causal mask, nanovllm/layers/attention.py:64-70).
//
// The 128-row query tile of the prefill kernel would spend 7/8 of its MFMA
// and LDS work on empty rows here, and one tile per (sequence, kv head) cannot
// fill the GPU.  This kernel works like the decode kernel instead:
//   * a wave owns all 16 rows of a (sequence, kv head) group and streams its
//     keys in chunks of 32; the chunks of all groups are cut into equal
//     contiguous ranges, one per wave of a persistent grid of one workgroup
//     per CU (stream-K), so every wave moves the same number of bytes;
//   * S^T = K Q^T on v_mfma_f32_16x16x32_bf16 with K in the A-operand
//     layout: lane (g, r) holds key row r of a 16-key block, k-step ks
//     covering d = 32ks + 8g .. +7.  The head dimension is permuted the same
//     way in Q, which leaves q . k unchanged.  When a wave streams many
//     chunks, K goes through LDS like V (full 256-byte rows per DMA load,
//     16-byte chunks XOR-swizzled by row & 15, then one ds_read_b128 per
//     operand); for short ranges it is loaded straight into the operand
//     layout (the four lanes of a key read 64 contiguous bytes per load), one
//     LDS round trip less per chunk.  Measured (interleaved A/B): 32 x 6
//     queries over U{1024..8192} 114.1 -> 109.2 us, 64 x 4 over U{512..4096}
//     127.2 -> 121.3 us; 8 x 6 over U{1024..4096} 29.4 us in registers
//     against 31.1 us through LDS;
//   * the next chunk's K loads go out as soon as the S products have consumed
//     the registers, its V loads once the P V products have read the LDS
//     buffer, so a wave always has a chunk in flight;
//   * the accumulator gives lane (g, r) keys 4g..4g+3 of row r, so P^T for a
//     pair of 16-key blocks is the B operand of O^T += V^T P^T with the keys
//     in the order {block 0: 4g..4g+3, block 1: 4g..4g+3}; V^T in that key
//     order comes from the wave's LDS copy of the chunk by two
//     ds_read_b64_tr_b16 per operand (16-byte chunks of each 256-byte row
//     XOR-swizzled by 2*(row & 7): conflict-free);
//   * online softmax per chunk in log2 units; groups cut between waves leave
//     (O, m, l) records that a combine kernel merges, as in the decode (with
//     16 waves folding interleaved slices of the parts when groups are cut
//     into many).
#include "nvk_common.h"
#include "short_query.h"

namespace {

constexpr int HD = 128;
constexpr int kR = 16;                        // rows per wave (tokens x heads of a kv head)
// Chunks of 32 keys on one workgroup per CU (1024 waves, 16 KiB of K and V
// in flight per wave).  Measured on MI355X (interleaved A/B, 32 sequences x 6
// queries over U{1024..8192}; 8 x 6 over U{1024..4096}): 64-key chunks on two
// workgroups per CU 121.0 / 33.1 us, on one 114.7 / 30.4 us; 32-key chunks on
// two 119.2 / 33.4 us, on one 113.6 / 29.6 us; 384 workgroups (uneven over
// the CUs) 134.6 us.  More bytes in flight than this only queue up.
constexpr int kCK = 32;                       // keys per chunk
constexpr int kKB = kCK / 16;                 // 16-key blocks of a chunk
constexpr int kPairs = kCK / 32;              // 32-key pairs (one P.V k-step each)
constexpr int kWavesPerWG = 4;
constexpr int kMaxWGs = 256;                  // one workgroup per CU
constexpr int kMinChunks = 2;                 // a wave streams at least this many chunks
#ifndef NVK_SQ_KLDS_MIN
#define NVK_SQ_KLDS_MIN 32
#endif
constexpr int kKldsMinChunks = NVK_SQ_KLDS_MIN;  // chunks per wave (static bound) for K in LDS
constexpr int kMaxBatch = 2048;
constexpr int kRowBytes = HD * 2;
constexpr int kChunkBytes = kCK * kRowBytes;  // a wave's V staging in LDS
constexpr int kRec = HD + 4;                  // record floats per row: O, m, l, pad

typedef __attribute__((address_space(4))) const int32_t sq_const_i32;
typedef __attribute__((address_space(3))) void* sq_lds_ptr;

struct SqArgs {
  ShortQueryParams p;
  float scale_log2;
  int G;
  int cap;             // max_blocks * block_size: keys a table can name
  int64_t row_elems;   // Hkv * HD
  uint32_t row_bytes;  // row_elems * 2
  int32_t* desc;       // [batch][Hkv] x 2: first and last wave of the group, -1 if empty
  float* rec;          // [n_waves][2][kR][kRec]
  int n_waves;
};

__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

__device__ __forceinline__ int seq_keys(const SqArgs& a, int s) {
  int lk = ((sq_const_i32*)a.p.cu_k)[s + 1] - ((sq_const_i32*)a.p.cu_k)[s];
  lk = lk < 0 ? 0 : lk;
  return lk > a.cap ? a.cap : lk;
}
__device__ __forceinline__ int seq_queries(const SqArgs& a, int s) {
  return ((sq_const_i32*)a.p.cu_q)[s + 1] - ((sq_const_i32*)a.p.cu_q)[s];
}
__device__ __forceinline__ int seq_chunks(const SqArgs& a, int s) {
  return seq_queries(a, s) > 0 ? (seq_keys(a, s) + kCK - 1) / kCK : 0;
}

// Exclusive prefix of chunks per sequence into s_cs[0..B]; returns the total.
__device__ int chunk_prefix(const SqArgs& a, int* s_cs, int* s_wsum) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int B = a.p.batch;
  const int per = (B + 255) / 256;
  const int b0 = tid * per;
  int local = 0;
  for (int i = 0; i < per; ++i)
    if (b0 + i < B) local += seq_chunks(a, b0 + i);
  const int x = nvk_wave_scan_add(local);  // inclusive over the wave
  if (lane == 63) s_wsum[wave] = x;
  __syncthreads();
  int run = x - local;
  for (int w = 0; w < wave; ++w) run += s_wsum[w];
  for (int i = 0; i < per; ++i) {
    if (b0 + i < B) {
      s_cs[b0 + i] = run;
      run += seq_chunks(a, b0 + i);
    }
  }
  const int total = s_wsum[0] + s_wsum[1] + s_wsum[2] + s_wsum[3];
  if (tid == 0) s_cs[B] = total;
  __syncthreads();
  return total;
}

__device__ __forceinline__ int64_t active_waves(int64_t T, int64_t P) {
  int64_t p = T / kMinChunks;
  if (p > P) p = P;
  return p < 1 ? 1 : p;
}
__device__ __forceinline__ int64_t range_begin(int64_t w, int64_t T, int64_t P) { return w * T / P; }
__device__ __forceinline__ int64_t chunk_owner(int64_t c, int64_t T, int64_t P) {
  return ((c + 1) * P - 1) / T;
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) { return (uint32_t)(size_t)(sq_lds_ptr)(p); }

// Raw buffer descriptor over [base, base + bytes) (loads past it return zeros).
__device__ __forceinline__ nvk_u32x4 rsrc_of(const uint16_t* base, uint32_t bytes) {
  const uint64_t b = (uint64_t)(uintptr_t)base;
  return nvk_u32x4{(uint32_t)uniform((int)(uint32_t)b), (uint32_t)uniform((int)((b >> 32) & 0xFFFFu)),
                   (uint32_t)uniform((int)bytes), 0x00020000u};
}
// 16 bytes per lane straight into LDS: lane l writes [dst + 16 l, +16).  The
// rows are read once: non-temporal (measured 6 % faster on the verification
// step than the default policy).
__device__ __forceinline__ void lds_load(const nvk_u32x4& rsrc, uint32_t voffset, uint32_t dst) {
  asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, 0 offen nt lds"
               :: "v"(voffset), "s"(rsrc), "s"(dst) : "memory", "m0");
}
__device__ __forceinline__ void wait_loads() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

__device__ __forceinline__ float sum_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float max_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// KLDS: K staged in LDS by full-row DMA loads like V (then read in the MFMA
// operand layout), instead of loaded straight into the operand layout.
template <bool F16, bool KLDS>
__global__ __launch_bounds__(64 * kWavesPerWG, 2) void short_query_kernel(SqArgs a) {
  using E = NvkElt<F16>;
  typedef typename E::vec8 vec8;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[(KLDS ? 2 : 1) * kWavesPerWG * kChunkBytes];
  __shared__ int s_cs[kMaxBatch + 1];
  __shared__ int s_wsum[kWavesPerWG];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int r = lane & 15, g = lane >> 4;
  const int Hkv = a.p.num_kv_heads;

  const int S = chunk_prefix(a, s_cs, s_wsum);
  if (blockIdx.x == 0) {  // groups no wave visits (no query or no key)
    for (int e = tid; e < a.p.batch * Hkv; e += 256) {
      const int b = e / Hkv;
      if (s_cs[b + 1] == s_cs[b]) *reinterpret_cast<int2*>(a.desc + 2 * e) = make_int2(-1, -1);
    }
  }
  const int64_t T = (int64_t)Hkv * S;
  const int64_t P = active_waves(T, a.n_waves);
  const int wave = uniform(tid >> 6);
  const int64_t w = (int64_t)blockIdx.x * kWavesPerWG + wave;
  if (w >= P || T == 0) return;
  const int64_t c0 = range_begin(w, T, P), c1 = range_begin(w + 1, T, P);
  if (c0 >= c1) return;

  // first chunk: last sequence s with Hkv * s_cs[s] <= c0
  int s = nvk_last_le(s_cs, a.p.batch, Hkv, c0, lane);
  int n = uniform(s_cs[s + 1] - s_cs[s]);
  int kvh, k;
  {
    const int rr = (int)(c0 - (int64_t)Hkv * s_cs[s]);
    kvh = uniform(rr / n);
    k = uniform(rr % n);
  }
  bool started_here = k == 0;

  uint8_t* vbuf = lds + wave * kChunkBytes;
  const uint32_t vbase = (uint32_t)uniform((int)lds_addr(vbuf));
  // V tr-read addresses of this lane (pair 0, d block 0): rows 4g + c/4 (lo)
  // and 16 + 4g + c/4 (hi), 8 bytes at logical column 4(c%4) of d block db,
  // physical byte row*256 + 32*(db ^ (row & 7)) + 8*(c%4).
  const int rlo = 4 * g + (r >> 2), rhi = 16 + rlo;
  const uint32_t tr_lo = vbase + rlo * kRowBytes + 8 * (r & 3);
  const uint32_t tr_hi = vbase + rhi * kRowBytes + 8 * (r & 3);
  const int sw_lo = rlo & 7, sw_hi = rhi & 7;
  // DMA lane offsets: load j covers rows 4j..4j+3, lane l -> row 4j + l/16,
  // slot l%16, logical chunk (l%16) ^ 2*(row & 7).
  uint32_t v_voff[kCK / 4], k_voff[kCK / 4];
#pragma unroll
  for (int j = 0; j < kCK / 4; ++j) {
    const int row = 4 * j + g;
    v_voff[j] = (uint32_t)row * a.row_bytes + 16u * (uint32_t)((r) ^ (2 * (row & 7)));
    k_voff[j] = (uint32_t)row * a.row_bytes + 16u * (uint32_t)(r ^ (row & 15));
  }
  // KLDS: slot c ^ (row & 15) of a K row holds its logical 16-byte chunk c, so
  // the operand reads (16 rows, one chunk each, per 16 lanes) are conflict free.
  const uint32_t kbase_l =
      KLDS ? (uint32_t)uniform((int)lds_addr(lds + (kWavesPerWG + wave) * kChunkBytes)) : 0u;

  // per-group state
  vec8 qf[HD / 32];
  nvk_f32x4 acc_o[HD / 16];
  float m_run = -INFINITY, l_part = 0.f;
  int q_row0 = 0, Lq = 0, nkeys = 0, diag = 0, tok = 0, head = 0;
  bool row_valid = false;
  const int32_t* bt_row = nullptr;

  auto start_group = [&]() {
    q_row0 = ((sq_const_i32*)a.p.cu_q)[s];
    Lq = seq_queries(a, s);
    const int lk_raw = ((sq_const_i32*)a.p.cu_k)[s + 1] - ((sq_const_i32*)a.p.cu_k)[s];
    nkeys = seq_keys(a, s);
    diag = lk_raw - Lq;
    tok = r / a.G;
    head = kvh * a.G + r % a.G;
    row_valid = tok < Lq;
    bt_row = a.p.block_tables + (int64_t)s * a.p.bt_stride;
    // Q in the permuted head-dimension order of the K operand (see below)
    const uint16_t* qp = a.p.q + (int64_t)(q_row0 + tok) * a.p.q_stride_tok +
                         (int64_t)head * a.p.q_stride_head + 8 * g;
#pragma unroll
    for (int ks = 0; ks < HD / 32; ++ks) {
      nvk_u32x4 v = {0u, 0u, 0u, 0u};
      if (row_valid) v = *reinterpret_cast<const nvk_u32x4*>(qp + 32 * ks);
      qf[ks] = __builtin_bit_cast(vec8, v);
    }
#pragma unroll
    for (int db = 0; db < HD / 16; ++db) acc_o[db] = nvk_f32x4{0.f, 0.f, 0.f, 0.f};
    m_run = -INFINITY;
    l_part = 0.f;
  };

  // Sources of chunk kk of group (sequence ss, kv head hh): the K rows this
  // lane loads and the V buffer descriptor (rows past the keys read zeros).
  struct ChunkSrc {
    const uint16_t* k;  // this lane's K row (a dummy in-bounds row for a missing key)
    nvk_u32x4 kr;       // KLDS: the K rows' buffer descriptor (SGPRs)
    nvk_u32x4 v;        // SGPRs
  };
  auto chunk_src = [&](int ss, int hh, int kk, const int32_t* btr, int nk) {
    const int kbase = kk * kCK;
    const int logical = kbase / a.p.block_size;
    const int page = ((sq_const_i32*)btr)[logical];
    const bool page_ok = page >= 0 && page < a.p.num_blocks;
    int rem = nk - kbase;
    rem = rem > kCK ? kCK : rem;
    rem = page_ok ? rem : 0;
    const int64_t row0 =
        page_ok ? (int64_t)page * a.p.block_size + (kbase - logical * a.p.block_size) : 0;
    (void)ss;
    ChunkSrc cs;
    cs.k = (r < rem ? a.p.k_cache + (row0 + r) * a.row_elems + hh * HD : a.p.k_cache) + 8 * g;
    // key blocks 1..3 are rows 16, 32, 48 further; a missing one reads the dummy row
    if constexpr (KLDS)
      cs.kr = rsrc_of(a.p.k_cache + row0 * a.row_elems + hh * HD, (uint32_t)rem * a.row_bytes);
    cs.v = rsrc_of(a.p.v_cache + row0 * a.row_elems + hh * HD, (uint32_t)rem * a.row_bytes);
    return cs;
  };
  // K of a chunk into the A-operand layout: lane (g, r) of key block kb holds
  // key 16 kb + r, and its k-step ks covers d = 32 ks + 8 g .. +7 (the head
  // dimension is permuted identically in Q, which leaves q . k unchanged), so
  // the four lanes of a key read 64 contiguous bytes per load.
  auto issue_k = [&](const ChunkSrc& cs, int rem_rows, vec8 (&kf)[kKB][HD / 32]) {
    if constexpr (KLDS) {
#pragma unroll
      for (int j = 0; j < kCK / 4; ++j) lds_load(cs.kr, k_voff[j], kbase_l + j * 4 * kRowBytes);
      return;
    }
#pragma unroll
    for (int kb = 0; kb < kKB; ++kb) {
      const bool ok = 16 * kb + r < rem_rows;
      const uint16_t* src = ok ? cs.k + (int64_t)16 * kb * a.row_elems : a.p.k_cache + 8 * g;
#pragma unroll
      for (int ks = 0; ks < HD / 32; ++ks)
        kf[kb][ks] = __builtin_bit_cast(vec8, *reinterpret_cast<const nvk_u32x4*>(src + 32 * ks));
    }
  };
  auto issue_v = [&](const ChunkSrc& cs) {
#pragma unroll
    for (int j = 0; j < kCK / 4; ++j) lds_load(cs.v, v_voff[j], vbase + j * 4 * kRowBytes);
  };
  auto rows_of = [&](int kk, const int32_t* btr, int nk) {
    const int kbase = kk * kCK;
    const int page = ((sq_const_i32*)btr)[kbase / a.p.block_size];
    int rem = nk - kbase;
    rem = rem > kCK ? kCK : rem;
    return (page >= 0 && page < a.p.num_blocks) ? rem : 0;
  };

  start_group();
  vec8 kf[kKB][HD / 32];
  {
    const ChunkSrc cs = chunk_src(s, kvh, k, bt_row, nkeys);
    issue_k(cs, rows_of(k, bt_row, nkeys), kf);
    issue_v(cs);
  }

  for (int64_t c = c0;; ++c) {
    wait_loads();  // K registers and the V buffer of chunk k
    const int kbase = k * kCK;

    // ---- S^T = K Q^T (lane: keys 16kb + 4g + i of row r)
    nvk_f32x4 sacc[kKB];
#pragma unroll
    for (int kb = 0; kb < kKB; ++kb) {
      sacc[kb] = nvk_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < HD / 32; ++ks) {
        if constexpr (KLDS) {
          const uint32_t ka = kbase_l + (16 * kb + r) * kRowBytes + 16 * ((4 * ks + g) ^ r);
          kf[kb][ks] = *reinterpret_cast<const __attribute__((address_space(3))) vec8*>((size_t)ka);
        }
        sacc[kb] = E::mfma16x16x32(kf[kb][ks], qf[ks], sacc[kb]);
      }
    }

    // ---- the next chunk's position; its K loads go out now (kf is free)
    const bool last = c + 1 == c1;
    const bool group_end = k == n - 1;
    int ns = s, nkvh = kvh, nk = k + 1, nn = n;
    if (group_end) {
      nk = 0;
      if (++nkvh == Hkv) {
        nkvh = 0;
        int b = s + 1;
        if (!last)
          while (s_cs[b + 1] == s_cs[b]) ++b;  // a next chunk exists
        ns = uniform(b);
        nn = last ? 0 : uniform(s_cs[ns + 1] - s_cs[ns]);
      }
    }
    ChunkSrc nsrc;
    if (!last) {
      const int32_t* nbt = a.p.block_tables + (int64_t)ns * a.p.bt_stride;
      const int nkeys_n = ns == s ? nkeys : seq_keys(a, ns);
      nsrc = chunk_src(ns, nkvh, nk, nbt, nkeys_n);
      // KLDS: this chunk's K reads are done before its buffer is refilled
      if constexpr (KLDS) asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      issue_k(nsrc, rows_of(nk, nbt, nkeys_n), kf);
    }

    // ---- mask, row max, online softmax
    const int row_limit = tok + diag;  // last visible key of the row
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < kKB; ++kb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = kbase + 16 * kb + 4 * g + i;
        const bool vis = row_valid && key < nkeys && key <= row_limit;
        sacc[kb][i] = vis ? sacc[kb][i] : -INFINITY;
        mx = fmaxf(mx, sacc[kb][i]);
      }
    }
    mx = nvk_max_xor32(max_xor16(mx));
    const float mt = mx == -INFINITY ? -INFINITY : mx * a.scale_log2;
    const float m_new = fmaxf(m_run, mt);
    const float moff = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = nvk_fast_exp2(m_run - moff);  // 0 while nothing was visible
    m_run = m_new;
    l_part *= alpha;
#pragma unroll
    for (int db = 0; db < HD / 16; ++db) acc_o[db] *= alpha;
    constexpr uint32_t kOnes = E::kOnes;  // the pair (1, 1)
    vec8 pf[kPairs];
#pragma unroll
    for (int p = 0; p < kPairs; ++p) {
      uint32_t wds[4];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const nvk_f32x4& sv = sacc[2 * p + h];
        const uint32_t w0 = E::pack2(nvk_fast_exp2(fmaf(sv[0], a.scale_log2, -moff)),
                                            nvk_fast_exp2(fmaf(sv[1], a.scale_log2, -moff)));
        const uint32_t w1 = E::pack2(nvk_fast_exp2(fmaf(sv[2], a.scale_log2, -moff)),
                                            nvk_fast_exp2(fmaf(sv[3], a.scale_log2, -moff)));
        l_part = E::dot2(w0, kOnes, l_part);
        l_part = E::dot2(w1, kOnes, l_part);
        wds[2 * h] = w0;
        wds[2 * h + 1] = w1;
      }
      pf[p] = __builtin_bit_cast(vec8, nvk_u32x4{wds[0], wds[1], wds[2], wds[3]});
    }
    // ---- O^T += V^T P^T
#pragma unroll
    for (int p = 0; p < kPairs; ++p) {
#pragma unroll
      for (int db = 0; db < HD / 16; ++db) {
        const uint32_t a_lo = tr_lo + p * 32 * kRowBytes + 32 * (db ^ sw_lo);
        const uint32_t a_hi = tr_hi + p * 32 * kRowBytes + 32 * (db ^ sw_hi);
        const nvk_i16x4 vlo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) nvk_i16x4*)(size_t)a_lo);
        const nvk_i16x4 vhi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) nvk_i16x4*)(size_t)a_hi);
        const nvk_i16x8 vv = {vlo[0], vlo[1], vlo[2], vlo[3], vhi[0], vhi[1], vhi[2], vhi[3]};
        acc_o[db] = E::mfma16x16x32(__builtin_bit_cast(vec8, vv), pf[p], acc_o[db]);
      }
    }
    // the V buffer is free again: the next chunk's V goes out
    if (!last) issue_v(nsrc);

    // ---- group end or range end
    if (group_end || last) {
      const float l_tot = nvk_sum_xor32(sum_xor16(l_part));
      const bool whole = group_end && started_here;
      if (whole) {
        if (row_valid) {
          const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
          uint16_t* op = a.p.out + (int64_t)(q_row0 + tok) * a.p.out_stride_tok +
                         (int64_t)head * a.p.out_stride_head + 4 * g;
#pragma unroll
          for (int db = 0; db < HD / 16; ++db) {
            nvk_u32x2 wv;
            wv.x = E::pack2(acc_o[db][0] * inv, acc_o[db][1] * inv);
            wv.y = E::pack2(acc_o[db][2] * inv, acc_o[db][3] * inv);
            *reinterpret_cast<nvk_u32x2*>(op + 16 * db) = wv;
          }
        }
      } else if (row_valid) {  // the combine reads the valid rows only
        float* rec = a.rec + ((w * 2 + (started_here ? 0 : 1)) * kR + r) * (int64_t)kRec;
#pragma unroll
        for (int db = 0; db < HD / 16; ++db) *reinterpret_cast<nvk_f32x4*>(rec + 16 * db + 4 * g) = acc_o[db];
        if (g == 0) {
          rec[HD] = m_run;
          rec[HD + 1] = l_tot;
        }
      }
      if (lane == 0) {
        const int64_t gfirst = (int64_t)Hkv * s_cs[s] + (int64_t)kvh * n;
        const int p1 = (int)chunk_owner(gfirst, T, P);
        const int p2 = (int)chunk_owner(gfirst + n - 1, T, P);
        *reinterpret_cast<int2*>(a.desc + 2 * (s * Hkv + kvh)) = make_int2(p1, p2);
      }
      if (last) return;
      s = ns;
      kvh = uniform(nkvh);
      n = nn;
      k = 0;
      started_here = true;
      start_group();
    } else {
      k = uniform(nk);
    }
  }
}

// Merges the records of groups cut between waves and writes the zero rows of
// groups with no key.
// Merge of one row's 4 output columns over the parts of a cut group (wave
// p1's head record, slot 0, then the continuation records, slot 1): slice s
// of S folds parts p1+s, p1+s+S, ..., kBatch parts per round trip; returns
// the unnormalised sum O, its L and the reference max M.
template <int kBatch>
__device__ __forceinline__ void sq_merge_parts(const SqArgs& a, int row, int d0, int p1, int p2,
                                               int s, int S, float& M, float& L, nvk_f32x4& O) {
  M = -INFINITY;
  L = 0.f;
  O = nvk_f32x4{0.f, 0.f, 0.f, 0.f};
  for (int base = p1 + s; base <= p2; base += kBatch * S) {
    float mv[kBatch], lv[kBatch];
    nvk_f32x4 ov[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int p = base + u * S;
      const bool ok = p <= p2;
      const int pr = ok ? p : p1;
      const float* rec = a.rec + (((int64_t)pr * 2 + (pr == p1 ? 0 : 1)) * kR + row) * kRec;
      mv[u] = ok ? rec[HD] : -INFINITY;
      lv[u] = rec[HD + 1];
      ov[u] = *reinterpret_cast<const nvk_f32x4*>(rec + d0);
    }
    float mb = M;
#pragma unroll
    for (int u = 0; u < kBatch; ++u) mb = fmaxf(mb, mv[u]);
    if (mb == -INFINITY) continue;
    const float rs = nvk_fast_exp2(M - mb);
    L *= rs;
    O *= rs;
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const float wt = nvk_fast_exp2(mv[u] - mb);
      L += lv[u] * wt;
      O += wt * ov[u];
    }
    M = mb;
  }
}

template <bool F16>
__device__ __forceinline__ void sq_write_row(uint16_t* op, float L, const nvk_f32x4& O) {
  const float inv = L > 0.f ? 1.f / L : 0.f;
  nvk_u32x2 wv;
  wv.x = NvkElt<F16>::pack2(O[0] * inv, O[1] * inv);
  wv.y = NvkElt<F16>::pack2(O[2] * inv, O[3] * inv);
  *reinterpret_cast<nvk_u32x2*>(op) = wv;
}

// grid = (Hkv, batch), 512 threads: thread t owns row t / 32 and
// d = 4 (t % 32) .. +3.
template <bool F16>
__global__ __launch_bounds__(512) void short_query_combine_kernel(SqArgs a) {
  const int kvh = blockIdx.x, s = blockIdx.y;
  const int row = threadIdx.x >> 5, d0 = 4 * (threadIdx.x & 31);
  const int Lq = seq_queries(a, s);
  const int tok = row / a.G;
  if (tok >= Lq) return;
  const int head = kvh * a.G + row % a.G;
  uint16_t* op = a.p.out + (int64_t)(a.p.cu_q[s] + tok) * a.p.out_stride_tok +
                 (int64_t)head * a.p.out_stride_head + d0;
  const int2 desc = *reinterpret_cast<const int2*>(a.desc + 2 * (s * a.p.num_kv_heads + kvh));
  if (desc.x < 0) {
    *reinterpret_cast<nvk_u32x2*>(op) = nvk_u32x2{0u, 0u};
    return;
  }
  const int p1 = desc.x, p2 = desc.y;
  if (p1 == p2) return;  // finished inside one wave
  // records fetched per round trip: the smallest batch that holds every part
  // (16 for groups cut into more; uniform over the workgroup)
  float M, L;
  nvk_f32x4 O;
  const int parts = p2 - p1 + 1;
  if (parts <= 4)
    sq_merge_parts<4>(a, row, d0, p1, p2, 0, 1, M, L, O);
  else if (parts <= 8)
    sq_merge_parts<8>(a, row, d0, p1, p2, 0, 1, M, L, O);
  else
    sq_merge_parts<16>(a, row, d0, p1, p2, 0, 1, M, L, O);
  sq_write_row<F16>(op, L, O);
}

// Combine of steps whose groups are cut into many parts (one to four
// sequences over long contexts: 1 x 16 K keys cuts each group into 128).
// grid = (Hkv * kR/2, batch), kSqSlices waves: a workgroup owns two rows of
// one (sequence, kv head), wave s folds parts p1+s, p1+s+kSqSlices, ... (half
// a wave per row, 4 columns per lane), and wave 0 merges the waves' states
// through LDS.
constexpr int kSqSlices = 16;
template <bool F16>
__global__ __launch_bounds__(64 * kSqSlices) void short_query_combine_sliced_kernel(SqArgs a) {
  const int kvh = blockIdx.x / (kR / 2), s = blockIdx.y;
  const int lane = threadIdx.x & 63, slice = threadIdx.x >> 6;
  const int row = 2 * (blockIdx.x % (kR / 2)) + (lane >> 5), d0 = 4 * (lane & 31);
  const int Lq = seq_queries(a, s);
  if (2 * (blockIdx.x % (kR / 2)) >= Lq * a.G) return;  // both rows empty (uniform)
  const bool row_ok = row < Lq * a.G;
  const int tok = row / a.G;
  const int head = kvh * a.G + row % a.G;
  uint16_t* op = a.p.out + (int64_t)(a.p.cu_q[s] + tok) * a.p.out_stride_tok +
                 (int64_t)head * a.p.out_stride_head + d0;
  const int2 desc = *reinterpret_cast<const int2*>(a.desc + 2 * (s * a.p.num_kv_heads + kvh));
  if (desc.x < 0) {  // uniform over the workgroup
    if (slice == 0 && row_ok) *reinterpret_cast<nvk_u32x2*>(op) = nvk_u32x2{0u, 0u};
    return;
  }
  const int p1 = desc.x, p2 = desc.y;
  if (p1 == p2) return;  // finished inside one wave (uniform)
  float M, L;
  nvk_f32x4 O;
  const int per_slice = (p2 - p1 + kSqSlices) / kSqSlices;  // ceil(parts / kSqSlices)
  if (per_slice <= 4)
    sq_merge_parts<4>(a, row, d0, p1, p2, slice, kSqSlices, M, L, O);
  else if (per_slice <= 8)
    sq_merge_parts<8>(a, row, d0, p1, p2, slice, kSqSlices, M, L, O);
  else
    sq_merge_parts<16>(a, row, d0, p1, p2, slice, kSqSlices, M, L, O);
  __shared__ float sm[kSqSlices][64], sl[kSqSlices][64];
  __shared__ nvk_f32x4 so[kSqSlices][64];
  sm[slice][lane] = M;
  sl[slice][lane] = L;
  so[slice][lane] = O;
  __syncthreads();
  if (slice != 0 || !row_ok) return;
  float mx = sm[0][lane];
#pragma unroll
  for (int i = 1; i < kSqSlices; ++i) mx = fmaxf(mx, sm[i][lane]);
  const float mref = mx == -INFINITY ? 0.f : mx;
  L = 0.f;
  O = nvk_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < kSqSlices; ++i) {
    const float wt = nvk_fast_exp2(sm[i][lane] - mref);
    L += sl[i][lane] * wt;
    O += wt * so[i][lane];
  }
  sq_write_row<F16>(op, L, O);
}

int sq_waves(int batch, int64_t max_keys, int num_kv_heads) {
  const int64_t chunks = (max_keys + kCK - 1) / kCK;
  const int64_t t_max = chunks * batch * num_kv_heads;
  int64_t wgs = (t_max / kMinChunks + kWavesPerWG - 1) / kWavesPerWG;
  if (wgs > kMaxWGs) wgs = kMaxWGs;
  if (wgs < 1) wgs = 1;
  return (int)wgs * kWavesPerWG;
}

size_t sq_desc_bytes(int batch, int num_kv_heads) {
  return ((size_t)batch * num_kv_heads * 8 + 255) / 256 * 256;
}

}  // namespace

bool short_query_applies(bool paged, int block_size, int max_seqlen_q, int num_q_heads,
                         int num_kv_heads, int head_dim, int batch) {
  if (!paged || head_dim != HD || block_size <= 0 || block_size % kCK) return false;
  if (num_kv_heads <= 0 || num_q_heads % num_kv_heads) return false;
  const int G = num_q_heads / num_kv_heads;
  return max_seqlen_q > 0 && (int64_t)max_seqlen_q * G <= kR && batch > 0 && batch <= kMaxBatch;
}

size_t short_query_ws_bytes(int batch, int64_t max_keys, int num_q_heads, int num_kv_heads) {
  (void)num_q_heads;
  if (batch <= 0 || num_kv_heads <= 0 || max_keys <= 0) return 0;
  return sq_desc_bytes(batch, num_kv_heads) +
         (size_t)sq_waves(batch, max_keys, num_kv_heads) * 2 * kR * kRec * sizeof(float);
}

int short_query_launch(const ShortQueryParams& p, int64_t max_keys, void* ws, hipStream_t s) {
  SqArgs a;
  a.p = p;
  a.scale_log2 = p.scale * NVK_LOG2E;
  a.G = p.num_q_heads / p.num_kv_heads;
  const int64_t cap = (int64_t)p.max_blocks * p.block_size;
  a.cap = (int)(cap < INT32_MAX ? cap : INT32_MAX);
  a.row_elems = (int64_t)p.num_kv_heads * HD;
  a.row_bytes = (uint32_t)(a.row_elems * 2);
  a.desc = static_cast<int32_t*>(ws);
  a.rec = reinterpret_cast<float*>(static_cast<char*>(ws) + sq_desc_bytes(p.batch, p.num_kv_heads));
  a.n_waves = sq_waves(p.batch, max_keys, p.num_kv_heads);
  // K through LDS when a wave may stream many chunks (its full-row loads
  // stream faster); straight into registers for short ranges (one LDS round
  // trip less per chunk).  Bound from the static sizes.
  const int64_t chunks_bound = (max_keys + kCK - 1) / kCK * p.batch * p.num_kv_heads;
  const bool klds = chunks_bound >= (int64_t)kKldsMinChunks * a.n_waves;
  const dim3 grid(a.n_waves / kWavesPerWG), block(64 * kWavesPerWG);
  if (p.f16) {
    if (klds) hipLaunchKernelGGL((short_query_kernel<true, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((short_query_kernel<true, false>), grid, block, 0, s, a);
  } else {
    if (klds) hipLaunchKernelGGL((short_query_kernel<false, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((short_query_kernel<false, false>), grid, block, 0, s, a);
  }
  int st = nvk_launch_status();
  if (st != NVK_OK) return st;
  // At least 32 waves per (sequence, kv head) group: its parts are folded in
  // slices.
  const bool sliced = a.n_waves >= 32 * (int64_t)p.batch * p.num_kv_heads;
  const dim3 sgrid(p.num_kv_heads * (kR / 2), p.batch), cgrid(p.num_kv_heads, p.batch);
  if (sliced && p.f16)
    hipLaunchKernelGGL(short_query_combine_sliced_kernel<true>, sgrid, dim3(64 * kSqSlices), 0, s,
                       a);
  else if (sliced)
    hipLaunchKernelGGL(short_query_combine_sliced_kernel<false>, sgrid, dim3(64 * kSqSlices), 0,
                       s, a);
  else if (p.f16)
    hipLaunchKernelGGL(short_query_combine_kernel<true>, cgrid, dim3(32 * kR), 0, s, a);
  else
    hipLaunchKernelGGL(short_query_combine_kernel<false>, cgrid, dim3(32 * kR), 0, s, a);
  return nvk_launch_status();
}
