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
//     is token r/G, head r%G; wave w owns rows 32w..32w+31.
//   * K and V tiles of 64 keys go from HBM straight into LDS (buffer/global
//     loads with the LDS destination, 16 bytes per lane), row-major [key][d]
//     with 256-byte rows whose 16-byte chunks are XOR-swizzled by the row, so
//     both MFMA operand reads below are bank-conflict free.
//   * S^T = K Q^T: v_mfma_f32_32x32x16_bf16 with K (LDS) as the A operand and
//     the wave's Q fragment (registers, loaded once) as B.  Each lane then
//     holds 32 keys of ONE query row; the row max / sum need one exchange of
//     the wave halves (v_permlane32_swap).
//   * O^T += V^T P^T: the same MFMA with V^T as A, read with the transposing
//     LDS load (ds_read_b64_tr_b16), and P as B straight from the S^T
//     accumulators (P never leaves the registers).
//   * Software pipeline, one barrier per key tile: while tile t is in its
//     softmax (VALU) and PV product, the S MFMAs of tile t+1 run and the loads
//     of K(t+2) and V(t+1) are in flight into the free LDS stages.
//   * Softmax in log2 units with a lazily updated reference max (rescaling
//     only when a tile raises the max by more than 2^8), row sums by
//     v_dot2_f32_bf16 over the packed probabilities.
//   * The grid runs the query tiles nearest the end of each sequence (the
//     ones with most keys) first.
//   * The normalised output rows go back through LDS (each wave's 32 rows in
//     the K stages, free in a range's last step), so each store writes four
//     whole 256-byte rows.  Stored straight from the accumulator layout, a
//     lane wrote 8 bytes to 16 places and each store covered 16 bytes of 32
//     rows; the workgroup's end, and with it the start of the next one in its
//     slot, waited for those partial-line writes.
#include <type_traits>

#include "nvk_common.h"
#include "short_query.h"

namespace {

constexpr int HD = 128;
constexpr int kWaves = 4;                    // waves per workgroup
constexpr int kRows = 32 * kWaves;           // query rows per workgroup (32 per wave)
constexpr int kTileRowsPerWave = 64 / kWaves;      // key rows of a tile each wave loads
constexpr int kLoadsPerWave = kTileRowsPerWave / 4;  // 4-row (1 KiB) loads per wave
constexpr int kKeys = 64;                    // keys per tile
constexpr int kRowBytes = HD * 2;            // LDS bytes of one key row
constexpr int kTileBytes = kKeys * kRowBytes;
constexpr float kLazy = 8.f;                 // log2 headroom of the lazy softmax max

// How a workgroup finds its keys.
enum KvMode {
  kDense = 0,         // k / v rows of the step, key j of sequence s = row cu_k[s] + j
  kPagedAligned = 1,  // paged, block_size a multiple of 64: a key tile lies in one page
  kPagedAny = 2,      // paged, any other block size
};

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
  int out_rows16;  // out 16-byte aligned, strides multiples of 8: whole-row stores
  int n_qtiles;
  // Split-K over key tiles (short query ranges over long contexts): blockIdx.z
  // = qtile * n_splits + split, split j owning key tiles
  // [j*tiles_per_split, (j+1)*tiles_per_split) (the last one: to the end).
  // With n_splits > 1 every row's partial (O unnormalised, m, l) goes to `ws`
  // and prefill_combine_kernel writes `out`.
  int n_splits, tiles_per_split;
  float* ws;
  // Longest-first order of the (sequence, query tile) pairs, pair = qt * batch
  // + s, written by prefill_tile_order_kernel; null: the grid order.  Only
  // with n_splits == 1.
  const int32_t* order;
};

constexpr int kRecFloats = HD + 4;  // partial record of one row: O[HD], m, l, pad
constexpr int kMaxSplits = 16;      // key-range splits of one query tile

// ---- longest-first order of the query tiles ----------------------------------
// The hardware starts workgroups in blockIdx order as slots free up.  Ranking
// the (sequence, query tile) pairs by their number of key tiles, largest
// first, is the longest-processing-time rule: the last workgroups to start
// are short and the step ends with little idle time.  Measured on MI355X
// (interleaved A/B, same process): 32 sequences of 512 cached + 100-1024 new
// tokens 206 -> 194 us, 64 sequences of 256 + 16-512 130 -> 117 us, 16 of
// 1024 + 256-2048 452 -> 375 us, 128 sequences of 16-400 tokens 141 -> 139
// us, this kernel included; outputs bit-identical (every tile is computed
// the same way whatever runs when).  One workgroup counting-sorts the pairs by cost (ties in any
// order: any permutation of the pairs gives the same output).
constexpr int kOrderThreads = 1024;
constexpr int kOrderBuckets = 4096;      // costs above kOrderBuckets - 1 share the last
constexpr int kOrderMaxBatch = 4096;     // sequence bounds staged in LDS
constexpr int64_t kOrderMaxPairs = 1 << 22;
// Below two rounds of the workgroup slots (256 CUs x 2) every tile starts at
// once and the order cannot shorten the step: no extra kernel then.
constexpr int64_t kOrderMinWgs = 1024;
// Tag stored after the last pair of an order: batch < 2^13, n_qtiles < 2^16.
__host__ __device__ __forceinline__ int32_t order_tag(int batch, int n_qtiles) {
  return (int32_t)(0xA0000000u | ((uint32_t)batch << 16) | (uint32_t)n_qtiles);
}
static bool use_order(int batch, int64_t pairs, int num_kv_heads) {
  return batch > 1 && batch <= kOrderMaxBatch && pairs <= kOrderMaxPairs &&
         pairs * num_kv_heads > kOrderMinWgs;
}

__global__ __launch_bounds__(kOrderThreads) void prefill_tile_order_kernel(
    const int32_t* cu_q, const int32_t* cu_k, int batch, int n_qtiles, int tq, int32_t* order) {
  constexpr int kPer = kOrderBuckets / kOrderThreads;
  __shared__ int hist[kOrderBuckets];
  __shared__ int lq[kOrderMaxBatch], lk[kOrderMaxBatch];
  __shared__ int wsum[kOrderThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int P = batch * n_qtiles;
  for (int i = tid; i < kOrderBuckets; i += kOrderThreads) hist[i] = 0;
  for (int i = tid; i < batch; i += kOrderThreads) {
    lq[i] = cu_q[i + 1] - cu_q[i];
    lk[i] = cu_k[i + 1] - cu_k[i];
  }
  __syncthreads();
  // cost of pair p = qt * batch + s: 1 + key tiles of its last query row, 0
  // for a query tile past the sequence (it returns at once)
  auto cost = [&](int p) {
    const int qt = p / batch, sq = p - qt * batch;
    const int Lq = lq[sq], Lk = lk[sq];
    const int q0 = Lq - (qt + 1) * tq;
    if (Lq <= 0 || q0 + tq <= 0) return 0;
    int n = q0 + tq + (Lk - Lq);
    n = n < Lk ? n : Lk;
    n = n > 0 ? n : 0;
    const int c = 1 + (n + kKeys - 1) / kKeys;
    return c < kOrderBuckets - 1 ? c : kOrderBuckets - 1;
  };
  for (int p = tid; p < P; p += kOrderThreads) atomicAdd(&hist[cost(p)], 1);
  __syncthreads();
  // first rank of each bucket = pairs of higher cost; thread t owns buckets
  // [kPer t, kPer t + kPer), so those above its buckets are the ones of the
  // threads above it
  int loc[kPer];
  int sum = 0;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    loc[i] = hist[kPer * tid + i];
    sum += loc[i];
  }
  int x = sum;  // inclusive scan over the wave
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  if (lane == 63) wsum[w] = x;
  __syncthreads();
  int total = 0, before = 0;
#pragma unroll
  for (int i = 0; i < kOrderThreads / 64; ++i) {
    total += wsum[i];
    before += i < w ? wsum[i] : 0;
  }
  int run = total - (before + x);  // pairs in the buckets of threads above this one
  int start[kPer];
#pragma unroll
  for (int i = kPer - 1; i >= 0; --i) {
    start[i] = run;
    run += loc[i];
  }
  __syncthreads();  // every thread has read hist
#pragma unroll
  for (int i = 0; i < kPer; ++i) hist[kPer * tid + i] = start[i];  // cursors
  __syncthreads();
  for (int p = tid; p < P; p += kOrderThreads) order[atomicAdd(&hist[cost(p)], 1)] = p;
  if (tid == 0) order[P] = order_tag(batch, n_qtiles);
}
// An order is the pairs [0, batch * n_qtiles) in some permutation, followed by
// the tag of (batch, n_qtiles).  Any permutation of the same pairs gives the
// same output, so an order ranked for other lengths but the same batch and
// tile count is still correct; one whose tag differs is ignored (grid order).
static size_t order_bytes(int64_t pairs) { return (size_t)((pairs + 1) * 4 + 255) / 256 * 256; }

// Key range of one (sequence, query tile): shared by the attention and the
// combine kernels.
struct QTile {
  int q_row0, Lq, k_row0, Lk;
  int q0;            // first query token of the tile (may be < 0)
  int diag;          // row i sees keys j <= i + diag
  int n_keys;        // keys visible to the last row of the tile (clamped)
  int unmasked_keys; // keys visible to every row of the tile
  bool live;         // the tile holds at least one query token
};

template <int MODE>
__device__ __forceinline__ QTile qtile_info(const PrefillArgs& a, int s, int qt, int TQ) {
  QTile t;
  t.q_row0 = a.cu_q[s];
  t.Lq = a.cu_q[s + 1] - t.q_row0;
  t.k_row0 = a.cu_k[s];
  t.Lk = a.cu_k[s + 1] - t.k_row0;
  t.q0 = t.Lq - (qt + 1) * TQ;
  t.live = t.Lq > 0 && t.q0 + TQ > 0;
  int Lk_eff = t.Lk;
  if (MODE != kDense) {
    const int64_t cap = (int64_t)a.max_blocks * a.block_size;
    if ((int64_t)Lk_eff > cap) Lk_eff = (int)cap;
  } else {
    const int64_t cap = a.total_k - t.k_row0;  // rows past the end of k / v are absent
    if ((int64_t)Lk_eff > cap) Lk_eff = cap > 0 ? (int)cap : 0;
  }
  t.diag = t.Lk - t.Lq;
  int n_keys = (t.q0 + TQ - 1) + t.diag + 1;
  if (n_keys > Lk_eff) n_keys = Lk_eff;
  t.n_keys = n_keys < 0 ? 0 : n_keys;
  t.unmasked_keys = (t.q0 < 0 ? 0 : t.q0) + t.diag + 1;
  return t;
}

// Raw buffer descriptor over [b, b + bytes) for a byte address b (stride 0,
// dword3 0x00020000 = 32-bit data format, the gfx9 setting for untyped buffer
// access).
__device__ __forceinline__ nvk_u32x4 tile_rsrc(uint64_t b, uint32_t bytes) {
  return nvk_u32x4{(uint32_t)b, (uint32_t)(b >> 32) & 0xFFFFu, bytes, 0x00020000u};
}

// 16-byte chunk c of key row r sits at chunk c ^ swz(r) of the LDS row.  Over
// any 16 consecutive rows swz is a bijection (the K operand reads one chunk of
// 16 rows per 16 lanes) and over 4 consecutive rows it spreads 4 chunks over
// 16 slots (the transposing V reads).
__device__ __forceinline__ int swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

typedef __attribute__((address_space(3))) void* lds_ptr_t;

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(size_t)(lds_ptr_t)(p);
}

// Loads straight into LDS, 16 bytes per lane: lane l of the wave writes LDS
// bytes [dst + 16 l, dst + 16 l + 16).  Issued as inline asm so that the
// compiler does not order the wave's later LDS reads (of other stages) behind
// them; completion is awaited explicitly (vmcnt) before the publishing barrier.
// `rsrc`: a raw buffer descriptor (wave-uniform); loads at offsets >= its
// size write zeros.
// `rsrc` and `dst` must be wave-uniform values held in SGPRs (see uniform()).
// Load 16 bytes per lane from the buffer `rsrc` at byte `voffset` into LDS at
// dst + J KiB + 16 * lane (the LDS address formed in M0 by one scalar op).
template <int J>
__device__ __forceinline__ void lds_load_buffer_at(const nvk_u32x4& rsrc, uint32_t voffset,
                                                   uint32_t dst) {
  if constexpr (J == 0)
    asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
                 :: "v"(voffset), "s"(rsrc), "s"(dst) : "memory", "m0");
  else
    asm volatile("s_add_u32 m0, %2, %3\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
                 :: "v"(voffset), "s"(rsrc), "s"(dst), "n"(J * 1024) : "memory", "m0", "scc");
}
// readfirstlane of wave-uniform values the compiler may have computed with
// vector instructions (inline asm "s" operands need SGPRs).
__device__ __forceinline__ uint32_t uniform(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_readfirstlane((int)x);
}
__device__ __forceinline__ void lds_load_global(const void* src, uint32_t dst) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
               :: "v"(src), "s"((uint32_t)__builtin_amdgcn_readfirstlane((int)dst)) : "memory", "m0");
}
__device__ __forceinline__ void wait_lds_loads() {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

template <int G, int MODE, bool F16>
__global__ __launch_bounds__(64 * kWaves, 8 / kWaves) void varlen_prefill_kernel(PrefillArgs a) {
  constexpr int TQ = kRows / G;  // query tokens per workgroup
  using E = NvkElt<F16>;
  typedef typename E::vec8 vec8;

  const int kvh = blockIdx.x;
  int s = blockIdx.y, z = blockIdx.z;
  if (a.order) {  // one query tile per workgroup; a scalar read of its pair
    typedef __attribute__((address_space(4))) const int32_t const_i32;
    const int pairs = a.batch * a.n_qtiles;
    const int rank = blockIdx.y + a.batch * blockIdx.z;
    int p = ((const_i32*)a.order)[rank];
    const int32_t tag = ((const_i32*)a.order)[pairs];
    // an order of other sizes (tag) or a damaged one stays in bounds: grid order
    p = (unsigned)p < (unsigned)pairs && tag == order_tag(a.batch, a.n_qtiles) ? p : rank;
    z = p / a.batch;
    s = p - z * a.batch;
  }
  const int qt = z / a.n_splits;  // 0 = the tile that ends at the last query token
  const int split = z - qt * a.n_splits;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int half = lane >> 5;  // 0/1: which 8-wide k slice this lane feeds
  const int l32 = lane & 31;

  const QTile qi = qtile_info<MODE>(a, s, qt, TQ);
  if (!qi.live) return;
  const int q_row0 = qi.q_row0, Lq = qi.Lq, k_row0 = qi.k_row0;
  const int q0 = qi.q0, diag = qi.diag, n_keys = qi.n_keys;
  const int unmasked_keys = qi.unmasked_keys;
  const int n_tiles = (n_keys + kKeys - 1) / kKeys;
  // This workgroup's key tiles [t_begin, t_end).
  const int t_begin = split * a.tiles_per_split;
  const int t_end = split == a.n_splits - 1 ? n_tiles
                    : (t_begin + a.tiles_per_split < n_tiles ? t_begin + a.tiles_per_split
                                                             : n_tiles);
  if (a.n_splits > 1 && t_begin >= t_end) return;  // the combine skips empty splits

  // LDS: K stages 0/1, then V stages 0/1 (64 KB).
  __shared__ __attribute__((aligned(1024))) uint8_t lds[4 * kTileBytes];
  // LDS byte addresses of the stages, from one conversion of the array's
  // address (converting each stage pointer would re-check it for null)
  const uint32_t lds_base = lds_addr(lds);
  auto k_stage = [&](int st) { return lds_base + (uint32_t)(st * kTileBytes); };
  auto v_stage = [&](int st) { return lds_base + (uint32_t)((2 + st) * kTileBytes); };

  const int32_t* bt_row = MODE != kDense ? a.block_tables + (int64_t)s * a.bt_stride : nullptr;

  // ---- this lane's query row and its Q fragment (B operand of S^T) --------
  const int row = wave * 32 + l32;
  const int tok = q0 + row / G;
  const int head = kvh * G + row % G;
  const bool row_valid = tok >= 0 && tok < Lq;
  vec8 qf[HD / 16];
  {
    const int64_t qrow = (int64_t)q_row0 + tok;
    const bool ok = row_valid && qrow < a.total_q;
    const uint16_t* qp = a.q + qrow * a.q_stride_tok + (int64_t)head * a.q_stride_head + 8 * half;
#pragma unroll
    for (int ks = 0; ks < HD / 16; ++ks) {
      nvk_u32x4 w = {0, 0, 0, 0};
      if (ok) w = *reinterpret_cast<const nvk_u32x4*>(qp + 16 * ks);
      qf[ks] = __builtin_bit_cast(vec8, w);
    }
  }
  const int row_limit = tok + diag;  // last visible key of this row

  // ---- tile loads straight into LDS ---------------------------------------------
  // Wave w fills its kTileRowsPerWave rows of a stage (64 / kWaves, from row
  // w*kTileRowsPerWave) with loads of 4 rows; lane l writes LDS chunk l of
  // load j, i.e. row w*kTileRowsPerWave + 4j + l/16, slot l%16, so it fetches
  // chunk (l%16) ^ swz(row) of that key row.
  const int dma_rsub = lane >> 4;  // row within the 4-row block
  // first tile row of the wave's load j, and the chunk this lane fetches for it
  auto dma_row0 = [&](int j) { return kTileRowsPerWave * wave + 4 * j; };
  auto dma_chunk = [&](int j) { return (lane & 15) ^ ((dma_rsub << 2) | ((dma_row0(j) >> 2) & 3)); };
  const uint32_t k_row_bytes =
      MODE == kDense ? (uint32_t)a.k_stride_tok * 2u : (uint32_t)a.num_kv_heads * HD * 2u;
  const uint32_t v_row_bytes =
      MODE == kDense ? (uint32_t)a.v_stride_tok * 2u : (uint32_t)a.num_kv_heads * HD * 2u;
  const int64_t paged_row_elems = (int64_t)a.num_kv_heads * HD;
  // Aligned paged mode: the kv head's first element in page 0 and the page
  // stride in bytes (below 2^32, checked at launch), so a tile's address is
  // one 32 x 32 -> 64-bit product and two adds.
  const uint64_t head_k = (uint64_t)(uintptr_t)(a.k + kvh * HD);
  const uint64_t head_v = (uint64_t)(uintptr_t)(a.v + kvh * HD);
  const uint32_t page_bytes = (uint32_t)a.block_size * k_row_bytes;
  // kPagedAny: a key that does not exist reads the sequence's first q row
  // (finite); its score is masked to -inf and its probability is 0.
  const uint16_t* dummy = a.q + (int64_t)q_row0 * a.q_stride_tok;

  // A K or V tile load into one LDS stage, planned once per tile and issued as
  // kLoadsPerWave instructions per wave (load j: 4 rows), so the issues can be
  // spread over the MFMA work.  Dense / aligned paged: one buffer descriptor
  // over the tile's valid rows (rows past them load zeros; a tile that does
  // not exist has none), lane offsets fixed per load.  kPagedAny: per-row
  // global addresses, resolved when the plan is made.
  struct DmaPlan {
    nvk_u32x4 rsrc;                       // SGPRs
    uint32_t dst0;                        // LDS byte address of the wave's first row
    const uint16_t* rows[kLoadsPerWave];  // kPagedAny: this lane's source per load
  };
  uint32_t k_voff[kLoadsPerWave], v_voff[kLoadsPerWave];  // lane byte offset of load j
#pragma unroll
  for (int j = 0; j < kLoadsPerWave; ++j) {
    k_voff[j] = (uint32_t)(dma_row0(j) + dma_rsub) * k_row_bytes + 16u * (uint32_t)dma_chunk(j);
    v_voff[j] = (uint32_t)(dma_row0(j) + dma_rsub) * v_row_bytes + 16u * (uint32_t)dma_chunk(j);
  }
  // `page` / `in_page` (kPagedAligned): the tile's page id and its first key's
  // offset inside that page (multiples of 64, kept by the caller without
  // divisions).
  // Keys this workgroup loads: tiles past t_end and keys past n_keys get 0
  // bytes, so a tile's byte count is one clamp of key_end - its first key.
  const int key_end = n_keys < t_end * kKeys ? n_keys : t_end * kKeys;
  auto tile_keys = [&](int kt) {
    int rem = key_end - kt * kKeys;
    rem = rem < kKeys ? rem : kKeys;
    asm volatile("" : "+s"(rem));  // keeps the clamp scalar (as one op it is v_med3)
    return rem > 0 ? rem : 0;
  };
  // Dense mode: the kv head's first element of this sequence's key rows; tile
  // kt starts kt * 64 rows later.
  const uint64_t dense_k = MODE == kDense ? (uint64_t)(uintptr_t)(a.k + (int64_t)k_row0 * a.k_stride_tok +
                                                                  (int64_t)kvh * a.kv_stride_head) : 0;
  const uint64_t dense_v = MODE == kDense ? (uint64_t)(uintptr_t)(a.v + (int64_t)k_row0 * a.v_stride_tok +
                                                                  (int64_t)kvh * a.kv_stride_head) : 0;
  auto plan_tile = [&](int kt, uint32_t dst, bool is_v, int page, int in_page) {
    DmaPlan pl;
    const int base = kt * kKeys;
    const uint16_t* src = is_v ? a.v : a.k;
    pl.dst0 = uniform(dst + (uint32_t)(kTileRowsPerWave * wave * kRowBytes));
    const int rem = tile_keys(kt);
    if constexpr (MODE == kPagedAny) {
      pl.rsrc = nvk_u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int j = 0; j < kLoadsPerWave; ++j) {
        const int pos = base + dma_row0(j) + dma_rsub;
        const int64_t prow = pos < n_keys ? nvk_paged_row(bt_row, pos, a.block_size, a.bs_shift,
                                                          a.num_blocks) : -1;
        pl.rows[j] = (prow >= 0 ? src + prow * paged_row_elems + kvh * HD : dummy) +
                     8 * dma_chunk(j);
      }
    } else {
      uint32_t bytes = (uint32_t)rem * (is_v ? v_row_bytes : k_row_bytes);
      nvk_u32x4 r;
      if constexpr (MODE == kDense) {
        const uint32_t row_bytes = is_v ? v_row_bytes : k_row_bytes;
        r = tile_rsrc((is_v ? dense_v : dense_k) + (uint64_t)(uint32_t)base * row_bytes, bytes);
      } else {
        const bool ok = (uint32_t)page < (uint32_t)a.num_blocks;
        const uint64_t off = (uint64_t)(uint32_t)page * page_bytes + (uint32_t)in_page * k_row_bytes;
        r = tile_rsrc((is_v ? head_v : head_k) + (ok ? off : 0), ok ? bytes : 0u);  // no branch
      }
      pl.rsrc = nvk_u32x4{uniform(r.x), uniform(r.y), uniform(r.z), uniform(r.w)};
    }
    return pl;
  };
  // Aligned paged mode: a tile's byte offset from the kv head's first element
  // of page 0 and its byte count (both 0 when the page id is outside the
  // pool; 0 bytes past the tile range).  K and V rows share them, so each
  // step computes one (the K tile's) and the next step's V plan reuses it.
  struct TileOff {
    uint64_t off;
    uint32_t bytes;
  };
  auto tile_off = [&](int kt, int page, int in_page) {
    const int rem = tile_keys(kt);
    const bool ok = (uint32_t)page < (uint32_t)a.num_blocks;
    // an invalid page loads nothing (0 bytes); its offset is then irrelevant
    const uint32_t pg = ok ? (uint32_t)page : 0u;
    TileOff t;
    t.off = (uint64_t)pg * page_bytes + (uint32_t)in_page * k_row_bytes;
    t.bytes = ok ? (uint32_t)rem * k_row_bytes : 0u;
    return t;
  };
  auto plan_at = [&](const TileOff& t, uint32_t dst, bool is_v) {
    DmaPlan pl;
    pl.dst0 = uniform(dst + (uint32_t)(kTileRowsPerWave * wave * kRowBytes));
    const nvk_u32x4 r = tile_rsrc((is_v ? head_v : head_k) + t.off, t.bytes);
    pl.rsrc = nvk_u32x4{uniform(r.x), uniform(r.y), uniform(r.z), r.w};
    return pl;
  };
  static_assert(4 * kRowBytes == 1024 && kLoadsPerWave <= 4, "load j lands at dst0 + j KiB");
  auto issue_load = [&](const DmaPlan& pl, int j, bool is_v) {
    if constexpr (MODE == kPagedAny) {
      lds_load_global(pl.rows[j], pl.dst0 + 4 * j * kRowBytes);
    } else {
      const uint32_t vo = is_v ? v_voff[j] : k_voff[j];
      switch (j) {  // j is a constant wherever the loop schedule is unrolled
        case 0: lds_load_buffer_at<0>(pl.rsrc, vo, pl.dst0); break;
        case 1: lds_load_buffer_at<1>(pl.rsrc, vo, pl.dst0); break;
        case 2: lds_load_buffer_at<2>(pl.rsrc, vo, pl.dst0); break;
        default: lds_load_buffer_at<3>(pl.rsrc, vo, pl.dst0); break;
      }
    }
  };

  // Page ids (kPagedAligned): read one step before the tile's load is issued;
  // `logical` is the tile's page index in the sequence, kept by the caller.
  const int last_page = n_keys > 0 ? (n_keys - 1) / a.block_size : 0;
  auto fetch_page = [&](int logical) -> int {
    logical = logical < last_page ? logical : last_page;
    asm volatile("" : "+v"(logical));  // keep the table read a vector load
    return bt_row[logical];
  };
  // The first tiles' page ids: scalar loads, so that waiting for them does not
  // also wait for the Q loads issued before them (vector loads complete in
  // order).  Measured on MI355X (interleaved A/B, bit-identical): 32 sequences
  // of 512 cached + 100-1024 new tokens 191.2 -> 190.0 us, 64 of 256 + 16-512
  // 116.2 -> 113.0 us.
  auto first_page = [&](int kt) -> int {
    typedef __attribute__((address_space(4))) const int32_t const_i32;
    int logical = a.bs_shift >= 0 ? (kt * kKeys) >> a.bs_shift : (kt * kKeys) / a.block_size;
    logical = logical < last_page ? logical : last_page;
    return ((const_i32*)bt_row)[logical];
  };

  // ---- S^T = K Q^T for one tile: two 32-key blocks ---------------------------
  // Lane reads key row 32 mb + l32, logical chunk 2 ks + half, i.e. byte
  // row*256 + 16*((2 ks + half) ^ swz(row)) = k_addr ^ (32 ks) (+ 8192 mb).
  const int k_swz = swz(l32);
  const uint32_t k_addr0 = lds_base + l32 * kRowBytes + 16 * ((half ^ k_swz) & 1) +
                           32 * (k_swz >> 1);
  // The XOR touches bits 5-7 only and the stage / block offsets are multiples
  // of 8 KiB, so the address of fragment ks in stage st, block mb is
  // k_addr[ks] + st * kTileBytes + 8192 mb: a constant offset of the read.
  uint32_t k_addr[HD / 16];
#pragma unroll
  for (int ks = 0; ks < HD / 16; ++ks) k_addr[ks] = k_addr0 ^ (32u * ks);
  auto compute_s = [&](auto stage, nvk_f32x16 (&acc)[2]) {
    constexpr int ST = decltype(stage)::value;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) acc[mb] = nvk_f32x16{};
#pragma unroll
    for (int ks = 0; ks < HD / 16; ++ks) {
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        const vec8 kf = *reinterpret_cast<const __attribute__((address_space(3))) vec8*>(
            (size_t)(k_addr[ks] + ST * kTileBytes + 32 * kRowBytes * mb));
        acc[mb] = E::mfma32x32x16(kf, qf[ks], acc[mb]);
      }
    }
  };

  // ---- O^T += V^T P^T -----------------------------------------------------------
  // A operand lane l: V^T[d = 32 db + l%32][8 keys], from two ds_read_b64_tr_b16:
  // inside a 16-lane group, source lane c names the 4 elements at key kb + c/4,
  // d d0 + 4(c%4), and lane i receives V[kb + 0..3][d0 + i].  The fragment's
  // keys are {4h..4h+3, 8+4h..8+4h+3} (h = lane/32) of the 16-key step: the
  // order in which the S^T accumulator holds P.  Byte address of the lo/hi read
  // for d block db: v_lo/hi ^ (64 db) (+ 4096 ks).
  nvk_f32x16 acc_o[HD / 32];
#pragma unroll
  for (int db = 0; db < HD / 32; ++db) acc_o[db] = nvk_f32x16{};
  uint32_t v_lo0, v_hi0;
  {
    const int tr_key = (lane & 15) >> 2;                          // row within the 4-row group
    const int tr_c0 = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);  // chunk within 32 d
    const int sw_lo = swz(4 * half + tr_key), sw_hi = swz(8 + 4 * half + tr_key);
    const uint32_t v0 = lds_base + 2 * kTileBytes + 8 * (lane & 1);
    v_lo0 = v0 + (4 * half + tr_key) * kRowBytes + 16 * (tr_c0 ^ (sw_lo & 3)) + 64 * (sw_lo >> 2);
    v_hi0 = v0 + (8 + 4 * half + tr_key) * kRowBytes + 16 * (tr_c0 ^ (sw_hi & 3)) +
            64 * (sw_hi >> 2);
  }
  // V read addresses of d block db in stage 0 (bits 6-7 XORed; stage and k-step
  // offsets are multiples of 4 KiB and become constant offsets of the reads)
  uint32_t v_lo[HD / 32], v_hi[HD / 32];
#pragma unroll
  for (int db = 0; db < HD / 32; ++db) {
    v_lo[db] = v_lo0 ^ (64u * db);
    v_hi[db] = v_hi0 ^ (64u * db);
  }
  // Online softmax in log2 units with a lazily updated reference max: the
  // probabilities are exp2(score - m_ref) with m_ref at most kLazy below the
  // true running max, so they stay <= 2^kLazy; m_ref (and the accumulators)
  // are only rescaled when a tile's max exceeds m_ref + kLazy.
  float m_ref = -INFINITY;
  float l_part[2] = {0.f, 0.f};  // this lane's share of the row sum (two chains)

  // Scores of keys a row may not see -> -inf (boundary tiles only; uniform).
  // Score i of block mb is key kbase + 4 half + c with the constant c below:
  // it stays iff c <= min(row_limit, n_keys - 1) - kbase - 4 half, one
  // compare and one select per score.
  auto mask_tile = [&](nvk_f32x16 (&sc)[2], int kt) {
    const int kbase = kt * kKeys;
    if (kbase + kKeys > unmasked_keys || kbase + kKeys > n_keys) {
      const int lim = (row_limit < n_keys - 1 ? row_limit : n_keys - 1) - kbase - 4 * half;
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int c = 32 * mb + 8 * (i >> 2) + (i & 3);
          sc[mb][i] = c <= lim ? sc[mb][i] : -INFINITY;
        }
      }
    }
  };
  // Row max of a tile (score i of the 32 is sc[i / 16][i % 16]) in four
  // chains, chain c over scores 8c..8c+6 in three v_max3 steps, then a join
  // with scores 7, 15, 23, 31.  The steps can be spread over MFMAs, and two
  // chains advance side by side: a v_max3 (inline asm) that reads the result
  // of the one just before it costs a wait state.
  auto max_chain = [&](const nvk_f32x16 (&sc)[2], float x, int c, int st) -> float {
    auto v = [&](int i) { return sc[i >> 4][i & 15]; };
    const int b = 8 * c;
    return st == 0 ? nvk_max3(v(b), v(b + 1), v(b + 2))
                   : nvk_max3(x, v(b + 2 * st + 1), v(b + 2 * st + 2));
  };
  auto max_join_a = [&](const nvk_f32x16 (&sc)[2], const float (&ch)[4], float (&t)[2]) {
    t[0] = nvk_max3(ch[0], ch[1], sc[0][7]);
    t[1] = nvk_max3(ch[2], ch[3], sc[0][15]);
  };
  auto max_join_b = [&](const nvk_f32x16 (&sc)[2], const float (&t)[2]) -> float {
    const float u = nvk_max3(t[0], t[1], sc[1][7]);
    return nvk_max_xor32(fmaxf(u, sc[1][15])) * a.scale_log2;  // tile max, log2 units
  };
  // Lazy rescale for a tile whose row max (log2 units) is mt; returns the
  // offset for exp2.
  auto rescale = [&](float mt) -> float {
    const bool need = mt > m_ref + kLazy;
    if (__builtin_amdgcn_ballot_w64(need)) {
      // Lanes that do not need it keep alpha = 1 (a row with no visible key so
      // far has m_ref = -inf, and exp2(-inf - -inf) would be NaN).
      const float m_new = need ? mt : m_ref;
      const float alpha = need ? nvk_fast_exp2(m_ref - m_new) : 1.f;  // 0 when m_ref = -inf
      m_ref = m_new;
#pragma unroll
      for (int j = 0; j < 2; ++j) l_part[j] *= alpha;
#pragma unroll
      for (int db = 0; db < HD / 32; ++db) acc_o[db] *= alpha;
    }
    return m_ref == -INFINITY ? 0.f : m_ref;  // row masked so far: p = 0
  };
  // Word n = 4p + e of the tile's probabilities (word e of P fragment p: keys
  // 16p..16p+15 of the tile, in accumulator order): exp2(score * scale_log2 -
  // moff) of two scores packed to bf16; the row sum accumulates the same
  // rounded values that enter the PV product.  A word is made in two halves,
  // the exp2 pair (exp_start) and the packing (exp_finish), and the loop
  // starts word n + 1 before it finishes word n: a packing that reads an
  // exp2 result in the next instruction waits a cycle (an s_nop per word).
  struct ExpPair {
    float p0, p1;
  };
  auto exp_start = [&](const nvk_f32x16 (&sc)[2], float moff, int n) -> ExpPair {
    const int p = n >> 2, e = n & 3;
    const int mb = p >> 1, i = 8 * (p & 1) + 2 * e;
    ExpPair x;
    x.p0 = nvk_fast_exp2(fmaf(sc[mb][i], a.scale_log2, -moff));
    x.p1 = nvk_fast_exp2(fmaf(sc[mb][i + 1], a.scale_log2, -moff));
    asm volatile("" : "+v"(x.p0), "+v"(x.p1));  // issued here
    return x;
  };
  auto exp_finish = [&](ExpPair x, int n) -> uint32_t {
    // packed no earlier than here (a fence, not an asm statement: the hazard
    // check would take an asm writing p0 / p1 for a transcendental)
    __builtin_amdgcn_sched_barrier(0);
    uint32_t w = E::pack2(x.p0, x.p1);
    l_part[n & 1] = E::dot2(w, E::kOnes, l_part[n & 1]);  // the pair (1, 1)
    // keep this word where it is placed among the MFMAs (no sinking to its use)
    asm volatile("" : "+v"(w), "+v"(l_part[n & 1]));
    return w;
  };

  // The MFMA work of step kt, software-pipelined by hand (sched_barrier(0)
  // fences keep the order; the compiler would otherwise group the MFMAs).
  // P fragment f holds keys 16f..16f+15 of tile kt; fragments 0-1 come from
  // score block 0, fragments 2-3 from block 1.  Order:
  //   exp2 of fragment 0;
  //   O k-step 0 (4 MFMAs) with the exp2 of fragment 1;
  //   S(kt+1) block 0 (8 MFMAs, into the consumed score block 0) with the
  //     exp2 of fragments 2-3;
  //   S(kt+1) block 1 (8);
  //   mask of S(kt+1) (boundary tiles only);
  //   O k-steps 1-3 (12) with the row max of S(kt+1).
  // Between the MFMAs: the loads of V(kt+1) and K(kt+2) and, in SALU, the
  // plans of the next step's loads (V(kt+2), K(kt+3); pages pg_v / pg_k).
  // LDS operands are read two MFMAs ahead.
  // Stages: tile t sits in stage (t - t_begin) & 1, so the step loop runs
  // two steps per pass and every stage offset is a constant (P: the stage of
  // tile kt).
  // LAST: the step of the range's last tile, which has no S(kt+1), row max or
  // loads of its own to make.
  auto mma_step = [&](auto par, auto last, int kt, nvk_f32x16 (&sc)[2], float moff,
                      const DmaPlan& plan_v, const DmaPlan& plan_k, int pg_v, int ip_v, int pg_k,
                      int ip_k, DmaPlan& next_v, DmaPlan& next_k, float& mt_next, TileOff& toff) {
    constexpr int P = decltype(par)::value;
    constexpr bool LAST = decltype(last)::value;
    auto rd_k = [&](int ks, int mb) {  // K of tile kt+1
      return *reinterpret_cast<const __attribute__((address_space(3))) vec8*>(
          (size_t)(k_addr[ks] + (1 - P) * kTileBytes + 32 * kRowBytes * mb));
    };
    auto rd_v = [&](int db, int ks) {  // V of tile kt
      const nvk_i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) nvk_i16x4*)(size_t)(v_lo[db] + P * kTileBytes +
                                                                  16 * ks * kRowBytes));
      const nvk_i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) nvk_i16x4*)(size_t)(v_hi[db] + P * kTileBytes +
                                                                  16 * ks * kRowBytes));
      const nvk_i16x8 w = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      return __builtin_bit_cast(vec8, w);
    };
    auto pack = [](const uint32_t (&w)[4]) {
      return __builtin_bit_cast(vec8, nvk_u32x4{w[0], w[1], w[2], w[3]});
    };
    // loads of this step: V(kt+1) during the O MFMAs, K(kt+2) during the S MFMAs
    auto v_load_at = [&](int idx) {  // O MFMA index -> load number or -1
      constexpr int kAt[4] = {1, 3, 5, 9};
      for (int j = 0; j < kLoadsPerWave; ++j)
        if (kAt[kLoadsPerWave > 2 ? j : 2 * j] == idx) return j;
      return -1;
    };
    auto k_load_at = [&](int i) {  // S MFMA index (0..15) -> load number or -1
      constexpr int kAt[4] = {2, 6, 10, 14};
      for (int j = 0; j < kLoadsPerWave; ++j)
        if (kAt[kLoadsPerWave > 2 ? j : 2 * j] == i) return j;
      return -1;
    };
    vec8 pf[4];
    uint32_t pw[4], pw3[4];
    vec8 vf[3];
    vf[0] = rd_v(0, 0);
    vf[1] = rd_v(1, 0);
    // words 0-3 (fragment 0) before the first MFMA; word n lives in xp[n & 1]
    // from its start to its finish
    ExpPair xp[2];
    xp[0] = exp_start(sc, moff, 0);
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      xp[(n + 1) & 1] = exp_start(sc, moff, n + 1);
      pw[n] = exp_finish(xp[n & 1], n);
    }
    pf[0] = pack(pw);
    __builtin_amdgcn_sched_barrier(0);
    constexpr int kO = (kKeys / 16) * (HD / 32);
    auto o_mfma = [&](int idx) {  // idx = ks*4 + db; reads V two MFMAs ahead
      const int ks = idx / (HD / 32), db = idx % (HD / 32);
      if (idx + 2 < kO) vf[(idx + 2) % 3] = rd_v((idx + 2) % (HD / 32), (idx + 2) / (HD / 32));
      __builtin_amdgcn_sched_barrier(0);
      acc_o[db] = E::mfma32x32x16(vf[idx % 3], pf[ks], acc_o[db]);
      const int j = v_load_at(idx);
      if (j >= 0 && !LAST) issue_load(plan_v, j, true);
    };
    // O k-step 0 with fragment 1 (words 4-7; word 8 started).
#pragma unroll
    for (int idx = 0; idx < 4; ++idx) {
      o_mfma(idx);
      pw[idx] = exp_finish(xp[idx & 1], 4 + idx);
      xp[(5 + idx) & 1] = exp_start(sc, moff, 5 + idx);
      __builtin_amdgcn_sched_barrier(0);
    }
    pf[1] = pack(pw);
    // S(kt+1), block 0 then block 1 (LAST: only the exp2 of fragments 2-3).
    vec8 kf[3];
#pragma unroll
    for (int mb = 0; mb < (LAST ? 1 : 2); ++mb) {
      if constexpr (!LAST) {
        kf[0] = rd_k(0, mb);
        kf[1] = rd_k(1, mb);
        sc[mb] = nvk_f32x16{};
      }
#pragma unroll
      for (int ks = 0; ks < HD / 16; ++ks) {
        if constexpr (!LAST) {
          if (ks + 2 < HD / 16) kf[(ks + 2) % 3] = rd_k(ks + 2, mb);
          __builtin_amdgcn_sched_barrier(0);
          sc[mb] = E::mfma32x32x16(kf[ks % 3], qf[ks], sc[mb]);
        }
        if (mb == 0) {  // fragments 2-3: words 8-15
          const uint32_t w = exp_finish(xp[ks & 1], 8 + ks);
          if (ks < 4) pw[ks] = w;
          else pw3[ks - 4] = w;
          if (ks < 7) xp[(9 + ks) & 1] = exp_start(sc, moff, 9 + ks);
        }
        const int j = k_load_at(8 * mb + ks);
        if (j >= 0 && !LAST) issue_load(plan_k, j, false);
        if constexpr (!LAST && MODE == kPagedAligned) {  // toff: tile kt+2 in, tile kt+3 out
          if (mb == 0 && ks == 5) next_v = plan_at(toff, v_stage(P), true);
          if (mb == 1 && ks == 1) {
            toff = tile_off(kt + 3, pg_k, ip_k);
            next_k = plan_at(toff, k_stage(1 - P), false);
          }
        } else if constexpr (!LAST && MODE == kDense) {
          if (mb == 0 && ks == 5) next_v = plan_tile(kt + 2, v_stage(P), true, pg_v, ip_v);
          if (mb == 1 && ks == 1)
            next_k = plan_tile(kt + 3, k_stage(1 - P), false, pg_k, ip_k);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      if (mb == 0) {
        pf[2] = pack(pw);
        pf[3] = pack(pw3);
      }
    }
    if constexpr (!LAST) mask_tile(sc, kt + 1);
    // O k-steps 1-3 with the row max of S(kt+1): chains 0-1 (score block 0)
    // beside MFMAs 4-6, chains 2-3 (block 1, just computed) beside 8-10, the
    // join beside 11-12.
    float ch[4] = {0.f, 0.f, 0.f, 0.f}, tj[2];
#pragma unroll
    for (int idx = 4; idx < kO; ++idx) {
      o_mfma(idx);
      if constexpr (!LAST) {
        if (idx >= 4 && idx < 7) {
          ch[0] = max_chain(sc, ch[0], 0, idx - 4);
          ch[1] = max_chain(sc, ch[1], 1, idx - 4);
        }
        if (idx >= 8 && idx < 11) {
          ch[2] = max_chain(sc, ch[2], 2, idx - 8);
          ch[3] = max_chain(sc, ch[3], 3, idx - 8);
        }
        if (idx == 11) max_join_a(sc, ch, tj);
        if (idx == 12) mt_next = max_join_b(sc, tj);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // ---- pipelined main loop ------------------------------------------------------
  // Step kt (one barrier): S(kt) and its row max are in registers, V(kt) and
  // K(kt+1) are in LDS.  The step loads V(kt+1) into V stage (kt+1)&1 and
  // K(kt+2) into K stage kt&1 while it computes O += V(kt) P(kt) and S(kt+1).
  // The barrier at the top of a step publishes the previous step's loads
  // (each wave waits for its own first) and guarantees that every wave has
  // finished reading the stages this step's loads overwrite.  Page ids
  // (aligned paged mode) are read two steps before their tile's plan.
  if (t_begin < t_end) {
    nvk_f32x16 sc[2];
    const int tb = t_begin;
    int pg[4] = {0, 0, 0, 0};  // pages of tiles tb .. tb+3
    int ip[4] = {0, 0, 0, 0};  // and their first keys' offsets in those pages
    if constexpr (MODE == kPagedAligned) {
#pragma unroll
      for (int i = 0; i < 4; ++i) pg[i] = first_page(tb + i);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pg[i] = __builtin_amdgcn_readfirstlane(pg[i]);
        ip[i] = ((tb + i) * kKeys) % a.block_size;
      }
    }
    auto next_in_page = [&](int x) { return x + kKeys == a.block_size ? 0 : x + kKeys; };
    {
      const DmaPlan k0 = plan_tile(tb, k_stage(0), false, pg[0], ip[0]);
      const DmaPlan v0 = plan_tile(tb, v_stage(0), true, pg[0], ip[0]);
      const DmaPlan k1 = plan_tile(tb + 1, k_stage(1), false, pg[1], ip[1]);
#pragma unroll
      for (int j = 0; j < kLoadsPerWave; ++j) {
        issue_load(k0, j, false);
        issue_load(v0, j, true);
        issue_load(k1, j, false);
      }
    }
    DmaPlan plan_v = plan_tile(tb + 1, v_stage(1), true, pg[1], ip[1]);
    TileOff toff = tile_off(tb + 2, pg[2], ip[2]);  // aligned paged: tile kt+2 of the step
    DmaPlan plan_k = MODE == kPagedAligned ? plan_at(toff, k_stage(0), false)
                                           : plan_tile(tb + 2, k_stage(0), false, pg[2], ip[2]);
    int page_a = pg[2], page_b = pg[3];  // pages of tiles kt+2, kt+3
    int ip_a = ip[2], ip_b = ip[3];
    // page index of tile kt+3 in the sequence (aligned paged mode), advanced
    // with the in-page offsets instead of a division per step
    int lp_b = MODE == kPagedAligned ? ((tb + 3) * kKeys) / a.block_size : 0;
    wait_lds_loads();
    __syncthreads();
    compute_s(std::integral_constant<int, 0>{}, sc);
    mask_tile(sc, tb);
    float mt;
    {
      float ch[4] = {0.f, 0.f, 0.f, 0.f}, tj[2];
#pragma unroll
      for (int st = 0; st < 3; ++st)
#pragma unroll
        for (int c = 0; c < 4; ++c) ch[c] = max_chain(sc, ch[c], c, st);
      max_join_a(sc, ch, tj);
      mt = max_join_b(sc, tj);
    }
    // The first tile sets the reference max: the accumulators and row sums
    // are still zero, so the rescale the first step would run (alpha = 0)
    // changes nothing and is skipped.  A row that sees no key of the tile
    // keeps -inf.
    m_ref = mt;
    auto step = [&](auto par, auto last, int kt) {
      constexpr int P = decltype(par)::value;
      constexpr bool LAST = decltype(last)::value;
      wait_lds_loads();
      __syncthreads();
      int page_c = 0;
      const int ip_c = next_in_page(ip_b);               // tile kt+4
      const int lp_c = ip_c == 0 ? lp_b + 1 : lp_b;
      if constexpr (MODE == kPagedAligned) {
        page_a = __builtin_amdgcn_readfirstlane(page_a);
        page_b = __builtin_amdgcn_readfirstlane(page_b);
        if (kt + 4 < t_end) page_c = fetch_page(lp_c);
      }
      if constexpr (MODE == kPagedAny && !LAST) {
        plan_v = plan_tile(kt + 1, v_stage(1 - P), true, 0, 0);
        plan_k = plan_tile(kt + 2, k_stage(P), false, 0, 0);
      }
      const float moff = rescale(mt);
      DmaPlan next_v = plan_v, next_k = plan_k;
      mma_step(par, last, kt, sc, moff, plan_v, plan_k, page_a, ip_a, page_b, ip_b, next_v, next_k,
               mt, toff);
      plan_v = next_v;
      plan_k = next_k;
      page_a = page_b;
      page_b = page_c;
      ip_a = ip_b;
      ip_b = ip_c;
      lp_b = lp_c;
    };
    const std::integral_constant<int, 0> p0;
    const std::integral_constant<int, 1> p1;
    const std::false_type more;
    const std::true_type last;
    int kt = tb;
    for (; kt + 2 < t_end; kt += 2) {
      step(p0, more, kt);
      step(p1, more, kt + 1);
    }
    if (kt + 1 < t_end) {  // two tiles left
      step(p0, more, kt);
      step(p1, last, kt + 1);
    } else {
      step(p0, last, kt);
    }
  }

  // ---- epilogue: normalise and store the rows ----------------------------------
  if (a.n_splits > 1) {  // partial record: O^T column (unnormalised), m_ref, l
    if (!row_valid) return;
    const float l_tot = nvk_sum_xor32(l_part[0] + l_part[1]);
    float* rec = a.ws + ((((int64_t)s * a.num_kv_heads + kvh) * a.n_qtiles + qt) * a.n_splits +
                         split) * (int64_t)kRows * kRecFloats +
                 (int64_t)row * kRecFloats;
#pragma unroll
    for (int db = 0; db < HD / 32; ++db) {
#pragma unroll
      for (int grp = 0; grp < 4; ++grp) {
        const nvk_f32x4 o4 = {acc_o[db][4 * grp], acc_o[db][4 * grp + 1], acc_o[db][4 * grp + 2],
                              acc_o[db][4 * grp + 3]};
        *reinterpret_cast<nvk_f32x4*>(rec + 32 * db + 8 * grp + 4 * half) = o4;
      }
    }
    if (half == 0) {
      rec[HD] = m_ref;
      rec[HD + 1] = l_tot;
    }
    return;
  }
  const float l_tot = nvk_sum_xor32(l_part[0] + l_part[1]);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  // Lane (half, l32) holds d = 32 db + 8 grp + 4 half .. +3 of its row.
  auto packed = [&](int db, int grp) {
    nvk_u32x2 w;
    w.x = E::pack2(acc_o[db][4 * grp] * inv, acc_o[db][4 * grp + 1] * inv);
    w.y = E::pack2(acc_o[db][4 * grp + 2] * inv, acc_o[db][4 * grp + 3] * inv);
    return w;
  };
  if (!a.out_rows16) {  // 8 bytes per lane and store (16 per row and instruction)
    if (!row_valid) return;
    uint16_t* op = a.out + ((int64_t)q_row0 + tok) * a.out_stride_tok + (int64_t)head * a.out_stride_head;
#pragma unroll
    for (int db = 0; db < HD / 32; ++db)
#pragma unroll
      for (int grp = 0; grp < 4; ++grp)
        *reinterpret_cast<nvk_u32x2*>(op + 32 * db + 8 * grp + 4 * half) = packed(db, grp);
    return;
  }
  // The wave's 32 rows go through its own HD * 64 bytes of the K stages, so
  // that each store writes four whole rows (half as many store instructions,
  // every 128-byte line written whole).  No wave reads a K stage in a range's
  // last step, and the stages' last loads were awaited before that step's
  // barrier.  16-byte chunk c of row r sits at chunk c ^ (r & 15): two-way
  // bank conflicts on the writes, none on the reads.
  constexpr uint32_t kRowB = HD * 2;
  const uint32_t ebase = lds_base + (uint32_t)wave * 32u * kRowB;
  typedef __attribute__((address_space(3))) nvk_u32x2 lds_u32x2;
  typedef __attribute__((address_space(3))) nvk_u32x4 lds_u32x4;
#pragma unroll
  for (int db = 0; db < HD / 32; ++db)
#pragma unroll
    for (int grp = 0; grp < 4; ++grp) {
      const uint32_t c = (uint32_t)((4 * db + grp) ^ (l32 & 15));
      *(lds_u32x2*)(size_t)(ebase + (uint32_t)l32 * kRowB + 16u * c + 8u * (uint32_t)half) =
          packed(db, grp);
    }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  const int c = lane & 15;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int rr = 4 * j + (lane >> 4);
    const nvk_u32x4 v = *(lds_u32x4*)(size_t)(ebase + (uint32_t)rr * kRowB +
                                               16u * (uint32_t)(c ^ (rr & 15)));
    const int r_row = wave * 32 + rr;
    const int r_tok = q0 + r_row / G;
    if (r_tok >= 0 && r_tok < Lq)
      *reinterpret_cast<nvk_u32x4*>(a.out + ((int64_t)q_row0 + r_tok) * a.out_stride_tok +
                                    (int64_t)(kvh * G + r_row % G) * a.out_stride_head + 8 * c) = v;
  }
}

// Merges the split-K partial records of one (sequence, kv head, query tile):
// thread t handles row t/8 and d range 16*(t%8) .. +15.  The m of every live
// split is fetched in one round trip, then the splits are folded in order,
// kFoldBatch at a time with all their loads in flight (left to itself the
// compiler waits for each split's m in turn and keeps four of a split's
// loads in flight).
constexpr int kFoldBatch = 4;
template <int G, int MODE, bool F16>
__global__ __launch_bounds__(8 * kRows) void prefill_combine_kernel(PrefillArgs a) {
  constexpr int TQ = kRows / G;
  const int kvh = blockIdx.x, s = blockIdx.y, qt = blockIdx.z;
  const QTile qi = qtile_info<MODE>(a, s, qt, TQ);
  if (!qi.live) return;
  const int r = threadIdx.x >> 3, dq = threadIdx.x & 7;
  const int tok = qi.q0 + r / G;
  if (tok < 0 || tok >= qi.Lq) return;
  const int head = kvh * G + r % G;
  const int n_tiles = (qi.n_keys + kKeys - 1) / kKeys;
  // splits that own at least one tile (the others wrote nothing)
  int n_live = a.tiles_per_split > 0 ? (n_tiles + a.tiles_per_split - 1) / a.tiles_per_split : 0;
  if (n_live > a.n_splits) n_live = a.n_splits;
  const float* rec0 = a.ws + (((int64_t)s * a.num_kv_heads + kvh) * a.n_qtiles + qt) *
                                 a.n_splits * (int64_t)kRows * kRecFloats +
                      (int64_t)r * kRecFloats;
  const int64_t split_stride = (int64_t)kRows * kRecFloats;
  float mv[kMaxSplits];
#pragma unroll
  for (int j = 0; j < kMaxSplits; ++j) {
    const float m = rec0[(j < n_live ? j : 0) * split_stride + HD];
    mv[j] = j < n_live ? m : -INFINITY;
  }
  float M = -INFINITY;
#pragma unroll
  for (int j = 0; j < kMaxSplits; ++j) M = fmaxf(M, mv[j]);
  float L = 0.f;
  nvk_f32x4 acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = nvk_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j0 = 0; j0 < kMaxSplits; j0 += kFoldBatch) {
    if (j0 >= n_live) break;
    float lv[kFoldBatch];
    nvk_f32x4 ov[kFoldBatch][4];
#pragma unroll
    for (int u = 0; u < kFoldBatch; ++u) {
      const int j = j0 + u < n_live ? j0 + u : j0;  // past the last live split: reread j0, weight 0
      const float* rec = rec0 + j * split_stride;
      lv[u] = rec[HD + 1];
#pragma unroll
      for (int i = 0; i < 4; ++i) ov[u][i] = *reinterpret_cast<const nvk_f32x4*>(rec + 16 * dq + 4 * i);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < kFoldBatch; ++u) {
      if (j0 + u >= n_live) break;
      const float m = mv[j0 + u];
      const float w = m == -INFINITY ? 0.f : nvk_fast_exp2(m - M);
      L += w * lv[u];
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] += w * ov[u][i];
    }
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  uint16_t* op = a.out + ((int64_t)qi.q_row0 + tok) * a.out_stride_tok +
                 (int64_t)head * a.out_stride_head + 16 * dq;
#pragma unroll
  for (int i = 0; i < 4; ++i) {  // 8-byte stores: out is only required 8-byte aligned
    nvk_u32x2 w;
    w.x = NvkElt<F16>::pack2(acc[i][0] * inv, acc[i][1] * inv);
    w.y = NvkElt<F16>::pack2(acc[i][2] * inv, acc[i][3] * inv);
    *reinterpret_cast<nvk_u32x2*>(op + 4 * i) = w;
  }
}

template <int G, int MODE, bool F16>
int launch_mode(const PrefillArgs& a, hipStream_t stream) {
  dim3 grid(a.num_kv_heads, a.batch, a.n_qtiles * a.n_splits);
  hipLaunchKernelGGL((varlen_prefill_kernel<G, MODE, F16>), grid, dim3(64 * kWaves), 0, stream,
                     a);
  if (a.n_splits > 1) {
    const int st = nvk_launch_status();
    if (st != NVK_OK) return st;
    dim3 cgrid(a.num_kv_heads, a.batch, a.n_qtiles);
    hipLaunchKernelGGL((prefill_combine_kernel<G, MODE, F16>), cgrid, dim3(8 * kRows), 0, stream,
                       a);
  }
  return nvk_launch_status();
}

template <int G, bool F16>
int launch_prefill(const PrefillArgs& a, hipStream_t stream) {
  if (!a.block_tables) return launch_mode<G, kDense, F16>(a, stream);
  // aligned pages whose byte size fits 32 bits (tile addresses in 32 x 32-bit products)
  if (a.block_size % kKeys == 0 &&
      (uint64_t)a.block_size * a.num_kv_heads * HD * 2 <= UINT32_MAX)
    return launch_mode<G, kPagedAligned, F16>(a, stream);
  return launch_mode<G, kPagedAny, F16>(a, stream);
}

template <bool F16>
int launch_prefill_g(const PrefillArgs& a, int G, hipStream_t s) {
  switch (G) {
    case 1: return launch_prefill<1, F16>(a, s);
    case 2: return launch_prefill<2, F16>(a, s);
    case 4: return launch_prefill<4, F16>(a, s);
    default: return launch_prefill<8, F16>(a, s);
  }
}


// Split-K plan for a launch: split the key range when the query ranges are
// short (at most half a query tile, so partial records stay small next to the
// keys they summarise) and the query tiles alone give fewer than ~4
// workgroups per CU, keeping at least 8 key tiles (512 keys) per split.
// Deterministic in its arguments, so the workspace query and the launch agree.
struct SplitPlan {
  int n_qtiles, n_splits, tiles_per_split;
};
static SplitPlan plan_splits(int batch, int max_seqlen_q, int64_t max_keys, int num_q_heads,
                             int num_kv_heads) {
  SplitPlan p;
  const int G = num_q_heads / num_kv_heads;
  const int TQ = kRows / G;
  p.n_qtiles = (max_seqlen_q + TQ - 1) / TQ;
  p.n_splits = 1;
  const int64_t max_tiles = (max_keys + kKeys - 1) / kKeys;
  const int64_t wgs = (int64_t)num_kv_heads * batch * p.n_qtiles;
  constexpr int64_t kTargetWgs = 1024, kMinTilesPerSplit = 8;
  if (wgs > 0 && wgs < kTargetWgs && max_tiles >= 2 * kMinTilesPerSplit &&
      2 * max_seqlen_q <= TQ) {
    int64_t n = (kTargetWgs + wgs - 1) / wgs;
    if (n > max_tiles / kMinTilesPerSplit) n = max_tiles / kMinTilesPerSplit;
    if (n > kMaxSplits) n = kMaxSplits;
    if (p.n_qtiles * n > 65535) n = 1;
    p.n_splits = n < 1 ? 1 : (int)n;
  }
  p.tiles_per_split = (int)((max_tiles + p.n_splits - 1) / p.n_splits);
  return p;
}
static size_t split_workspace_bytes(const SplitPlan& p, int batch, int num_kv_heads) {
  if (p.n_splits <= 1) return 0;
  return (size_t)num_kv_heads * batch * p.n_qtiles * p.n_splits * kRows * kRecFloats *
         sizeof(float);
}

}  // namespace

extern "C" size_t nvk_varlen_prefill_workspace_size(int32_t batch, int32_t max_seqlen_q,
                                                    int32_t max_seqlen_k, int32_t num_q_heads,
                                                    int32_t num_kv_heads, int32_t head_dim) {
  if (batch <= 0 || max_seqlen_q <= 0 || max_seqlen_k <= 0 || num_q_heads <= 0 ||
      num_kv_heads <= 0 || head_dim != HD || num_q_heads % num_kv_heads)
    return 0;
  const int G = num_q_heads / num_kv_heads;
  if (G != 1 && G != 2 && G != 4 && G != 8) return 0;
  const size_t split = split_workspace_bytes(
      plan_splits(batch, max_seqlen_q, max_seqlen_k, num_q_heads, num_kv_heads), batch,
      num_kv_heads);
  // short query ranges over paged keys take the short-query kernels (pages of
  // a multiple of 64 keys; the size does not depend on the page size)
  const size_t sq = short_query_applies(true, 64, max_seqlen_q, num_q_heads, num_kv_heads,
                                        head_dim, batch)
                        ? short_query_ws_bytes(batch, max_seqlen_k, num_q_heads, num_kv_heads)
                        : 0;
  // room for the longest-first tile order (multi-sequence prefills)
  const SplitPlan pl = plan_splits(batch, max_seqlen_q, max_seqlen_k, num_q_heads, num_kv_heads);
  const int64_t pairs = (int64_t)batch * pl.n_qtiles;
  const size_t ord = use_order(batch, pairs, num_kv_heads) ? order_bytes(pairs) : 0;
  size_t need = split > sq ? split : sq;
  return ord > need ? ord : need;
}

namespace {

// Bytes of the longest-first order a launch of these sizes uses (0: it runs
// its query tiles in grid order).  The same decision varlen_prefill_impl takes.
size_t order_bytes_for(int32_t batch, int32_t max_seqlen_q, int64_t max_keys, int32_t num_q_heads,
                       int32_t num_kv_heads, bool paged, int32_t block_size) {
  if (batch <= 0 || max_seqlen_q <= 0 || max_keys <= 0 || num_q_heads <= 0 ||
      num_kv_heads <= 0 || num_q_heads % num_kv_heads)
    return 0;
  if (paged && short_query_applies(true, block_size, max_seqlen_q, num_q_heads, num_kv_heads, HD,
                                   batch))
    return 0;  // the short-query kernels take these
  const SplitPlan sp = plan_splits(batch, max_seqlen_q, max_keys, num_q_heads, num_kv_heads);
  const int64_t pairs = (int64_t)batch * sp.n_qtiles;
  if (sp.n_splits != 1 || !use_order(batch, pairs, num_kv_heads)) return 0;
  return order_bytes(pairs);
}

int varlen_prefill_impl(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                        int64_t total_q, const void* k, const void* v, int64_t k_stride_tok,
                        int64_t v_stride_tok, int64_t kv_stride_head, int64_t total_k,
                        const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int32_t batch,
                        int32_t max_seqlen_q, int32_t max_seqlen_k, const int32_t* block_tables,
                        int64_t bt_stride, int32_t max_blocks, int32_t block_size,
                        int32_t num_blocks, int32_t num_q_heads, int32_t num_kv_heads,
                        int32_t head_dim, float scale, void* out, int64_t out_stride_tok,
                        int64_t out_stride_head, void* workspace, size_t workspace_bytes,
                        int32_t dtype, void* stream, const int32_t* given_order,
                        size_t given_order_bytes) {
  if (batch < 0 || max_seqlen_q < 0 || max_seqlen_k < 0 || num_q_heads <= 0 ||
      num_kv_heads <= 0 || total_q < 0 || total_k < 0)
    return NVK_EINVAL;
  if (!(scale > 0.f)) return NVK_EINVAL;  // the row max is taken before scaling
  if (dtype != NVK_DTYPE_BF16 && dtype != NVK_DTYPE_F16) return NVK_EUNSUPPORTED;
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
  if (workspace && (uintptr_t)workspace % 256) return NVK_EALIGN;

  // Keys per sequence are bounded by max_seqlen_k (when given) and by the table
  // (paged) or the k rows (dense).
  int64_t max_keys = block_tables ? (int64_t)max_blocks * block_size : total_k;
  if (max_seqlen_k > 0 && max_seqlen_k < max_keys) max_keys = max_seqlen_k;

  // Short query ranges (<= 16 rows per kv head) over paged keys: the stream-K
  // short-query kernels, when the workspace holds their records.
  if (num_blocks > 0 && max_keys > 0 &&
      short_query_applies(block_tables != nullptr, block_size, max_seqlen_q, num_q_heads,
                          num_kv_heads, head_dim, batch) &&
      workspace && workspace_bytes >= short_query_ws_bytes(batch, max_keys, num_q_heads,
                                                           num_kv_heads)) {
    ShortQueryParams sp;
    sp.q = static_cast<const uint16_t*>(q);
    sp.q_stride_tok = q_stride_tok;
    sp.q_stride_head = q_stride_head;
    sp.k_cache = static_cast<const uint16_t*>(k);
    sp.v_cache = static_cast<const uint16_t*>(v);
    sp.cu_q = cu_seqlens_q;
    sp.cu_k = cu_seqlens_k;
    sp.batch = batch;
    sp.block_tables = block_tables;
    sp.bt_stride = bt_stride;
    sp.max_blocks = max_blocks;
    sp.block_size = block_size;
    sp.num_blocks = num_blocks;
    sp.num_q_heads = num_q_heads;
    sp.num_kv_heads = num_kv_heads;
    sp.scale = scale;
    sp.out = static_cast<uint16_t*>(out);
    sp.out_stride_tok = out_stride_tok;
    sp.out_stride_head = out_stride_head;
    sp.f16 = dtype == NVK_DTYPE_F16;
    return short_query_launch(sp, max_keys, workspace, reinterpret_cast<hipStream_t>(stream));
  }
  SplitPlan sp = plan_splits(batch, max_seqlen_q, max_keys, num_q_heads, num_kv_heads);
  if (sp.n_qtiles > 65535) return NVK_EINVAL;
  if (sp.n_splits > 1 && (!workspace || workspace_bytes < split_workspace_bytes(sp, batch,
                                                                                num_kv_heads))) {
    sp.n_splits = 1;  // no room for partials: one workgroup per query tile
    sp.tiles_per_split = (int)((max_keys + kKeys - 1) / kKeys);
  }

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
  a.out_rows16 = (uintptr_t)out % 16 == 0 && out_stride_tok % 8 == 0 && out_stride_head % 8 == 0;
  a.n_qtiles = sp.n_qtiles;
  a.n_splits = sp.n_splits;
  a.tiles_per_split = sp.n_splits > 1 ? sp.tiles_per_split : 1 << 30;
  a.ws = static_cast<float*>(workspace);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  // One query tile per workgroup, a grid of several rounds and room in the
  // workspace: rank the tiles longest first (one more small kernel).  One
  // sequence: the grid order (last query tile first) already is.
  a.order = nullptr;
  const int64_t pairs = (int64_t)batch * sp.n_qtiles;
  if (sp.n_splits == 1 && use_order(batch, pairs, num_kv_heads)) {
    if (given_order) {
      if (given_order_bytes < order_bytes(pairs)) return NVK_EWORKSPACE;
      if ((uintptr_t)given_order % 4) return NVK_EALIGN;
      a.order = given_order;  // ranked once for every layer of the step
    } else if (workspace && workspace_bytes >= order_bytes(pairs)) {
      int32_t* order = static_cast<int32_t*>(workspace);
      hipLaunchKernelGGL(prefill_tile_order_kernel, dim3(1), dim3(kOrderThreads), 0, s,
                         cu_seqlens_q, cu_seqlens_k, batch, sp.n_qtiles, kRows / G, order);
      const int st = nvk_launch_status();
      if (st != NVK_OK) return st;
      a.order = order;
    }
  }
  return dtype == NVK_DTYPE_F16 ? launch_prefill_g<true>(a, G, s) : launch_prefill_g<false>(a, G, s);
}

}  // namespace

extern "C" int nvk_varlen_prefill(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                                  int64_t total_q, const void* k, const void* v,
                                  int64_t k_stride_tok, int64_t v_stride_tok,
                                  int64_t kv_stride_head, int64_t total_k,
                                  const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                  int32_t batch, int32_t max_seqlen_q, int32_t max_seqlen_k,
                                  const int32_t* block_tables, int64_t bt_stride,
                                  int32_t max_blocks, int32_t block_size, int32_t num_blocks,
                                  int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                  float scale, void* out, int64_t out_stride_tok,
                                  int64_t out_stride_head, void* workspace,
                                  size_t workspace_bytes, int32_t dtype, void* stream) {
  return varlen_prefill_impl(q, q_stride_tok, q_stride_head, total_q, k, v, k_stride_tok,
                             v_stride_tok, kv_stride_head, total_k, cu_seqlens_q, cu_seqlens_k,
                             batch, max_seqlen_q, max_seqlen_k, block_tables, bt_stride,
                             max_blocks, block_size, num_blocks, num_q_heads, num_kv_heads,
                             head_dim, scale, out, out_stride_tok, out_stride_head, workspace,
                             workspace_bytes, dtype, stream, nullptr, 0);
}

extern "C" int nvk_varlen_prefill_ordered(
    const void* q, int64_t q_stride_tok, int64_t q_stride_head, int64_t total_q, const void* k,
    const void* v, int64_t k_stride_tok, int64_t v_stride_tok, int64_t kv_stride_head,
    int64_t total_k, const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int32_t batch,
    int32_t max_seqlen_q, int32_t max_seqlen_k, const int32_t* block_tables, int64_t bt_stride,
    int32_t max_blocks, int32_t block_size, int32_t num_blocks, int32_t num_q_heads,
    int32_t num_kv_heads, int32_t head_dim, float scale, void* out, int64_t out_stride_tok,
    int64_t out_stride_head, void* workspace, size_t workspace_bytes, const int32_t* order,
    size_t order_bytes_, int32_t dtype, void* stream) {
  return varlen_prefill_impl(q, q_stride_tok, q_stride_head, total_q, k, v, k_stride_tok,
                             v_stride_tok, kv_stride_head, total_k, cu_seqlens_q, cu_seqlens_k,
                             batch, max_seqlen_q, max_seqlen_k, block_tables, bt_stride,
                             max_blocks, block_size, num_blocks, num_q_heads, num_kv_heads,
                             head_dim, scale, out, out_stride_tok, out_stride_head, workspace,
                             workspace_bytes, dtype, stream, order, order_bytes_);
}

extern "C" size_t nvk_prefill_tile_order_size(int32_t batch, int32_t max_seqlen_q,
                                              int32_t max_keys, int32_t num_q_heads,
                                              int32_t num_kv_heads, int32_t block_size) {
  return order_bytes_for(batch, max_seqlen_q, max_keys, num_q_heads, num_kv_heads,
                         block_size > 0, block_size);
}

extern "C" int nvk_prefill_tile_order(const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                      int32_t batch, int32_t max_seqlen_q, int32_t max_keys,
                                      int32_t num_q_heads, int32_t num_kv_heads,
                                      int32_t block_size, int32_t* order, size_t order_bytes_,
                                      void* stream) {
  const size_t need = order_bytes_for(batch, max_seqlen_q, max_keys, num_q_heads, num_kv_heads,
                                      block_size > 0, block_size);
  if (need == 0) return NVK_OK;  // nothing to rank: the prefill runs in grid order
  if (!cu_seqlens_q || !cu_seqlens_k || !order) return NVK_EINVAL;
  if (order_bytes_ < need) return NVK_EWORKSPACE;
  const int G = num_q_heads / num_kv_heads;
  if (G != 1 && G != 2 && G != 4 && G != 8) return NVK_EUNSUPPORTED;
  const SplitPlan sp = plan_splits(batch, max_seqlen_q, max_keys, num_q_heads, num_kv_heads);
  hipLaunchKernelGGL(prefill_tile_order_kernel, dim3(1), dim3(kOrderThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), cu_seqlens_q, cu_seqlens_k, batch,
                     sp.n_qtiles, kRows / G, order);
  return nvk_launch_status();
}
