// Device-side builders of a step's attention metadata for gfx950.
//
// The reference builds slot_mapping, positions, cu_seqlens and the padded
// block tables with per-token Python loops on the host
// (nanovllm/engine/model_runner.py:123-188) and uploads them.  Here the host
// sends only per-sequence numbers (cached / new token counts or lengths) and
// the block tables in compressed rows (offsets + ids, one list concatenation),
// and one kernel expands them, with the reference's exact formulas:
//
//   prefill (model_runner.py:129-170): for sequence s with start = cached
//     tokens and n = scheduled tokens,
//       cu_seqlens_q[s+1] = cu_seqlens_q[s] + n, cu_seqlens_k[s+1] = cu_seqlens_k[s] + start + n,
//       positions of its tokens = start .. start+n-1,
//       slot of position p = block_table[p / bs] * bs + p % bs   (lines 151-161)
//     a sequence without a block table (warmup, line 149) gets slot -1;
//   decode (model_runner.py:172-188): context_lens = len, positions = len-1,
//       slot = block_table[-1] * bs + last_block_num_tokens - 1
//            = block_table[-1] * bs + (len - 1) % bs            (sequence.py:59-65);
//   block tables (model_runner.py:123-127): row s = the sequence's pages,
//       padded with -1 to the table width.
// The decode builder can write straight into a captured graph's static
// buffers: rows [batch, padded_batch) get slot -1 and context length 0, and
// only the live [:batch, :width] rectangle of the table is written
// (model_runner.py:204-210).
//
// Work split: every workgroup rebuilds the exclusive prefix of the per-
// sequence token counts in LDS (batch <= kMaxBatch, one pass), then a
// grid-stride loop maps each token to its sequence by binary search over that
// prefix.  The step is latency bound (a few KB to a few hundred KB of output).
#include "nvk_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kMaxBatch = 8192;
constexpr int kMaxGrid = 1024;

// Exclusive prefix of value(0..B) into s[0..B] (s[B] = total) by one
// workgroup; ends with a barrier.
template <typename F>
__device__ void block_prefix(F value, int B, int* s, int* s_wsum) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int per = (B + kThreads - 1) / kThreads;
  const int b0 = tid * per;
  int local = 0;
  for (int i = 0; i < per; ++i)
    if (b0 + i < B) local += value(b0 + i);
  int x = local;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off);
    if (lane >= off) x += y;
  }
  if (lane == 63) s_wsum[wave] = x;
  __syncthreads();
  int run = x - local;
  for (int w = 0; w < wave; ++w) run += s_wsum[w];
  for (int i = 0; i < per; ++i) {
    if (b0 + i < B) {
      s[b0 + i] = run;
      run += value(b0 + i);
    }
  }
  if (tid == kThreads - 1) s[B] = run;
  __syncthreads();
}

// Padded block-table rows [0, B) x [0, W) from compressed rows.
__device__ void write_tables(const int32_t* __restrict__ off, const int32_t* __restrict__ ids,
                             int B, int W, int64_t stride, int32_t* __restrict__ tables) {
  const int64_t n = (int64_t)B * W;
  for (int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x; e < n;
       e += (int64_t)gridDim.x * kThreads) {
    const int b = (int)(e / W), i = (int)(e - (int64_t)b * W);
    const int lo = off[b], len = off[b + 1] - lo;
    tables[(int64_t)b * stride + i] = i < len ? ids[lo + i] : -1;
  }
}

struct PrefillMetaArgs {
  const int32_t* num_cached;
  const int32_t* num_new;
  const int32_t* bt_off;
  const int32_t* bt_ids;
  int batch, block_size, width;
  int64_t n_tokens;
  int32_t* cu_q;
  int32_t* cu_k;
  int64_t* positions;
  int32_t* slots;
  int32_t* tables;  // may be null
};

__global__ __launch_bounds__(kThreads) void prefill_metadata_kernel(PrefillMetaArgs a) {
  __shared__ int s_cu[kMaxBatch + 1];
  __shared__ int s_wsum[kThreads / 64];
  const int B = a.batch;
  block_prefix([&](int b) { return a.num_new[b]; }, B, s_cu, s_wsum);
  if (blockIdx.x == 0)
    for (int b = threadIdx.x; b <= B; b += kThreads) a.cu_q[b] = s_cu[b];
  const int64_t T = a.n_tokens;
  for (int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x; t < T;
       t += (int64_t)gridDim.x * kThreads) {
    int lo = 0, hi = B - 1;  // sequence of token t: last s with s_cu[s] <= t
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if ((int64_t)s_cu[mid] <= t) lo = mid; else hi = mid - 1;
    }
    const int64_t pos = (int64_t)a.num_cached[lo] + (t - s_cu[lo]);
    a.positions[t] = pos;
    const int off = a.bt_off[lo], len = a.bt_off[lo + 1] - off;
    const int64_t blk = pos / a.block_size;
    a.slots[t] = blk < len ? a.bt_ids[off + blk] * a.block_size + (int32_t)(pos - blk * a.block_size)
                           : -1;
  }
  if (a.tables) write_tables(a.bt_off, a.bt_ids, B, a.width, a.width, a.tables);
  if (blockIdx.x == 0) {  // cu_seqlens_k: prefix of cached + new, in the same LDS
    __syncthreads();
    block_prefix([&](int b) { return a.num_cached[b] + a.num_new[b]; }, B, s_cu, s_wsum);
    for (int b = threadIdx.x; b <= B; b += kThreads) a.cu_k[b] = s_cu[b];
  }
}

struct DecodeMetaArgs {
  const int32_t* seq_lens;
  const int32_t* bt_off;
  const int32_t* bt_ids;
  int batch, padded_batch, block_size, width;
  int64_t table_stride;
  int32_t* context_lens;
  int64_t* positions;
  int32_t* slots;
  int32_t* tables;
};

__global__ __launch_bounds__(kThreads) void decode_metadata_kernel(DecodeMetaArgs a) {
  for (int b = blockIdx.x * kThreads + threadIdx.x; b < a.padded_batch; b += gridDim.x * kThreads) {
    if (b < a.batch) {
      const int n = a.seq_lens[b];
      const int last = a.bt_off[b + 1] - 1;
      a.context_lens[b] = n;
      a.positions[b] = (int64_t)n - 1;
      a.slots[b] = (n >= 1 && last >= a.bt_off[b])
                       ? a.bt_ids[last] * a.block_size + (n - 1) % a.block_size
                       : -1;
    } else {  // graph padding rows
      a.context_lens[b] = 0;
      a.slots[b] = -1;
    }
  }
  write_tables(a.bt_off, a.bt_ids, a.batch, a.width, a.table_stride, a.tables);
}

// cu_seqlens of a uniform query block per sequence over its cache lengths
// (seqlen_q queries at the end of each sequence's seqlens_k keys): one
// workgroup, cu_q[b] = b * seqlen_q, cu_k = exclusive prefix of seqlens_k.
__global__ __launch_bounds__(kThreads) void uniform_cu_seqlens_kernel(const int32_t* seqlens_k,
                                                                     int B, int seqlen_q,
                                                                     int32_t* cu_q,
                                                                     int32_t* cu_k) {
  __shared__ int s_cu[kMaxBatch + 1];
  __shared__ int s_wsum[kThreads / 64];
  block_prefix([&](int b) { return seqlens_k[b]; }, B, s_cu, s_wsum);
  for (int b = threadIdx.x; b <= B; b += kThreads) {
    cu_q[b] = b * seqlen_q;
    cu_k[b] = s_cu[b];
  }
}

// Refresh of a captured decode graph's static metadata: slot -1 and context 0
// past the live batch up to the static rows, the live block-table rectangle
// copied (the rest of the table left as it is).
struct GraphRefreshArgs {
  const int64_t* src_pos;
  const int32_t* src_slot;
  const int32_t* src_ctx;
  const int32_t* src_bt;
  int64_t src_bt_stride;
  int batch, width, static_rows;
  int64_t* pos;
  int32_t* slot;
  int32_t* ctx;
  int32_t* bt;
  int64_t bt_stride;
};

__global__ __launch_bounds__(kThreads) void decode_graph_refresh_kernel(GraphRefreshArgs a) {
  const int64_t cells = (int64_t)a.batch * a.width;
  const int64_t n = cells > a.static_rows ? cells : a.static_rows;
  for (int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x; e < n;
       e += (int64_t)gridDim.x * kThreads) {
    if (e < a.static_rows) {
      const int b = (int)e;
      const bool live = b < a.batch;
      a.slot[b] = live ? a.src_slot[b] : -1;
      a.ctx[b] = live ? a.src_ctx[b] : 0;
      if (live) a.pos[b] = a.src_pos[b];
    }
    if (e < cells) {
      const int64_t b = e / a.width, j = e - b * a.width;
      a.bt[b * a.bt_stride + j] = a.src_bt[b * a.src_bt_stride + j];
    }
  }
}

}  // namespace

extern "C" int nvk_prefill_metadata(const int32_t* num_cached, const int32_t* num_new,
                                    const int32_t* bt_offsets, const int32_t* bt_ids,
                                    int32_t batch, int32_t block_size, int32_t table_width,
                                    int64_t n_tokens, int32_t* cu_seqlens_q,
                                    int32_t* cu_seqlens_k, int64_t* positions,
                                    int32_t* slot_mapping, int32_t* block_tables, void* stream) {
  if (batch < 0 || block_size <= 0 || n_tokens < 0 || table_width < 0) return NVK_EINVAL;
  if (batch > kMaxBatch) return NVK_EUNSUPPORTED;
  if (batch == 0) return NVK_OK;
  if (!num_cached || !num_new || !bt_offsets || !cu_seqlens_q || !cu_seqlens_k) return NVK_EINVAL;
  if (n_tokens > 0 && (!positions || !slot_mapping)) return NVK_EINVAL;
  if (block_tables && table_width == 0) return NVK_EINVAL;
  PrefillMetaArgs a;
  a.num_cached = num_cached;
  a.num_new = num_new;
  a.bt_off = bt_offsets;
  a.bt_ids = bt_ids;
  a.batch = batch;
  a.block_size = block_size;
  a.width = table_width;
  a.n_tokens = n_tokens;
  a.cu_q = cu_seqlens_q;
  a.cu_k = cu_seqlens_k;
  a.positions = positions;
  a.slots = slot_mapping;
  a.tables = block_tables;
  int64_t work = n_tokens > (int64_t)batch * table_width ? n_tokens : (int64_t)batch * table_width;
  int64_t grid = (work + kThreads - 1) / kThreads;
  grid = grid < 1 ? 1 : (grid > kMaxGrid ? kMaxGrid : grid);
  hipLaunchKernelGGL(prefill_metadata_kernel, dim3((unsigned)grid), dim3(kThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), a);
  return nvk_launch_status();
}

extern "C" int nvk_decode_metadata(const int32_t* seq_lens, const int32_t* bt_offsets,
                                   const int32_t* bt_ids, int32_t batch, int32_t padded_batch,
                                   int32_t block_size, int32_t table_width,
                                   int64_t table_row_stride, int32_t* context_lens,
                                   int64_t* positions, int32_t* slot_mapping,
                                   int32_t* block_tables, void* stream) {
  if (batch < 0 || padded_batch < batch || block_size <= 0 || table_width < 0 ||
      table_row_stride < table_width)
    return NVK_EINVAL;
  if (padded_batch == 0) return NVK_OK;
  if (!context_lens || !positions || !slot_mapping) return NVK_EINVAL;
  if (batch > 0 && (!seq_lens || !bt_offsets || !bt_ids || !block_tables || table_width == 0))
    return NVK_EINVAL;
  DecodeMetaArgs a;
  a.seq_lens = seq_lens;
  a.bt_off = bt_offsets;
  a.bt_ids = bt_ids;
  a.batch = batch;
  a.padded_batch = padded_batch;
  a.block_size = block_size;
  a.width = table_width;
  a.table_stride = table_row_stride;
  a.context_lens = context_lens;
  a.positions = positions;
  a.slots = slot_mapping;
  a.tables = block_tables;
  int64_t work = (int64_t)batch * table_width > padded_batch ? (int64_t)batch * table_width
                                                             : padded_batch;
  int64_t grid = (work + kThreads - 1) / kThreads;
  grid = grid < 1 ? 1 : (grid > kMaxGrid ? kMaxGrid : grid);
  hipLaunchKernelGGL(decode_metadata_kernel, dim3((unsigned)grid), dim3(kThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), a);
  return nvk_launch_status();
}

extern "C" int nvk_uniform_cu_seqlens(const int32_t* seqlens_k, int32_t batch, int32_t seqlen_q,
                                      int32_t* cu_seqlens_q, int32_t* cu_seqlens_k,
                                      void* stream) {
  if (batch < 0 || seqlen_q < 0 || batch > kMaxBatch) return NVK_EINVAL;
  if ((int64_t)batch * seqlen_q > INT32_MAX) return NVK_EINVAL;
  if (!cu_seqlens_q || !cu_seqlens_k || (batch > 0 && !seqlens_k)) return NVK_EINVAL;
  hipLaunchKernelGGL(uniform_cu_seqlens_kernel, dim3(1), dim3(kThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), seqlens_k, batch, seqlen_q,
                     cu_seqlens_q, cu_seqlens_k);
  return nvk_launch_status();
}

extern "C" int nvk_decode_graph_refresh(const int64_t* src_positions,
                                        const int32_t* src_slot_mapping,
                                        const int32_t* src_context_lens,
                                        const int32_t* src_block_tables, int64_t src_bt_stride,
                                        int32_t batch, int32_t width, int64_t* positions,
                                        int32_t* slot_mapping, int32_t* context_lens,
                                        int32_t* block_tables, int64_t bt_stride,
                                        int32_t static_rows, void* stream) {
  if (batch < 0 || width < 0 || static_rows < 0 || batch > static_rows) return NVK_EINVAL;
  if (static_rows == 0) return NVK_OK;
  if (!positions || !slot_mapping || !context_lens) return NVK_EINVAL;
  if (batch > 0 && (!src_positions || !src_slot_mapping || !src_context_lens)) return NVK_EINVAL;
  if (batch > 0 && width > 0) {
    if (!src_block_tables || !block_tables) return NVK_EINVAL;
    if (src_bt_stride < width || bt_stride < width) return NVK_EINVAL;
  }
  GraphRefreshArgs a;
  a.src_pos = src_positions;
  a.src_slot = src_slot_mapping;
  a.src_ctx = src_context_lens;
  a.src_bt = src_block_tables;
  a.src_bt_stride = src_bt_stride;
  a.batch = batch;
  a.width = batch > 0 ? width : 0;
  a.static_rows = static_rows;
  a.pos = positions;
  a.slot = slot_mapping;
  a.ctx = context_lens;
  a.bt = block_tables;
  a.bt_stride = bt_stride;
  const int64_t cells = (int64_t)a.batch * a.width;
  const int64_t n = cells > static_rows ? cells : static_rows;
  int64_t grid = (n + kThreads - 1) / kThreads;
  grid = grid > kMaxGrid ? kMaxGrid : grid;
  hipLaunchKernelGGL(decode_graph_refresh_kernel, dim3((unsigned)grid), dim3(kThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), a);
  return nvk_launch_status();
}
