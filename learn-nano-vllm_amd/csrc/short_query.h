// Internal: attention for steps whose query ranges are short (at most 16 rows
// of query tokens x query heads per kv head), e.g. speculative-decode
// verification.  Used by nvk_varlen_prefill; not part of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

struct ShortQueryParams {
  const uint16_t* q;
  int64_t q_stride_tok, q_stride_head;
  const uint16_t* k_cache;
  const uint16_t* v_cache;
  const int32_t* cu_q;
  const int32_t* cu_k;
  int batch;
  const int32_t* block_tables;
  int64_t bt_stride;
  int max_blocks, block_size, num_blocks;
  int num_q_heads, num_kv_heads;
  float scale;
  uint16_t* out;
  int64_t out_stride_tok, out_stride_head;
  bool f16;  // elements are f16 (else bf16)
};

// True when the short-query kernels cover a launch of these sizes: paged keys
// with 64-aligned pages, max_seqlen_q * G <= 16 rows, head_dim 128.
bool short_query_applies(bool paged, int block_size, int max_seqlen_q, int num_q_heads,
                         int num_kv_heads, int head_dim, int batch);

// Workspace bytes (descriptors + partial records) for these static sizes.
size_t short_query_ws_bytes(int batch, int64_t max_keys, int num_q_heads, int num_kv_heads);

// Enqueues the two kernels (stream-K pass, combine).  ws: 256-byte aligned,
// short_query_ws_bytes() bytes.  Returns NVK_OK or a hipError_t.
int short_query_launch(const ShortQueryParams& p, int64_t max_keys, void* ws, hipStream_t s);
