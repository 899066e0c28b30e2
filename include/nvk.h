/*
 * nvk.h — C ABI of the MI355X (gfx950) KV-cache hot path of nano-vLLM.
 *
 * Three entry points replace the three GPU calls that
 * nanovllm/layers/attention.py makes per decoder layer:
 *
 *   nvk_kv_store        <- store_kvcache_kernel / store_kvcache
 *                          (nanovllm/layers/attention.py:10-40)
 *   nvk_paged_decode    <- flash_attn_with_kvcache(q.unsqueeze(1), k_cache, v_cache,
 *                          cache_seqlens=context_lens, block_table=block_tables,
 *                          softmax_scale, causal=True)
 *                          (nanovllm/layers/attention.py:72-74)
 *   nvk_varlen_prefill  <- flash_attn_varlen_func(q, k, v, max_seqlen_q, cu_seqlens_q,
 *                          max_seqlen_k, cu_seqlens_k, softmax_scale, causal=True,
 *                          block_table)
 *                          (nanovllm/layers/attention.py:64-70)
 *
 * and one more fuses the steps just before them:
 *
 *   nvk_qk_norm_rope_store <- q_norm / k_norm / rotary_emb of Qwen3Attention.forward
 *                          (nanovllm/models/qwen3.py:79-86) + the store of
 *                          attention.py:62-63
 *   nvk_paged_decode_prologue <- the same prologue + the decode call of a
 *                          decode step, in one decode kernel
 *
 * Conventions shared by every entry point
 *   - All pointers are device pointers (hipMalloc / torch CUDA tensors) except
 *     where stated.  Strides are in ELEMENTS, not bytes.
 *   - Nothing is allocated and nothing is synchronised: the work is enqueued on
 *     `stream` (a hipStream_t passed as void*; NULL = the null stream), so every
 *     entry point may be captured into a hipGraph.  No device metadata is read
 *     on the host.
 *   - Return value: 0 = enqueued; a negative NVK_E* code = the arguments were
 *     rejected before anything was launched; a positive value = the hipError_t
 *     reported by the launch.
 *   - The library keeps no pointer after it returns and has no global state
 *     but the static scratch of nvk_paged_decode_noalloc (one per GPU), so
 *     calls from several host threads on distinct streams, each with its own
 *     workspace, are independent.
 *   - KV-cache layout (nanovllm/engine/model_runner.py:115-121): per layer
 *     k_cache / v_cache are contiguous [num_blocks][block_size][num_kv_heads][head_dim];
 *     the flat token slot s = page * block_size + offset addresses row s of a
 *     [num_blocks*block_size][num_kv_heads*head_dim] view.
 */
#ifndef NVK_H_
#define NVK_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* error codes (negative; positive values are hipError_t) */
#define NVK_OK 0
#define NVK_EINVAL (-1)       /* null pointer, negative size, inconsistent shape   */
#define NVK_EUNSUPPORTED (-2) /* head_dim / group size / dtype not built          */
#define NVK_EALIGN (-3)       /* pointer or stride misaligned for the element type */
#define NVK_EWORKSPACE (-4)   /* workspace missing or smaller than required       */
#define NVK_ESCRATCH (-5)     /* sizes exceed the no-allocation entry's scratch    */

/* element types of q / k / v / caches / outputs */
#define NVK_DTYPE_BF16 0
#define NVK_DTYPE_F16 1
#define NVK_DTYPE_F32 2

/* Human-readable text for an NVK_E* code or a hipError_t. Never NULL. */
const char* nvk_strerror(int code);

/* gfx target the library was built for, e.g. "gfx950". */
const char* nvk_build_target(void);

/*
 * KV-store scatter.
 * Replaces store_kvcache_kernel (nanovllm/layers/attention.py:10-30) and its
 * launcher store_kvcache (attention.py:33-40).
 *
 * For every token t in [0, n_tokens):
 *     s = slot_mapping[t];
 *     if s == -1: skip                                  (attention.py:22-23)
 *     k_cache[s*row_elems : (s+1)*row_elems] = key  [t*key_row_stride   : +row_elems]
 *     v_cache[s*row_elems : (s+1)*row_elems] = value[t*value_row_stride : +row_elems]
 *
 * row_elems = num_kv_heads*head_dim (the Triton kernel's D).  Each token row of
 * key / value must be contiguous (the reference asserts stride(-1)==1 and
 * stride(1)==head_dim, attention.py:36-37); the row strides are free, which
 * covers the value view of the packed qkv (row stride (Hq+2*Hkv)*head_dim).
 * cache_slots = num_blocks*block_size.  A slot outside [0, cache_slots) is
 * skipped like -1: the reference writes out of bounds there, this library
 * writes nothing.  Duplicate slots are a race (one of the rows wins), never a
 * fault.  elem_bytes is 2 (bf16/f16) or 4 (f32).
 */
int nvk_kv_store(const void* key, int64_t key_row_stride,
                 const void* value, int64_t value_row_stride,
                 void* k_cache, void* v_cache,
                 const int32_t* slot_mapping, int64_t n_tokens,
                 int32_t row_elems, int32_t elem_bytes, int64_t cache_slots,
                 void* stream);

/*
 * Paged GQA decode attention, one query token per sequence.
 * Replaces flash_attn_with_kvcache(q.unsqueeze(1), k_cache, v_cache,
 *     cache_seqlens=context_lens, block_table=block_tables,
 *     softmax_scale=scale, causal=True)      (nanovllm/layers/attention.py:72-74)
 *
 *   out[b, h, :] = softmax_j( scale * q[b,h,:] . K[b, j, h/G, :] ) V[b, j, h/G, :]
 *   over j < context_lens[b], with K[b, j] = k_cache[block_tables[b, j/block_size]]
 *   [j % block_size] and G = num_q_heads / num_kv_heads.
 *
 * q:   [batch][num_q_heads][head_dim] with strides (q_stride_tok, q_stride_head, 1).
 * out: same shape, strides (out_stride_tok, out_stride_head, 1).
 * block_tables: int32 [batch][max_blocks] with row stride bt_stride; entries at
 *   or beyond ceil(context_lens[b]/block_size) are never read (they may be -1
 *   or stale, model_runner.py:123-127, 204-211).
 * context_lens: int32 [batch]; it counts the token just stored
 *   (model_runner.py:180).  context_lens[b] == 0 (a padded graph row) writes
 *   zeros.  Lengths above max_blocks*block_size are clamped to it.  A page id
 *   outside [0, num_blocks) is never dereferenced; the output of a context
 *   that names one is unspecified (the reference reads out of bounds there).
 * workspace: device scratch of nvk_paged_decode_workspace_size() bytes, 256-byte
 *   aligned (per-context descriptors and the partial results of contexts split
 *   between waves); it need not be initialised, every call writes what it
 *   reads.  Two calls in flight at once need two workspaces.
 * Two kernels are enqueued: the balanced split-K pass and a combine pass.
 * scale must be > 0.  dtype: NVK_DTYPE_BF16 or NVK_DTYPE_F16 (q, caches and
 * out alike; f32 accumulation either way).  head_dim: 128 or 64.
 * G: 1, 2, 4 or 8.  batch <= 2048.  q, k_cache, v_cache and out 16-byte
 * aligned, token / head strides multiples of 8 elements.
 */
int nvk_paged_decode(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                     const void* k_cache, const void* v_cache,
                     const int32_t* block_tables, int64_t bt_stride,
                     const int32_t* context_lens,
                     int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                     int32_t head_dim, int32_t block_size, int32_t max_blocks,
                     int32_t num_blocks, float scale,
                     void* out, int64_t out_stride_tok, int64_t out_stride_head,
                     void* workspace, size_t workspace_bytes,
                     int32_t dtype, void* stream);

/* Bytes of workspace nvk_paged_decode needs for these sizes (0 on bad input). */
size_t nvk_paged_decode_workspace_size(int32_t batch, int32_t num_q_heads,
                                       int32_t num_kv_heads, int32_t head_dim,
                                       int32_t block_size, int32_t max_blocks);

/*
 * nvk_paged_decode without a workspace argument: it allocates nothing.
 * No counterpart in the reference.  For callers that cannot allocate device
 * memory: code under HIP graph capture that may not call hipMalloc, serving
 * loops and harnesses that forbid allocation.
 *
 * Same arguments, kernels and results (bit for bit) as nvk_paged_decode; the
 * workspace is instead a static device array of NVK_NOALLOC_SCRATCH_BYTES
 * inside the library, one per GPU, held until the process ends.  Sizes whose
 * nvk_paged_decode_workspace_size() exceeds it are rejected with
 * NVK_ESCRATCH before anything is launched (Qwen3-0.6B shapes need at most
 * 4.5 MB at batch 2048; group size 8 at most 17.5 MB).  The scratch of the
 * current device is used (looked up once per device), and `stream` must
 * belong to that device (else NVK_EINVAL).  Every call on one GPU shares its
 * scratch: two calls that overlap on one GPU (different streams, or two host
 * threads) race and give undefined results; calls ordered on one stream are
 * safe.  Nothing in the scratch needs clearing between calls.
 *
 * nvk_paged_decode_noalloc_init: looks up the current device's scratch now
 * (hipGetSymbolAddress) instead of at that device's first call.  Call it once
 * per device, with the device current, before capturing
 * nvk_paged_decode_noalloc into a graph, so that nothing but the kernel
 * launches happens under capture.  Returns 0 or a hipError_t.
 */
#define NVK_NOALLOC_SCRATCH_BYTES (20u << 20)
int nvk_paged_decode_noalloc_init(void);
int nvk_paged_decode_noalloc(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                             const void* k_cache, const void* v_cache,
                             const int32_t* block_tables, int64_t bt_stride,
                             const int32_t* context_lens,
                             int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                             int32_t head_dim, int32_t block_size, int32_t max_blocks,
                             int32_t num_blocks, float scale,
                             void* out, int64_t out_stride_tok, int64_t out_stride_head,
                             int32_t dtype, void* stream);

/*
 * Varlen causal attention over new tokens, with or without a paged prefix.
 * Replaces flash_attn_varlen_func(q, k, v, max_seqlen_q=..., cu_seqlens_q=...,
 *     max_seqlen_k=..., cu_seqlens_k=..., softmax_scale=scale, causal=True,
 *     block_table=block_tables)               (nanovllm/layers/attention.py:64-70)
 *
 * Sequence s has Lq = cu_seqlens_q[s+1]-cu_seqlens_q[s] query rows and
 * Lk = cu_seqlens_k[s+1]-cu_seqlens_k[s] keys.  Query row i sees key j iff
 * j <= i + Lk - Lq (bottom-right aligned causal mask, the flash-attn 2.x
 * convention); a row that sees no key is written as zeros.
 *
 * q:   [total_q][num_q_heads][head_dim], strides (q_stride_tok, q_stride_head, 1).
 * out: [total_q][num_q_heads][head_dim], strides (out_stride_tok, out_stride_head, 1).
 * Paged mode (block_tables != NULL): k / v are the caches
 *   [num_blocks][block_size][num_kv_heads][head_dim] (contiguous; k_stride_tok,
 *   v_stride_tok and kv_stride_head are ignored) and key j of sequence s lives
 *   in page block_tables[s*bt_stride + j/block_size].  Lk is clamped to
 *   max_blocks*block_size.  A page id outside [0, num_blocks) is never
 *   dereferenced; the output of a sequence that names one is unspecified.
 * Dense mode (block_tables == NULL): k / v are [total_k][num_kv_heads][head_dim]
 *   with row strides k_stride_tok / v_stride_tok and head stride kv_stride_head;
 *   key j of sequence s is row cu_seqlens_k[s] + j (rows >= total_k are
 *   treated as absent).
 * max_seqlen_q sizes the grid and max_seqlen_k (0 = unknown) bounds the keys
 *   of a sequence; both are host values, as in the reference's Context
 *   (context.py:8-11).  max_seqlen_k only steers the split-K plan: every key
 *   is still attended if a sequence has more.
 * workspace: optional device scratch (256-byte aligned) of
 *   nvk_varlen_prefill_workspace_size() bytes.  When the query tiles alone
 *   cannot fill the GPU (few, short query ranges over long contexts, e.g.
 *   speculative-decode verification) the key range is split across
 *   workgroups whose partial results go to the workspace, and a second kernel
 *   merges them.  NULL (or too small) = no split; the result is the same up
 *   to rounding.  Otherwise, for a multi-sequence prefill whose grid takes
 *   more than two rounds of workgroups, a one-workgroup kernel first ranks
 *   the (sequence, query tile) pairs by their key count into the workspace
 *   and the attention kernel runs them longest first; without the workspace
 *   they run in grid order, with the same output bits.  Two calls in flight
 *   at once need two workspaces.
 * scale must be > 0.  dtype: NVK_DTYPE_BF16 or NVK_DTYPE_F16 (q, k / v and
 * out alike; f32 accumulation either way).  head_dim: 128.  G: 1, 2, 4 or 8.
 */
int nvk_varlen_prefill(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                       int64_t total_q,
                       const void* k, const void* v,
                       int64_t k_stride_tok, int64_t v_stride_tok,
                       int64_t kv_stride_head, int64_t total_k,
                       const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                       int32_t batch, int32_t max_seqlen_q, int32_t max_seqlen_k,
                       const int32_t* block_tables, int64_t bt_stride,
                       int32_t max_blocks, int32_t block_size, int32_t num_blocks,
                       int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                       float scale,
                       void* out, int64_t out_stride_tok, int64_t out_stride_head,
                       void* workspace, size_t workspace_bytes,
                       int32_t dtype, void* stream);

/* Bytes of workspace nvk_varlen_prefill uses to split these sizes (0 = it
 * does not split them, or bad input).  max_seqlen_k: as in nvk_varlen_prefill
 * (for a paged call, at most max_blocks*block_size). */
size_t nvk_varlen_prefill_workspace_size(int32_t batch, int32_t max_seqlen_q,
                                         int32_t max_seqlen_k, int32_t num_q_heads,
                                         int32_t num_kv_heads, int32_t head_dim);

/*
 * The longest-first order of a prefill's query tiles, ranked once for every
 * layer of a step.  Every decoder layer of a model step calls the prefill
 * with the same cu_seqlens (nanovllm/layers/attention.py:67-70, once per
 * layer of nanovllm/models/qwen3.py:180-181); nvk_varlen_prefill ranks them
 * in each call, these rank them once.
 *
 * nvk_prefill_tile_order_size: bytes of the order a prefill of these sizes
 *   uses, 0 when it runs its query tiles in grid order (few tiles, short
 *   query ranges split across workgroups or taken by the short-query
 *   kernels).  max_keys: the per-sequence key bound the prefill call will
 *   use (min(max_seqlen_k, max_blocks*block_size) paged, min(max_seqlen_k,
 *   total_k) dense); block_size: the page size, 0 for dense keys.
 * nvk_prefill_tile_order: writes that order (one kernel; nothing when the
 *   size is 0): a permutation of the (sequence, query tile) pairs followed by
 *   a tag of the batch and the tile count.  order: device int32, 16-byte
 *   aligned, order_bytes >= size.
 * nvk_varlen_prefill_ordered: nvk_varlen_prefill with the order given; it
 *   launches no ranking kernel.  order_bytes: the bytes of the order buffer;
 *   when the call would use an order and order_bytes is below
 *   nvk_prefill_tile_order_size() of its sizes, it returns NVK_EWORKSPACE
 *   and launches nothing.  The order should come from nvk_prefill_tile_order
 *   with the same metadata; the output is the same for any order: an order
 *   ranked for other lengths of the same batch and tile count only runs the
 *   tiles in a slower order, and one whose tag names another batch or tile
 *   count is ignored (the tiles then run in grid order).  NULL =
 *   nvk_varlen_prefill.  Outputs are bit-identical to nvk_varlen_prefill's.
 */
size_t nvk_prefill_tile_order_size(int32_t batch, int32_t max_seqlen_q, int32_t max_keys,
                                   int32_t num_q_heads, int32_t num_kv_heads, int32_t block_size);
int nvk_prefill_tile_order(const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                           int32_t batch, int32_t max_seqlen_q, int32_t max_keys,
                           int32_t num_q_heads, int32_t num_kv_heads, int32_t block_size,
                           int32_t* order, size_t order_bytes, void* stream);
int nvk_varlen_prefill_ordered(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                               int64_t total_q,
                               const void* k, const void* v,
                               int64_t k_stride_tok, int64_t v_stride_tok,
                               int64_t kv_stride_head, int64_t total_k,
                               const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                               int32_t batch, int32_t max_seqlen_q, int32_t max_seqlen_k,
                               const int32_t* block_tables, int64_t bt_stride,
                               int32_t max_blocks, int32_t block_size, int32_t num_blocks,
                               int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                               float scale,
                               void* out, int64_t out_stride_tok, int64_t out_stride_head,
                               void* workspace, size_t workspace_bytes, const int32_t* order,
                               size_t order_bytes, int32_t dtype, void* stream);

/*
 * Fused attention prologue: q/k RMSNorm + rotary embedding + KV-store.
 * Replaces, per decoder layer, the steps between the qkv projection and the
 * attention kernels: nanovllm/models/qwen3.py:79-86 (split, q_norm, k_norm,
 * rotary_emb), i.e. RMSNorm.rms_forward (nanovllm/layers/layernorm.py:16-26),
 * RotaryEmbedding.forward / apply_rotary_emb (rotary_embedding.py:6-14,
 * 37-48), and the store_kvcache call of Attention.forward (attention.py:62-63).
 *
 * For every token t in [0, n_tokens) and head row of qkv[t] =
 * [q (num_q_heads rows) | k (num_kv_heads rows) | v (num_kv_heads rows)],
 * each row head_dim elements of type T (bf16 or f16) contiguous, token row
 * stride qkv_row_stride:
 *     q, k rows: x = float(row); x *= rsqrt(mean(x^2) + eps); x = T(x);
 *                x = T(x * weight)               (q_norm_weight / k_norm_weight, T)
 *                rotated by cos_sin_cache[positions[t]] (halves cos | sin,
 *                rotate-half convention) and rounded to T
 *     q_out[t, h]                      = rotated q row h
 *     k_out[t, h]                      = rotated k row h        (k_out may be NULL)
 *     k_cache row slot_mapping[t], h   = rotated k row h        (slot -1 skipped)
 *     v_cache row slot_mapping[t], h   = v row h (bit copy)     (slot -1 skipped)
 * Every f32 product and sum is rounded separately, as the reference's tensor
 * operations are.  cos_sin_cache: float32 [max_position][row stride >=
 * head_dim] (the reference's cos_sin_cache buffer, [max_position, 1,
 * head_dim]); a position outside [0, max_position) is clamped into it (output
 * unspecified, no out-of-bounds read).  slot_mapping NULL = no store (the
 * reference skips the store while the caches are empty, attention.py:62);
 * otherwise caches as in nvk_kv_store with cache_slots = num_blocks*block_size
 * and slots outside [0, cache_slots) skipped.  positions: int64 [n_tokens].
 * dtype (T of qkv, the weights, q_out, k_out and the caches): NVK_DTYPE_BF16
 * or NVK_DTYPE_F16 (the model's dtype, model_runner.py:29).  head_dim: 128.
 * Pointers 16-byte aligned, strides multiples of 8 elements
 * (cos_sin_row_stride of 4), n_tokens < 2^31.  One kernel (one workgroup per
 * token), nothing allocated.
 */
int nvk_qk_norm_rope_store(const void* qkv, int64_t qkv_row_stride, int64_t n_tokens,
                           const int64_t* positions, const void* q_norm_weight,
                           const void* k_norm_weight, float eps, const float* cos_sin_cache,
                           int64_t cos_sin_row_stride, int64_t max_position,
                           int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                           void* q_out, int64_t q_out_stride_tok, int64_t q_out_stride_head,
                           void* k_out, int64_t k_out_stride_tok, int64_t k_out_stride_head,
                           void* k_cache, void* v_cache, const int32_t* slot_mapping,
                           int64_t cache_slots, int32_t dtype, void* stream);

/*
 * Decode step with the attention prologue applied inside the decode kernel:
 * nvk_qk_norm_rope_store followed by nvk_paged_decode for one new token per
 * sequence (qwen3.py:79-86 then attention.py:62-63 and 72-74 in a decode
 * step), without materialising q and with one launch fewer.
 * Row b of qkv is sequence b's new token (row stride qkv_row_stride, layout
 * as in nvk_qk_norm_rope_store).  q is normed and rotated at positions[b] in
 * the kernel; the new token's k (normed, rotated) and v are stored at cache
 * row slot_mapping[b] (skipped when outside [0, cache_slots)) and used from
 * registers for key context_lens[b] - 1, which must be that cache row (as
 * model_runner.prepare_decode builds it: slot = the row of position
 * len - 1, context_lens = len); a sequence of context length 0 (a graph
 * padding row) stores nothing.  Output, caches, block tables, context
 * lengths, workspace (nvk_paged_decode_workspace_size) and empty contexts as
 * in nvk_paged_decode; norm weights, eps, cos_sin_cache and positions as in
 * nvk_qk_norm_rope_store.  The result equals the two calls' bit for bit.
 * dtype: NVK_DTYPE_BF16 or NVK_DTYPE_F16 (qkv, weights, caches and out
 * alike).  head_dim: 128.  Two kernels are enqueued (decode with prologue,
 * combine).
 */
int nvk_paged_decode_prologue(
    const void* qkv, int64_t qkv_row_stride, const int64_t* positions, const void* q_norm_weight,
    const void* k_norm_weight, float eps, const float* cos_sin_cache, int64_t cos_sin_row_stride,
    int64_t max_position, void* k_cache, void* v_cache, const int32_t* slot_mapping,
    int64_t cache_slots, const int32_t* block_tables, int64_t bt_stride,
    const int32_t* context_lens, int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
    int32_t head_dim, int32_t block_size, int32_t max_blocks, int32_t num_blocks, float scale,
    void* out, int64_t out_stride_tok, int64_t out_stride_head, void* workspace,
    size_t workspace_bytes, int32_t dtype, void* stream);

/*
 * Device-side step metadata.
 * Replaces the per-token host loops of ModelRunner.prepare_prefill /
 * prepare_decode / prepare_block_tables (nanovllm/engine/model_runner.py:
 * 123-188) and the graph-buffer refresh of run_model (model_runner.py:
 * 204-210).  Block tables come compressed: row b is
 * bt_ids[bt_offsets[b] .. bt_offsets[b+1]) (int32 [batch+1] offsets).
 *
 * nvk_prefill_metadata: per sequence b, num_cached[b] cached and num_new[b]
 * new (scheduled) tokens; n_tokens = sum(num_new).  Writes
 *   cu_seqlens_q [batch+1] = exclusive prefix of num_new,
 *   cu_seqlens_k [batch+1] = exclusive prefix of num_cached + num_new,
 *   positions    [n_tokens] int64: num_cached[b] .. num_cached[b]+num_new[b]-1,
 *   slot_mapping [n_tokens]: block_table[p / block_size] * block_size + p % block_size
 *                (-1 for a sequence without pages, or past its table),
 *   block_tables [batch][table_width], -1 padded (NULL = not written; the
 *                reference builds it only when some sequence has cached tokens).
 * batch <= 8192.  bt_ids may be NULL when no sequence has pages.
 *
 * nvk_decode_metadata: per sequence b of length seq_lens[b] (counting the new
 * token), rows b < batch: context_lens = len, positions = len - 1,
 *   slot = block_table[-1] * block_size + (len - 1) % block_size (the
 *   reference's block_table[-1]*bs + last_block_num_tokens - 1), and
 *   block_tables row b = its pages, -1 padded to table_width (row stride
 *   table_row_stride; columns >= table_width untouched);
 * rows batch <= b < padded_batch (graph padding): slot -1, context 0;
 *   positions and table rows there are untouched.
 * Both: one kernel, nothing allocated, asynchronous on `stream`.
 */
int nvk_prefill_metadata(const int32_t* num_cached, const int32_t* num_new,
                         const int32_t* bt_offsets, const int32_t* bt_ids, int32_t batch,
                         int32_t block_size, int32_t table_width, int64_t n_tokens,
                         int32_t* cu_seqlens_q, int32_t* cu_seqlens_k, int64_t* positions,
                         int32_t* slot_mapping, int32_t* block_tables, void* stream);

int nvk_decode_metadata(const int32_t* seq_lens, const int32_t* bt_offsets,
                        const int32_t* bt_ids, int32_t batch, int32_t padded_batch,
                        int32_t block_size, int32_t table_width, int64_t table_row_stride,
                        int32_t* context_lens, int64_t* positions, int32_t* slot_mapping,
                        int32_t* block_tables, void* stream);

/*
 * Refresh of a captured decode graph's static metadata before a replay, the
 * copies of ModelRunner.run_model (nanovllm/engine/model_runner.py:200-211)
 * in one kernel: for b < static_rows
 *   slot_mapping[b] = b < batch ? src_slot_mapping[b] : -1,
 *   context_lens[b] = b < batch ? src_context_lens[b] : 0,
 *   positions[b]    = src_positions[b] for b < batch (rows above untouched),
 * and block_tables[b][j] = src_block_tables[b][j] for b < batch, j < width
 * (row strides bt_stride / src_bt_stride; everything else untouched, as the
 * reference leaves it).  batch <= static_rows.  Nothing allocated,
 * asynchronous on `stream`.
 */
int nvk_decode_graph_refresh(const int64_t* src_positions, const int32_t* src_slot_mapping,
                             const int32_t* src_context_lens, const int32_t* src_block_tables,
                             int64_t src_bt_stride, int32_t batch, int32_t width,
                             int64_t* positions, int32_t* slot_mapping, int32_t* context_lens,
                             int32_t* block_tables, int64_t bt_stride, int32_t static_rows,
                             void* stream);

/*
 * cu_seqlens of a query block of seqlen_q tokens at the end of every
 * sequence's seqlens_k[b] keys (speculative-decode verification through
 * flash_attn_with_kvcache with seqlen_q > 1, whose cache_seqlens
 * nanovllm/layers/attention.py:72-74 passes): cu_seqlens_q[b] = b*seqlen_q,
 * cu_seqlens_k = exclusive prefix of seqlens_k ([batch+1] int32 each).  One
 * kernel; batch <= 8192.
 */
int nvk_uniform_cu_seqlens(const int32_t* seqlens_k, int32_t batch, int32_t seqlen_q,
                           int32_t* cu_seqlens_q, int32_t* cu_seqlens_k, void* stream);

/*
 * LM-head last-token gather (nanovllm/layers/embed_head.py:56-60): in a
 * prefill step, out[b] = x[cu_seqlens_q[b+1] - 1] (row b of [batch][hidden]
 * bf16 or f16 (dtype), row strides in elements).  A sequence with
 * cu_seqlens_q[b+1] == 0 leaves its output row unwritten.  hidden and strides
 * multiples of 8.
 */
int nvk_gather_last_tokens(const void* x, int64_t x_row_stride, const int32_t* cu_seqlens_q,
                           int32_t batch, int32_t hidden, int32_t dtype, void* out,
                           int64_t out_row_stride, void* stream);

/*
 * Temperature sampling (nanovllm/layers/sampler.py:7-12):
 *   tokens[b] = argmax_i softmax(logits[b] / temperatures[b])_i / max(E_i, 1e-10)
 * with E_i ~ Exp(1): token i is drawn with probability softmax(logits[b] / T)_i.
 * noise != NULL: E = noise[b][i] (float32, row stride noise_row_stride), and
 * the argmax is evaluated as argmax_i logits[b][i] / T - log max(E_i, 1e-10)
 * (the same maximiser: the softmax normaliser is one constant per row); ties
 * go to the smallest index.
 * noise == NULL: the same distribution drawn by inverse transform with
 * uniforms from Philox4x32-10 keyed by seed at counters (offset, b, w) for
 * w < 2 + ceil(vocab / 2048): calls that must draw independently use
 * different offsets.  Non-finite logits carry no mass.
 * Rows without a finite logit give token 0.
 * logits: bf16, f16 or f32 (dtype) [batch][row_stride]; tokens: int64 [batch].
 * workspace: nvk_sample_workspace_size() bytes (16-byte aligned; three 4-byte
 * slots per row and 2048 logits), need not be initialised.
 * Two kernels: one workgroup per row and 8192 logits, then one wave per row.
 */
size_t nvk_sample_workspace_size(int32_t batch, int32_t vocab);
int nvk_sample(const void* logits, int64_t row_stride, int32_t batch, int32_t vocab,
               int32_t dtype, const float* temperatures, const float* noise,
               int64_t noise_row_stride, uint64_t seed, uint64_t offset, int64_t* tokens,
               void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NVK_H_ */
