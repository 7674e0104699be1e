/*
 * rlt_kv: C ABI of the MI355X (gfx950) depth-aware paged-KV hot path.
 *
 * Every buffer is caller-owned device memory passed as a raw pointer; the
 * library never allocates or frees device memory and never synchronises the
 * host.  All work is enqueued on the caller's HIP stream (`stream`, a
 * hipStream_t passed as void*; NULL is the default stream).
 *
 * Strides are in ELEMENTS, not bytes, and are 64-bit everywhere: a block id
 * multiplied by a block stride is computed in int64 before any addition, so
 * pools whose element offsets exceed 2^31 (or byte offsets above 2^32) are
 * addressed correctly.
 *
 * Pool layout (per tensor, K and V identical):
 *   [num_blocks, num_layers, page_size, num_kv_heads, head_dim]
 * as created by vllm_rlt/core/kv_cache_manager.py:132-134.  A "layer slice"
 * is key_cache[:, layer], i.e. [num_blocks, page_size, num_kv_heads, head_dim]
 * with the pool's block stride.
 *
 * Return value of every entry point: RLT_OK (0) on success, a negative
 * rlt_status otherwise.  rlt_last_error() returns a message for the calling
 * thread's last failure.  RLT_EINVAL means nothing was enqueued.
 */
#ifndef RLT_KV_H
#define RLT_KV_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  RLT_OK = 0,
  RLT_EINVAL = -1,      /* invalid argument; nothing enqueued */
  RLT_EUNSUPPORTED = -2, /* valid but unsupported shape/dtype; nothing enqueued */
  RLT_ELAUNCH = -3,     /* the HIP runtime rejected a launch */
  RLT_EWORKSPACE = -4   /* workspace too small; nothing enqueued */
} rlt_status;

/* Storage dtypes accepted for K/V/q/out (vllm_rlt/core/kv_cache_manager.py:111-112). */
typedef enum { RLT_FLOAT32 = 0, RLT_FLOAT16 = 1, RLT_BFLOAT16 = 2 } rlt_dtype;

/* Message describing the calling thread's most recent failure ("" if none). */
const char* rlt_last_error(void);

/* Library version string, e.g. "rlt_kv 0.1 gfx950". */
const char* rlt_version(void);

/*
 * KV append / scatter of one layer.
 * Replaces the two index_put launches of _write_prepared
 *   vllm_rlt/core/kv_cache_manager.py:531-532
 * and the captured equivalent in vllm_rlt/worker/cuda_graph.py:16-20:
 *   key_cache[write_blocks[i], layer, write_offsets[i]]   = k[i]
 *   value_cache[write_blocks[i], layer, write_offsets[i]] = v[i]
 * for i < n_rows (padding rows beyond n_rows are never written).  A bitwise
 * copy; the caller guarantees (block, offset) pairs are distinct
 * (kv_cache_manager.py:416-419).
 *   cache_strides[5]: block, layer, token, head, dim strides of key/value cache
 *   k_strides[3], v_strides[3]: row, head, dim strides of k / v ([n, hkv, d]).
 *   write_blocks, write_offsets: device int64 [n_rows].
 */
int rlt_kv_append(void* key_cache, void* value_cache, const int64_t* cache_strides,
                  const void* k, const int64_t* k_strides, const void* v,
                  const int64_t* v_strides, const int64_t* write_blocks,
                  const int64_t* write_offsets, int64_t n_rows, int64_t layer,
                  int64_t num_layers, int64_t num_blocks, int64_t page_size,
                  int64_t num_kv_heads, int64_t head_dim, int dtype, void* stream);

/*
 * Rotary position embedding of q and k fused with the KV append of one layer.
 * Replaces, per layer, the rotation of Ouro's attention
 *   q = q * cos + rotate_half(q) * sin;  k = k * cos + rotate_half(k) * sin
 *     vllm_rlt/models/ouro.py:104-109 (rotate_half at :73-75)
 * followed by the append of _write_prepared (vllm_rlt/core/kv_cache_manager.py:
 * 531-532) and its captured form (vllm_rlt/worker/cuda_graph.py:16-20):
 *   q_out[i] = rot(q[i])                                       for i < n_rows
 *   key_cache[write_blocks[i], layer, write_offsets[i]] = rot(k[i])  i < n_write
 *   value_cache[write_blocks[i], layer, write_offsets[i]] = v[i]     i < n_write
 * rot(x)[j] = x[j] * cos[j] + rotate_half(x)[j] * sin[j], where each product and
 * the sum round to the storage dtype as the reference's elementwise tensor ops
 * do, so q_out and the pages are bit-identical to the unfused sequence given
 * the same cos / sin (the reference computes them once per traversal,
 * vllm_rlt/models/ouro.py:209-213, and they are inputs here).  q_out may be q.
 *   q_strides / k_strides / v_strides / q_out_strides[3]: row, head, dim.
 *   cos_sin_strides[2]: row, dim strides shared by cos and sin ([n_rows, d]).
 *   head_dim must be even.
 */
int rlt_rope_kv_append(void* key_cache, void* value_cache, const int64_t* cache_strides,
                       const void* q, const int64_t* q_strides, const void* k,
                       const int64_t* k_strides, const void* v, const int64_t* v_strides,
                       const void* cos, const void* sin, const int64_t* cos_sin_strides,
                       void* q_out, const int64_t* q_out_strides,
                       const int64_t* write_blocks, const int64_t* write_offsets,
                       int64_t n_rows, int64_t n_write, int64_t layer, int64_t num_layers,
                       int64_t num_blocks, int64_t page_size, int64_t num_q_heads,
                       int64_t num_kv_heads, int64_t head_dim, int dtype, void* stream);

/*
 * Gather of slot-indexed per-request rows into batch order.
 * Replaces gather_kernel (vllm_rlt/kernels/routing.py:45-59), launched by
 * RoutingBank.gather (vllm_rlt/worker/async_state.py:93-102):
 *   out[r] = pool[slots[r]]  for r < count;  out[r] = 0 for count <= r < size
 * Rows are row_bytes long (hidden states, int64 tokens, any dtype); strides are
 * in bytes.  A slot outside [0, num_slots) reads as zeros.
 */
int rlt_gather_rows(const void* pool, int64_t pool_row_bytes_stride, int64_t num_slots,
                    const int64_t* slots, int64_t count, int64_t size, void* out,
                    int64_t out_row_bytes_stride, int64_t row_bytes, void* stream);

/*
 * Scatter of batch rows back to their request slots.
 * Replaces scatter_kernel (vllm_rlt/kernels/routing.py:62-76), launched by
 * RoutingBank.scatter (vllm_rlt/worker/async_state.py:104-112):
 *   pool[slots[r]] = values[r]  for r < count
 * Strides in bytes; a slot outside [0, num_slots) is skipped.
 */
int rlt_scatter_rows(const void* values, int64_t values_row_bytes_stride, const int64_t* slots,
                     int64_t count, void* pool, int64_t pool_row_bytes_stride, int64_t num_slots,
                     int64_t row_bytes, void* stream);

/*
 * Device-resident page tables updated in place from (index, value) pairs.
 * Replaces the per-request table uploads of RoutingBank.transfer
 * (vllm_rlt/worker/async_state.py:46-49: one pinned tensor and one copy
 * `tables[slot, :, :width] = table` for every request whose table changed):
 *   tables[patches[2i]] = (int32) patches[2i + 1]  for i < n
 * over the flat int32 tables [slots, planes, width].  A caller ships only the
 * entries the device does not hold yet (a new request's whole table, a
 * growing request's new pages), all requests of a step in one launch.
 * patches: int64 [n, 2], device or pinned host memory (read in place).
 * Indices within one call must be distinct; one outside [0, table_elems) is
 * skipped.
 */
int rlt_patch_tables(const int64_t* patches, int64_t n, int32_t* tables, int64_t table_elems,
                     void* stream);

/*
 * Whole-page export / import of the K and V pools (all layers of a page are one
 * contiguous block).  Replaces the page-by-page copies of preemption
 *   keys[row] = key_cache[block]   (vllm_rlt/engine/preemption.py:85-89)
 *   key_cache[block] = keys[row]   (vllm_rlt/engine/preemption.py:130-132)
 * and the whole-page segments of kv_segments (vllm_rlt/pd/transport.py:35-37):
 *   export: dst_keys[i] = key_cache[blocks[i]], dst_values[i] = value_cache[blocks[i]]
 *   import: key_cache[blocks[i]] = src_keys[i], value_cache[blocks[i]] = src_values[i]
 * for i < n, page_bytes per page.  Strides in bytes.  The packed rows may be
 * device memory or pinned host memory.  A block id outside [0, num_blocks) is
 * skipped.
 */
int rlt_kv_export_pages(const void* key_cache, const void* value_cache, int64_t pool_stride_bytes,
                        int64_t page_bytes, int64_t num_blocks, const int64_t* blocks, int64_t n,
                        void* dst_keys, void* dst_values, int64_t dst_stride_bytes, void* stream);
int rlt_kv_import_pages(void* key_cache, void* value_cache, int64_t pool_stride_bytes,
                        int64_t page_bytes, int64_t num_blocks, const int64_t* blocks, int64_t n,
                        const void* src_keys, const void* src_values, int64_t src_stride_bytes,
                        void* stream);

/*
 * Batched byte-range copy: dst_addresses[i][0:bytes[i]] = src_addresses[i][0:bytes[i]]
 * for i < n, one launch.  Executes the (address, size) descriptor lists of
 * kv_segments / partition_segments (vllm_rlt/pd/transport.py:18-68) for a
 * transfer the device can address directly (same device, or peer / pinned
 * host memory mapped to it).  The three arrays are device or pinned host
 * memory; max_bytes (the largest bytes[i]) only sizes the grid.  The caller
 * guarantees every range lies inside its allocation.
 */
int rlt_copy_segments(const int64_t* src_addresses, const int64_t* dst_addresses,
                      const int64_t* bytes, int64_t n, int64_t max_bytes, void* stream);

/*
 * Workspace bytes rlt_paged_decode needs for n_rows rows.  Depends only on the
 * shape, never on context lengths, so a caller can size it without a sync.
 */
int64_t rlt_paged_decode_workspace_bytes(int64_t n_rows, int64_t num_q_heads,
                                         int64_t num_kv_heads, int64_t head_dim);

/*
 * Single-query paged GQA decode attention over per-row block tables.
 * Replaces the attention callable contract
 *   attention(q, key_cache, value_cache, block_tables, context_lengths)
 * of vllm_rlt/kernels/paged_attention.py:12-36 (torch reference),
 * vllm_rlt/kernels/triton_attention.py:100-125 (Triton) and
 * vllm_rlt/kernels/flash_attention.py:98-130 (FlashAttention decode).
 * Row r attends q[r, hq, :] to tokens 0..context_lengths[r]-1 of its table;
 * q head j uses KV head j / (num_q_heads / num_kv_heads).  Softmax and both
 * products accumulate in fp32 with scale applied to q.k; the output is
 * rounded (nearest-even) to the storage dtype.  context_lengths[r] == 0 gives
 * an all-zero row.  Table entries at index >= ceil(len / page_size) are never
 * read, so padding may be -1 or 0.
 *   q_strides[3], out_strides[3]: row, head, dim strides.
 *   kv_strides[4]: block, token, head, dim strides of the LAYER SLICE; key and
 *     value slices must share them.  key_cache/value_cache point at the slice.
 *   block_tables: device int32 [n_rows, >= ceil(max_len/page)], row stride
 *     table_stride.  context_lengths: device int32 [n_rows].
 *   max_table_width: block_tables' column count; bounds the launch grid, and a
 *     length above max_table_width * page_size is clamped to it.
 *   workspace: device memory of >= rlt_paged_decode_workspace_bytes() bytes.
 * Results are independent of batch composition: a row's output bits depend
 * only on that row's inputs.
 */
int rlt_paged_decode(const void* q, const int64_t* q_strides, const void* key_cache,
                     const void* value_cache, const int64_t* kv_strides,
                     const int32_t* block_tables, int64_t table_stride,
                     int64_t max_table_width, const int32_t* context_lengths, void* out,
                     const int64_t* out_strides, int64_t n_rows, int64_t num_q_heads,
                     int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                     int64_t num_blocks, float scale, int dtype, void* workspace,
                     int64_t workspace_bytes, void* stream);

/*
 * KV append and decode attention of one layer in one launch.
 * Replaces, for a decode batch, the pair _write_prepared then _attend_prepared
 * (vllm_rlt/core/kv_cache_manager.py:520-534 and 559-586): first
 *   key_cache[write_blocks[i], write_offsets[i]] = k_new[i]  (and V), i < n_write
 * on the layer slices, then rlt_paged_decode over the updated pages; the pages
 * and the output equal that sequence's bit for bit.  Inside the launch a row
 * whose write slot is its own last token's slot (table[(len-1)/page],
 * (len-1) % page) reads that token from k_new / v_new, and the pages are
 * written after every split has read its keys (when max_table_width x
 * page_size <= 256 every row is one split, which stores its row's token
 * after its own reads, and no merge kernel runs).  So the caller guarantees that
 * no row reads a slot another row writes in this launch (true of a decode
 * batch with one row per request and depth; a packed chunk, where a row reads
 * the tokens of the rows before it, must use rlt_kv_append then
 * rlt_paged_decode).  Shapes the tiled kernel does not cover, or k_new / v_new
 * rows that are not 16-byte aligned with a unit dim stride, run the append
 * first and then the decode.
 *   key_cache / value_cache: the layer slices, written.
 *   k_new / v_new: [n_rows or more, num_kv_heads, head_dim], strides (row,
 *     head, dim) in elements.  write_blocks / write_offsets: device int64
 *     [n_write]; a slot outside the pool is skipped.  n_write <= n_rows.
 *   workspace: as rlt_paged_decode.
 */
int rlt_paged_decode_append(const void* q, const int64_t* q_strides, void* key_cache,
                            void* value_cache, const int64_t* kv_strides,
                            const int32_t* block_tables, int64_t table_stride,
                            int64_t max_table_width, const int32_t* context_lengths, void* out,
                            const int64_t* out_strides, int64_t n_rows, int64_t num_q_heads,
                            int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                            int64_t num_blocks, float scale, int dtype, const void* k_new,
                            const int64_t* k_new_strides, const void* v_new,
                            const int64_t* v_new_strides, const int64_t* write_blocks,
                            const int64_t* write_offsets, int64_t n_write, void* workspace,
                            int64_t workspace_bytes, void* stream);

/*
 * rlt_paged_decode without a workspace argument: allocates nothing.
 * No counterpart in the reference.  It is for callers that cannot allocate
 * device memory: code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc.  Same arguments (minus the workspace), contract and
 * output bits as rlt_paged_decode.
 * The split-K partials live in a static 64 MiB device array of the library.
 * Each device holds its own copy from the library's first use there until the
 * process ends.  Its address is looked up once per device.  The stream must
 * belong to the current device.
 * Rows go through in chunks of rlt_paged_decode_no_alloc_rows_per_launch()
 * rows (126 at 16 q heads x head_dim 128), one chunk after another on the
 * stream.  A shape whose single row needs more than 64 MiB of partials is
 * rejected with RLT_EUNSUPPORTED before anything is enqueued.
 * Every call on one device shares the array: calls that overlap on one device
 * (different streams, or several host threads) race and give wrong results.
 * Nothing in the array has to start at zero.
 */
int rlt_paged_decode_no_alloc(const void* q, const int64_t* q_strides, const void* key_cache,
                              const void* value_cache, const int64_t* kv_strides,
                              const int32_t* block_tables, int64_t table_stride,
                              int64_t max_table_width, const int32_t* context_lengths, void* out,
                              const int64_t* out_strides, int64_t n_rows, int64_t num_q_heads,
                              int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                              int64_t num_blocks, float scale, int dtype, void* stream);

/* Device bytes the library holds on every device it runs on, whether or not
 * rlt_paged_decode_no_alloc is called: the static scratch array above (64 MiB),
 * part of the code object loaded on the device.  No counterpart in the
 * reference; memory planners subtract it from the KV budget. */
int64_t rlt_static_device_bytes(void);

/* Rows per launch of rlt_paged_decode_no_alloc for this head geometry (0 when
 * even one row exceeds the static scratch or the heads are invalid). */
int64_t rlt_paged_decode_no_alloc_rows_per_launch(int64_t num_q_heads, int64_t num_kv_heads,
                                                  int64_t head_dim);

/*
 * rlt_paged_decode (with the append of rlt_paged_decode_append when n_write
 * > 0) for a batch whose rows alias prefix-cache pages (shared read-only,
 * vllm_rlt/core/kv_cache_manager.py:211-293: under LAST-EXITED every plane
 * has its own prefix pages, so a mixed-depth batch has one aliasing group per
 * plane and per distinct prefix).  Same contract and result as
 * rlt_paged_decode / rlt_paged_decode_append, which it replaces for such a
 * batch; the reference reads shared pages once per row, this reads each
 * group's pages once per launch.
 *   prefix_groups: device int32 buffer, in order:
 *     row_group[n_rows]           group of each row, -1 for none;
 *     groups[n_groups][5]         (first member index, member count, first
 *                                  page index, page count, split length);
 *     item_start[n_groups + 1]    prefix sums of the prefix pass's work items,
 *                                  items of group g = min(page count x page /
 *                                  split length, 63) x ceil(members x G / 64);
 *     members[n_members]          the rows of every group, group after group;
 *     pages[n_pages]              the shared page ids of every group.
 *   n_items = item_start[n_groups], with n_items x num_kv_heads < 2^31.  The
 *   members of group g must be exactly the rows with row_group == g; the split
 *   length is the decode split plan's for the members (256 << k: a function
 *   of a row's length alone).
 * A member's splits inside its group's pages are computed once for all
 * members (bf16 or fp16, head_dim 128, q heads per KV head 1/2/4/8, page 16;
 * other shapes ignore the hint) and merged with each row's remaining splits.
 * A split is taken from the prefix pass only if the row uses the group's split
 * length, the split is not the row's last, and the row's table entries for it
 * equal the group's pages, so an inexact page list costs speed, not
 * correctness.  A row's result depends on its own q, pages and group only, not
 * on the rest of the batch.  Every index in the buffer is bounds-checked on
 * the device: out-of-range groups, members and pages are ignored.  Rows must
 * not be more than 8192.
 */
int rlt_paged_decode_shared_prefix(const void* q, const int64_t* q_strides, void* key_cache,
                                   void* value_cache, const int64_t* kv_strides,
                                   const int32_t* block_tables, int64_t table_stride,
                                   int64_t max_table_width, const int32_t* context_lengths,
                                   void* out, const int64_t* out_strides, int64_t n_rows,
                                   int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                                   int64_t page_size, int64_t num_blocks, float scale, int dtype,
                                   const void* k_new, const int64_t* k_new_strides,
                                   const void* v_new, const int64_t* v_new_strides,
                                   const int64_t* write_blocks, const int64_t* write_offsets,
                                   int64_t n_write, const int32_t* prefix_groups,
                                   int64_t n_groups, int64_t n_members, int64_t n_pages,
                                   int64_t n_items, void* workspace, int64_t workspace_bytes,
                                   void* stream);

/*
 * Workspace bytes rlt_paged_prefill needs (shape-only, no sync needed).  Zero
 * for the MFMA path (bf16/fp16, head_dim 64 or 128, page 16, 16-byte aligned
 * rows); otherwise the size of the per-token decode-row path.
 */
int64_t rlt_paged_prefill_workspace_bytes(int64_t total_q, int64_t num_seqs,
                                          int64_t max_table_width, int64_t num_q_heads,
                                          int64_t num_kv_heads, int64_t head_dim,
                                          int64_t page_size, int dtype);

/*
 * Packed chunked-prefill attention over paged prefixes, bottom-right causal.
 * Replaces FlashPagedAttention.prefill, vllm_rlt/kernels/flash_attention.py:
 * 66-96 (FA4 varlen with cu_seqlens_q, seqused_k, page_table, causal=True),
 * selected by _attend_prepared when the batch carries cu_seqlens_q
 * (vllm_rlt/core/kv_cache_manager.py:570-579).  Sequence s owns query rows
 * [cu_seqlens_q[s], cu_seqlens_q[s+1]) of q and attends through
 * block_tables[s]; context_lengths[s] is its key length (prefix + chunk), so
 * query row i sees the first context_lengths[s] - (cu[s+1] - 1 - i) keys.
 * The chunk's own K/V must already be in the pool.  scale must be finite and
 * nonzero (RLT_EINVAL otherwise); negative scales are exact.
 *   cu_seqlens_q: device int32 [num_seqs + 1], cu[0] == 0, cu[num_seqs] == total_q.
 *   block_tables: device int32 [num_seqs, max_table_width] (row stride table_stride).
 */
int rlt_paged_prefill(const void* q, const int64_t* q_strides, const void* key_cache,
                      const void* value_cache, const int64_t* kv_strides,
                      const int32_t* block_tables, int64_t table_stride,
                      int64_t max_table_width, const int32_t* context_lengths,
                      const int32_t* cu_seqlens_q, int64_t num_seqs, int64_t total_q,
                      int64_t max_seqlen_q, void* out, const int64_t* out_strides,
                      int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                      int64_t page_size, int64_t num_blocks, float scale, int dtype,
                      void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Batched LAST-EXITED exit copies from device-resident descriptors.
 * Replaces finalize_kernel, vllm_rlt/kernels/routing.py:80-109 (launched at
 * vllm_rlt/worker/model_runner.py:543-557).  For every descriptor i with
 * (slot, depth, pos) = descriptors[3i .. 3i+2] and every target plane
 * depth < target < max_loops, copies the token's K and V at ALL layers:
 *   src = tables[(slot*planes + depth )*table_width + pos/page_size]
 *   dst = tables[(slot*planes + target)*table_width + pos/page_size]
 *   cache[dst, :, pos % page_size] = cache[src, :, pos % page_size]
 *   descriptors: device (or device-visible pinned) int64 [n, 3].
 *   tables: device int32 [num_slots, planes, table_width].
 * Descriptors whose slot, page or table entries fall outside the tables or
 * the pool are skipped (never dereferenced).
 */
int rlt_kv_finalize(const int64_t* descriptors, int64_t n, const int32_t* tables,
                    int64_t table_width, int64_t planes, int64_t num_slots,
                    void* key_cache, void* value_cache, const int64_t* cache_strides,
                    int64_t num_layers, int64_t num_blocks, int64_t num_kv_heads,
                    int64_t head_dim, int64_t page_size, int64_t max_loops, int dtype,
                    void* stream);

/*
 * Synchronous exit copy of one token with host-known pages.
 * Replaces the basic-index copies of finalize_token,
 * vllm_rlt/core/kv_cache_manager.py:601-611:
 *   cache[dst_blocks[j], :, offset] = cache[src_block, :, offset], j < n_dst
 * dst_blocks is a HOST array (n_dst <= 64) passed by value in the launch, so
 * no host-to-device index upload precedes the copy.
 */
int rlt_kv_copy_token(void* key_cache, void* value_cache, const int64_t* cache_strides,
                      int64_t src_block, const int64_t* dst_blocks, int64_t n_dst,
                      int64_t offset, int64_t num_layers, int64_t num_blocks,
                      int64_t page_size, int64_t num_kv_heads, int64_t head_dim, int dtype,
                      void* stream);

/*
 * Gather one (request, plane, layer) history in position order.
 * Replaces read(), vllm_rlt/core/kv_cache_manager.py:616-637:
 *   out_k[t] = key_cache[table[t / page], layer, t % page], t < length
 * (same for V).  table: device int32; out_k/out_v: contiguous
 * [length, num_kv_heads, head_dim].
 */
int rlt_kv_gather(const void* key_cache, const void* value_cache,
                  const int64_t* cache_strides, int64_t layer, const int32_t* table,
                  int64_t length, void* out_k, void* out_v, int64_t num_layers,
                  int64_t num_blocks, int64_t page_size, int64_t num_kv_heads,
                  int64_t head_dim, int dtype, void* stream);

/*
 * GPU-resident decode metadata from (slot, depth, pos) descriptors.
 * Replaces metadata_kernel, vllm_rlt/kernels/routing.py:8-41 (launched at
 * vllm_rlt/worker/async_state.py:59-75).  For row < size:
 *   valid = row < count;  (slot, depth, pos) = valid ? descriptors[3row..] : 0
 *   plane = planes > 1 ? depth : 0;  base = (slot*planes + plane)*table_width
 *   slots[row] = slot; positions[row] = pos; lengths[row] = valid ? pos+1 : 0
 *   if valid: blocks[row] = tables[base + pos/page]; offsets[row] = pos % page
 *   out_tables[row*out_table_stride + c] = valid ? tables[base + c] : 0,
 *     c < out_width
 * tables: device int32 [num_slots, planes, table_width].  A descriptor whose
 * slot, plane or page lies outside the tables is handled like a padding row
 * (length 0, zero table row, no write address) after slots/positions store it.
 */
int rlt_build_decode_metadata(const int64_t* descriptors, int64_t count, int64_t size,
                              const int32_t* tables, int64_t num_slots,
                              int64_t table_width, int64_t planes,
                              int64_t page_size, int64_t* slots, int64_t* positions,
                              int32_t* lengths, int64_t* blocks, int64_t* offsets,
                              int32_t* out_tables, int64_t out_table_stride,
                              int64_t out_width, void* stream);

/*
 * Stage a packed int64 blob into device int64 and int32 copies.
 * Replaces stage_prefill, vllm_rlt/kernels/prefill_metadata.py:8-12.
 * source may be device memory or device-visible pinned host memory.
 */
int rlt_stage_prefill(const int64_t* source, int64_t* target, int32_t* target32,
                      int64_t n, void* stream);

/*
 * Expand packed prefill (position, sequence) pairs into write addresses.
 * Replaces expand_prefill, vllm_rlt/kernels/prefill_metadata.py:16-32:
 *   blocks[i] = tables[sequences[i]*table_width + positions[i]/page]
 *   offsets[i] = positions[i] % page
 * tables: device int32 [num_sequences, table_width]; an entry outside the
 * tables yields block -1.
 */
int rlt_expand_prefill(const int64_t* positions, const int64_t* sequences,
                       const int32_t* tables, int64_t num_sequences, int64_t table_width,
                       int64_t page_size, int64_t* blocks, int64_t* offsets, int64_t n,
                       void* stream);

#ifdef __cplusplus
}
#endif

#endif /* RLT_KV_H */
