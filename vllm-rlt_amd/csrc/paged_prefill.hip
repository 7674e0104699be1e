// Packed chunked-prefill attention over paged prefixes (bottom-right causal).
//
// Sequence s owns query rows [cu[s], cu[s+1]); its keys end at its last query
// position, so query row i sees len_k[s] - (cu[s+1] - 1 - i) keys.  This file
// expands every query row into a decode row (its own length and a copy of its
// sequence's table row) in the workspace and runs the split-K decode kernels
// on them -- the same per-token causal rows the reference's non-FA4 backends
// use for prefill.
#include <algorithm>

#include "common.hpp"

namespace rlt {
namespace {

constexpr int kThreads = 256;

struct ExpandArgs {
  const int32_t* cu;
  const int32_t* lens;
  const int32_t* tables;
  int64_t table_stride, width;
  int num_seqs;
  int32_t* row_lens;
  int32_t* row_tables;  // [total_q, width]
};

// grid (total_q): one workgroup per query row.
__global__ __launch_bounds__(kThreads) void expand_rows_kernel(ExpandArgs a) {
  const int row = blockIdx.x;
  int lo = 0, hi = a.num_seqs;  // find s with cu[s] <= row < cu[s+1]
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (a.cu[mid] <= row) lo = mid;
    else hi = mid;
  }
  const int s = lo;
  if (threadIdx.x == 0) {
    const int64_t n = static_cast<int64_t>(a.lens[s]) - (a.cu[s + 1] - 1 - row);
    a.row_lens[row] = static_cast<int32_t>(n < 0 ? 0 : n);
  }
  const int32_t* src = a.tables + s * a.table_stride;
  int32_t* dst = a.row_tables + static_cast<int64_t>(row) * a.width;
  for (int64_t c = threadIdx.x; c < a.width; c += kThreads) dst[c] = src[c];
}

int64_t expand_bytes(int64_t total_q, int64_t width) {
  const int64_t lens = (total_q * 4 + 255) / 256 * 256;
  const int64_t tables = (total_q * std::max<int64_t>(width, 1) * 4 + 255) / 256 * 256;
  return lens + tables;
}

}  // namespace
}  // namespace rlt

using namespace rlt;

extern "C" int64_t rlt_paged_prefill_workspace_bytes(int64_t total_q, int64_t num_seqs, int64_t max_table_width,
                                                     int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim) {
  if (total_q <= 0 || num_seqs <= 0) return 0;
  return expand_bytes(total_q, max_table_width) +
         rlt_paged_decode_workspace_bytes(total_q, num_q_heads, num_kv_heads, head_dim);
}

extern "C" int rlt_paged_prefill(const void* q, const int64_t* q_strides, const void* key_cache,
                                 const void* value_cache, const int64_t* kv_strides, const int32_t* block_tables,
                                 int64_t table_stride, int64_t max_table_width, const int32_t* context_lengths,
                                 const int32_t* cu_seqlens_q, int64_t num_seqs, int64_t total_q, int64_t max_seqlen_q,
                                 void* out, const int64_t* out_strides, int64_t num_q_heads, int64_t num_kv_heads,
                                 int64_t head_dim, int64_t page_size, int64_t num_blocks, float scale, int dtype,
                                 void* workspace, int64_t workspace_bytes, void* stream) {
  if (!dtype_size(dtype)) return fail(RLT_EINVAL, "rlt_paged_prefill: unknown dtype %d", dtype);
  if (num_seqs < 0 || total_q < 0 || max_seqlen_q < 0)
    return fail(RLT_EINVAL, "rlt_paged_prefill: negative sizes");
  if (max_table_width < 0 || table_stride < max_table_width)
    return fail(RLT_EINVAL, "rlt_paged_prefill: bad table shape");
  if (total_q == 0 || num_seqs == 0) return RLT_OK;
  if (!cu_seqlens_q || !block_tables || !context_lengths)
    return fail(RLT_EINVAL, "rlt_paged_prefill: NULL pointer argument");
  if (total_q > 0x7fffffff || num_seqs > 0x7fffffff)
    return fail(RLT_EUNSUPPORTED, "rlt_paged_prefill: too many rows");
  const int64_t need = rlt_paged_prefill_workspace_bytes(total_q, num_seqs, max_table_width, num_q_heads,
                                                         num_kv_heads, head_dim);
  if (!workspace || workspace_bytes < need)
    return fail(RLT_EWORKSPACE, "rlt_paged_prefill: workspace of %lld bytes < required %lld",
                (long long)workspace_bytes, (long long)need);
  if (!aligned16(workspace)) return fail(RLT_EINVAL, "rlt_paged_prefill: workspace must be 16-byte aligned");
  const int64_t width = std::max<int64_t>(max_table_width, 1);
  char* ws = static_cast<char*>(workspace);
  ExpandArgs e{};
  e.cu = cu_seqlens_q;
  e.lens = context_lengths;
  e.tables = block_tables;
  e.table_stride = table_stride;
  e.width = max_table_width;
  e.num_seqs = static_cast<int>(num_seqs);
  e.row_lens = reinterpret_cast<int32_t*>(ws);
  e.row_tables = reinterpret_cast<int32_t*>(ws + (total_q * 4 + 255) / 256 * 256);
  hipLaunchKernelGGL(expand_rows_kernel, dim3(static_cast<unsigned>(total_q)), dim3(kThreads), 0, as_stream(stream), e);
  if (int rc = check_launch("rlt_paged_prefill(expand)")) return rc;
  char* decode_ws = ws + expand_bytes(total_q, max_table_width);
  return rlt_paged_decode(q, q_strides, key_cache, value_cache, kv_strides, e.row_tables, width, max_table_width,
                          e.row_lens, out, out_strides, total_q, num_q_heads, num_kv_heads, head_dim, page_size,
                          num_blocks, scale, dtype, decode_ws, workspace_bytes - expand_bytes(total_q, max_table_width),
                          stream);
}
