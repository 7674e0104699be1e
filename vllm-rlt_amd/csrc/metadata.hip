// GPU-resident routing metadata: per-row write addresses, context lengths and
// depth-resolved block tables built on the device from compact
// (slot, depth, position) descriptors, plus the packed-prefill staging and
// expansion.  All integer work; results are bit-exact by construction.
#include "common.hpp"

namespace rlt {
namespace {

constexpr int kThreads = 256;

struct DecodeMetaArgs {
  const int64_t* desc;
  const int32_t* tables;
  int64_t num_slots, table_width, planes, page;
  int64_t count;
  int64_t* slots;
  int64_t* positions;
  int32_t* lengths;
  int64_t* blocks;
  int64_t* offsets;
  int32_t* out_tables;
  int64_t out_stride, out_width;
};

// grid (size): one workgroup per output row; padding rows (row >= count)
// get slot = pos = length = 0, no write address, and an all-zero table row.
// A descriptor that points outside the tables is treated as padding after its
// slot and position are recorded, so no table read leaves the tables.
__global__ __launch_bounds__(kThreads) void decode_metadata_kernel(DecodeMetaArgs a) {
  const int64_t row = blockIdx.x;
  const bool real = row < a.count;
  const int64_t slot = real ? a.desc[3 * row] : 0;
  const int64_t depth = real ? a.desc[3 * row + 1] : 0;
  const int64_t pos = real ? a.desc[3 * row + 2] : 0;
  const int64_t plane = a.planes > 1 ? depth : 0;
  const bool valid = real && slot >= 0 && slot < a.num_slots && plane >= 0 && plane < a.planes && pos >= 0 &&
                     pos / a.page < a.table_width;
  const int32_t* src = a.tables + (valid ? (slot * a.planes + plane) * a.table_width : 0);
  if (threadIdx.x == 0) {
    a.slots[row] = slot;
    a.positions[row] = pos;
    a.lengths[row] = valid ? static_cast<int32_t>(pos + 1) : 0;
    if (valid) {
      a.blocks[row] = src[pos / a.page];
      a.offsets[row] = pos % a.page;
    }
  }
  int32_t* dst = a.out_tables + row * a.out_stride;
  for (int64_t c = threadIdx.x; c < a.out_width; c += kThreads) dst[c] = valid ? src[c] : 0;
}

__global__ __launch_bounds__(kThreads) void stage_prefill_kernel(const int64_t* src, int64_t* dst, int32_t* dst32,
                                                               int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= n) return;
  const int64_t x = src[i];
  dst[i] = x;
  dst32[i] = static_cast<int32_t>(x);
}

// Entries whose (sequence, page) fall outside the tables get block -1.
__global__ __launch_bounds__(kThreads) void expand_prefill_kernel(const int64_t* positions, const int64_t* sequences,
                                                                const int32_t* tables, int64_t num_seqs, int64_t width,
                                                                int64_t page, int64_t* blocks, int64_t* offsets,
                                                                int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= n) return;
  const int64_t pos = positions[i];
  const int64_t seq = sequences[i];
  const bool ok = seq >= 0 && seq < num_seqs && pos >= 0 && pos / page < width;
  blocks[i] = ok ? tables[seq * width + pos / page] : -1;
  offsets[i] = pos % page;
}

unsigned blocks_for(int64_t n) { return static_cast<unsigned>((n + kThreads - 1) / kThreads); }

}  // namespace
}  // namespace rlt

using namespace rlt;

extern "C" int rlt_build_decode_metadata(const int64_t* descriptors, int64_t count, int64_t size,
                                         const int32_t* tables, int64_t num_slots, int64_t table_width, int64_t planes,
                                         int64_t page_size, int64_t* slots, int64_t* positions, int32_t* lengths,
                                         int64_t* blocks, int64_t* offsets, int32_t* out_tables,
                                         int64_t out_table_stride, int64_t out_width, void* stream) {
  if (count < 0 || size < count) return fail(RLT_EINVAL, "rlt_build_decode_metadata: need 0 <= count <= size");
  if (num_slots <= 0 || table_width <= 0 || planes <= 0 || page_size <= 0)
    return fail(RLT_EINVAL, "rlt_build_decode_metadata: table shape and page_size must be positive");
  if (out_width < 0 || out_width > table_width || out_table_stride < out_width)
    return fail(RLT_EINVAL, "rlt_build_decode_metadata: need out_width <= table_width and <= out_table_stride");
  if (size == 0) return RLT_OK;
  if (!tables || !slots || !positions || !lengths || !out_tables || (count && (!descriptors || !blocks || !offsets)))
    return fail(RLT_EINVAL, "rlt_build_decode_metadata: NULL pointer argument");
  if (size > 0x7fffffff) return fail(RLT_EUNSUPPORTED, "rlt_build_decode_metadata: too many rows");
  DecodeMetaArgs a{descriptors, tables,  num_slots, table_width, planes,     page_size,        count,    slots,
                   positions,   lengths, blocks,    offsets,     out_tables, out_table_stride, out_width};
  hipLaunchKernelGGL(decode_metadata_kernel, dim3(static_cast<unsigned>(size)), dim3(kThreads), 0, as_stream(stream), a);
  return check_launch("rlt_build_decode_metadata");
}

extern "C" int rlt_stage_prefill(const int64_t* source, int64_t* target, int32_t* target32, int64_t n, void* stream) {
  if (n < 0) return fail(RLT_EINVAL, "rlt_stage_prefill: n is negative");
  if (n == 0) return RLT_OK;
  if (!source || !target || !target32) return fail(RLT_EINVAL, "rlt_stage_prefill: NULL pointer argument");
  hipLaunchKernelGGL(stage_prefill_kernel, dim3(blocks_for(n)), dim3(kThreads), 0, as_stream(stream), source, target,
                     target32, n);
  return check_launch("rlt_stage_prefill");
}

extern "C" int rlt_expand_prefill(const int64_t* positions, const int64_t* sequences, const int32_t* tables,
                                  int64_t num_sequences, int64_t table_width, int64_t page_size, int64_t* blocks,
                                  int64_t* offsets, int64_t n, void* stream) {
  if (n < 0) return fail(RLT_EINVAL, "rlt_expand_prefill: n is negative");
  if (num_sequences <= 0 || table_width <= 0 || page_size <= 0)
    return fail(RLT_EINVAL, "rlt_expand_prefill: bad table shape");
  if (n == 0) return RLT_OK;
  if (!positions || !sequences || !tables || !blocks || !offsets)
    return fail(RLT_EINVAL, "rlt_expand_prefill: NULL pointer argument");
  hipLaunchKernelGGL(expand_prefill_kernel, dim3(blocks_for(n)), dim3(kThreads), 0, as_stream(stream), positions,
                     sequences, tables, num_sequences, table_width, page_size, blocks, offsets, n);
  return check_launch("rlt_expand_prefill");
}
