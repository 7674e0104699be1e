// Page movement for preemption snapshots and prefill-to-decode transfer.
//
// Whole pages: export copies page blocks[i] of the K and V pools (all layers,
// one contiguous block) to row i of a destination array, import copies row i
// back to page blocks[i].  The destination may be device memory or pinned
// host memory the device can address, so a snapshot to host needs no device
// temporary.  Block ids are bounds-checked on the device: an out-of-range id
// is skipped.
//
// Segments: a batch of (source address, destination address, bytes) triples,
// the byte ranges kv_segments produces for partially filled pages, copied by
// one launch.  Addresses are plain device-visible addresses; the caller
// guarantees each range lies in its allocation.
//
// Both copy 16-byte packets when source, destination and length are 16-byte
// aligned, else bytes.  Copies are bitwise.
#include <algorithm>

#include "common.hpp"

namespace rlt {
namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;
constexpr int64_t kChunkBytes = int64_t(kThreads) * kUnroll * 16;  // bytes per workgroup and pass

__device__ __forceinline__ void copy_range(char* dst, const char* src, int64_t bytes, int64_t chunk) {
  const int64_t begin = chunk * kChunkBytes;
  if (begin >= bytes) return;
  const int64_t end = min(bytes, begin + kChunkBytes);
  const bool vec = ((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src) |
                     static_cast<uintptr_t>(bytes)) & 15u) == 0;
  if (vec) {
    const u32x4* s = reinterpret_cast<const u32x4*>(src + begin);
    u32x4* d = reinterpret_cast<u32x4*>(dst + begin);
    const int64_t n = (end - begin) / 16;
    u32x4 tmp[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = threadIdx.x + int64_t(u) * kThreads;
      if (i < n) tmp[u] = s[i];
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = threadIdx.x + int64_t(u) * kThreads;
      if (i < n) d[i] = tmp[u];
    }
  } else {
    for (int64_t i = begin + threadIdx.x; i < end; i += kThreads) dst[i] = src[i];
  }
}

struct PageCopyArgs {
  char* pool[2];         // K, V pools
  int64_t pool_stride;   // bytes between pages
  int64_t page_bytes;    // bytes copied per page
  int64_t num_blocks;
  const int64_t* blocks;
  char* rows[2];         // packed rows for K, V
  int64_t row_stride;    // bytes
  int export_pages;      // 1: pool -> rows, 0: rows -> pool
};

// grid (n, 2, chunks): page i, tensor (K or V), chunk of the page.
__global__ __launch_bounds__(kThreads) void page_copy_kernel(PageCopyArgs a) {
  const int64_t i = blockIdx.x;
  const int which = blockIdx.y;
  const int64_t block = a.blocks[i];
  if (block < 0 || block >= a.num_blocks) return;
  char* page = a.pool[which] + block * a.pool_stride;
  char* row = a.rows[which] + i * a.row_stride;
  if (a.export_pages) copy_range(row, page, a.page_bytes, blockIdx.z);
  else copy_range(page, row, a.page_bytes, blockIdx.z);
}

struct SegmentArgs {
  const int64_t* src;
  const int64_t* dst;
  const int64_t* bytes;
};

// grid (n, chunks): segment i; workgroup y copies chunks y, y + gridDim.y, ...
// so a segment longer than the grid's chunks is still copied whole.
__global__ __launch_bounds__(kThreads) void segment_copy_kernel(SegmentArgs a) {
  const int64_t i = blockIdx.x;
  const int64_t bytes = a.bytes[i];
  char* dst = reinterpret_cast<char*>(a.dst[i]);
  const char* src = reinterpret_cast<const char*>(a.src[i]);
  for (int64_t chunk = blockIdx.y; chunk * kChunkBytes < bytes; chunk += gridDim.y) copy_range(dst, src, bytes, chunk);
}

int chunks_for(int64_t bytes) { return static_cast<int>((bytes + kChunkBytes - 1) / kChunkBytes); }

}  // namespace
}  // namespace rlt

using namespace rlt;

namespace {
int page_copy(void* key_cache, void* value_cache, int64_t pool_stride_bytes, int64_t page_bytes,
              int64_t num_blocks, const int64_t* blocks, int64_t n, void* rows_k, void* rows_v,
              int64_t row_stride_bytes, int export_pages, void* stream, const char* name) {
  if (n < 0 || page_bytes < 0 || num_blocks < 0 || pool_stride_bytes < page_bytes || row_stride_bytes < page_bytes)
    return fail(RLT_EINVAL, "%s: bad page geometry", name);
  if (n == 0 || page_bytes == 0) return RLT_OK;
  if (!key_cache || !value_cache || !blocks || !rows_k || !rows_v) return fail(RLT_EINVAL, "%s: NULL pointer argument", name);
  const int64_t chunks = chunks_for(page_bytes);
  if (n > 0x7fffffff || chunks > 65535) return fail(RLT_EUNSUPPORTED, "%s: too many pages or too large a page", name);
  PageCopyArgs a{};
  a.pool[0] = static_cast<char*>(key_cache);
  a.pool[1] = static_cast<char*>(value_cache);
  a.pool_stride = pool_stride_bytes;
  a.page_bytes = page_bytes;
  a.num_blocks = num_blocks;
  a.blocks = blocks;
  a.rows[0] = static_cast<char*>(rows_k);
  a.rows[1] = static_cast<char*>(rows_v);
  a.row_stride = row_stride_bytes;
  a.export_pages = export_pages;
  hipLaunchKernelGGL(page_copy_kernel, dim3(static_cast<unsigned>(n), 2, static_cast<unsigned>(chunks)),
                     dim3(kThreads), 0, as_stream(stream), a);
  return check_launch(name);
}
}  // namespace

extern "C" int rlt_kv_export_pages(const void* key_cache, const void* value_cache, int64_t pool_stride_bytes,
                                   int64_t page_bytes, int64_t num_blocks, const int64_t* blocks, int64_t n,
                                   void* dst_keys, void* dst_values, int64_t dst_stride_bytes, void* stream) {
  return page_copy(const_cast<void*>(key_cache), const_cast<void*>(value_cache), pool_stride_bytes, page_bytes,
                   num_blocks, blocks, n, dst_keys, dst_values, dst_stride_bytes, 1, stream, "rlt_kv_export_pages");
}

extern "C" int rlt_kv_import_pages(void* key_cache, void* value_cache, int64_t pool_stride_bytes, int64_t page_bytes,
                                   int64_t num_blocks, const int64_t* blocks, int64_t n, const void* src_keys,
                                   const void* src_values, int64_t src_stride_bytes, void* stream) {
  return page_copy(key_cache, value_cache, pool_stride_bytes, page_bytes, num_blocks, blocks, n,
                   const_cast<void*>(src_keys), const_cast<void*>(src_values), src_stride_bytes, 0, stream,
                   "rlt_kv_import_pages");
}

extern "C" int rlt_copy_segments(const int64_t* src_addresses, const int64_t* dst_addresses, const int64_t* bytes,
                                 int64_t n, int64_t max_bytes, void* stream) {
  if (n < 0 || max_bytes < 0) return fail(RLT_EINVAL, "rlt_copy_segments: negative sizes");
  if (n == 0) return RLT_OK;
  if (!src_addresses || !dst_addresses || !bytes) return fail(RLT_EINVAL, "rlt_copy_segments: NULL pointer argument");
  const int64_t chunks = std::max<int64_t>(1, std::min<int64_t>(chunks_for(max_bytes), 4096));
  if (n > 0x7fffffff) return fail(RLT_EUNSUPPORTED, "rlt_copy_segments: too many segments");
  SegmentArgs a{src_addresses, dst_addresses, bytes};
  hipLaunchKernelGGL(segment_copy_kernel, dim3(static_cast<unsigned>(n), static_cast<unsigned>(chunks)), dim3(kThreads),
                     0, as_stream(stream), a);
  return check_launch("rlt_copy_segments");
}
