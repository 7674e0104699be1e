// Per-request state routing between the slot-indexed pools a runner keeps on
// the device (hidden states [max_seqs, hidden], tokens [max_seqs, 1]) and the
// row-ordered batch: gather (pool rows -> batch rows) and scatter (batch rows
// -> pool rows).  Byte-exact copies of whole rows; dtype never matters.
//
// Rows move as 16-byte packets when every row start is 16-byte aligned and
// the row length is a multiple of 16 bytes, else as 4-byte words when that
// alignment holds, else byte by byte.  Slots are bounds-checked: a gather row
// whose slot is outside the pool reads as zeros, a scatter row with such a
// slot is skipped.
#include "common.hpp"

namespace rlt {
namespace {

constexpr int kThreads = 256;

struct RowCopyArgs {
  const char* src;
  int64_t src_stride;  // bytes
  char* dst;
  int64_t dst_stride;  // bytes
  const int64_t* slots;
  int64_t num_slots;
  int64_t count;  // gather: rows [count, size) are zero-filled
  int64_t row_units;
};

template <typename U>
__device__ __forceinline__ U zero_unit() {
  return U{};
}
template <>
__device__ __forceinline__ u32x4 zero_unit<u32x4>() {
  return u32x4{0u, 0u, 0u, 0u};
}

// grid (size, column chunks): out[row] = pool[slots[row]] for row < count,
// zeros otherwise (vllm_rlt/kernels/routing.py:45-59).
template <typename U>
__global__ __launch_bounds__(kThreads) void gather_rows_kernel(RowCopyArgs a) {
  const int64_t row = blockIdx.x;
  const int64_t col = static_cast<int64_t>(blockIdx.y) * kThreads + threadIdx.x;
  if (col >= a.row_units) return;
  U value = zero_unit<U>();
  if (row < a.count) {
    const int64_t slot = a.slots[row];
    if (slot >= 0 && slot < a.num_slots) value = reinterpret_cast<const U*>(a.src + slot * a.src_stride)[col];
  }
  reinterpret_cast<U*>(a.dst + row * a.dst_stride)[col] = value;
}

// grid (count, column chunks): pool[slots[row]] = in[row]
// (vllm_rlt/kernels/routing.py:62-76).
template <typename U>
__global__ __launch_bounds__(kThreads) void scatter_rows_kernel(RowCopyArgs a) {
  const int64_t row = blockIdx.x;
  const int64_t col = static_cast<int64_t>(blockIdx.y) * kThreads + threadIdx.x;
  if (col >= a.row_units) return;
  const int64_t slot = a.slots[row];
  if (slot < 0 || slot >= a.num_slots) return;
  reinterpret_cast<U*>(a.dst + slot * a.dst_stride)[col] = reinterpret_cast<const U*>(a.src + row * a.src_stride)[col];
}

// grid ceil(n / kThreads): tables[index_i] = value_i for the (index, value)
// int64 pairs i < n.  The pairs may sit in pinned host memory, read in place.
// An index outside [0, table_elems) is skipped.
__global__ __launch_bounds__(kThreads) void patch_tables_kernel(const int64_t* patches, int64_t n, int32_t* tables,
                                                                int64_t table_elems) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= n) return;
  const int64_t index = patches[2 * i];
  if (index < 0 || index >= table_elems) return;
  tables[index] = static_cast<int32_t>(patches[2 * i + 1]);
}

int unit_bytes(const void* p, const void* q, int64_t s0, int64_t s1, int64_t row_bytes) {
  const uintptr_t bits = reinterpret_cast<uintptr_t>(p) | reinterpret_cast<uintptr_t>(q) |
                         static_cast<uintptr_t>(s0) | static_cast<uintptr_t>(s1) | static_cast<uintptr_t>(row_bytes);
  if ((bits & 15u) == 0) return 16;
  if ((bits & 3u) == 0) return 4;
  return 1;
}

template <bool GATHER, typename U>
void launch_unit(const dim3& grid, hipStream_t stream, const RowCopyArgs& a) {
  if constexpr (GATHER) hipLaunchKernelGGL(gather_rows_kernel<U>, grid, dim3(kThreads), 0, stream, a);
  else hipLaunchKernelGGL(scatter_rows_kernel<U>, grid, dim3(kThreads), 0, stream, a);
}

template <bool GATHER>
int launch_rows(RowCopyArgs a, int64_t rows, int64_t row_bytes, int unit, hipStream_t stream, const char* name) {
  a.row_units = row_bytes / unit;
  const int64_t chunks = (a.row_units + kThreads - 1) / kThreads;
  if (rows > 0x7fffffff || chunks > 65535) return fail(RLT_EUNSUPPORTED, "%s: too many rows or too wide a row", name);
  const dim3 grid(static_cast<unsigned>(rows), static_cast<unsigned>(chunks));
  switch (unit) {
    case 16: launch_unit<GATHER, u32x4>(grid, stream, a); break;
    case 4: launch_unit<GATHER, uint32_t>(grid, stream, a); break;
    default: launch_unit<GATHER, uint8_t>(grid, stream, a); break;
  }
  return check_launch(name);
}

}  // namespace
}  // namespace rlt

using namespace rlt;

extern "C" int rlt_gather_rows(const void* pool, int64_t pool_row_bytes_stride, int64_t num_slots,
                               const int64_t* slots, int64_t count, int64_t size, void* out,
                               int64_t out_row_bytes_stride, int64_t row_bytes, void* stream) {
  if (count < 0 || size < count) return fail(RLT_EINVAL, "rlt_gather_rows: need 0 <= count <= size");
  if (row_bytes < 0 || num_slots < 0 || pool_row_bytes_stride < 0 || out_row_bytes_stride < row_bytes)
    return fail(RLT_EINVAL, "rlt_gather_rows: bad row geometry");
  if (size == 0 || row_bytes == 0) return RLT_OK;
  if (!out || (count > 0 && (!pool || !slots))) return fail(RLT_EINVAL, "rlt_gather_rows: NULL pointer argument");
  RowCopyArgs a{};
  a.src = static_cast<const char*>(pool);
  a.src_stride = pool_row_bytes_stride;
  a.dst = static_cast<char*>(out);
  a.dst_stride = out_row_bytes_stride;
  a.slots = slots;
  a.num_slots = num_slots;
  a.count = count;
  const int unit = unit_bytes(pool, out, pool_row_bytes_stride, out_row_bytes_stride, row_bytes);
  return launch_rows<true>(a, size, row_bytes, unit, as_stream(stream), "rlt_gather_rows");
}

extern "C" int rlt_scatter_rows(const void* values, int64_t values_row_bytes_stride, const int64_t* slots,
                                int64_t count, void* pool, int64_t pool_row_bytes_stride, int64_t num_slots,
                                int64_t row_bytes, void* stream) {
  if (count < 0 || row_bytes < 0 || num_slots < 0 || values_row_bytes_stride < 0 || pool_row_bytes_stride < row_bytes)
    return fail(RLT_EINVAL, "rlt_scatter_rows: bad row geometry");
  if (count == 0 || row_bytes == 0) return RLT_OK;
  if (!values || !slots || !pool) return fail(RLT_EINVAL, "rlt_scatter_rows: NULL pointer argument");
  RowCopyArgs a{};
  a.src = static_cast<const char*>(values);
  a.src_stride = values_row_bytes_stride;
  a.dst = static_cast<char*>(pool);
  a.dst_stride = pool_row_bytes_stride;
  a.slots = slots;
  a.num_slots = num_slots;
  a.count = count;
  const int unit = unit_bytes(values, pool, values_row_bytes_stride, pool_row_bytes_stride, row_bytes);
  return launch_rows<false>(a, count, row_bytes, unit, as_stream(stream), "rlt_scatter_rows");
}

extern "C" int rlt_patch_tables(const int64_t* patches, int64_t n, int32_t* tables, int64_t table_elems,
                                void* stream) {
  if (n < 0 || table_elems < 0) return fail(RLT_EINVAL, "rlt_patch_tables: n and table_elems must be >= 0");
  if (n == 0) return RLT_OK;
  if (!patches || !tables) return fail(RLT_EINVAL, "rlt_patch_tables: NULL pointer argument");
  const int64_t blocks = (n + kThreads - 1) / kThreads;
  if (blocks > 0x7fffffff) return fail(RLT_EUNSUPPORTED, "rlt_patch_tables: too many patches");
  hipLaunchKernelGGL(patch_tables_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, as_stream(stream),
                     patches, n, tables, table_elems);
  return check_launch("rlt_patch_tables");
}
