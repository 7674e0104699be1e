// Byte-exact KV movement on the paged pool: append (scatter of the new
// token's K/V), LAST-EXITED exit copies, and the ordered gather behind read().
//
// Each token slot of one layer holds a [num_kv_heads, head_dim] slab (4 KiB
// for Ouro in bf16).  When the slab is contiguous on both sides every lane
// moves 16-byte packets (global_load/store_dwordx4); otherwise a strided
// element loop is used.  Block ids and offsets read from device memory are
// bounds-checked against the pool before any address is formed: an
// out-of-range entry is skipped, never dereferenced.
#include "common.hpp"

namespace rlt {
namespace {

constexpr int kThreads = 256;

struct SlabGeom {
  int64_t head_stride;  // elements
  int64_t dim_stride;   // elements
};

// Copy one [hkv, d] slab.  VEC: both sides contiguous and 16-byte aligned;
// the slab is then nvec packets of 16 bytes.
template <typename E, bool VEC>
__device__ __forceinline__ void copy_slab(E* dst, SlabGeom dg, const E* src, SlabGeom sg, int hkv, int d,
                                          int nvec) {
  if constexpr (VEC) {
    u32x4* out = reinterpret_cast<u32x4*>(dst);
    const u32x4* in = reinterpret_cast<const u32x4*>(src);
    for (int c = threadIdx.x; c < nvec; c += kThreads) out[c] = in[c];
  } else {
    const int total = hkv * d;
    for (int e = threadIdx.x; e < total; e += kThreads) {
      const int h = e / d, i = e - (e / d) * d;
      dst[h * dg.head_stride + i * dg.dim_stride] = src[h * sg.head_stride + i * sg.dim_stride];
    }
  }
}

struct PoolGeom {
  int64_t block, layer, token;  // element strides
  SlabGeom slab;
  int64_t num_blocks;
  int64_t num_layers;
  int64_t page;
};

__device__ __forceinline__ int64_t slot_offset(const PoolGeom& g, int64_t block, int64_t layer, int64_t token) {
  return block * g.block + layer * g.layer + token * g.token;
}

// ---------------------------------------------------------------------------
// Append: grid (n_rows, 2); y selects K (0) or V (1).
struct AppendArgs {
  void* cache[2];
  const void* src[2];
  int64_t src_row[2];
  SlabGeom src_slab[2];
  const int64_t* blocks;
  const int64_t* offsets;
  PoolGeom pool;
  int64_t layer;
  int hkv, d, nvec;
};

template <typename E, bool VEC>
__global__ __launch_bounds__(kThreads) void kv_append_kernel(AppendArgs a) {
  const int64_t row = blockIdx.x;
  const int which = blockIdx.y;
  const int64_t block = a.blocks[row];
  const int64_t offset = a.offsets[row];
  if (block < 0 || block >= a.pool.num_blocks || offset < 0 || offset >= a.pool.page) return;
  E* dst = static_cast<E*>(a.cache[which]) + slot_offset(a.pool, block, a.layer, offset);
  const E* src = static_cast<const E*>(a.src[which]) + row * a.src_row[which];
  copy_slab<E, VEC>(dst, a.pool.slab, src, a.src_slab[which], a.hkv, a.d, a.nvec);
}

// ---------------------------------------------------------------------------
// One token's exit copy with host-known pages: grid (n_dst, num_layers, 2).
constexpr int kMaxCopyTargets = 64;
struct CopyTokenArgs {
  void* cache[2];
  PoolGeom pool;
  int64_t src_block;
  int64_t offset;
  int64_t dst_blocks[kMaxCopyTargets];
  int hkv, d, nvec;
};

template <typename E, bool VEC>
__global__ __launch_bounds__(kThreads) void kv_copy_token_kernel(CopyTokenArgs a) {
  const int64_t layer = blockIdx.y;
  E* base = static_cast<E*>(a.cache[blockIdx.z]);
  const int64_t dst_block = a.dst_blocks[blockIdx.x];
  const E* src = base + slot_offset(a.pool, a.src_block, layer, a.offset);
  E* dst = base + slot_offset(a.pool, dst_block, layer, a.offset);
  copy_slab<E, VEC>(dst, a.pool.slab, src, a.pool.slab, a.hkv, a.d, a.nvec);
}

// ---------------------------------------------------------------------------
// Batched exit copies from device descriptors: grid (n, max_loops, num_layers),
// K and V handled by the same workgroup.
struct FinalizeArgs {
  void* cache[2];
  PoolGeom pool;
  const int64_t* desc;
  const int32_t* tables;
  int64_t table_width, planes, num_slots, max_loops;
  int hkv, d, nvec;
};

template <typename E, bool VEC>
__global__ __launch_bounds__(kThreads) void kv_finalize_kernel(FinalizeArgs a) {
  const int64_t row = blockIdx.x;
  const int64_t target = blockIdx.y;
  const int64_t layer = blockIdx.z;
  const int64_t slot = a.desc[3 * row];
  const int64_t depth = a.desc[3 * row + 1];
  const int64_t pos = a.desc[3 * row + 2];
  if (target <= depth || depth < 0 || slot < 0 || slot >= a.num_slots || pos < 0) return;
  const int64_t page = pos / a.pool.page;
  if (page >= a.table_width) return;
  const int64_t src_block = a.tables[(slot * a.planes + depth) * a.table_width + page];
  const int64_t dst_block = a.tables[(slot * a.planes + target) * a.table_width + page];
  if (src_block < 0 || src_block >= a.pool.num_blocks || dst_block < 0 || dst_block >= a.pool.num_blocks) return;
  const int64_t offset = pos - page * a.pool.page;
#pragma unroll
  for (int which = 0; which < 2; ++which) {
    E* base = static_cast<E*>(a.cache[which]);
    copy_slab<E, VEC>(base + slot_offset(a.pool, dst_block, layer, offset), a.pool.slab,
                      base + slot_offset(a.pool, src_block, layer, offset), a.pool.slab, a.hkv, a.d, a.nvec);
  }
}

// ---------------------------------------------------------------------------
// Ordered gather of one (table, layer): grid (length, 2).
struct GatherArgs {
  const void* cache[2];
  void* out[2];
  PoolGeom pool;
  const int32_t* table;
  int64_t layer;
  int hkv, d, nvec;
};

template <typename E, bool VEC>
__global__ __launch_bounds__(kThreads) void kv_gather_kernel(GatherArgs a) {
  const int64_t t = blockIdx.x;
  const int which = blockIdx.y;
  const int64_t page = t / a.pool.page;
  const int64_t block = a.table[page];
  E* dst = static_cast<E*>(a.out[which]) + t * static_cast<int64_t>(a.hkv) * a.d;
  const SlabGeom packed{a.d, 1};
  if (block < 0 || block >= a.pool.num_blocks) return;
  const E* src = static_cast<const E*>(a.cache[which]) + slot_offset(a.pool, block, a.layer, t - page * a.pool.page);
  copy_slab<E, VEC>(dst, packed, src, a.pool.slab, a.hkv, a.d, a.nvec);
}

// ---------------------------------------------------------------------------
// Host helpers.
bool slab_contiguous(SlabGeom s, int d) { return s.dim_stride == 1 && s.head_stride == d; }

int pool_from(const int64_t* st, int64_t num_blocks, int64_t num_layers, int64_t page, PoolGeom* g) {
  if (!st) return fail(RLT_EINVAL, "cache_strides is NULL");
  for (int i = 0; i < 5; ++i)
    if (st[i] < 0) return fail(RLT_EINVAL, "cache_strides[%d] is negative", i);
  if (num_blocks <= 0 || num_layers <= 0 || page <= 0) return fail(RLT_EINVAL, "pool dimensions must be positive");
  *g = PoolGeom{st[0], st[1], st[2], SlabGeom{st[3], st[4]}, num_blocks, num_layers, page};
  return RLT_OK;
}

// True when every slab start of the pool is 16-byte aligned and contiguous.
bool pool_vec_ok(const PoolGeom& g, const void* a, const void* b, int hkv, int d, int esize) {
  if (!slab_contiguous(g.slab, d)) return false;
  if ((static_cast<int64_t>(hkv) * d * esize) % 16) return false;
  if (!aligned16(a) || !aligned16(b)) return false;
  return (g.block * esize) % 16 == 0 && (g.layer * esize) % 16 == 0 && (g.token * esize) % 16 == 0;
}

int check_heads(int64_t hkv, int64_t d) {
  if (hkv <= 0 || d <= 0) return fail(RLT_EINVAL, "num_kv_heads and head_dim must be positive");
  if (hkv * d > (1 << 24)) return fail(RLT_EUNSUPPORTED, "num_kv_heads*head_dim too large");
  return RLT_OK;
}

#define RLT_DISPATCH_ESIZE(ESIZE, VEC, LAUNCH)         \
  do {                                                 \
    if ((ESIZE) == 2) {                                \
      if (VEC) { LAUNCH(uint16_t, true); }             \
      else { LAUNCH(uint16_t, false); }                \
    } else {                                           \
      if (VEC) { LAUNCH(uint32_t, true); }             \
      else { LAUNCH(uint32_t, false); }                \
    }                                                  \
  } while (0)

}  // namespace
}  // namespace rlt

using namespace rlt;

extern "C" int rlt_kv_append(void* key_cache, void* value_cache, const int64_t* cache_strides, const void* k,
                             const int64_t* k_strides, const void* v, const int64_t* v_strides,
                             const int64_t* write_blocks, const int64_t* write_offsets, int64_t n_rows,
                             int64_t layer, int64_t num_layers, int64_t num_blocks, int64_t page_size,
                             int64_t num_kv_heads, int64_t head_dim, int dtype, void* stream) {
  const int esize = dtype_size(dtype);
  if (!esize) return fail(RLT_EINVAL, "rlt_kv_append: unknown dtype %d", dtype);
  if (n_rows < 0) return fail(RLT_EINVAL, "rlt_kv_append: n_rows is negative");
  if (int rc = check_heads(num_kv_heads, head_dim)) return rc;
  PoolGeom pool;
  if (int rc = pool_from(cache_strides, num_blocks, num_layers, page_size, &pool)) return rc;
  if (layer < 0 || layer >= num_layers) return fail(RLT_EINVAL, "rlt_kv_append: layer %lld out of range", (long long)layer);
  if (n_rows == 0) return RLT_OK;
  if (!key_cache || !value_cache || !k || !v || !write_blocks || !write_offsets || !k_strides || !v_strides)
    return fail(RLT_EINVAL, "rlt_kv_append: NULL pointer argument");
  if (n_rows > 0x7fffffff) return fail(RLT_EUNSUPPORTED, "rlt_kv_append: too many rows");
  AppendArgs a{};
  a.cache[0] = key_cache;
  a.cache[1] = value_cache;
  a.src[0] = k;
  a.src[1] = v;
  a.src_row[0] = k_strides[0];
  a.src_row[1] = v_strides[0];
  a.src_slab[0] = SlabGeom{k_strides[1], k_strides[2]};
  a.src_slab[1] = SlabGeom{v_strides[1], v_strides[2]};
  a.blocks = write_blocks;
  a.offsets = write_offsets;
  a.pool = pool;
  a.layer = layer;
  a.hkv = static_cast<int>(num_kv_heads);
  a.d = static_cast<int>(head_dim);
  a.nvec = static_cast<int>(num_kv_heads * head_dim * esize / 16);
  const bool vec = pool_vec_ok(pool, key_cache, value_cache, a.hkv, a.d, esize) &&
                   slab_contiguous(a.src_slab[0], a.d) && slab_contiguous(a.src_slab[1], a.d) && aligned16(k) &&
                   aligned16(v) && (k_strides[0] * esize) % 16 == 0 && (v_strides[0] * esize) % 16 == 0;
  const dim3 grid(static_cast<unsigned>(n_rows), 2);
#define LAUNCH(E, V) hipLaunchKernelGGL((kv_append_kernel<E, V>), grid, dim3(kThreads), 0, as_stream(stream), a)
  RLT_DISPATCH_ESIZE(esize, vec, LAUNCH);
#undef LAUNCH
  return check_launch("rlt_kv_append");
}

extern "C" int rlt_kv_copy_token(void* key_cache, void* value_cache, const int64_t* cache_strides, int64_t src_block,
                                 const int64_t* dst_blocks, int64_t n_dst, int64_t offset, int64_t num_layers,
                                 int64_t num_blocks, int64_t page_size, int64_t num_kv_heads, int64_t head_dim,
                                 int dtype, void* stream) {
  const int esize = dtype_size(dtype);
  if (!esize) return fail(RLT_EINVAL, "rlt_kv_copy_token: unknown dtype %d", dtype);
  if (int rc = check_heads(num_kv_heads, head_dim)) return rc;
  PoolGeom pool;
  if (int rc = pool_from(cache_strides, num_blocks, num_layers, page_size, &pool)) return rc;
  if (n_dst < 0 || n_dst > kMaxCopyTargets)
    return fail(RLT_EINVAL, "rlt_kv_copy_token: n_dst must be in [0, %d]", kMaxCopyTargets);
  if (n_dst == 0) return RLT_OK;
  if (!key_cache || !value_cache || !dst_blocks) return fail(RLT_EINVAL, "rlt_kv_copy_token: NULL pointer argument");
  if (src_block < 0 || src_block >= num_blocks) return fail(RLT_EINVAL, "rlt_kv_copy_token: source block out of range");
  if (offset < 0 || offset >= page_size) return fail(RLT_EINVAL, "rlt_kv_copy_token: offset out of range");
  CopyTokenArgs a{};
  a.cache[0] = key_cache;
  a.cache[1] = value_cache;
  a.pool = pool;
  a.src_block = src_block;
  a.offset = offset;
  for (int64_t j = 0; j < n_dst; ++j) {
    if (dst_blocks[j] < 0 || dst_blocks[j] >= num_blocks)
      return fail(RLT_EINVAL, "rlt_kv_copy_token: destination block %lld out of range", (long long)dst_blocks[j]);
    if (dst_blocks[j] == src_block) return fail(RLT_EINVAL, "rlt_kv_copy_token: destination equals source");
    a.dst_blocks[j] = dst_blocks[j];
  }
  a.hkv = static_cast<int>(num_kv_heads);
  a.d = static_cast<int>(head_dim);
  a.nvec = static_cast<int>(num_kv_heads * head_dim * esize / 16);
  const bool vec = pool_vec_ok(pool, key_cache, value_cache, a.hkv, a.d, esize);
  const dim3 grid(static_cast<unsigned>(n_dst), static_cast<unsigned>(num_layers), 2);
#define LAUNCH(E, V) hipLaunchKernelGGL((kv_copy_token_kernel<E, V>), grid, dim3(kThreads), 0, as_stream(stream), a)
  RLT_DISPATCH_ESIZE(esize, vec, LAUNCH);
#undef LAUNCH
  return check_launch("rlt_kv_copy_token");
}

extern "C" int rlt_kv_finalize(const int64_t* descriptors, int64_t n, const int32_t* tables, int64_t table_width,
                               int64_t planes, int64_t num_slots, void* key_cache, void* value_cache,
                               const int64_t* cache_strides, int64_t num_layers, int64_t num_blocks,
                               int64_t num_kv_heads, int64_t head_dim, int64_t page_size, int64_t max_loops,
                               int dtype, void* stream) {
  const int esize = dtype_size(dtype);
  if (!esize) return fail(RLT_EINVAL, "rlt_kv_finalize: unknown dtype %d", dtype);
  if (int rc = check_heads(num_kv_heads, head_dim)) return rc;
  PoolGeom pool;
  if (int rc = pool_from(cache_strides, num_blocks, num_layers, page_size, &pool)) return rc;
  if (n < 0) return fail(RLT_EINVAL, "rlt_kv_finalize: n is negative");
  if (max_loops <= 0 || planes < max_loops)
    return fail(RLT_EINVAL, "rlt_kv_finalize: planes (%lld) must cover max_loops (%lld)", (long long)planes,
                (long long)max_loops);
  if (table_width <= 0 || num_slots <= 0) return fail(RLT_EINVAL, "rlt_kv_finalize: table shape must be positive");
  if (n == 0) return RLT_OK;
  if (!descriptors || !tables || !key_cache || !value_cache)
    return fail(RLT_EINVAL, "rlt_kv_finalize: NULL pointer argument");
  if (n > 0x7fffffff || max_loops > 65535 || num_layers > 65535)
    return fail(RLT_EUNSUPPORTED, "rlt_kv_finalize: launch too large");
  FinalizeArgs a{};
  a.cache[0] = key_cache;
  a.cache[1] = value_cache;
  a.pool = pool;
  a.desc = descriptors;
  a.tables = tables;
  a.table_width = table_width;
  a.planes = planes;
  a.num_slots = num_slots;
  a.max_loops = max_loops;
  a.hkv = static_cast<int>(num_kv_heads);
  a.d = static_cast<int>(head_dim);
  a.nvec = static_cast<int>(num_kv_heads * head_dim * esize / 16);
  const bool vec = pool_vec_ok(pool, key_cache, value_cache, a.hkv, a.d, esize);
  const dim3 grid(static_cast<unsigned>(n), static_cast<unsigned>(max_loops), static_cast<unsigned>(num_layers));
#define LAUNCH(E, V) hipLaunchKernelGGL((kv_finalize_kernel<E, V>), grid, dim3(kThreads), 0, as_stream(stream), a)
  RLT_DISPATCH_ESIZE(esize, vec, LAUNCH);
#undef LAUNCH
  return check_launch("rlt_kv_finalize");
}

extern "C" int rlt_kv_gather(const void* key_cache, const void* value_cache, const int64_t* cache_strides,
                             int64_t layer, const int32_t* table, int64_t length, void* out_k, void* out_v,
                             int64_t num_layers, int64_t num_blocks, int64_t page_size, int64_t num_kv_heads,
                             int64_t head_dim, int dtype, void* stream) {
  const int esize = dtype_size(dtype);
  if (!esize) return fail(RLT_EINVAL, "rlt_kv_gather: unknown dtype %d", dtype);
  if (int rc = check_heads(num_kv_heads, head_dim)) return rc;
  PoolGeom pool;
  if (int rc = pool_from(cache_strides, num_blocks, num_layers, page_size, &pool)) return rc;
  if (layer < 0 || layer >= num_layers) return fail(RLT_EINVAL, "rlt_kv_gather: layer out of range");
  if (length < 0) return fail(RLT_EINVAL, "rlt_kv_gather: length is negative");
  if (length == 0) return RLT_OK;
  if (!key_cache || !value_cache || !table || !out_k || !out_v)
    return fail(RLT_EINVAL, "rlt_kv_gather: NULL pointer argument");
  if (length > 0x7fffffff) return fail(RLT_EUNSUPPORTED, "rlt_kv_gather: length too large");
  GatherArgs a{};
  a.cache[0] = key_cache;
  a.cache[1] = value_cache;
  a.out[0] = out_k;
  a.out[1] = out_v;
  a.pool = pool;
  a.table = table;
  a.layer = layer;
  a.hkv = static_cast<int>(num_kv_heads);
  a.d = static_cast<int>(head_dim);
  a.nvec = static_cast<int>(num_kv_heads * head_dim * esize / 16);
  const bool vec = pool_vec_ok(pool, key_cache, value_cache, a.hkv, a.d, esize) && aligned16(out_k) && aligned16(out_v);
  const dim3 grid(static_cast<unsigned>(length), 2);
#define LAUNCH(E, V) hipLaunchKernelGGL((kv_gather_kernel<E, V>), grid, dim3(kThreads), 0, as_stream(stream), a)
  RLT_DISPATCH_ESIZE(esize, vec, LAUNCH);
#undef LAUNCH
  return check_launch("rlt_kv_gather");
}
