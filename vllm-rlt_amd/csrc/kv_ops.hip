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
// Rotary embedding fused with the append: grid (n_rows).  Row i rotates its q
// (all rows) and, for i < n_write, writes its rotated k and its v to the slot
// (write_blocks[i], layer, write_offsets[i]).  The rotation of a head vector x
// with per-row cos / sin (each D wide) is, for j < D/2 and h = D/2,
//   out[j]     = R(R(x[j] * cos[j])       + R(-x[j + h] * sin[j]))
//   out[j + h] = R(R(x[j + h] * cos[j + h]) + R(x[j] * sin[j + h]))
// where R rounds to the storage type: each product and the sum round exactly
// where the elementwise tensor ops x * cos + rotate_half(x) * sin do.  One
// thread owns both halves of its pair, so q_out may alias q.
struct RopeArgs {
  void* cache[2];
  PoolGeom pool;
  int64_t layer;
  const void* x[2];  // q, k
  int64_t x_row[2], x_head[2], x_dim[2];
  const void* v;
  int64_t v_row, v_head, v_dim;
  void* q_out;
  int64_t qo_row, qo_head, qo_dim;
  const void* cos;
  const void* sin;
  int64_t cs_row, cs_dim;
  const int64_t* blocks;
  const int64_t* offsets;
  int64_t n_write;
  int hq, hkv, d;
};

template <typename T> __device__ __forceinline__ float round_to(float x);
template <> __device__ __forceinline__ float round_to<bf16>(float x) { return __uint_as_float(f32_to_bf16_bits(x) << 16); }
template <> __device__ __forceinline__ float round_to<f16>(float x) { return static_cast<float>(static_cast<f16>(x)); }
template <> __device__ __forceinline__ float round_to<float>(float x) { return x; }

// (lo, hi) <- rotated (x_lo, x_hi) with the cos / sin of both halves.
template <typename T>
__device__ __forceinline__ void rotate_pair(float x_lo, float x_hi, float c_lo, float c_hi, float s_lo, float s_hi,
                                            float* lo, float* hi) {
#pragma clang fp contract(off)
  *lo = round_to<T>(round_to<T>(x_lo * c_lo) + round_to<T>(-x_hi * s_lo));
  *hi = round_to<T>(round_to<T>(x_hi * c_hi) + round_to<T>(x_lo * s_hi));
}

// VEC: every operand has unit dim stride and 16-byte aligned rows, heads and
// half-vectors, and the pool slab is contiguous; each thread then moves 16-byte
// packets.  Otherwise one thread per element (pair) with any strides.
template <typename T, bool VEC>
__global__ __launch_bounds__(kThreads) void rope_kv_append_kernel(RopeArgs a) {
  using PK = Packet<T>;
  constexpr int EPV = VEC ? PK::N : 1;  // elements per work unit
  const int64_t row = blockIdx.x;
  const int half = a.d / 2;
  const int pair_units = half / EPV;
  int64_t block = -1, offset = 0;
  bool write = row < a.n_write;
  if (write) {
    block = a.blocks[row];
    offset = a.offsets[row];
    write = block >= 0 && block < a.pool.num_blocks && offset >= 0 && offset < a.pool.page;
  }
  const T* cs_c = static_cast<const T*>(a.cos) + row * a.cs_row;
  const T* cs_s = static_cast<const T*>(a.sin) + row * a.cs_row;
  const int q_units = a.hq * pair_units;
  const int k_units = write ? a.hkv * pair_units : 0;
  const int v_units = write ? a.hkv * (a.d / EPV) : 0;
  const int total = q_units + k_units + v_units;
  for (int u = threadIdx.x; u < total; u += kThreads) {
    if (u < q_units + k_units) {
      const int which = u < q_units ? 0 : 1;
      const int w = which ? u - q_units : u;
      const int head = w / pair_units;
      const int j0 = (w - head * pair_units) * EPV;
      const T* x = static_cast<const T*>(a.x[which]) + row * a.x_row[which] + head * a.x_head[which];
      T* dst;
      int64_t dst_dim;
      if (which == 0) {
        dst = static_cast<T*>(a.q_out) + row * a.qo_row + head * a.qo_head;
        dst_dim = a.qo_dim;
      } else {
        dst = static_cast<T*>(a.cache[0]) + slot_offset(a.pool, block, a.layer, offset) + head * a.pool.slab.head_stride;
        dst_dim = a.pool.slab.dim_stride;
      }
      if constexpr (VEC) {
        float xl[EPV], xh[EPV], cl[EPV], ch[EPV], sl[EPV], sh[EPV], ol[EPV], oh[EPV];
        PK::unpack(*reinterpret_cast<const u32x4*>(x + j0), xl);
        PK::unpack(*reinterpret_cast<const u32x4*>(x + half + j0), xh);
        PK::unpack(*reinterpret_cast<const u32x4*>(cs_c + j0), cl);
        PK::unpack(*reinterpret_cast<const u32x4*>(cs_c + half + j0), ch);
        PK::unpack(*reinterpret_cast<const u32x4*>(cs_s + j0), sl);
        PK::unpack(*reinterpret_cast<const u32x4*>(cs_s + half + j0), sh);
#pragma unroll
        for (int e = 0; e < EPV; ++e) rotate_pair<T>(xl[e], xh[e], cl[e], ch[e], sl[e], sh[e], &ol[e], &oh[e]);
        *reinterpret_cast<u32x4*>(dst + j0) = PK::pack(ol);
        *reinterpret_cast<u32x4*>(dst + half + j0) = PK::pack(oh);
      } else {
        const int64_t xd = a.x_dim[which];
        float lo, hi;
        rotate_pair<T>(load_elem(x + j0 * xd), load_elem(x + (half + j0) * xd), load_elem(cs_c + j0 * a.cs_dim),
                       load_elem(cs_c + (half + j0) * a.cs_dim), load_elem(cs_s + j0 * a.cs_dim),
                       load_elem(cs_s + (half + j0) * a.cs_dim), &lo, &hi);
        store_elem(dst + j0 * dst_dim, lo);
        store_elem(dst + (half + j0) * dst_dim, hi);
      }
    } else {
      const int w = u - q_units - k_units;
      const int units_per_head = a.d / EPV;
      const int head = w / units_per_head;
      const int j0 = (w - head * units_per_head) * EPV;
      const T* src = static_cast<const T*>(a.v) + row * a.v_row + head * a.v_head;
      T* dst = static_cast<T*>(a.cache[1]) + slot_offset(a.pool, block, a.layer, offset) + head * a.pool.slab.head_stride;
      if constexpr (VEC) {
        *reinterpret_cast<u32x4*>(dst + j0) = *reinterpret_cast<const u32x4*>(src + j0);
      } else {
        dst[j0 * a.pool.slab.dim_stride] = src[j0 * a.v_dim];  // bitwise copy
      }
    }
  }
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

extern "C" int rlt_rope_kv_append(void* key_cache, void* value_cache, const int64_t* cache_strides, const void* q,
                                  const int64_t* q_strides, const void* k, const int64_t* k_strides, const void* v,
                                  const int64_t* v_strides, const void* cos, const void* sin,
                                  const int64_t* cos_sin_strides, void* q_out, const int64_t* q_out_strides,
                                  const int64_t* write_blocks, const int64_t* write_offsets, int64_t n_rows,
                                  int64_t n_write, int64_t layer, int64_t num_layers, int64_t num_blocks,
                                  int64_t page_size, int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                                  int dtype, void* stream) {
  const int esize = dtype_size(dtype);
  if (!esize) return fail(RLT_EINVAL, "rlt_rope_kv_append: unknown dtype %d", dtype);
  if (n_rows < 0 || n_write < 0 || n_write > n_rows)
    return fail(RLT_EINVAL, "rlt_rope_kv_append: need 0 <= n_write <= n_rows");
  if (int rc = check_heads(num_kv_heads, head_dim)) return rc;
  if (head_dim % 2) return fail(RLT_EINVAL, "rlt_rope_kv_append: head_dim must be even for split-half rotation");
  if (num_q_heads <= 0 || num_q_heads * head_dim > (1 << 24))
    return fail(RLT_EINVAL, "rlt_rope_kv_append: bad num_q_heads");
  PoolGeom pool;
  if (int rc = pool_from(cache_strides, num_blocks, num_layers, page_size, &pool)) return rc;
  if (layer < 0 || layer >= num_layers)
    return fail(RLT_EINVAL, "rlt_rope_kv_append: layer %lld out of range", (long long)layer);
  if (n_rows == 0) return RLT_OK;
  if (!key_cache || !value_cache || !q || !k || !v || !cos || !sin || !q_out || !q_strides || !k_strides ||
      !v_strides || !cos_sin_strides || !q_out_strides || (n_write > 0 && (!write_blocks || !write_offsets)))
    return fail(RLT_EINVAL, "rlt_rope_kv_append: NULL pointer argument");
  if (n_rows > 0x7fffffff) return fail(RLT_EUNSUPPORTED, "rlt_rope_kv_append: too many rows");
  RopeArgs a{};
  a.cache[0] = key_cache;
  a.cache[1] = value_cache;
  a.pool = pool;
  a.layer = layer;
  a.x[0] = q;
  a.x[1] = k;
  a.x_row[0] = q_strides[0], a.x_head[0] = q_strides[1], a.x_dim[0] = q_strides[2];
  a.x_row[1] = k_strides[0], a.x_head[1] = k_strides[1], a.x_dim[1] = k_strides[2];
  a.v = v;
  a.v_row = v_strides[0], a.v_head = v_strides[1], a.v_dim = v_strides[2];
  a.q_out = q_out;
  a.qo_row = q_out_strides[0], a.qo_head = q_out_strides[1], a.qo_dim = q_out_strides[2];
  a.cos = cos;
  a.sin = sin;
  a.cs_row = cos_sin_strides[0], a.cs_dim = cos_sin_strides[1];
  a.blocks = write_blocks;
  a.offsets = write_offsets;
  a.n_write = n_write;
  a.hq = static_cast<int>(num_q_heads);
  a.hkv = static_cast<int>(num_kv_heads);
  a.d = static_cast<int>(head_dim);
  auto vec_tensor = [&](const void* p, const int64_t* st, int n) {
    if (!aligned16(p) || st[n - 1] != 1) return false;
    for (int i = 0; i + 1 < n; ++i)
      if ((st[i] * esize) % 16) return false;
    return true;
  };
  const bool vec = (head_dim / 2 * esize) % 16 == 0 && pool_vec_ok(pool, key_cache, value_cache, a.hkv, a.d, esize) &&
                   vec_tensor(q, q_strides, 3) && vec_tensor(k, k_strides, 3) && vec_tensor(v, v_strides, 3) &&
                   vec_tensor(q_out, q_out_strides, 3) && vec_tensor(cos, cos_sin_strides, 2) &&
                   vec_tensor(sin, cos_sin_strides, 2);
  const dim3 grid(static_cast<unsigned>(n_rows));
  hipStream_t st = as_stream(stream);
#define LAUNCH(T)                                                                                        \
  do {                                                                                                   \
    if (vec) hipLaunchKernelGGL((rope_kv_append_kernel<T, true>), grid, dim3(kThreads), 0, st, a);       \
    else hipLaunchKernelGGL((rope_kv_append_kernel<T, false>), grid, dim3(kThreads), 0, st, a);          \
  } while (0)
  switch (dtype) {
    case RLT_BFLOAT16: LAUNCH(bf16); break;
    case RLT_FLOAT16: LAUNCH(f16); break;
    default: LAUNCH(float); break;
  }
#undef LAUNCH
  return check_launch("rlt_rope_kv_append");
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
