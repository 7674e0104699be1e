// Single-query paged GQA decode attention for gfx950.
//
// Work decomposition.  A row's context [0, len) is cut into fixed splits of
// kSplitTokens tokens; rows longer than kMaxSplits splits double the split
// length until kMaxSplits cover them.  The split plan of a row depends only on
// that row's length, so a row's output bits never depend on the rest of the
// batch, and rows of similar length cut at the same token offsets.  One
// wavefront processes one (row, kv_head, split) item.  When the kv head count
// is a multiple of the workgroup's 4 waves, a workgroup owns one (row, split,
// block of 4 heads) and workgroups are laid out so that each XCD serves whole
// (split, head block) groups with all rows of a group back to back: rows whose
// tables alias the same pages (a shared prefix) read them at the same time
// through one L2.  Otherwise the four waves of a workgroup walk the compact
// item list (rows x splits x kv_heads, kv_head innermost) in grid-stride order,
// after each workgroup builds the exclusive prefix of split counts over rows
// in LDS; neither schedule needs host-side length information.
//
// Inside an item.  Lanes form 64/LPT token groups of LPT lanes; lane (g, s)
// owns dims [s*EPL, s*EPL+EPL) of tokens g, g+TPI, ... of every tile.  One
// load instruction therefore reads TPI consecutive tokens that all lie in the
// same page, so the page's base address is wave-uniform: the split's table
// entries are fetched once (one per lane) and picked out with readlane, and
// K/V move as global_load_dwordx4 with an SGPR page base.  Each lane group keeps its own
// running max / normaliser / accumulator (exp2 domain, fp32), so a tile needs
// no cross-group traffic; the groups are merged once per item.  Tokens past
// the split end re-read the split's last valid token (in bounds, finite) and
// are masked to probability 0, so table entries past ceil(len/page) are never
// read and uninitialised pool memory never reaches the arithmetic.  A length
// larger than the table covers is clamped to it.
//
// Multi-split rows write (max, sum, unnormalised acc) partials to the
// workspace; a second kernel merges them in split order.  Single-split rows
// write their output directly and an empty row is one item that writes zeros.
// (Merging inside the split kernel, by the last split to finish, needs an
// agent-scope release/acquire per split -- an L2 writeback and invalidate
// across the 8 XCDs -- and measured 3x slower than the separate merge.)
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "common.hpp"
#include "mfma.hpp"

// Split-K partials of rlt_paged_decode_no_alloc: a fixed per-device array in
// place of a caller workspace (64 MiB; see rlt_kv.h for the row chunking it
// implies).  Host code never passes `scratch` itself to a kernel -- on the
// host it is only a stand-in for the device symbol -- but the address
// hipGetSymbolAddress returns for the current device.
constexpr int64_t kNoAllocScratchBytes = int64_t(64) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace rlt {
namespace {

// Tuning constants (overridable at compile time for measurement builds).
#ifndef RLT_DECODE_SPLIT_TOKENS
#define RLT_DECODE_SPLIT_TOKENS 256
#endif
#ifndef RLT_DECODE_TILE
#define RLT_DECODE_TILE 32
#endif
#ifndef RLT_DECODE_NT_LOADS
#define RLT_DECODE_NT_LOADS 1
#endif

constexpr int kWaves = 4;
constexpr int kSplitTokens = RLT_DECODE_SPLIT_TOKENS;
constexpr int kTile = RLT_DECODE_TILE;
constexpr int kMaxSplits = 64;
// Shared-prefix pass (head_dim 128): keys per tile, padded LDS rows
// (conflict-light K and transposing V reads), LDS elements of a workgroup
// (a K and a V tile per key half).
constexpr int kPrefixBK = 32;
constexpr int kPrefixKRow = 128 + 8, kPrefixVRow = 128 + 32;
constexpr int kPrefixTileElems = 2 * kPrefixBK * (kPrefixKRow + kPrefixVRow);
// A query's running maximum (prefix pass, grouped-query split pass) moves only
// when a tile exceeds it by more than this many powers of two.
constexpr float kPrefixRescale = 8.f;
#ifndef RLT_DECODE_PREFIX_WORKERS
#define RLT_DECODE_PREFIX_WORKERS 128
#endif
constexpr int kPrefixWorkers = RLT_DECODE_PREFIX_WORKERS;
static_assert(kPrefixWorkers > 0 && kPrefixWorkers % 8 == 0, "whole rounds of the 8 XCDs");
constexpr int kMaxRowsPerLaunch = 8192;
#ifndef RLT_DECODE_MAX_GRID
#define RLT_DECODE_MAX_GRID 4096
#endif
constexpr int kMaxGrid = RLT_DECODE_MAX_GRID;
#ifndef RLT_DECODE_XCD_SCHEDULE
#define RLT_DECODE_XCD_SCHEDULE 1
#endif
constexpr int kXcds = 8;  // MI355X: 8 XCDs, workgroups dispatched round-robin
constexpr float kLog2e = 1.4426950408889634f;

__host__ __device__ inline void split_plan(int len, int* split_len, int* nsplit) {
  // Rows longer than kMaxSplits splits double the split length until
  // kMaxSplits cover the row, so rows of similar length cut their contexts at
  // the same token offsets (an aliased prefix then falls into the same splits
  // of every row).  The doubling count is the smallest k >= 0 with
  // kMaxSplits * (kSplitTokens << k) >= len, taken from a leading-zero count
  // so the plan has no loop (the merge kernel issues its loads around it).
  // An empty row is one item that writes the all-zero row.
  constexpr unsigned kCover = static_cast<unsigned>(kMaxSplits) * kSplitTokens;
  const unsigned m = len > 0 ? (static_cast<unsigned>(len) + kCover - 1) / kCover : 1u;
  const int k = m <= 1 ? 0 : 32 - __builtin_clz(m - 1);
  const int per = kSplitTokens << k;
  *split_len = per;
  *nsplit = len > 0 ? (len + per - 1) / per : 1;
}

struct DecodeArgs {
  const void* q;
  int64_t q_row, q_head, q_dim;
  const void* k;
  const void* v;
  int64_t kv_block, kv_token, kv_head, kv_dim;
  const int32_t* tables;
  int64_t table_stride;
  const int32_t* lens;
  void* out;
  int64_t o_row, o_head, o_dim;
  float* ws_acc;  // [rows][hkv][kMaxSplits][G][D]
  float2* ws_ml;  // [rows][hkv][kMaxSplits][G]  (max in log2 units, sum)
  int n_rows, hkv, hq, d, page;
  int xcd_groups;  // > 0: XCD-affine schedule over this many (split, head block) groups
  int64_t num_blocks;
  int64_t max_len;  // table width * page: lengths are clamped to what the table covers
  float qscale;     // softmax scale * log2(e)
  // Prefix groups (all null / 0 when absent; the layout of the hint buffer is
  // documented at rlt_paged_decode_shared_prefix in rlt_kv.h): row r belongs
  // to group pg_row_group[r] (-1: none); group g's record is (first member,
  // member count, first page, page count, split length) at pg_groups[5g];
  // its member rows and shared page ids are slices of pg_members / pg_pages;
  // pg_item_start[g] is the first prefix-pass work item of group g.  The
  // splits of a member row inside its group's pages (at the group's split
  // length) come from the prefix workers (shared_prefix_item) instead of
  // the split pass.
  const int32_t* pg_row_group;
  const int32_t* pg_groups;
  const int32_t* pg_item_start;
  const int32_t* pg_members;
  const int32_t* pg_pages;
  int pg_n_groups, pg_n_members, pg_n_pages, pg_n_items;
  // Workgroups 0 .. pg_workers - 1 of the split pass compute the prefix
  // pass's items (item w, w + pg_workers, ...) while the others stream the
  // rest; a multiple of the XCD count, so the split pass's XCD mapping holds.
  int pg_workers;
  // Fused KV append (rlt_paged_decode_append; null / 0 otherwise): row
  // r < n_write stores its new token k_new[r] / v_new[r] ([hkv, D], strides
  // in elements, dim stride 1) at slot (write_blocks[r], write_offsets[r]) of
  // the layer slices.  The split pass reads a row's own new token from
  // k_new / v_new (its last token, when the write slot is the row's last
  // token slot) and the merge kernel stores it into the pages after every
  // split has read them (in a single-split launch the row's one item stores
  // it after its own reads), so no slot is written before it is read.
  const void* k_new;
  const void* v_new;
  int64_t kn_row, kn_head, kn_dim, vn_row, vn_head, vn_dim;
  const int64_t* write_blocks;
  const int64_t* write_offsets;
  int n_write;
};

// A row's effective context length; never reaches past its table row.
__device__ __forceinline__ int row_length(const DecodeArgs& a, int r) {
  const int64_t len = a.lens[r];
  return static_cast<int>(len < a.max_len ? len : a.max_len);
}

// Group record fields (pg_groups[5g + field]).
constexpr int kGroupMember0 = 0, kGroupMembers = 1, kGroupPage0 = 2, kGroupPages = 3, kGroupSplit = 4;
constexpr int kGroupFields = 5;

// The record of group g when its member and page slices lie inside the hint
// buffers and its split length is one the decode plan uses; null otherwise
// (the group is then ignored).
__device__ __forceinline__ const int32_t* group_record(const DecodeArgs& a, int g) {
  if (g < 0 || g >= a.pg_n_groups) return nullptr;
  const int32_t* rec = a.pg_groups + kGroupFields * g;
  const int m0 = rec[kGroupMember0], mn = rec[kGroupMembers], p0 = rec[kGroupPage0], pn = rec[kGroupPages];
  const int split = rec[kGroupSplit];
  const bool ok = m0 >= 0 && mn >= 0 && m0 <= a.pg_n_members - mn && p0 >= 0 && pn >= 0 && p0 <= a.pg_n_pages - pn &&
                  split >= kSplitTokens && (split & (split - 1)) == 0;
  return ok ? rec : nullptr;
}

// The record of row r's group when split sp of the row (split_len tokens, ns
// splits) can go to the prefix pass: the group uses the row's split length, and
// the split lies inside the group's pages, within the prefix pass's items
// (splits below kMaxSplits - 1), and is not the row's last split (so the row
// goes through the merge).  Null otherwise.
__device__ __forceinline__ const int32_t* prefix_candidate(const DecodeArgs& a, int r, int sp, int split_len, int ns) {
  if (!a.pg_row_group) return nullptr;
  const int32_t* rec = group_record(a, a.pg_row_group[r]);
  if (!rec || rec[kGroupSplit] != split_len) return nullptr;
  const int64_t covered = static_cast<int64_t>(rec[kGroupPages]) * a.page / split_len;
  if (sp >= covered || sp >= ns - 1 || sp >= kMaxSplits - 1) return nullptr;
  return rec;
}

// True when split sp of row r is computed by the prefix pass rather than by
// the split pass: it is a candidate and the row's table holds exactly the
// group's pages there.  All of it depends on the row and its own group only.
// Both passes evaluate it, so every split is produced exactly once.
__device__ bool prefix_takes(const DecodeArgs& a, int r, int sp, int split_len, int ns) {
  const int32_t* rec = prefix_candidate(a, r, sp, split_len, ns);
  if (!rec) return false;
  const int pages = split_len / a.page;
  const int32_t* trow = a.tables + static_cast<int64_t>(r) * a.table_stride + sp * pages;
  const int32_t* shared = a.pg_pages + rec[kGroupPage0] + sp * pages;
  // Entries in batches of 16 loads issued together: one memory round trip per
  // batch rather than one per page.
  constexpr int kBatch = 16;
  bool same = true;
  int i = 0;
  for (; i + kBatch <= pages; i += kBatch) {
    int32_t tv[kBatch], gv[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      tv[u] = trow[i + u];
      gv[u] = shared[i + u];
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) same &= tv[u] == gv[u];
  }
  for (; i < pages; ++i) same &= trow[i] == shared[i];
  return same;
}

// K/V page reads: each byte is read once per launch.
__device__ __forceinline__ u32x4 load_page(const u32x4* p) {
#if RLT_DECODE_NT_LOADS
  return __builtin_nontemporal_load(p);
#else
  return *p;
#endif
}

// Split partials: written once and read once, by the merge kernel.  Marked
// non-temporal (0.4-0.5% shorter launches on the LAST-EXITED and SHARED
// decode workloads than plain stores, same bits).
__device__ __forceinline__ void store_partial(float* p, const u32x4 w) {
  __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(p));
}

// Builds prefix[0..n] = exclusive scan of split counts in LDS; returns total.
__device__ int build_split_prefix(const DecodeArgs& a, int* prefix) {
  const int n = a.n_rows;
  __shared__ int wave_totals[kWaves];
  const int per = (n + blockDim.x - 1) / blockDim.x;
  const int lo = min(n, static_cast<int>(threadIdx.x) * per);
  const int hi = min(n, lo + per);
  int local = 0;
  for (int r = lo; r < hi; ++r) {
    int sl, ns;
    split_plan(row_length(a, r), &sl, &ns);
    local += ns;
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int incl = local;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o, 64);
    if (lane >= o) incl += y;
  }
  if (lane == 63) wave_totals[wave] = incl;
  __syncthreads();
  int base = 0;
  for (int w = 0; w < wave; ++w) base += wave_totals[w];
  int run = base + incl - local;
  for (int r = lo; r < hi; ++r) {
    prefix[r] = run;
    int sl, ns;
    split_plan(row_length(a, r), &sl, &ns);
    run += ns;
  }
  int total = 0;
  for (int w = 0; w < kWaves; ++w) total += wave_totals[w];
  if (threadIdx.x == 0) prefix[n] = total;
  __syncthreads();
  return total;
}

// Largest r in [0, n) with prefix[r] <= x (prefix non-decreasing, x < prefix[n]).
__device__ __forceinline__ int find_row(const int* prefix, int n, int x) {
  int lo = 0, hi = n;  // invariant: prefix[lo] <= x < prefix[hi]
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (prefix[mid] <= x) lo = mid;
    else hi = mid;
  }
  return lo;
}

// Merges the split partials of (row r, kv head h, q head j) into the output
// when the row has ns >= 2 splits.  Lane sp holds split sp's (max, sum)
// (kMaxSplits == 64 == wave size), so the global max and the normaliser are
// two wave reductions.  The accumulators are read 16 bytes per lane: lane
// (q, c) of a load reads dims 4c .. 4c + 3 of split i * SPI + q, so one load
// instruction covers SPI whole splits.  Each lane sums its splits in split
// order, then the SPI lanes of one chunk are added by a fixed butterfly, so
// the result depends only on the row's own partials.  The (max, sum) of all
// 64 slots and the first batch of SPB splits are loaded whatever ns is (every
// slot lies inside the workspace) and the slots past ns are selected away
// afterwards, so none of these loads waits for the row's length: the merge
// costs one round trip to memory for the common split counts.
template <int D>
struct MergeLoads {
  static constexpr int CH = D / 4;     // 16-byte chunks of one split's accumulators
  static constexpr int SPI = 64 / CH;  // splits per load instruction
  // The first batch covers 16 splits (rows up to 4096 tokens at 256-token
  // splits): a larger one reads more slots past ns than a second round trip
  // for the longer rows costs.  Later batches take up to 24 loads per lane,
  // so rows of up to 64 splits need one more round trip at D = 64 or 128.
  static constexpr int SPB = 16;
  static constexpr int NB = SPB / SPI;
  static constexpr int NB2 = (kMaxSplits - SPB) / SPI < 24 ? (kMaxSplits - SPB) / SPI : 24;
  static constexpr int FB = NB2 * SPI;  // splits per later batch: 48, 48, 24 for D = 64, 128, 256
  float2 ml;                            // this lane's split's (max, sum)
  u32x4 x[NB];                          // the first batch of accumulators
};

template <int D>
__device__ __forceinline__ MergeLoads<D> load_partials(const DecodeArgs& a, int r, int h, int j, int lane) {
  using L = MergeLoads<D>;
  static_assert(D % 64 == 0 && D <= 256 && L::SPB % L::SPI == 0 && L::SPB <= kMaxSplits, "whole chunks and splits");
  const int G = a.hq / a.hkv;
  const int64_t slot0 = (static_cast<int64_t>(r) * a.hkv + h) * kMaxSplits;
  const int64_t split_stride = static_cast<int64_t>(G) * D;
  const float* base = a.ws_acc + (slot0 * G + j) * D + 4 * (lane % L::CH) + (lane / L::CH) * split_stride;
  L v;
  v.ml = a.ws_ml[(slot0 + lane) * G + j];
#pragma unroll
  for (int i = 0; i < L::NB; ++i) v.x[i] = *reinterpret_cast<const u32x4*>(base + i * L::SPI * split_stride);
  return v;
}

template <typename T, int D>
__device__ void merge_partials(const DecodeArgs& a, int r, int h, int j, int ns, int lane, MergeLoads<D> v) {
  using L = MergeLoads<D>;
  // ns < 2: nothing to merge (the split pass wrote the row); only the store is skipped, so the
  // loads of v stay unconditional.
  const bool live = ns > 1;
  static_assert(kMaxSplits == 64, "one lane per split");
  const int G = a.hq / a.hkv;
  const int64_t slot0 = (static_cast<int64_t>(r) * a.hkv + h) * kMaxSplits;
  const int64_t split_stride = static_cast<int64_t>(G) * D;
  const int c = lane % L::CH, q = lane / L::CH;
  T* orow = static_cast<T*>(a.out) + r * a.o_row + static_cast<int64_t>(h * G + j) * a.o_head;
  const float* base = a.ws_acc + (slot0 * G + j) * D + 4 * c + q * split_stride;
  const float2 ml = lane < ns ? v.ml : make_float2(-INFINITY, 0.f);
  const float M = strided_max<1>(ml.x);
  const float w = lane < ns ? fast_exp2(ml.x - M) : 0.f;
  const float inv = 1.f / group_sum<64>(ml.y * w);
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < L::NB; ++i) {
    const int u = i * L::SPI + q;
    const float wu = __shfl(w, u, 64);
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] = fmaf(u < ns ? __uint_as_float(v.x[i][e]) : 0.f, wu, acc[e]);
  }
  // Further splits (rows of more than SPB splits), a whole batch of loads in flight at a time.
  for (int sp0 = L::SPB; live && sp0 < ns; sp0 += L::FB) {
    u32x4 x[L::NB2];
#pragma unroll
    for (int i = 0; i < L::NB2; ++i) {
      const int u = sp0 + i * L::SPI + q;
      x[i] = u < ns ? *reinterpret_cast<const u32x4*>(base + (sp0 + i * L::SPI) * split_stride) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < L::NB2; ++i) {
      const float wu = __shfl(w, (sp0 + i * L::SPI + q) & 63, 64);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] = fmaf(__uint_as_float(x[i][e]), wu, acc[e]);
    }
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) acc[e] = strided_sum<L::CH>(acc[e]);
  if (live && q == 0) {
#pragma unroll
    for (int e = 0; e < 4; ++e) store_elem(orow + (4 * c + e) * a.o_dim, acc[e] * inv);
  }
}

// The prefix pass's work item (defined with the prefix pass below).
template <typename T, int G>
__device__ __forceinline__ void shared_prefix_item(const DecodeArgs& a, int item, int h, uint16_t* tiles);

// The split pass over workgroups block = 0 .. blocks - 1 of a 256-thread
// launch (the kernels below map their workgroups onto it).  ONE_SPLIT: every
// row is a single split (the tables span at most one split), so each row's one
// item stores the row's new token itself (APPEND), after its own reads, and no
// merge kernel runs.
template <typename T, int D, int G, int P, int TILE, bool XCD, bool PREFIX, bool APPEND, bool ONE_SPLIT = false>
__device__ __forceinline__ void split_pass(DecodeArgs a, const int block, const int blocks) {
  using PK = Packet<T>;
  constexpr int EPL = PK::N;      // elements of one token a lane owns
  constexpr int LPT = D / EPL;    // lanes per token
  constexpr int TPI = 64 / LPT;   // tokens per load instruction
  constexpr int IPP = P / TPI;    // load instructions per page
  constexpr int PPT = TILE / P;   // pages per tile
  constexpr int NI = TILE / TPI;  // load instructions per tile (per tensor)
  static_assert(D % EPL == 0 && 64 % LPT == 0 && LPT >= 1, "head_dim must map onto whole lanes");
  static_assert(P % TPI == 0 && TILE % P == 0 && kSplitTokens % TILE == 0, "tile geometry");

  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int g = lane / LPT;
  const int s = lane % LPT;
  const uint32_t lane_dim = static_cast<uint32_t>(s * EPL);

  // A one-split launch's append: row r's new token of kv head h into its
  // write slot (skipped when the slot is outside the pool), by the lanes of
  // one token, after the item has read its pages.
  auto store_new_token = [&](const int r, const int h) {
    if constexpr (APPEND && ONE_SPLIT) {
      if (r >= a.n_write || g != 0) return;
      const int64_t b = a.write_blocks[r], o = a.write_offsets[r];
      if (b < 0 || b >= a.num_blocks || o < 0 || o >= a.page) return;
      const int64_t slot = b * a.kv_block + o * a.kv_token + static_cast<int64_t>(h) * a.kv_head + lane_dim;
      const u32x4 kt = *reinterpret_cast<const u32x4*>(static_cast<const T*>(a.k_new) + r * a.kn_row +
                                                        static_cast<int64_t>(h) * a.kn_head + lane_dim);
      const u32x4 vt = *reinterpret_cast<const u32x4*>(static_cast<const T*>(a.v_new) + r * a.vn_row +
                                                        static_cast<int64_t>(h) * a.vn_head + lane_dim);
      *reinterpret_cast<u32x4*>(const_cast<T*>(static_cast<const T*>(a.k)) + slot) = kt;
      *reinterpret_cast<u32x4*>(const_cast<T*>(static_cast<const T*>(a.v)) + slot) = vt;
    }
  };

  // One (row r, kv head h, split sp) item per wave.
  auto process = [&](const int r, const int h, const int sp, const int len, const int split_len, const int ns) {
    if (len <= 0) {
      if (g == 0) {
        T* orow = static_cast<T*>(a.out) + r * a.o_row + static_cast<int64_t>(h) * G * a.o_head + lane_dim;
        const u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int j = 0; j < G; ++j) *reinterpret_cast<u32x4*>(orow + j * a.o_head) = zero;
      }
      store_new_token(r, h);
      return;
    }
    const int t_begin = sp * split_len;
    const int t_end = min(len, t_begin + split_len);
    const int last = t_end - 1;
    // Fused append: the row's write slot, read up front when this is its last split.
    int64_t wb = -1, wo = -1;
    if constexpr (APPEND) {
      if (t_end == len && r < a.n_write) {
        wb = a.write_blocks[r];
        wo = a.write_offsets[r];
      }
    }

    // q for the G query heads of this kv head, pre-scaled into log2 units.
    float qv[G][EPL];
    {
      const T* qrow = static_cast<const T*>(a.q) + r * a.q_row + static_cast<int64_t>(h) * G * a.q_head + lane_dim;
#pragma unroll
      for (int j = 0; j < G; ++j) {
        const u32x4 p = *reinterpret_cast<const u32x4*>(qrow + j * a.q_head);
        PK::unpack(p, qv[j]);
#pragma unroll
        for (int e = 0; e < EPL; ++e) qv[j][e] *= a.qscale;
      }
    }

    float m[G], l[G], acc[G][EPL];
#pragma unroll
    for (int j = 0; j < G; ++j) {
      m[j] = -INFINITY;
      l[j] = 0.f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[j][e] = 0.f;
    }

    const int32_t* trow = a.tables + r * a.table_stride;
    const T* kbase = static_cast<const T*>(a.k) + static_cast<int64_t>(h) * a.kv_head;
    const T* vbase = static_cast<const T*>(a.v) + static_cast<int64_t>(h) * a.kv_head;
    const uint32_t tok_stride = static_cast<uint32_t>(a.kv_token);

    // Loads of tile t + 1 are issued while tile t computes: K(t+1) after the
    // scores of tile t, V(t+1) after its value accumulation.  The loop body
    // holds no conditional load (table entries are fetched per 64-page chunk
    // before its tiles, and the chunk's last tile is peeled), so the compiler
    // waits only for the tile being consumed and never drains the pipeline.
    auto scores = [&](const u32x4 (&kt)[NI], int t0, float (&sc)[G][NI]) {
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        float x[EPL];
        PK::unpack(kt[i], x);
        const bool valid = t0 + i * TPI + g <= last;
#pragma unroll
        for (int j = 0; j < G; ++j) {
          float dot = 0.f;
#pragma unroll
          for (int e = 0; e < EPL; ++e) dot = fmaf(qv[j][e], x[e], dot);
          dot = group_sum<LPT>(dot);
          sc[j][i] = valid ? dot : -INFINITY;
        }
      }
    };
    auto accumulate = [&](const u32x4 (&vt)[NI], int t0, const float (&sc)[G][NI]) {
      float p[G][NI];
#pragma unroll
      for (int j = 0; j < G; ++j) {
        float tmax = sc[j][0];
#pragma unroll
        for (int i = 1; i < NI; ++i) tmax = fmaxf(tmax, sc[j][i]);
        const float mn = fmaxf(m[j], tmax);
        const float corr = (mn == -INFINITY) ? 1.f : fast_exp2(m[j] - mn);
        float psum = 0.f;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          const bool valid = t0 + i * TPI + g <= last;
          p[j][i] = valid ? fast_exp2(sc[j][i] - mn) : 0.f;
          psum += p[j][i];
        }
        l[j] = l[j] * corr + psum;
        m[j] = mn;
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[j][e] *= corr;
      }
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        float y[EPL];
        PK::unpack(vt[i], y);
#pragma unroll
        for (int j = 0; j < G; ++j)
#pragma unroll
          for (int e = 0; e < EPL; ++e) acc[j][e] = fmaf(p[j][i], y[e], acc[j][e]);
      }
    };

    constexpr int kChunkTokens = 64 * P;  // one table entry per lane
    for (int c0 = t_begin; c0 < t_end; c0 += kChunkTokens) {
      const int c1 = min(t_end, c0 + kChunkTokens);
      const int chunk_page = c0 / P;
      const int chunk_last = (c1 - 1) / P - chunk_page;  // <= 63
      const int table_entry = lane <= chunk_last ? trow[chunk_page + lane] : 0;
      auto tile_pages = [&](int t0, int64_t (&blk)[PPT]) {
        const int rel0 = (t0 - c0) / P;
#pragma unroll
        for (int pg = 0; pg < PPT; ++pg) {
          const int64_t b = __builtin_amdgcn_readlane(table_entry, min(rel0 + pg, chunk_last));
          blk[pg] = (b < 0 || b >= a.num_blocks) ? 0 : b;
        }
      };
      auto issue = [&](u32x4 (&dst)[NI], const T* base, const int64_t (&blk)[PPT], int t0) {
#pragma unroll
        for (int pg = 0; pg < PPT; ++pg) {
          const T* page = base + blk[pg] * a.kv_block;
#pragma unroll
          for (int i = 0; i < IPP; ++i) {
            const int tok = min(t0 + pg * P + i * TPI + g, last);
            const uint32_t off = static_cast<uint32_t>(tok & (P - 1)) * tok_stride + lane_dim;
            dst[pg * IPP + i] = load_page(reinterpret_cast<const u32x4*>(page + off));
          }
        }
      };
      // The final tile of a row whose new token is fused in: the lanes of
      // token len - 1 load it from `fresh_row` (k_new / v_new) instead of the
      // page slot, within the tile's own load stream.
      auto issue_fresh = [&](u32x4 (&dst)[NI], const T* base, const T* fresh_row, const int64_t (&blk)[PPT],
                             int t0) {
#pragma unroll
        for (int pg = 0; pg < PPT; ++pg) {
          const T* page = base + blk[pg] * a.kv_block;
#pragma unroll
          for (int i = 0; i < IPP; ++i) {
            const int tok = min(t0 + pg * P + i * TPI + g, last);
            const uint32_t off = static_cast<uint32_t>(tok & (P - 1)) * tok_stride + lane_dim;
            const T* src = tok == len - 1 ? fresh_row + lane_dim : page + off;
            dst[pg * IPP + i] = *reinterpret_cast<const u32x4*>(src);
          }
        }
      };
      const int ntiles = (c1 - c0 + TILE - 1) / TILE;
      // Whether this chunk ends the row and the row's write slot is its last
      // token's slot (page id from the chunk's table entries): then the new
      // token comes from k_new / v_new.
      bool fresh = false;
      const T* kn_row = nullptr;
      const T* vn_row = nullptr;
      if constexpr (APPEND) {
        fresh = c1 == len && wb >= 0 && wo == (len - 1) % P &&
                wb == static_cast<int64_t>(__builtin_amdgcn_readlane(table_entry, chunk_last));
        kn_row = static_cast<const T*>(a.k_new) + r * a.kn_row + static_cast<int64_t>(h) * a.kn_head;
        vn_row = static_cast<const T*>(a.v_new) + r * a.vn_row + static_cast<int64_t>(h) * a.vn_head;
      }
      u32x4 kp[NI], vp[NI];
      int64_t blk[PPT];
      // sched_barrier keeps every K load of a tile ahead of its V loads in
      // issue order, so waiting for K never waits for V.
      tile_pages(c0, blk);
      if (APPEND && fresh && ntiles == 1) {
        issue_fresh(kp, kbase, kn_row, blk, c0);
        __builtin_amdgcn_sched_barrier(0);
        issue_fresh(vp, vbase, vn_row, blk, c0);
      } else {
        issue(kp, kbase, blk, c0);
        __builtin_amdgcn_sched_barrier(0);
        issue(vp, vbase, blk, c0);
      }
      int t0 = c0;
      // With a fused token the iteration that issues the final tile is peeled.
      const int steady = (APPEND && fresh) ? ntiles - 1 : ntiles;
      for (int it = 1; it < steady; ++it, t0 += TILE) {
        float sc[G][NI];
        scores(kp, t0, sc);
        tile_pages(t0 + TILE, blk);
        issue(kp, kbase, blk, t0 + TILE);
        __builtin_amdgcn_sched_barrier(0);
        accumulate(vp, t0, sc);
        issue(vp, vbase, blk, t0 + TILE);
        __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (APPEND) {
        if (fresh && ntiles > 1) {
          float sc[G][NI];
          scores(kp, t0, sc);
          tile_pages(t0 + TILE, blk);
          issue_fresh(kp, kbase, kn_row, blk, t0 + TILE);
          __builtin_amdgcn_sched_barrier(0);
          accumulate(vp, t0, sc);
          issue_fresh(vp, vbase, vn_row, blk, t0 + TILE);
          __builtin_amdgcn_sched_barrier(0);
          t0 += TILE;
        }
      }
      float sc[G][NI];
      scores(kp, t0, sc);
      accumulate(vp, t0, sc);
    }

    // Merge the token groups (lanes that share s).
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const float M = strided_max<LPT>(m[j]);
      const float f = (m[j] == -INFINITY) ? 0.f : fast_exp2(m[j] - M);
      l[j] = strided_sum<LPT>(l[j] * f);
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[j][e] = strided_sum<LPT>(acc[j][e] * f);
      m[j] = M;
    }

    if (ns == 1) {
      if (g == 0) {
        T* orow = static_cast<T*>(a.out) + r * a.o_row + static_cast<int64_t>(h) * G * a.o_head + lane_dim;
#pragma unroll
        for (int j = 0; j < G; ++j) {
          float o[EPL];
          const float inv = 1.f / l[j];
#pragma unroll
          for (int e = 0; e < EPL; ++e) o[e] = acc[j][e] * inv;
          *reinterpret_cast<u32x4*>(orow + j * a.o_head) = PK::pack(o);
        }
      }
      store_new_token(r, h);
    } else {
      const int64_t slot = (static_cast<int64_t>(r) * a.hkv + h) * kMaxSplits + sp;
      if (g == 0) {
        float* dst = a.ws_acc + slot * G * D + lane_dim;
#pragma unroll
        for (int j = 0; j < G; ++j)
#pragma unroll
          for (int e = 0; e < EPL; e += 4) {
            u32x4 w;
            w[0] = __float_as_uint(acc[j][e]);
            w[1] = __float_as_uint(acc[j][e + 1]);
            w[2] = __float_as_uint(acc[j][e + 2]);
            w[3] = __float_as_uint(acc[j][e + 3]);
            store_partial(dst + j * D + e, w);
          }
      }
      if (lane == 0) {
#pragma unroll
        for (int j = 0; j < G; ++j) a.ws_ml[slot * G + j] = make_float2(m[j], l[j]);
      }
    }
  };

  // Grouped-query items (4 or 8 q heads per kv head, head_dim 128, page 16,
  // 16-bit types) on the matrix cores instead.  Per 32-token tile the wave
  // loads the K and V rows four whole rows per instruction and stages them in
  // its own LDS rows, one after the other.  It forms S^T = K Q^T with
  // v_mfma_f32_32x32x16 (A = K from the staged rows: lane (token c, half)
  // reads dims 16ks + 8half .. + 7 of row c; B = q, column c being q head
  // c % G, so columns G..31 repeat the heads and are dropped), keeps an online
  // softmax per column in log2 units (the running maximum moves only by more
  // than 2^kPrefixRescale), and accumulates O^T += V^T P^T with P rounded to T
  // and V^T from transposing reads of the staged V rows; the row sums come from
  // the same P (v_dot2 against ones).  Loads of tile t + 1 go out while tile t
  // computes (K after its scores, V after its staging).  Same partials,
  // outputs and fused-append handling as `process`.
  constexpr bool kMfma = (G == 4 || G == 8) && D == 128 && P == 16 && !std::is_same_v<T, float>;
  constexpr int kMfmaTile = 32;
  // Each wave's staged rows: a tile's K rows (kPrefixKRow apart), then its V
  // rows over them (kPrefixVRow apart).
  __shared__ __align__(16) uint16_t gqa_rows[kMfma ? kWaves * kMfmaTile * kPrefixVRow : 1];
  auto process_mfma = [&](const int r, const int h, const int sp, const int len, const int split_len, const int ns) {
    if constexpr (kMfma) {
      using Ops = MfmaOps<T>;
      using V8 = typename Ops::V8;
      constexpr int BK = kMfmaTile, KSTEPS = D / 16, DTILES = D / 32, VROW = kPrefixVRow;
      if (len <= 0) {  // a row with no keys is written as zeros
        if (g == 0) {
          T* orow = static_cast<T*>(a.out) + r * a.o_row + static_cast<int64_t>(h) * G * a.o_head + lane_dim;
          const u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
          for (int jj = 0; jj < G; ++jj) *reinterpret_cast<u32x4*>(orow + jj * a.o_head) = zero;
        }
        store_new_token(r, h);
        return;
      }
      const int t_begin = sp * split_len;
      const int t_end = min(len, t_begin + split_len);
      const int last = t_end - 1;
      int64_t wb = -1, wo = -1;
      if constexpr (APPEND) {
        if (t_end == len && r < a.n_write) {
          wb = a.write_blocks[r];
          wo = a.write_offsets[r];
        }
      }
      const int half = lane >> 5;
      const int col = lane & 31;
      const int j = col % G;
      uint16_t* const rows_lds = gqa_rows + wave * BK * VROW;

      u32x4 qb[KSTEPS];
      {
        const T* qrow = static_cast<const T*>(a.q) + r * a.q_row + static_cast<int64_t>(h * G + j) * a.q_head;
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) qb[ks] = *reinterpret_cast<const u32x4*>(qrow + ks * 16 + half * 8);
      }
      const int grp = lane >> 4, gl = lane & 15;
      const int tr_off = (4 * (grp >> 1) + (gl >> 2)) * VROW + 16 * (grp & 1) + 4 * (gl & 3);
      f32x16 acc_o[DTILES];
#pragma unroll
      for (int c = 0; c < DTILES; ++c) acc_o[c] = f32x16{};
      // This lane's share of its column's row sum (the lane 32 away holds the
      // other keys), from the same rounded P that weights V.
      float lsum = 0.f;
      float m = -INFINITY;

      const int32_t* trow = a.tables + r * a.table_stride;
      const T* kbase = static_cast<const T*>(a.k) + static_cast<int64_t>(h) * a.kv_head;
      const T* vbase = static_cast<const T*>(a.v) + static_cast<int64_t>(h) * a.kv_head;
      const T* kn_row = nullptr;
      const T* vn_row = nullptr;
      if constexpr (APPEND) {
        kn_row = static_cast<const T*>(a.k_new) + r * a.kn_row + static_cast<int64_t>(h) * a.kn_head;
        vn_row = static_cast<const T*>(a.v_new) + r * a.vn_row + static_cast<int64_t>(h) * a.vn_head;
      }
      const uint32_t tok_stride = static_cast<uint32_t>(a.kv_token);

      constexpr int kChunkTokens = 64 * P;  // one table entry per lane
      for (int c0 = t_begin; c0 < t_end; c0 += kChunkTokens) {
        const int c1 = min(t_end, c0 + kChunkTokens);
        const int chunk_page = c0 / P;
        const int chunk_last = (c1 - 1) / P - chunk_page;  // <= 63
        const int table_entry = lane <= chunk_last ? trow[chunk_page + lane] : 0;
        // The row's new token comes from k_new / v_new when this chunk ends
        // the row and the write slot is its last token's slot.
        bool fresh = false;
        if constexpr (APPEND)
          fresh = c1 == len && wb >= 0 && wo == (len - 1) % P &&
                  wb == static_cast<int64_t>(__builtin_amdgcn_readlane(table_entry, chunk_last));
        // Pages of the tile at t0 (two 16-token pages), clamped into the pool.
        auto tile_blocks = [&](int t0, int64_t& b0, int64_t& b1) {
          const int rel = (t0 - c0) / P;
          const int64_t x0 = __builtin_amdgcn_readlane(table_entry, min(rel, chunk_last));
          const int64_t x1 = __builtin_amdgcn_readlane(table_entry, min(rel + 1, chunk_last));
          b0 = (x0 < 0 || x0 >= a.num_blocks) ? 0 : x0;
          b1 = (x1 < 0 || x1 >= a.num_blocks) ? 0 : x1;
        };
        // Token t of the tile at t0 (clamped to the split's last token) at
        // element offset dim: its page slot, or k_new / v_new for a fresh token.
        auto src = [&](const T* base, const T* fresh_row, int64_t b0, int64_t b1, int t0, int t, int dim) {
          const int tok = min(t, last);
          const int64_t blk = ((tok - t0) >> 4) ? b1 : b0;
          const T* p = base + blk * a.kv_block + static_cast<uint32_t>(tok & (P - 1)) * tok_stride + dim;
          if constexpr (APPEND) {
            if (fresh && tok == len - 1) p = fresh_row + dim;
          }
          return reinterpret_cast<const u32x4*>(p);
        };
        // K and V rows in natural layout: lane (row (lane >> 4) + 4i, chunk
        // lane & 15), four whole rows per load.
        auto load_rows = [&](u32x4 (&rows)[BK / 4], const T* base, const T* fresh_row, int t0) {
          int64_t b0, b1;
          tile_blocks(t0, b0, b1);
#pragma unroll
          for (int i = 0; i < BK / 4; ++i)
            rows[i] = load_page(src(base, fresh_row, b0, b1, t0, t0 + (lane >> 4) + 4 * i, (lane & 15) * 8));
        };
        auto stage_rows = [&](const u32x4 (&rows)[BK / 4], int stride) {
#pragma unroll
          for (int i = 0; i < BK / 4; ++i)
            *reinterpret_cast<u32x4*>(&rows_lds[((lane >> 4) + 4 * i) * stride + (lane & 15) * 8]) = rows[i];
        };
        const int ntiles = (c1 - c0 + BK - 1) / BK;
        u32x4 kt[BK / 4], vt[BK / 4];
        load_rows(kt, kbase, kn_row, c0);
        __builtin_amdgcn_sched_barrier(0);
        load_rows(vt, vbase, vn_row, c0);
        for (int it = 0; it < ntiles; ++it) {
          const int t0 = c0 + it * BK;
          // K goes through the wave's LDS rows into operand layout (the
          // previous tile's V reads of those rows were issued before, and LDS
          // runs one wave's operations in order).
          stage_rows(kt, kPrefixKRow);
          u32x4 ka[KSTEPS];
#pragma unroll
          for (int ks = 0; ks < KSTEPS; ++ks)
            ka[ks] = *reinterpret_cast<const u32x4*>(&rows_lds[col * kPrefixKRow + ks * 16 + half * 8]);
          f32x16 sacc = f32x16{};
#pragma unroll
          for (int ks = 0; ks < KSTEPS; ++ks) sacc = Ops::mma(as_v8<V8>(ka[ks]), as_v8<V8>(qb[ks]), sacc);
          if (it + 1 < ntiles) load_rows(kt, kbase, kn_row, t0 + BK);
          __builtin_amdgcn_sched_barrier(0);
          // Element e of this lane is token t0 + 8(e/4) + 4half + e%4.
          float tmax = -INFINITY;
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const bool valid = t0 + 8 * (e >> 2) + 4 * half + (e & 3) <= last;
            sacc[e] = valid ? sacc[e] * a.qscale : -INFINITY;
            tmax = fmaxf(tmax, sacc[e]);
          }
          tmax = max_across_halves(tmax);
          const bool move = tmax > m + kPrefixRescale;
          if (__builtin_amdgcn_ballot_w64(move) != 0) {
            const float mn = move ? fmaxf(m, tmax) : m;
            const float corr = (!move || mn == -INFINITY) ? 1.f : fast_exp2(m - mn);
#pragma unroll
            for (int c = 0; c < DTILES; ++c)
#pragma unroll
              for (int e = 0; e < 16; ++e) acc_o[c][e] *= corr;
            lsum *= corr;
            m = mn;
          }
          const float mb = (m == -INFINITY) ? 0.f : m;
          u32x4 pb[2];
#pragma unroll
          for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              pb[ks][e] = Ops::pack2(fast_exp2(sacc[ks * 8 + 2 * e] - mb), fast_exp2(sacc[ks * 8 + 2 * e + 1] - mb));
          // Stage this tile's V over its K rows (read above), then send the
          // next tile's V loads.
          stage_rows(vt, VROW);
          if (it + 1 < ntiles) load_rows(vt, vbase, vn_row, t0 + BK);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
            for (int c = 0; c < DTILES; ++c) {
              const uint16_t* vlo = &rows_lds[tr_off + ks * 16 * VROW + c * 32];
              const u32x2 lo = lds_read_tr(vlo);
              const u32x2 hi = lds_read_tr(vlo + 8 * VROW);
              const u32x4 va = {lo[0], lo[1], hi[0], hi[1]};
              acc_o[c] = Ops::mma(as_v8<V8>(va), as_v8<V8>(pb[ks]), acc_o[c]);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) lsum = Ops::sum2(pb[ks][e], lsum);
          }
        }
      }

      // Columns 0 .. G-1 hold the q heads.  O^T element e of dim tile c is dim
      // 32c + 8(e/4) + 4half + e%4.
      const float l = lsum + __shfl_xor(lsum, 32, 64);
      if (col < G) {
        if (ns == 1) {
          T* orow = static_cast<T*>(a.out) + r * a.o_row + static_cast<int64_t>(h * G + j) * a.o_head + 4 * half;
          const float inv = 1.f / l;
#pragma unroll
          for (int c = 0; c < DTILES; ++c)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
              const u32x2 w2 = {Ops::pack2(acc_o[c][4 * g4] * inv, acc_o[c][4 * g4 + 1] * inv),
                                Ops::pack2(acc_o[c][4 * g4 + 2] * inv, acc_o[c][4 * g4 + 3] * inv)};
              *reinterpret_cast<u32x2*>(orow + 32 * c + 8 * g4) = w2;
            }
        } else {
          const int64_t slot = (static_cast<int64_t>(r) * a.hkv + h) * kMaxSplits + sp;
          float* dst = a.ws_acc + (slot * G + j) * D + 4 * half;
#pragma unroll
          for (int c = 0; c < DTILES; ++c)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
              u32x4 w;
#pragma unroll
              for (int e = 0; e < 4; ++e) w[e] = __float_as_uint(acc_o[c][4 * g4 + e]);
              store_partial(dst + 32 * c + 8 * g4, w);
            }
          if (half == 0) a.ws_ml[slot * G + j] = make_float2(m, l);
        }
      }
      if (ns == 1) store_new_token(r, h);
    }
  };
  auto run_item = [&](const int r, const int h, const int sp, const int len, const int split_len, const int ns) {
    if constexpr (kMfma) process_mfma(r, h, sp, len, split_len, ns);
    else process(r, h, sp, len, split_len, ns);
  };

  if constexpr (XCD) {
    // XCD-affine schedule: workgroup b runs on XCD b % kXcds (the dispatcher's
    // round-robin; b counts from the first split-pass workgroup, after a whole
    // number of rounds of prefix workers) and owns one (row, split, block of
    // kWaves heads).  Groups
    // gi = split * head_blocks + block are dealt out in rounds of kXcds; in
    // round k XCD x serves group k * kXcds + (x - k) mod kXcds, so every XCD
    // takes early and late splits alike (later splits have fewer rows).  Each
    // XCD walks its groups in order with all rows of a group back to back, so
    // rows that alias the same pages in the same split read them together
    // from one L2.  Items past a row's split count exit at once.
    const int b = block;
    const int t = b / kXcds;
    const int r = t % a.n_rows;
    const int round = t / a.n_rows;
    const int gi = kXcds * round + (b % kXcds + kXcds - round % kXcds) % kXcds;
    if (gi >= a.xcd_groups) return;
    const int head_blocks = a.hkv / kWaves;
    const int sp = gi / head_blocks;
    const int h = (gi - sp * head_blocks) * kWaves + wave;
    const int len = uniform(row_length(a, r));
    int split_len, ns;
    split_plan(len, &split_len, &ns);
    if (sp < ns && !(PREFIX && uniform(prefix_takes(a, r, sp, split_len, ns)))) run_item(r, h, sp, len, split_len, ns);
  } else {
    // Packed schedule (any head count): the compact list of rows x splits x
    // kv heads, kv head innermost, walked in grid-stride order.
    extern __shared__ int prefix[];
    const int total_splits = build_split_prefix(a, prefix);
    const int total = total_splits * a.hkv;
    for (int item = block * kWaves + wave; item < total; item += blocks * kWaves) {
      const int qi = item / a.hkv;
      const int h = item - qi * a.hkv;
      const int r = uniform(find_row(prefix, a.n_rows, qi));
      const int sp = uniform(qi - prefix[r]);
      const int len = uniform(row_length(a, r));
      int split_len, ns;
      split_plan(len, &split_len, &ns);
      if (!(PREFIX && uniform(prefix_takes(a, r, sp, split_len, ns)))) run_item(r, h, sp, len, split_len, ns);
    }
  }
}

template <typename T, int D, int G, int P, int TILE, bool XCD, bool APPEND, bool ONE_SPLIT>
__global__ __launch_bounds__(256) void paged_decode_kernel(DecodeArgs a) {
  split_pass<T, D, G, P, TILE, XCD, false, APPEND, ONE_SPLIT>(a, blockIdx.x, gridDim.x);
}

// The split pass for the grouped-query items on the matrix cores (4 or 8 q
// heads per kv head, head_dim 128, 16-bit types), held to two waves per SIMD.
template <typename T, int D, int G, int P, int TILE, bool XCD, bool APPEND, bool ONE_SPLIT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void paged_decode_gqa_kernel(DecodeArgs a) {
  split_pass<T, D, G, P, TILE, XCD, false, APPEND, ONE_SPLIT>(a, blockIdx.x, gridDim.x);
}

// The split pass with prefix groups: its first pg_workers workgroups compute
// the prefix pass's items (w, w + pg_workers, ...) while the rest run the split
// pass, which skips exactly the splits they take (prefix_takes, evaluated
// alike on both sides).  Two waves per SIMD, as the prefix items need.
template <typename T, int D, int G, int P, int TILE, bool XCD, bool APPEND>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void paged_decode_prefix_kernel(DecodeArgs a) {
  if (static_cast<int>(blockIdx.x) < a.pg_workers) {
    __shared__ __align__(16) uint16_t tiles[kPrefixTileElems];
    const int total = a.pg_n_items * a.hkv;
    for (int w = blockIdx.x; w < total; w += a.pg_workers) shared_prefix_item<T, G>(a, w / a.hkv, w % a.hkv, tiles);
    return;
  }
  split_pass<T, D, G, P, TILE, XCD, true, APPEND>(a, blockIdx.x - a.pg_workers, gridDim.x - a.pg_workers);
}

// Merge kernel: one wavefront per (row, q head) of a row with more than one
// split (the q heads of one kv head in parallel); with a fused append (APPEND)
// the wave of each (row, kv_head)'s first q head also writes that row's new
// token for the kv head: 16-byte chunks of the [D] slab from k_new / v_new to
// (write_blocks[r], write_offsets[r]), skipped when the slot is outside the
// pool.  All loads go out before the first wait: the row's length, the write
// slot and the new token (read from a clamped row and chunk, so no load needs
// a branch) and the partials (merge_partials).  The token is stored last: a
// store ahead of the partial loads would hold them back, since the compiler
// cannot tell the pool from the workspace.
template <typename T, int D, bool APPEND>
__global__ __launch_bounds__(256) void paged_decode_merge_kernel(DecodeArgs a) {
  constexpr int kChunks = D * static_cast<int>(sizeof(T)) / 16;
  static_assert(kChunks <= 64 && 64 % kChunks == 0, "whole chunks per lane group");
  const int item = blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (item >= a.n_rows * a.hq) return;
  const int G = a.hq / a.hkv;
  const int r = item / a.hq;
  const int qh = item - r * a.hq;
  const int h = qh / G;
  const int j = qh - h * G;
  const int lane = threadIdx.x & 63;
  const int len = row_length(a, r);
  int64_t b = -1, o = -1;
  u32x4 kt = {}, vt = {};
  if constexpr (APPEND) {  // a.n_write >= 1
    const int rw = min(r, a.n_write - 1);
    const int chunk = lane % kChunks;
    b = a.write_blocks[rw];
    o = a.write_offsets[rw];
    kt = reinterpret_cast<const u32x4*>(static_cast<const T*>(a.k_new) + rw * a.kn_row +
                                        static_cast<int64_t>(h) * a.kn_head)[chunk];
    vt = reinterpret_cast<const u32x4*>(static_cast<const T*>(a.v_new) + rw * a.vn_row +
                                        static_cast<int64_t>(h) * a.vn_head)[chunk];
  }
  const MergeLoads<D> first = load_partials<D>(a, r, h, j, lane);
  __builtin_amdgcn_sched_barrier(0);  // every load above is issued before the first wait
  int split_len, ns;
  split_plan(len, &split_len, &ns);
  merge_partials<T, D>(a, r, h, j, ns, lane, first);
  if (APPEND && j == 0 && r < a.n_write && lane < kChunks && b >= 0 && b < a.num_blocks && o >= 0 && o < a.page) {
    const int64_t slot = b * a.kv_block + o * a.kv_token + static_cast<int64_t>(h) * a.kv_head;
    reinterpret_cast<u32x4*>(const_cast<T*>(static_cast<const T*>(a.k) + slot))[lane] = kt;
    reinterpret_cast<u32x4*>(const_cast<T*>(static_cast<const T*>(a.v) + slot))[lane] = vt;
  }
}

// Shared-prefix pass: the split partials of the splits that prefix_takes()
// gives it, for every group at once, computed by the first workgroups of the
// split pass's launch (paged_decode_prefix_kernel).  Work item i belongs to the
// group g with item_start[g] <= i < item_start[g + 1]; its offset in the group
// is (split sp, block b of 64 queries), b fastest.  Item (i, h) owns
// split sp of group g's pages (keys [sp * S, (sp + 1) * S), S the group's
// split length) under kv head h, for 64 queries: (row, q head) pairs
// b * 64 .. b * 64 + 63 of the group's members x G.  Wave w takes queries
// 32(w % 2) .. + 31 over key half w / 2 of the split; the two halves merge
// their (max, sum, acc) through LDS at the end.  K and V of each 32-key tile
// are read once into LDS (row-major, padded rows) and serve all 64 queries,
// so a prefix is read from memory once per launch instead of once per row.
// Per tile a wave forms S^T = K Q^T with v_mfma_f32_32x32x16 (A = 32 K rows,
// B = its 32 queries' q), keeps an online softmax in log2 units, and
// accumulates O^T += V^T P^T with P rounded to T and V^T from transposing LDS
// reads; the row sums come from the same rounded P through one MFMA against
// ones.  A query's running maximum moves only when a tile exceeds it by
// 2^kRescale, decided per query: with every MFMA column computed on its own,
// a query's result depends on its own q and keys only, not on which queries
// share the workgroup (so not on the batch).  The result is written as the
// split pass would: (max, sum) and the unnormalised accumulator in the decode
// workspace slot of (row, h, sp).
// Work item `item` of the prefix pass under kv head h, by the 256 threads of a
// workgroup with `tiles` (kPrefixTileElems elements) of LDS.  Every thread of
// the workgroup calls it with the same arguments; it leaves the LDS free for
// the next call once all threads have passed its first barrier.
template <typename T, int G>
__device__ __forceinline__ void shared_prefix_item(const DecodeArgs& a, const int item, const int h, uint16_t* tiles) {
  using Ops = MfmaOps<T>;
  using V8 = typename Ops::V8;
  constexpr int D = 128, KSTEPS = D / 16, DTILES = D / 32;
  constexpr int KROW = kPrefixKRow, VROW = kPrefixVRow;
  constexpr int KTILE = kPrefixBK * KROW, VTILE = kPrefixBK * VROW;
  constexpr int MERGE_FLOATS = 2 + 16 * DTILES;  // (max, sum, acc) per lane
  static_assert(2 * 64 * MERGE_FLOATS * 4 <= 2 * (KTILE + VTILE) * 2, "merge fits in the tile buffers");
  static_assert(kPrefixTileElems == 2 * (KTILE + VTILE), "tile buffer size");

  const int tid = threadIdx.x;
  // The item's group: the last g with item_start[g] <= item.
  int g = 0;
  {
    int hi = a.pg_n_groups;
    while (hi - g > 1) {
      const int mid = (g + hi) >> 1;
      if (a.pg_item_start[mid] <= item) g = mid;
      else hi = mid;
    }
  }
  const int32_t* rec = group_record(a, g);
  if (!rec) return;
  const int S = rec[kGroupSplit];
  const int n_members = rec[kGroupMembers];
  const int qblocks = (n_members * G + 63) / 64;
  const int local = item - a.pg_item_start[g];
  if (local < 0 || qblocks == 0) return;
  const int sp = local / qblocks;
  const int qblock = local - sp * qblocks;
  const int lane = tid & 63;
  const int wave = uniform(tid >> 6);
  const int qw = wave & 1;   // query half
  const int kh = wave >> 1;  // key half
  const int half = lane >> 5;
  const int col = lane & 31;
  uint16_t* const k_lds = tiles + kh * (KTILE + VTILE);
  uint16_t* const v_lds = k_lds + KTILE;

  // An item past the group's whole splits (the host's item count may cover
  // more query blocks than there are) has nothing to do.
  if (static_cast<int64_t>(sp + 1) * S > static_cast<int64_t>(rec[kGroupPages]) * a.page) return;

  // Staging: within a key half, thread t (of 128) moves 16-byte chunk
  // (t + 128i) % 16 of tile row (t + 128i) / 16, i = 0..3, for K and for V.
  // The split lies inside the group's pages, so every page id read is one of them.
  const int32_t* group_pages = a.pg_pages + rec[kGroupPage0];
  const int ntiles = S / kPrefixBK / 2;  // per key half
  const int key0 = sp * S + kh * ntiles * kPrefixBK;
  const int ltid = tid & 127;
  const T* kbase = static_cast<const T*>(a.k) + static_cast<int64_t>(h) * a.kv_head;
  const T* vbase = static_cast<const T*>(a.v) + static_cast<int64_t>(h) * a.kv_head;
  // Two tiles of loads in flight: tile t's registers are slot t % 2.
  u32x4 kreg[2][4], vreg[2][4];
  auto load_tile = [&](int t, u32x4 (&kr)[4], u32x4 (&vr)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = ltid + 128 * i;
      const int key = key0 + t * kPrefixBK + (c >> 4);
      const int64_t b = group_pages[key / a.page];
      const int64_t blk = (b < 0 || b >= a.num_blocks) ? 0 : b;
      const int64_t off = blk * a.kv_block + static_cast<int64_t>(key % a.page) * a.kv_token + (c & 15) * 8;
      kr[i] = load_page(reinterpret_cast<const u32x4*>(kbase + off));
      vr[i] = load_page(reinterpret_cast<const u32x4*>(vbase + off));
    }
  };
  // The first two tiles depend on the group alone: their loads go out before
  // the membership checks below, whose chain of dependent reads they overlap.
  // (S = 256 << k keys, so each key half has at least two tiles.)
  load_tile(0, kreg[0], vreg[0]);
  load_tile(1, kreg[1], vreg[1]);

  // This lane's query: (member qi / G of group g, q head h * G + qi % G).
  const int qi = qblock * 64 + qw * 32 + col;
  const bool listed = qi < n_members * G;
  const int r = a.pg_members[rec[kGroupMember0] + (listed ? qi / G : 0)];
  const int j = listed ? qi % G : 0;
  const bool row_ok = listed && r >= 0 && r < a.n_rows;
  const int rq = row_ok ? r : 0;
  // q as the B operand (lane (col, half) holds dims 16ks + 8half .. + 7),
  // loaded for every listed row before its membership is known.
  u32x4 qb[KSTEPS];
  {
    const T* qrow = static_cast<const T*>(a.q) + rq * a.q_row + static_cast<int64_t>(h * G + j) * a.q_head;
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) qb[ks] = *reinterpret_cast<const u32x4*>(qrow + ks * 16 + half * 8);
  }
  bool mine = false;
  if (row_ok && a.pg_row_group[r] == g) {
    int split_len, ns;
    split_plan(row_length(a, r), &split_len, &ns);
    mine = prefix_takes(a, r, sp, split_len, ns);
  }
  if (!__syncthreads_or(mine)) return;

  auto store_tile = [&](const u32x4 (&kr)[4], const u32x4 (&vr)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = ltid + 128 * i;
      *reinterpret_cast<u32x4*>(&k_lds[(c >> 4) * KROW + (c & 15) * 8]) = kr[i];
      *reinterpret_cast<u32x4*>(&v_lds[(c >> 4) * VROW + (c & 15) * 8]) = vr[i];
    }
  };

  // V^T A-operand reads: within k-step ks, lane (dim i, half kh) needs keys
  // 16ks + 4kh + {0..3} and 16ks + 8 + 4kh + {0..3}, the key order in which
  // the S^T accumulator leaves P.
  const int grp = lane >> 4, gl = lane & 15;
  const int tr_off = (4 * (grp >> 1) + (gl >> 2)) * VROW + 16 * (grp & 1) + 4 * (gl & 3);
  const uint32_t one2 = Ops::pack2(1.f, 1.f);
  const u32x4 ones = {one2, one2, one2, one2};

  f32x16 acc_o[DTILES];
#pragma unroll
  for (int c = 0; c < DTILES; ++c) acc_o[c] = f32x16{};
  f32x16 acc_l = f32x16{};
  float m = -INFINITY;

  auto compute_tile = [&]() __attribute__((always_inline)) {
    f32x16 sacc = f32x16{};
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      const u32x4 kv = *reinterpret_cast<const u32x4*>(&k_lds[col * KROW + ks * 16 + half * 8]);
      sacc = Ops::mma(as_v8<V8>(kv), as_v8<V8>(qb[ks]), sacc);
    }
    float tmax = -INFINITY;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      sacc[e] *= a.qscale;
      tmax = fmaxf(tmax, sacc[e]);
    }
    tmax = max_across_halves(tmax);
    // Both lanes of a query (col, col + 32) hold the same tmax and m, so they
    // decide alike; a query that does not move keeps corr = 1 (exact).
    const bool move = tmax > m + kPrefixRescale;
    if (__builtin_amdgcn_ballot_w64(move) != 0) {
      const float mn = move ? fmaxf(m, tmax) : m;
      const float corr = (!move || mn == -INFINITY) ? 1.f : fast_exp2(m - mn);
#pragma unroll
      for (int c = 0; c < DTILES; ++c)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc_o[c][e] *= corr;
#pragma unroll
      for (int e = 0; e < 16; ++e) acc_l[e] *= corr;
      m = mn;
    }
    const float mb = (m == -INFINITY) ? 0.f : m;
    u32x4 pb[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        pb[ks][e] = Ops::pack2(fast_exp2(sacc[ks * 8 + 2 * e] - mb), fast_exp2(sacc[ks * 8 + 2 * e + 1] - mb));
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
      for (int c = 0; c < DTILES; ++c) {
        const uint16_t* vlo = &v_lds[tr_off + ks * 16 * VROW + c * 32];
        const u32x2 lo = lds_read_tr(vlo);
        const u32x2 hi = lds_read_tr(vlo + 8 * VROW);
        const u32x4 va = {lo[0], lo[1], hi[0], hi[1]};
        acc_o[c] = Ops::mma(as_v8<V8>(va), as_v8<V8>(pb[ks]), acc_o[c]);
      }
      acc_l = Ops::mma(as_v8<V8>(ones), as_v8<V8>(pb[ks]), acc_l);
    }
  };
  // S = 256 << k keys, so each key half has an even tile count.
  for (int t = 0; t < ntiles; t += 2) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      __syncthreads();  // the previous tile's reads are done
      store_tile(kreg[u], vreg[u]);
      __syncthreads();
      if (t + u + 2 < ntiles) load_tile(t + u + 2, kreg[u], vreg[u]);
      compute_tile();
    }
  }

  // Key half 1 hands its (max, sum, acc) to key half 0 through LDS.
  __syncthreads();
  float* xs = reinterpret_cast<float*>(tiles) + qw * MERGE_FLOATS * 64 + lane;
  if (kh == 1) {
    xs[0] = m;
    xs[64] = acc_l[0];
#pragma unroll
    for (int c = 0; c < DTILES; ++c)
#pragma unroll
      for (int e = 0; e < 16; ++e) xs[(2 + 16 * c + e) * 64] = acc_o[c][e];
  }
  __syncthreads();
  if (kh == 1 || !mine) return;
  const float m1 = xs[0];
  const float mm = fmaxf(m, m1);
  const float c0 = (m == -INFINITY) ? 0.f : fast_exp2(m - mm);
  const float c1 = (m1 == -INFINITY) ? 0.f : fast_exp2(m1 - mm);
  const float l = acc_l[0] * c0 + xs[64] * c1;
#pragma unroll
  for (int c = 0; c < DTILES; ++c)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc_o[c][e] = acc_o[c][e] * c0 + xs[(2 + 16 * c + e) * 64] * c1;
  m = mm;
  // O^T element e of dim tile c is dim 32c + 8(e/4) + 4half + e%4.
  const int64_t slot = (static_cast<int64_t>(rq) * a.hkv + h) * kMaxSplits + sp;
  float* dst = a.ws_acc + (slot * G + j) * D + 4 * half;
#pragma unroll
  for (int c = 0; c < DTILES; ++c)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      u32x4 w;
#pragma unroll
      for (int e = 0; e < 4; ++e) w[e] = __float_as_uint(acc_o[c][4 * g4 + e]);
      *reinterpret_cast<u32x4*>(dst + 32 * c + 8 * g4) = w;
    }
  if (half == 0) a.ws_ml[slot * G + j] = make_float2(m, l);
}

// Generic kernel for shapes the tiled kernel does not cover (odd head_dim,
// strided dims, any page size or group size): one wavefront per (row, q head),
// tokens in order, same exp2-domain online softmax.  Correctness path only.
constexpr int kGenericMaxPerLane = 8;  // head_dim <= 512

template <typename T>
__global__ __launch_bounds__(64) void paged_decode_generic_kernel(DecodeArgs a) {
  const int r = blockIdx.x;
  const int hq = blockIdx.y;
  const int lane = threadIdx.x;
  const int G = a.hq / a.hkv;
  const int h = hq / G;
  const int len = row_length(a, r);
  T* orow = static_cast<T*>(a.out) + r * a.o_row + static_cast<int64_t>(hq) * a.o_head;
  if (len <= 0) {
    for (int d = lane; d < a.d; d += 64) store_elem(orow + d * a.o_dim, 0.f);
    return;
  }
  const T* qrow = static_cast<const T*>(a.q) + r * a.q_row + static_cast<int64_t>(hq) * a.q_head;
  float qv[kGenericMaxPerLane], acc[kGenericMaxPerLane];
#pragma unroll
  for (int c = 0; c < kGenericMaxPerLane; ++c) {
    const int d = lane + 64 * c;
    qv[c] = d < a.d ? load_elem(qrow + d * a.q_dim) * a.qscale : 0.f;
    acc[c] = 0.f;
  }
  const int32_t* trow = a.tables + r * a.table_stride;
  float m = -INFINITY, l = 0.f;
  for (int t = 0; t < len; ++t) {
    int64_t blk = trow[t / a.page];
    blk = (blk < 0 || blk >= a.num_blocks) ? 0 : blk;
    const int64_t base = blk * a.kv_block + static_cast<int64_t>(t % a.page) * a.kv_token +
                         static_cast<int64_t>(h) * a.kv_head;
    const T* kt = static_cast<const T*>(a.k) + base;
    const T* vt = static_cast<const T*>(a.v) + base;
    float dot = 0.f;
#pragma unroll
    for (int c = 0; c < kGenericMaxPerLane; ++c) {
      const int d = lane + 64 * c;
      if (d < a.d) dot = fmaf(qv[c], load_elem(kt + d * a.kv_dim), dot);
    }
    dot = group_sum<64>(dot);
    const float mn = fmaxf(m, dot);
    const float corr = fast_exp2(m - mn);
    const float p = fast_exp2(dot - mn);
    l = l * corr + p;
#pragma unroll
    for (int c = 0; c < kGenericMaxPerLane; ++c) {
      const int d = lane + 64 * c;
      const float vv = d < a.d ? load_elem(vt + d * a.kv_dim) : 0.f;
      acc[c] = fmaf(p, vv, acc[c] * corr);
    }
    m = mn;
  }
  const float inv = 1.f / l;
#pragma unroll
  for (int c = 0; c < kGenericMaxPerLane; ++c) {
    const int d = lane + 64 * c;
    if (d < a.d) store_elem(orow + d * a.o_dim, acc[c] * inv);
  }
}

// ---------------------------------------------------------------------------
// Host dispatch.
using DecodeKernel = void (*)(DecodeArgs);

template <typename T, int D, bool XCD, bool PREFIX, bool APPEND, bool ONE_SPLIT = false>
DecodeKernel pick_group(int G) {
  if constexpr (PREFIX) {
    switch (G) {
      case 1: return paged_decode_prefix_kernel<T, D, 1, 16, kTile, XCD, APPEND>;
      case 2: return paged_decode_prefix_kernel<T, D, 2, 16, kTile, XCD, APPEND>;
      case 4: return paged_decode_prefix_kernel<T, D, 4, 16, kTile, XCD, APPEND>;
      case 8: return paged_decode_prefix_kernel<T, D, 8, 16, kTile, XCD, APPEND>;
      default: return nullptr;
    }
  } else {
    constexpr bool kMfmaGroups = D == 128 && !std::is_same_v<T, float>;  // split_pass's grouped-query items
    switch (G) {
      case 1: return paged_decode_kernel<T, D, 1, 16, kTile, XCD, APPEND, ONE_SPLIT>;
      case 2: return paged_decode_kernel<T, D, 2, 16, kTile, XCD, APPEND, ONE_SPLIT>;
      case 4:
        if constexpr (kMfmaGroups) return paged_decode_gqa_kernel<T, D, 4, 16, kTile, XCD, APPEND, ONE_SPLIT>;
        return paged_decode_kernel<T, D, 4, 16, kTile, XCD, APPEND, ONE_SPLIT>;
      case 8:
        if constexpr (kMfmaGroups) return paged_decode_gqa_kernel<T, D, 8, 16, kTile, XCD, APPEND, ONE_SPLIT>;
        return paged_decode_kernel<T, D, 8, 16, kTile, XCD, APPEND, ONE_SPLIT>;
      default: return nullptr;
    }
  }
}

// The fused-append split pass is compiled for the XCD-affine schedule (with
// and without the shared-prefix check); other cases append first, then decode.
template <typename T, int D, bool PREFIX>
DecodeKernel pick_group(int G, bool xcd, bool append, bool one_split) {
  if (append) {
    if (!xcd) return nullptr;
    if constexpr (!PREFIX) {
      if (one_split) return pick_group<T, D, true, false, true, true>(G);
    }
    return pick_group<T, D, true, PREFIX, true>(G);
  }
  return xcd ? pick_group<T, D, true, PREFIX, false>(G) : pick_group<T, D, false, PREFIX, false>(G);
}

// The split pass with the shared-prefix check exists where the prefix pass
// does (16-bit types, head_dim 128); everywhere else it is compiled out.
template <typename T, int D>
DecodeKernel pick_group(int G, bool xcd, bool prefix, bool append, bool one_split) {
  if (prefix) {
    if constexpr (D == 128 && !std::is_same_v<T, float>) return pick_group<T, D, true>(G, xcd, append, one_split);
    return nullptr;
  }
  return pick_group<T, D, false>(G, xcd, append, one_split);
}

template <typename T>
DecodeKernel pick_tiled(int d, int G, bool xcd, bool prefix, bool append, bool one_split = false);
template <>
DecodeKernel pick_tiled<bf16>(int d, int G, bool xcd, bool prefix, bool append, bool one_split) {
  switch (d) {
    case 64: return pick_group<bf16, 64>(G, xcd, prefix, append, one_split);
    case 128: return pick_group<bf16, 128>(G, xcd, prefix, append, one_split);
    case 256: return pick_group<bf16, 256>(G, xcd, prefix, append, one_split);
    default: return nullptr;
  }
}
template <>
DecodeKernel pick_tiled<f16>(int d, int G, bool xcd, bool prefix, bool append, bool one_split) {
  switch (d) {
    case 64: return pick_group<f16, 64>(G, xcd, prefix, append, one_split);
    case 128: return pick_group<f16, 128>(G, xcd, prefix, append, one_split);
    case 256: return pick_group<f16, 256>(G, xcd, prefix, append, one_split);
    default: return nullptr;
  }
}
template <>
DecodeKernel pick_tiled<float>(int d, int G, bool xcd, bool prefix, bool append, bool one_split) {
  switch (d) {
    case 64: return pick_group<float, 64>(G, xcd, prefix, append, one_split);
    case 128: return pick_group<float, 128>(G, xcd, prefix, append, one_split);
    default: return nullptr;
  }
}

// Unfused append for shapes the fused path does not cover: grid (n_write,
// hkv), one wave copies row r's head h slab (any dim strides) into its slot.
template <typename T>
__global__ __launch_bounds__(64) void slice_append_kernel(DecodeArgs a) {
  const int r = blockIdx.x, h = blockIdx.y;
  const int64_t b = a.write_blocks[r], o = a.write_offsets[r];
  if (b < 0 || b >= a.num_blocks || o < 0 || o >= a.page) return;
  const int64_t slot = b * a.kv_block + o * a.kv_token + static_cast<int64_t>(h) * a.kv_head;
  T* kd = const_cast<T*>(static_cast<const T*>(a.k)) + slot;
  T* vd = const_cast<T*>(static_cast<const T*>(a.v)) + slot;
  const T* kn = static_cast<const T*>(a.k_new) + r * a.kn_row + static_cast<int64_t>(h) * a.kn_head;
  const T* vn = static_cast<const T*>(a.v_new) + r * a.vn_row + static_cast<int64_t>(h) * a.vn_head;
  for (int d = threadIdx.x; d < a.d; d += 64) {
    kd[d * a.kv_dim] = kn[d * a.kn_dim];
    vd[d * a.kv_dim] = vn[d * a.vn_dim];
  }
}

bool stride16(int64_t stride, int esize) { return (stride * esize) % 16 == 0; }


template <typename T>
int launch_decode(DecodeArgs a, int64_t max_table_width, hipStream_t stream) {
  const int esize = sizeof(T);
  const int G = a.hq / a.hkv;
  DecodeKernel tiled = nullptr;
  const bool layout_ok = a.page == 16 && a.q_dim == 1 && a.o_dim == 1 && a.kv_dim == 1 && aligned16(a.q) &&
                         aligned16(a.out) && aligned16(a.k) && aligned16(a.v) && stride16(a.q_row, esize) &&
                         stride16(a.q_head, esize) && stride16(a.o_row, esize) && stride16(a.o_head, esize) &&
                         stride16(a.kv_block, esize) && stride16(a.kv_token, esize) && stride16(a.kv_head, esize) &&
                         a.kv_token * a.page < (int64_t(1) << 31);
  const bool xcd = RLT_DECODE_XCD_SCHEDULE && a.hkv % kWaves == 0;
  // A table of at most one split's tokens makes every row a single split:
  // the split pass then writes every output itself and no merge runs.
  const int64_t max_tokens = max_table_width * a.page;
  const bool single_split = max_tokens <= kSplitTokens;
  // The prefix groups are served where the split pass with prefix workers
  // exists for this shape (16-bit types, head_dim 128, 1/2/4/8 q heads per kv
  // head) and rows span more than one split (a prefix split is never a row's
  // last); elsewhere the hint is dropped.
  const bool prefix = a.pg_row_group && a.pg_n_items > 0 && layout_ok && !single_split &&
                      pick_tiled<T>(a.d, G, xcd, true, false);
  if (!prefix) a.pg_row_group = nullptr;
  if (a.n_write > 0) {
    // The fused append needs the tiled kernel and 16-byte rows of k_new / v_new;
    // otherwise the new tokens are written first and the decode runs as usual.
    const bool fused = layout_ok && a.kn_dim == 1 && a.vn_dim == 1 && aligned16(a.k_new) && aligned16(a.v_new) &&
                       stride16(a.kn_row, esize) && stride16(a.kn_head, esize) && stride16(a.vn_row, esize) &&
                       stride16(a.vn_head, esize) && pick_tiled<T>(a.d, G, xcd, prefix, true) != nullptr;
    if (!fused) {
      hipLaunchKernelGGL(slice_append_kernel<T>, dim3(a.n_write, a.hkv), dim3(64), 0, stream, a);
      if (int rc = check_launch("rlt_paged_decode_append(append)")) return rc;
      a.n_write = 0;
    }
  }
  const bool append = a.n_write > 0;
  // One-split rows: each row's one item stores its new token after its reads.
  if (layout_ok) tiled = pick_tiled<T>(a.d, G, xcd, prefix, append, single_split);
  if (prefix) {
    // The prefix pass's items run in the split pass's first workgroups.  The
    // prefix splits are never a row's last split, which holds the new token,
    // so they read no slot the fused append writes.
    const int64_t items = static_cast<int64_t>(a.pg_n_items) * a.hkv;
    a.pg_workers = static_cast<int>(std::min<int64_t>(kPrefixWorkers, (items + kXcds - 1) / kXcds * kXcds));
  }
  if (!tiled) {
    if (a.d > 64 * kGenericMaxPerLane) return fail(RLT_EUNSUPPORTED, "rlt_paged_decode: head_dim > 512");
    if (a.hq > 65535) return fail(RLT_EUNSUPPORTED, "rlt_paged_decode: too many query heads");
    hipLaunchKernelGGL(paged_decode_generic_kernel<T>, dim3(a.n_rows, a.hq), dim3(64), 0, stream, a);
    return check_launch("rlt_paged_decode(generic)");
  }
  const int64_t splits_cap = std::min<int64_t>(kMaxSplits, (max_tokens + kSplitTokens - 1) / kSplitTokens);
  if (xcd) {
    const int64_t groups = std::max<int64_t>(splits_cap, 1) * (a.hkv / kWaves);
    const int64_t grid = static_cast<int64_t>(kXcds) * a.n_rows * ((groups + kXcds - 1) / kXcds) + a.pg_workers;
    if (grid > 0x7fffffff) return fail(RLT_EUNSUPPORTED, "rlt_paged_decode: too many work items");
    a.xcd_groups = static_cast<int>(groups);
    hipLaunchKernelGGL(tiled, dim3(static_cast<unsigned>(grid)), dim3(64 * kWaves), 0, stream, a);
  } else {
    const int64_t items = static_cast<int64_t>(a.n_rows) * a.hkv * std::max<int64_t>(splits_cap, 1);
    const int grid = static_cast<int>(std::min<int64_t>(kMaxGrid, (items + kWaves - 1) / kWaves)) + a.pg_workers;
    const size_t lds = static_cast<size_t>(a.n_rows + 1) * sizeof(int);
    a.xcd_groups = 0;
    hipLaunchKernelGGL(tiled, dim3(grid), dim3(64 * kWaves), lds, stream, a);
  }
  if (int rc = check_launch("rlt_paged_decode")) return rc;
  if (single_split) return RLT_OK;
  const int merge_grid = (a.n_rows * a.hq + kWaves - 1) / kWaves;
  const dim3 mgrid(merge_grid), mblock(64 * kWaves);
  if (append) {
    if (a.d == 64) hipLaunchKernelGGL((paged_decode_merge_kernel<T, 64, true>), mgrid, mblock, 0, stream, a);
    else if (a.d == 128) hipLaunchKernelGGL((paged_decode_merge_kernel<T, 128, true>), mgrid, mblock, 0, stream, a);
    else hipLaunchKernelGGL((paged_decode_merge_kernel<T, 256, true>), mgrid, mblock, 0, stream, a);
  } else {
    if (a.d == 64) hipLaunchKernelGGL((paged_decode_merge_kernel<T, 64, false>), mgrid, mblock, 0, stream, a);
    else if (a.d == 128) hipLaunchKernelGGL((paged_decode_merge_kernel<T, 128, false>), mgrid, mblock, 0, stream, a);
    else hipLaunchKernelGGL((paged_decode_merge_kernel<T, 256, false>), mgrid, mblock, 0, stream, a);
  }
  return check_launch("rlt_paged_decode(merge)");
}

int64_t round256(int64_t x) { return (x + 255) / 256 * 256; }

// Workspace layout: acc partials | (max, sum) partials.
struct WorkspaceLayout {
  int64_t acc, ml, total;
};
WorkspaceLayout workspace_layout(int64_t rows, int64_t hq, int64_t hkv, int64_t d) {
  rows = std::min<int64_t>(rows, kMaxRowsPerLaunch);
  const int64_t slots = rows * hkv * kMaxSplits * (hq / hkv);
  WorkspaceLayout w{};
  w.acc = 0;
  w.ml = round256(slots * d * static_cast<int64_t>(sizeof(float)));
  w.total = w.ml + round256(slots * static_cast<int64_t>(sizeof(float2)));
  return w;
}

int64_t workspace_bytes_for(int64_t rows, int64_t hq, int64_t hkv, int64_t d) {
  if (rows <= 0 || hq <= 0 || hkv <= 0 || d <= 0 || hq % hkv) return 0;
  return workspace_layout(rows, hq, hkv, d).total;
}

}  // namespace
}  // namespace rlt

using namespace rlt;

extern "C" int64_t rlt_paged_decode_workspace_bytes(int64_t n_rows, int64_t num_q_heads, int64_t num_kv_heads,
                                                    int64_t head_dim) {
  return workspace_bytes_for(n_rows, num_q_heads, num_kv_heads, head_dim);
}

namespace {

// Sections of the prefix-group hint buffer (rlt_kv.h).
struct PrefixHint {
  const int32_t* buffer;
  int64_t n_groups, n_members, n_pages, n_items;
};

struct AppendSource {
  const void* k_new;
  const int64_t* k_strides;  // row, head, dim (elements)
  const void* v_new;
  const int64_t* v_strides;
  const int64_t* write_blocks;
  const int64_t* write_offsets;
  int64_t n_write;
};

int paged_decode(const void* q, const int64_t* q_strides, const void* key_cache, const void* value_cache,
                 const int64_t* kv_strides, const int32_t* block_tables, int64_t table_stride, int64_t max_table_width,
                 const int32_t* context_lengths, void* out, const int64_t* out_strides, int64_t n_rows,
                 int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim, int64_t page_size, int64_t num_blocks,
                 float scale, int dtype, void* workspace, int64_t workspace_bytes, void* stream,
                 const PrefixHint* hint, const AppendSource* append = nullptr) {
  const int esize = dtype_size(dtype);
  if (!esize) return fail(RLT_EINVAL, "rlt_paged_decode: unknown dtype %d", dtype);
  if (n_rows < 0) return fail(RLT_EINVAL, "rlt_paged_decode: n_rows is negative");
  if (num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads)
    return fail(RLT_EINVAL, "rlt_paged_decode: query heads must be a positive multiple of KV heads");
  if (head_dim <= 0 || page_size <= 0 || num_blocks <= 0)
    return fail(RLT_EINVAL, "rlt_paged_decode: head_dim, page_size and num_blocks must be positive");
  if (max_table_width < 0 || table_stride < 0) return fail(RLT_EINVAL, "rlt_paged_decode: bad table shape");
  if (n_rows == 0) return RLT_OK;
  if (!q || !key_cache || !value_cache || !block_tables || !context_lengths || !out || !q_strides || !kv_strides ||
      !out_strides)
    return fail(RLT_EINVAL, "rlt_paged_decode: NULL pointer argument");
  if (num_q_heads > 4096 || head_dim > 4096 || page_size > (1 << 20))
    return fail(RLT_EUNSUPPORTED, "rlt_paged_decode: shape too large");
  const int64_t need = workspace_bytes_for(n_rows, num_q_heads, num_kv_heads, head_dim);
  if (workspace_bytes < need || (need && !workspace))
    return fail(RLT_EWORKSPACE, "rlt_paged_decode: workspace of %lld bytes < required %lld",
                (long long)workspace_bytes, (long long)need);
  if (!aligned16(workspace)) return fail(RLT_EINVAL, "rlt_paged_decode: workspace must be 16-byte aligned");

  DecodeArgs a{};
  a.q_row = q_strides[0];
  a.q_head = q_strides[1];
  a.q_dim = q_strides[2];
  a.k = key_cache;
  a.v = value_cache;
  a.kv_block = kv_strides[0];
  a.kv_token = kv_strides[1];
  a.kv_head = kv_strides[2];
  a.kv_dim = kv_strides[3];
  a.table_stride = table_stride;
  a.o_row = out_strides[0];
  a.o_head = out_strides[1];
  a.o_dim = out_strides[2];
  const WorkspaceLayout layout = workspace_layout(n_rows, num_q_heads, num_kv_heads, head_dim);
  char* ws = static_cast<char*>(workspace);
  a.ws_acc = reinterpret_cast<float*>(ws + layout.acc);
  a.ws_ml = reinterpret_cast<float2*>(ws + layout.ml);
  a.hkv = static_cast<int>(num_kv_heads);
  a.hq = static_cast<int>(num_q_heads);
  a.d = static_cast<int>(head_dim);
  a.page = static_cast<int>(page_size);
  a.num_blocks = num_blocks;
  a.max_len = max_table_width * page_size;
  a.qscale = scale * kLog2e;
  if (hint) {
    a.pg_row_group = hint->buffer;
    a.pg_groups = a.pg_row_group + n_rows;
    a.pg_item_start = a.pg_groups + kGroupFields * hint->n_groups;
    a.pg_members = a.pg_item_start + hint->n_groups + 1;
    a.pg_pages = a.pg_members + hint->n_members;
    a.pg_n_groups = static_cast<int>(hint->n_groups);
    a.pg_n_members = static_cast<int>(hint->n_members);
    a.pg_n_pages = static_cast<int>(hint->n_pages);
    a.pg_n_items = static_cast<int>(hint->n_items);
  }
  if (append) {
    if (append->n_write < 0 || append->n_write > n_rows)
      return fail(RLT_EINVAL, "rlt_paged_decode_append: n_write must be in [0, n_rows]");
    if (append->n_write > 0 && (!append->k_new || !append->v_new || !append->k_strides || !append->v_strides ||
                                !append->write_blocks || !append->write_offsets))
      return fail(RLT_EINVAL, "rlt_paged_decode_append: NULL append argument");
    if (append->n_write > 0) {
      a.kn_row = append->k_strides[0];
      a.kn_head = append->k_strides[1];
      a.kn_dim = append->k_strides[2];
      a.vn_row = append->v_strides[0];
      a.vn_head = append->v_strides[1];
      a.vn_dim = append->v_strides[2];
    }
  }
  hipStream_t s = as_stream(stream);
  for (int64_t r0 = 0; r0 < n_rows; r0 += kMaxRowsPerLaunch) {
    const int64_t rows = std::min<int64_t>(kMaxRowsPerLaunch, n_rows - r0);
    a.q = static_cast<const char*>(q) + r0 * q_strides[0] * esize;
    a.out = static_cast<char*>(out) + r0 * out_strides[0] * esize;
    a.tables = block_tables + r0 * table_stride;
    a.lens = context_lengths + r0;
    a.n_rows = static_cast<int>(rows);
    a.n_write = 0;
    if (append && append->n_write > r0) {
      a.n_write = static_cast<int>(std::min<int64_t>(rows, append->n_write - r0));
      a.k_new = static_cast<const char*>(append->k_new) + r0 * a.kn_row * esize;
      a.v_new = static_cast<const char*>(append->v_new) + r0 * a.vn_row * esize;
      a.write_blocks = append->write_blocks + r0;
      a.write_offsets = append->write_offsets + r0;
    }
    int rc = RLT_OK;
    switch (dtype) {
      case RLT_BFLOAT16: rc = launch_decode<bf16>(a, max_table_width, s); break;
      case RLT_FLOAT16: rc = launch_decode<f16>(a, max_table_width, s); break;
      default: rc = launch_decode<float>(a, max_table_width, s); break;
    }
    if (rc) return rc;
  }
  return RLT_OK;
}

}  // namespace

extern "C" int rlt_paged_decode(const void* q, const int64_t* q_strides, const void* key_cache,
                                const void* value_cache, const int64_t* kv_strides, const int32_t* block_tables,
                                int64_t table_stride, int64_t max_table_width, const int32_t* context_lengths,
                                void* out, const int64_t* out_strides, int64_t n_rows, int64_t num_q_heads,
                                int64_t num_kv_heads, int64_t head_dim, int64_t page_size, int64_t num_blocks,
                                float scale, int dtype, void* workspace, int64_t workspace_bytes, void* stream) {
  return paged_decode(q, q_strides, key_cache, value_cache, kv_strides, block_tables, table_stride, max_table_width,
                      context_lengths, out, out_strides, n_rows, num_q_heads, num_kv_heads, head_dim, page_size,
                      num_blocks, scale, dtype, workspace, workspace_bytes, stream, nullptr);
}

namespace rlt {
namespace {

// Device address of `scratch` on the current device, looked up once per
// device (each device holds its own copy of the array).
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch[kMaxDevices] = {};

int scratch_for_stream(void* stream, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(RLT_ELAUNCH, "rlt_paged_decode_no_alloc: no current HIP device");
  if (stream) {
    int stream_dev = -1;
    if (hipStreamGetDevice(as_stream(stream), &stream_dev) != hipSuccess)
      return fail(RLT_EINVAL, "rlt_paged_decode_no_alloc: invalid stream");
    if (stream_dev != dev)
      return fail(RLT_EINVAL, "rlt_paged_decode_no_alloc: the stream belongs to device %d, the current device is %d",
                  stream_dev, dev);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch[dev]) {
    void* ptr = nullptr;
    const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !ptr)
      return fail(RLT_ELAUNCH, "rlt_paged_decode_no_alloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                  hipGetErrorString(err));
    g_scratch[dev] = ptr;
  }
  *out = g_scratch[dev];
  return RLT_OK;
}

}  // namespace
}  // namespace rlt

extern "C" int64_t rlt_static_device_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int64_t rlt_paged_decode_no_alloc_rows_per_launch(int64_t num_q_heads, int64_t num_kv_heads,
                                                              int64_t head_dim) {
  if (num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || num_q_heads % num_kv_heads) return 0;
  // Largest row count whose workspace layout fits the scratch array (at most
  // one launch's worth of rows).
  int64_t lo = 0, hi = kMaxRowsPerLaunch;
  while (lo < hi) {
    const int64_t mid = (lo + hi + 1) / 2;
    if (workspace_bytes_for(mid, num_q_heads, num_kv_heads, head_dim) <= kNoAllocScratchBytes) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

extern "C" int rlt_paged_decode_no_alloc(const void* q, const int64_t* q_strides, const void* key_cache,
                                         const void* value_cache, const int64_t* kv_strides,
                                         const int32_t* block_tables, int64_t table_stride, int64_t max_table_width,
                                         const int32_t* context_lengths, void* out, const int64_t* out_strides,
                                         int64_t n_rows, int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                                         int64_t page_size, int64_t num_blocks, float scale, int dtype,
                                         void* stream) {
  const int esize = dtype_size(dtype);
  if (!esize) return fail(RLT_EINVAL, "rlt_paged_decode_no_alloc: unknown dtype %d", dtype);
  if (n_rows < 0) return fail(RLT_EINVAL, "rlt_paged_decode_no_alloc: n_rows is negative");
  if (num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads)
    return fail(RLT_EINVAL, "rlt_paged_decode_no_alloc: query heads must be a positive multiple of KV heads");
  if (head_dim <= 0) return fail(RLT_EINVAL, "rlt_paged_decode_no_alloc: head_dim must be positive");
  if (n_rows == 0) return RLT_OK;
  if (!q || !block_tables || !context_lengths || !out || !q_strides || !out_strides)
    return fail(RLT_EINVAL, "rlt_paged_decode_no_alloc: NULL pointer argument");
  const int64_t rows_per = rlt_paged_decode_no_alloc_rows_per_launch(num_q_heads, num_kv_heads, head_dim);
  if (rows_per < 1)
    return fail(RLT_EUNSUPPORTED,
                "rlt_paged_decode_no_alloc: one row needs %lld bytes of split partials, more than the %lld-byte "
                "static scratch; use rlt_paged_decode with a workspace",
                (long long)workspace_bytes_for(1, num_q_heads, num_kv_heads, head_dim),
                (long long)kNoAllocScratchBytes);
  void* ws = nullptr;
  if (int rc = scratch_for_stream(stream, &ws)) return rc;
  // Row chunks run in stream order and reuse the scratch: each chunk's merge
  // has finished before the next chunk's split pass overwrites the partials.
  for (int64_t r0 = 0; r0 < n_rows; r0 += rows_per) {
    const int64_t rows = std::min<int64_t>(rows_per, n_rows - r0);
    const int rc = paged_decode(static_cast<const char*>(q) + r0 * q_strides[0] * esize, q_strides, key_cache,
                                value_cache, kv_strides, block_tables + r0 * table_stride, table_stride,
                                max_table_width, context_lengths + r0, static_cast<char*>(out) + r0 * out_strides[0] * esize,
                                out_strides, rows, num_q_heads, num_kv_heads, head_dim, page_size, num_blocks, scale,
                                dtype, ws, kNoAllocScratchBytes, stream, nullptr);
    if (rc) return rc;
  }
  return RLT_OK;
}

extern "C" int rlt_paged_decode_append(
    const void* q, const int64_t* q_strides, void* key_cache, void* value_cache, const int64_t* kv_strides,
    const int32_t* block_tables, int64_t table_stride, int64_t max_table_width, const int32_t* context_lengths,
    void* out, const int64_t* out_strides, int64_t n_rows, int64_t num_q_heads, int64_t num_kv_heads,
    int64_t head_dim, int64_t page_size, int64_t num_blocks, float scale, int dtype, const void* k_new,
    const int64_t* k_new_strides, const void* v_new, const int64_t* v_new_strides, const int64_t* write_blocks,
    const int64_t* write_offsets, int64_t n_write, void* workspace, int64_t workspace_bytes, void* stream) {
  const AppendSource append{k_new, k_new_strides, v_new, v_new_strides, write_blocks, write_offsets, n_write};
  return paged_decode(q, q_strides, key_cache, value_cache, kv_strides, block_tables, table_stride, max_table_width,
                      context_lengths, out, out_strides, n_rows, num_q_heads, num_kv_heads, head_dim, page_size,
                      num_blocks, scale, dtype, workspace, workspace_bytes, stream, nullptr, &append);
}

extern "C" int rlt_paged_decode_shared_prefix(
    const void* q, const int64_t* q_strides, void* key_cache, void* value_cache, const int64_t* kv_strides,
    const int32_t* block_tables, int64_t table_stride, int64_t max_table_width, const int32_t* context_lengths,
    void* out, const int64_t* out_strides, int64_t n_rows, int64_t num_q_heads, int64_t num_kv_heads,
    int64_t head_dim, int64_t page_size, int64_t num_blocks, float scale, int dtype, const void* k_new,
    const int64_t* k_new_strides, const void* v_new, const int64_t* v_new_strides, const int64_t* write_blocks,
    const int64_t* write_offsets, int64_t n_write, const int32_t* prefix_groups, int64_t n_groups,
    int64_t n_members, int64_t n_pages, int64_t n_items, void* workspace, int64_t workspace_bytes, void* stream) {
  if (!prefix_groups) return fail(RLT_EINVAL, "rlt_paged_decode_shared_prefix: NULL prefix_groups");
  if (n_rows > kMaxRowsPerLaunch)
    return fail(RLT_EUNSUPPORTED, "rlt_paged_decode_shared_prefix: more than %d rows", kMaxRowsPerLaunch);
  if (n_groups < 1 || n_groups > n_rows)
    return fail(RLT_EINVAL, "rlt_paged_decode_shared_prefix: n_groups must be in [1, n_rows]");
  if (n_members < n_groups || n_members > n_rows)
    return fail(RLT_EINVAL, "rlt_paged_decode_shared_prefix: n_members must be in [n_groups, n_rows]");
  if (n_pages < 1 || n_pages > n_groups * max_table_width)
    return fail(RLT_EINVAL, "rlt_paged_decode_shared_prefix: n_pages must be in [1, n_groups x max_table_width]");
  // The prefix workers walk n_items x num_kv_heads items in 32-bit indices.
  if (n_items < 0 || n_items > 0x7fffffff / std::max<int64_t>(num_kv_heads, 1))
    return fail(RLT_EINVAL, "rlt_paged_decode_shared_prefix: n_items x num_kv_heads out of range");
  const PrefixHint hint{prefix_groups, n_groups, n_members, n_pages, n_items};
  const AppendSource append{k_new, k_new_strides, v_new, v_new_strides, write_blocks, write_offsets, n_write};
  return paged_decode(q, q_strides, key_cache, value_cache, kv_strides, block_tables, table_stride, max_table_width,
                      context_lengths, out, out_strides, n_rows, num_q_heads, num_kv_heads, head_dim, page_size,
                      num_blocks, scale, dtype, workspace, workspace_bytes, stream, &hint, &append);
}
