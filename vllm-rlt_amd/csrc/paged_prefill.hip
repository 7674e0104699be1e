// Packed chunked-prefill attention over paged prefixes (bottom-right causal).
//
// Sequence s owns query rows [cu[s], cu[s+1]); its keys end at its last query
// position, so chunk query i sees keys [0, len_k[s] - n_q + i].
//
// MFMA path (bf16 / fp16, head_dim 64 or 128, page 16).  A workgroup of 8
// waves owns 128 query rows of one (sequence, query head): two key groups of 4
// waves take the even and the odd 64-token key tiles (4 pages each), each wave
// 32 rows, and merge at the end.  Tiles are staged in LDS: for head_dim 128
// straight from global memory (swizzled rows, see below) with the two groups
// in ping-pong -- one group's MFMA phase beside the other's softmax phase on
// every SIMD -- otherwise through registers into padded rows.  Per tile a wave
// forms S^T = K Q^T with v_mfma_f32_32x32x16 (A = K rows from LDS, B = its 32
// q rows from registers), so every lane holds 16 keys of one query: the online
// softmax needs one exchange with the lane 32 away.  The exponentiated scores,
// rounded to the storage type, are already the B operand of O^T += V^T P^T:
// within each 16-key k-step lane half h element e holds key
// 16ks + 8(e/4) + 4h + e%4, and V^T's A operand is read from row-major V in
// that same key order with transposing LDS reads (ds_read_b64_tr_b16).  The
// running maximum moves only when a tile's maximum exceeds it by more than
// 2^kRescale, so the rescale of the accumulators is rare.  Only diagonal tiles
// are masked; tiles past a wave's last visible key are skipped.  Keys past the
// sequence re-read its last valid token, so no unwritten page is read.
// Workgroups are mapped XCD-major so one (head, sequence)'s query tiles share
// an L2 while they stream the same prefix.
//
// Other shapes expand each query row into a decode row (its own key length and
// a copy of its sequence's table row) in the workspace and run the split-K
// decode kernels -- the per-token causal rows the reference's non-FA4
// backends use for prefill.
#include <algorithm>
#include <cmath>
#include <type_traits>

#include "common.hpp"
#include "mfma.hpp"

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

// ---------------------------------------------------------------------------
// MFMA prefill kernel.

// Direct global->LDS loads.  They are written as assembly so that the
// compiler's wait analysis, which cannot tell the tile buffers apart, does not
// wait for a tile still in flight before reading the previous one: the
// kernel orders them itself with explicit vmcnt waits and barriers.  Lane l
// writes bytes [l*16, l*16 + 16) after the LDS byte address in M0.  The
// kernel uses M0 for nothing else.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_dma16(uint32_t lds_byte, uint32_t offset, uint64_t base) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds_byte), "v"(offset), "s"(base)
               : "memory", "m0");
}
#pragma clang diagnostic pop

template <typename P>
__device__ __forceinline__ uint32_t lds_address(P* p) {
  return static_cast<uint32_t>(uniform(static_cast<int>((uint32_t)(uintptr_t)(lds_u16*)(p))));
}

// Position of logical 16-byte chunk c of LDS row r (256 bytes) is
// c ^ lds_swizzle(r), with swizzle bits (b0, b1, b2, b3) = (r2, r0, r1,
// r0 ^ r1 ^ r3).  Its 4 bits are a bijection of r % 16 and its low 3 bits one
// of r % 8, so 16 (or 8) consecutive rows put one logical chunk in distinct
// 16-byte bank groups: the K reads (16 bytes per lane, one row per lane) are
// conflict-free whether a pass serves 16 lanes over 256 bytes of banks or 8
// lanes over 128.  Bits 1-2 and bits 2-3 are each a bijection of r % 4, so
// 4 consecutive rows from a multiple of 4 put an aligned chunk pair, and an
// aligned chunk quad, in distinct bank groups: the transposing V reads (4
// rows x 32 or 64 bytes per pass) are conflict-free too.  (Simpler swizzles
// that satisfy only one of the two bank models measure bank-conflict cycles
// on gfx950; this one measures none.)
__device__ __forceinline__ int lds_swizzle(int r) {
  return ((r >> 2) & 1) | ((r & 1) << 1) | (((r >> 1) & 1) << 2) | (((r ^ (r >> 1) ^ (r >> 3)) & 1) << 3);
}

constexpr int kBM = 128;  // query rows per workgroup
constexpr int kBN = 64;   // keys per tile
constexpr int kPage = 16;
constexpr float kLog2eP = 1.4426950408889634f;
// A row's running maximum is only moved (and its sums rescaled) when a tile's
// maximum exceeds it by more than this many powers of two; until then the
// exponentials stay below 2^kRescale, exact enough in fp32 sums and in the
// bf16/fp16 P operand.
constexpr float kRescale = 8.f;

bool stride16(int64_t stride, int esize) { return (stride * esize) % 16 == 0; }

struct PrefillArgs {
  const void* q;
  int64_t q_row, q_head;
  const void* k;
  const void* v;
  int64_t kv_block, kv_token, kv_head;  // elements
  const int32_t* tables;
  int64_t table_stride, width;
  const int32_t* lens;
  const int32_t* cu;
  void* out;
  int64_t o_row, o_head;
  int num_seqs, hq, hkv;
  int64_t num_blocks;
  int total_q;      // rows of q / out; cu_seqlens_q entries are clamped to it
  int ranked;       // work-list mode (see the kernel)
  int max_qt;       // direct mode: query tiles per sequence bound
  float qscale;     // |scale| * log2(e)
  uint32_t q_sign;  // 0x80008000 negates q (a negative scale), else 0
};

// Rows [row0, row0 + nq) of sequence s, clamped to [0, total_q] so that an
// inconsistent cu_seqlens_q cannot index outside q and out.
__device__ __forceinline__ void seq_rows(const PrefillArgs& a, int s, int& row0, int& nq) {
  row0 = min(max(a.cu[s], 0), a.total_q);
  nq = min(max(a.cu[s + 1], row0), a.total_q) - row0;
}

// Work list.  A work item is (sequence, query tile of kBM rows, query head).
// Ranked mode (few sequences, hq a multiple of the XCD count): every workgroup
// ranks the sequences by the key tiles of their last query tile, longest
// first.  Workgroup b runs on XCD b % 8 (the dispatcher's round-robin) and is
// that XCD's (b / 8)-th item; each XCD's queue walks the ranked sequences, for
// each its heads h == xcd (mod 8), and for each head the query tiles, last
// (longest) first.  So the dispatcher hands out the longest items first on
// every XCD (greedy LPT), and the query tiles that stream one (sequence,
// head)'s prefix run back to back on one XCD, sharing its L2.  Direct mode:
// item = (seq * max_qt + t) * hq + head; empty items exit.
constexpr int kXcds = 8;
constexpr int kRankSeqs = 512;  // ranked mode: at most this many sequences
constexpr int kTablePages = 4096;  // page ids staged in LDS per workgroup (65536 keys)

template <typename T, int D, bool DMA>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) void paged_prefill_mfma_kernel(PrefillArgs a) {
  using Ops = MfmaOps<T>;
  using V8 = typename Ops::V8;
  constexpr int KSTEPS = D / 16;  // q.k k-steps
  constexpr int DTILES = D / 32;  // output column tiles
  // DMA (head_dim 128, page table within kTablePages): K/V tiles go from global memory straight into LDS
  // (global_load_lds_dwordx4), unpadded 256-byte rows whose 16-byte chunks are
  // XOR-swizzled (chunk c of row r sits at position c ^ lds_swizzle(r)) so the
  // K reads and the transposing V reads stay free of bank conflicts.  Other
  // head sizes stage through registers into padded rows: K, a quarter-wave's
  // 16-byte reads of 16 rows land in distinct bank groups when the stride is
  // an odd multiple of 16 bytes; V, the transposing read takes 4 rows x 64
  // bytes per half-wave, so the stride is 64 (mod 256) bytes.
  static_assert(!DMA || D == 128, "direct-to-LDS staging is laid out for head_dim 128");
  constexpr int KROW = DMA ? D : D + 8;
  constexpr int VROW = DMA ? D : D + 32;
  constexpr int KT = kBN * KROW, VT = kBN * VROW;  // elements per K / V tile
  constexpr int CHUNKS = D / 8;  // 16-byte chunks per token row
  constexpr int TOKENS_PER_PASS = 256 / CHUNKS;
  constexpr int PAGES_PER_PASS = TOKENS_PER_PASS / kPage;
  constexpr int PASSES = kBN / TOKENS_PER_PASS;
  constexpr int TILES_PER_CHUNK = 64 / (kBN / kPage);  // table entries arrive 64 at a time
  constexpr int MERGE_FLOATS = 2 + 16 * DTILES;        // m, l, accumulators per lane
  static_assert(kBN % TOKENS_PER_PASS == 0 && TOKENS_PER_PASS % kPage == 0, "tile loads");
  static_assert(64 % CHUNKS == 0 && (64 / CHUNKS) <= kPage, "a wave's loads stay in one page");
  static_assert(4 * 64 * MERGE_FLOATS * 4 <= 4 * (KT + VT) * 2, "merge fits in the tile buffers");
  static_assert(4 * kRankSeqs * 4 <= 4 * (KT + VT) * 2, "ranking fits in the tile buffers");
  // Two key groups, each with two K and V tile buffers; reused for ranking
  // before the tile loop and for the key-group merge after it.
  __shared__ __align__(16) uint16_t lds[4 * (KT + VT)];
  // Page ids of the workgroup's key range (direct-to-LDS path), staged once so
  // that the tile loop reads them from LDS rather than global memory.
  __shared__ int32_t page_ids[DMA ? kTablePages : 1];

  const int tid = threadIdx.x;
  int seq, t, h;
  if (a.ranked) {
    int* s_qt = reinterpret_cast<int*>(lds);  // [kRankSeqs] query tiles per sequence
    int* s_cost = s_qt + kRankSeqs;            // key tiles of its last query tile
    int* s_order = s_cost + kRankSeqs;         // sequences, longest first
    int* s_scan = s_order + kRankSeqs;         // query tiles of the ranked sequences, prefix sums
    const int ns = a.num_seqs;
    if (tid < ns) {
      int r0, nq_s;
      seq_rows(a, tid, r0, nq_s);
      const int keys = static_cast<int>(min<int64_t>(a.lens[tid], a.width * kPage));
      s_qt[tid] = (nq_s + kBM - 1) / kBM;
      s_cost[tid] = keys > 0 ? (keys + kBN - 1) / kBN : 0;
    }
    __syncthreads();
    if (tid < ns) {
      const int c = s_cost[tid];
      int r = 0;
      for (int q = 0; q < ns; ++q) {
        const int cq = s_cost[q];
        r += (cq > c) || (cq == c && q < tid);
      }
      s_order[r] = tid;
    }
    __syncthreads();
    s_scan[tid] = tid < ns ? s_qt[s_order[tid]] : 0;
    __syncthreads();
    for (int off = 1; off < ns; off <<= 1) {  // inclusive scan of the ns ranked entries
      const int v = tid >= off ? s_scan[tid - off] : 0;
      __syncthreads();
      s_scan[tid] += v;
      __syncthreads();
    }
    // XCD b % 8 owns heads h == b % 8 (mod 8): hpx of them per sequence.
    const int hpx = a.hq / kXcds;
    const int xcd = static_cast<int>(blockIdx.x) % kXcds;
    const int pos = static_cast<int>(blockIdx.x) / kXcds;
    // Ranked sequence r covers positions [hpx * scan[r-1], hpx * scan[r]).
    int lo = 0, hi = ns;  // first r with hpx * scan[r] > pos
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (hpx * s_scan[mid] > pos) hi = mid;
      else lo = mid + 1;
    }
    if (lo >= ns) return;
    seq = s_order[lo];
    const int qt = s_qt[seq];
    const int local = pos - hpx * (lo > 0 ? s_scan[lo - 1] : 0);
    h = xcd + kXcds * (local / qt);
    t = qt - 1 - local % qt;
    __syncthreads();  // ranking arrays are dead before the tiles reuse them
  } else {
    const int w = blockIdx.x;
    h = w % a.hq;
    seq = w / a.hq / a.max_qt;
    t = w / a.hq % a.max_qt;
    if (seq >= a.num_seqs) return;
  }
  int row0, nq;
  seq_rows(a, seq, row0, nq);
  if (t * kBM >= nq) return;
  const int64_t max_len = a.width * kPage;
  const int len_k = static_cast<int>(min<int64_t>(a.lens[seq], max_len));
  const int prefix = len_k - nq;
  const int kvh = h / (a.hq / a.hkv);
  const int qt0 = t * kBM;                         // first chunk row of the workgroup
  const int wg_last_row = min(qt0 + kBM, nq) - 1;  // last chunk row of the workgroup
  const int wg_keys = prefix + wg_last_row + 1;    // <= len_k, so len_k >= 1 below
  if (wg_keys <= 0) {
    // No row of the tile sees a key (a context shorter than its chunk): the
    // rows are written as zeros, as a row that sees no key is below.
    constexpr int CH = D / 8;  // 16-byte chunks per row
    const int rows = wg_last_row + 1 - qt0;
    for (int i = tid; i < rows * CH; i += 512) {
      T* orow = static_cast<T*>(a.out) + (row0 + qt0 + i / CH) * a.o_row + static_cast<int64_t>(h) * a.o_head;
      *reinterpret_cast<u32x4*>(orow + (i % CH) * 8) = u32x4{0u, 0u, 0u, 0u};
    }
    return;
  }
  const int ntiles = (wg_keys + kBN - 1) / kBN;

  // Waves 0-3 take key tiles 0, 2, 4, ...; waves 4-7 tiles 1, 3, 5, ...; wave
  // w and w + 4 own the same 32 query rows and merge at the end.
  const int lane = tid & 63;
  const int wave = uniform(tid >> 6);  // scalar, so per-wave conditions branch on SCC
  const int kg = wave >> 2;   // key group
  const int qw = wave & 3;    // query wave within the group
  const int gtid = tid & 255; // thread within the key group
  const int half = lane >> 5;
  const int col = lane & 31;
  const int wave_row0 = qt0 + qw * 32;  // chunk row of the wave's column 0
  const bool wave_live = wave_row0 < nq;
  const int wave_last_key = prefix + min(wave_row0 + 31, nq - 1);
  const int my_row = wave_row0 + col;
  const bool row_valid = my_row < nq;
  const int my_key_limit = prefix + my_row;  // last visible key of this lane's query
  uint16_t* const group_lds = lds + kg * 2 * (KT + VT);  // buffer b: K at b*(KT+VT), V after it

  // Q^T B-operands: lane holds dims [ks*16 + half*8, +8) of query my_row.
  u32x4 qb[KSTEPS];
  {
    const int r = row0 + min(my_row, nq - 1);
    const T* qrow = static_cast<const T*>(a.q) + r * a.q_row + static_cast<int64_t>(h) * a.q_head;
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) qb[ks] = *reinterpret_cast<const u32x4*>(qrow + ks * 16 + half * 8) ^ a.q_sign;
  }

  // Tile loads: pass i of tile j reads page 4j + i*PAGES_PER_PASS + ld_page,
  // the same page for the whole wave, so its table entry and base address are
  // scalar and each lane adds a 32-bit offset.  Table entries arrive 64 at a
  // time (one per lane, a chunk ahead of use) and are picked with readlane.
  // Slots past the sequence's last key re-read its last key (masked, but
  // finite: no unwritten slot is read); out-of-range ids read block 0.
  const int32_t* trow = a.tables + static_cast<int64_t>(seq) * a.table_stride;
  const char* kbase = static_cast<const char*>(a.k) + static_cast<int64_t>(kvh) * a.kv_head * sizeof(T);
  const char* vbase = static_cast<const char*>(a.v) + static_cast<int64_t>(kvh) * a.kv_head * sizeof(T);
  const int64_t block_bytes = a.kv_block * static_cast<int64_t>(sizeof(T));
  const uint32_t nblocks = static_cast<uint32_t>(a.num_blocks);
  const int ld_tok = gtid / CHUNKS;
  const int ld_page = uniform(ld_tok / kPage);
  const int ld_slot = ld_tok % kPage;
  const int ld_chunk = gtid % CHUNKS;
  const int last_page = (len_k - 1) / kPage;
  const int last_slot = (len_k - 1) % kPage;
  const uint32_t off_full = static_cast<uint32_t>((ld_slot * a.kv_token + ld_chunk * 8) * sizeof(T));
  const uint32_t off_last = static_cast<uint32_t>((min(ld_slot, last_slot) * a.kv_token + ld_chunk * 8) * sizeof(T));
  auto table_chunk = [&](int c) { return trow[min(c * 64 + lane, last_page)]; };
  int32_t tab_cur = table_chunk(0), tab_next = table_chunk(1);
  u32x4 kreg[PASSES], vreg[PASSES];
  // Direct-to-LDS staging: wave qw of a key group fills page 4j + qw of tile
  // j, rows 16qw .. 16qw+15 of the K and V tiles, four rows per instruction.
  // Lane l writes row 16qw + 4i + l/16 at chunk position l%16, so it fetches
  // that token's logical chunk (l%16) ^ lds_swizzle(4i + l/16).
  auto dma_offset = [&](int ln, int i, int slot_limit) {
    const int slot = 4 * i + (ln >> 4);
    const int chunk = (ln & 15) ^ lds_swizzle(slot);
    return static_cast<uint32_t>((min(slot, slot_limit) * a.kv_token + chunk * 8) * sizeof(T));
  };
  // Page p of the sequence (p < 4 * ntiles, which the host keeps within
  // kTablePages); past the last valid page the last page's id.  page_slot
  // reads the entry into a vector register (its use can come a phase later),
  // page_id makes it scalar.
  auto page_slot = [&](int p) -> int32_t { return page_ids[min(p, kTablePages - 1)]; };
  auto page_id = [&](int p) -> uint32_t { return static_cast<uint32_t>(uniform(page_slot(p))); };
  // Page p of tile j that wave qw stages; tiles past the last are clamped.
  auto tile_page = [&](int j) { return min(j, ntiles - 1) * (kBN / kPage) + qw; };
  // Per-lane source offsets of the four staging instructions of a page, and
  // of the sequence's last page (whose slots past the last key re-read it).
  uint32_t dma_full[4], dma_last[4];
  if constexpr (DMA) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      dma_full[i] = dma_offset(lane, i, kPage - 1);
      dma_last[i] = dma_offset(lane, i, last_slot);
    }
  }
  // One staging half: the K (which 0) or V (which 1) rows of page p (id
  // `id`) bound for buffer b of the wave's key group, where wave qw fills
  // rows 16qw .. 16qw + 15; issue(i) sends rows 16qw + 4i .. + 3.
  struct StageHalf {
    uint32_t dst;   // LDS byte address of the wave's rows
    uint64_t src;   // page base in global memory
    bool last;      // page p is the sequence's last
  };
  auto stage_half = [&](int p, uint32_t id, int b, int which) -> StageHalf {
    const int64_t blk = id < nblocks ? id : 0;
    const char* src = (which ? vbase : kbase) + blk * block_bytes;
    return {lds_address(group_lds + b * (KT + VT) + which * KT + qw * 16 * KROW),
            static_cast<uint64_t>(uniform64(reinterpret_cast<int64_t>(src))), p >= last_page};
  };
  auto stage_issue = [&](const StageHalf& h, int i) __attribute__((always_inline)) {
    lds_dma16(h.dst + i * 4 * KROW * sizeof(uint16_t), h.last ? dma_last[i] : dma_full[i], h.src);
  };
  auto issue_half = [&](int p, uint32_t id, int b, int which) __attribute__((always_inline)) {
    const StageHalf h = stage_half(p, id, b, which);
#pragma unroll
    for (int i = 0; i < 4; ++i) stage_issue(h, i);
  };
  // Tiles of a key group arrive 2 apart: the group's first tile of chunk c
  // is 16c + kg.
  auto load_tile = [&](int j) {
    if (j % TILES_PER_CHUNK == kg && j >= TILES_PER_CHUNK) {
      tab_cur = tab_next;
      tab_next = table_chunk(j / TILES_PER_CHUNK + 1);
    }
#pragma unroll
    for (int i = 0; i < PASSES; ++i) {
      const int p = j * (kBN / kPage) + i * PAGES_PER_PASS + ld_page;
      const uint32_t id = static_cast<uint32_t>(__builtin_amdgcn_readlane(tab_cur, p % 64));
      const int64_t blk = id < nblocks ? id : 0;
      const uint32_t off = p >= last_page ? off_last : off_full;
      kreg[i] = *reinterpret_cast<const u32x4*>(kbase + blk * block_bytes + off);
      vreg[i] = *reinterpret_cast<const u32x4*>(vbase + blk * block_bytes + off);
    }
  };

  // V^T A-operand reads: within k-step ks, lane (dim i, half kh) needs keys
  // 16ks + 4kh + {0..3} (elements 0-3) and 16ks + 8 + 4kh + {0..3} (4-7) --
  // the key order of the P^T B operand below.
  const int grp = lane >> 4, gl = lane & 15;
  const int tr_off = (4 * (grp >> 1) + (gl >> 2)) * VROW + 16 * (grp & 1) + 4 * (gl & 3);
  // Swizzled layout: a lane's K row is col (+32), its logical chunk 2ks + half;
  // its V rows are rlo and rlo + 8, logical chunk 4c + 2(grp&1) + (gl&3)/2,
  // 8-byte half gl&1 (rows 16ks + r keep r's swizzle).
  // In bytes, with sw = lds_swizzle(row): chunk (2ks + half) ^ sw of K row
  // col sits at 32 (ks ^ sw/2) + 16 (half ^ sw%2); V chunk (4c + m0) ^ sw of
  // row rlo (and likewise rlo + 8, with its own swizzle) at 64 (c ^ sw/4) +
  // 16 (m0 ^ sw%4).
  // So each read is ((step << 5 or 6) ^ key) + base, one v_xad_u32.
  const int kswz = lds_swizzle(col);
  const int k_key = (kswz >> 1) << 5;
  const int k_base = col * KROW * 2 + 16 * (half ^ (kswz & 1));
  const int rlo = 4 * (grp >> 1) + (gl >> 2);
  const int m0 = 2 * (grp & 1) + ((gl & 3) >> 1);
  const int v_key = (lds_swizzle(rlo) >> 2) << 6;
  const int v_key_hi = (lds_swizzle(rlo + 8) >> 2) << 6;
  const int v_base_lo = rlo * KROW * 2 + 16 * (m0 ^ (lds_swizzle(rlo) & 3)) + 8 * (gl & 1);
  const int v_base_hi = (rlo + 8) * KROW * 2 + 16 * (m0 ^ (lds_swizzle(rlo + 8) & 3)) + 8 * (gl & 1);

  f32x16 acc_o[DTILES];
#pragma unroll
  for (int c = 0; c < DTILES; ++c) acc_o[c] = f32x16{};
  float m = -INFINITY;
  // This lane's share of its query's row sum: the keys it holds, summed from
  // the rounded P that also weights V (v_dot2 against ones, next to the P V
  // MFMAs; the lane 32 away holds the other keys).
  float lsum = 0.f;

  // Whether the wave computes tile j: it exists and holds a key visible to
  // one of the wave's queries.  Once false it stays false for later tiles.
  auto active = [&](int j) { return j < ntiles && wave_live && j * kBN <= wave_last_key; };
  // Register-staged path (padded rows): S^T = K Q^T for the tile's two 32-key
  // halves, as two interleaved MFMA chains.
  auto scores = [&](int b, f32x16 (&sacc)[2]) __attribute__((always_inline)) {
    const uint16_t* k_lds = group_lds + b * (KT + VT);
    f32x16 c[2] = {{}, {}};
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const u32x4 kv = *reinterpret_cast<const u32x4*>(&k_lds[(hh * 32 + col) * KROW + ks * 16 + half * 8]);
        c[hh] = Ops::mma(as_v8<V8>(kv), as_v8<V8>(qb[ks]), c[hh]);
      }
    sacc[0] = c[0];
    sacc[1] = c[1];
  };
  // Online softmax of tile key0: mask (diagonal tiles and the chunk's last
  // rows only), tile maximum, exponentials.  Leaves P^T in fp32 in sacc; the
  // P V step rounds it to T one 16-key k-step at a time, next to that step's
  // MFMAs, where the VALU work hides under them instead of lengthening this
  // phase.  Element r of half hh holds key
  // key0 + 32hh + 8(r/4) + 4half + r%4.  When the running maximum moves it
  // returns true with the accumulators' factor in corr, which the row sum takes
  // here and acc_o in the P V step.  hook(0) .. hook(7) run
  // at fixed points along the way (the staging loads of the direct-to-LDS
  // path, spread out so that they never queue up behind one another).
  auto softmax = [&](int key0, f32x16 (&sacc)[2], float& corr, auto&& hook)
                     __attribute__((always_inline)) -> bool {
    float tmax = -INFINITY;
    if (uniform(key0 + kBN - 1 > prefix + wave_row0 || wave_row0 + 31 >= nq)) {
      const int lim = row_valid ? my_key_limit - key0 - 4 * half : -1;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float x = (hh * 32 + (r / 4) * 8 + (r % 4) > lim) ? -INFINITY : sacc[hh][r];
          sacc[hh][r] = x;
          tmax = fmaxf(tmax, x);
        }
    } else {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int r = 0; r < 16; ++r) tmax = fmaxf(tmax, sacc[hh][r]);
    }
    hook(0);
    tmax = max_across_halves(tmax) * a.qscale;
    hook(1);
    const bool rescale = __builtin_amdgcn_ballot_w64(tmax > m + kRescale) != 0;
    if (rescale) {
      const float mn = fmaxf(m, tmax);
      corr = (mn == -INFINITY) ? 1.f : fast_exp2(m - mn);
      m = mn;
      lsum *= corr;
    }
    hook(2);
    // p = 2^(s * scale * log2(e) - m); a lane that has seen no key yet has
    // only -inf scores, which give 0 against any finite offset.
    const float mb = (m == -INFINITY) ? 0.f : m;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        sacc[hh][r] = fast_exp2(fmaf(sacc[hh][r], a.qscale, -mb));
        if (r == 5) hook(3 + 3 * hh);
        if (r == 11) hook(4 + 3 * hh);
      }
      if (hh == 0) hook(5);
    }
    return rescale;
  };
  // Register-staged path: O^T = O^T * corr (when softmax() moved the maximum)
  // + V^T P^T over the tile's four 16-key k-steps.  Each step packs its P^T
  // operand to T and adds exactly those rounded values to the row sum (v_dot2
  // against ones).
  auto accumulate = [&](int b, const f32x16 (&pt)[2], bool rescale, float corr) __attribute__((always_inline)) {
    if (rescale) {
#pragma unroll
      for (int c = 0; c < DTILES; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc_o[c][r] *= corr;
    }
    const uint16_t* v_lds = group_lds + b * (KT + VT) + KT;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      u32x4 pb;
#pragma unroll
      for (int e = 0; e < 4; ++e) pb[e] = Ops::pack2(pt[ks / 2][(ks % 2) * 8 + 2 * e], pt[ks / 2][(ks % 2) * 8 + 2 * e + 1]);
#pragma unroll
      for (int c = 0; c < DTILES; ++c) {
        const uint16_t* vlo = &v_lds[tr_off + ks * 16 * VROW + c * 32];
        const u32x2 lo = lds_read_tr(vlo);
        const u32x2 hi = lds_read_tr(vlo + 8 * VROW);
        const u32x4 va = {lo[0], lo[1], hi[0], hi[1]};
        acc_o[c] = Ops::mma(as_v8<V8>(va), as_v8<V8>(pb), acc_o[c]);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) lsum = Ops::sum2(pb[e], lsum);
    }
  };
  // Direct-to-LDS path: one MFMA phase as a single stream in issue order --
  // the P V MFMAs of tile j - 2 (k = 0..15: k-step k / 4, output tile k % 4),
  // then the S MFMAs of tile j (k = 16..31: k-step (k - 16) / 2, key half
  // k % 2).  Each MFMA's A operand (two transposing V reads, or one K read) is
  // read kStreamAhead MFMAs before it, and every read, pack and MFMA is pinned
  // in that order: left to itself the scheduler groups the reads of several
  // k-steps, and each MFMA's wait then covers reads it does not use.  P^T of
  // k-step ks is rounded to T one k-step early and added to the row sum
  // (v_dot2 against ones) after that step's MFMAs.
  constexpr int kStreamAhead = 4;
  auto mfma_phase = [&](auto pv_tag, auto s_tag, int b_pv, int b_s, f32x16 (&sacc)[2], bool rescale, float corr)
                        __attribute__((always_inline)) {
    constexpr bool PV = decltype(pv_tag)::value, S = decltype(s_tag)::value;
    constexpr int K0 = PV ? 0 : 16, K1 = S ? 32 : 16, R = kStreamAhead + 1;
    if (PV && rescale) {
#pragma unroll
      for (int c = 0; c < DTILES; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc_o[c][r] *= corr;
    }
    const char* v_rows = reinterpret_cast<const char*>(group_lds + b_pv * (KT + VT) + KT);
    const char* k_rows = reinterpret_cast<const char*>(group_lds + b_s * (KT + VT));
    const int vk = v_key, vk_hi = v_key_hi, kk = k_key;
    auto read = [&](int k) __attribute__((always_inline)) {
      if (k < 16) {
        const int ks = k >> 2, c = k & 3;
        const char* rows = v_rows + ks * 16 * VROW * 2;
        const u32x2 lo = lds_read_tr(reinterpret_cast<const uint16_t*>(rows + (((c << 6) ^ vk) + v_base_lo)));
        const u32x2 hi = lds_read_tr(reinterpret_cast<const uint16_t*>(rows + (((c << 6) ^ vk_hi) + v_base_hi)));
        return u32x4{lo[0], lo[1], hi[0], hi[1]};
      }
      const int ks = (k - 16) >> 1, hh = k & 1;
      return *reinterpret_cast<const u32x4*>(k_rows + hh * 32 * KROW * 2 + (((ks << 5) ^ kk) + k_base));
    };
    auto pack = [&](int ks) __attribute__((always_inline)) {
      u32x4 pb;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        pb[e] = Ops::pack2(sacc[ks / 2][(ks % 2) * 8 + 2 * e], sacc[ks / 2][(ks % 2) * 8 + 2 * e + 1]);
      return pb;
    };
    u32x4 ring[R];
    u32x4 pb[4];
    f32x16 c[2] = {{}, {}};
#pragma unroll
    for (int k = K0; k < K0 + kStreamAhead; ++k) {
      ring[k % R] = read(k);
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (PV) pb[0] = pack(0);
#pragma unroll
    for (int k = K0; k < K1; ++k) {
      if (k + kStreamAhead < K1) ring[(k + kStreamAhead) % R] = read(k + kStreamAhead);
      __builtin_amdgcn_sched_barrier(0);
      if (k < 16) {
        acc_o[k & 3] = Ops::mma(as_v8<V8>(ring[k % R]), as_v8<V8>(pb[k >> 2]), acc_o[k & 3]);
        if ((k & 3) == 1 && k < 12) pb[(k >> 2) + 1] = pack((k >> 2) + 1);
        if ((k & 3) == 3) {
#pragma unroll
          for (int e = 0; e < 4; ++e) lsum = Ops::sum2(pb[k >> 2][e], lsum);
        }
      } else {
        const int ks = (k - 16) >> 1, hh = k & 1;
        c[hh] = Ops::mma(as_v8<V8>(ring[k % R]), as_v8<V8>(qb[ks]), c[hh]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (S) {
      sacc[0] = c[0];
      sacc[1] = c[1];
    }
  };
  const int niter = (ntiles + 1) / 2;  // tiles per key group (the last of group 1 may not exist)

  if constexpr (DMA) {
    const int fill = min(4 * ntiles, kTablePages);
    for (int i = tid; i < fill; i += 512) page_ids[i] = trow[min(i, last_page)];
    {
      // The V tile of buffer 1, which the first MFMA phase reads (times P = 0)
      // before any tile is staged there: zero, so no stale NaN reaches acc_o.
      u32x4* vz = reinterpret_cast<u32x4*>(group_lds + (KT + VT) + KT);
      const u32x4 zero = {0u, 0u, 0u, 0u};
      for (int i = tid & 255; i < VT / 8; i += 256) vz[i] = zero;
    }
    __syncthreads();
    // Ping-pong.  Iteration t of key group g handles tile j = 2t + g in two
    // phases: an MFMA phase (P V of tile j - 2, then S of tile j) and a
    // softmax phase (tile j's exponentials, with the staging DMA of K of tile
    // j + 4 and V of tile j + 2 into the buffers the MFMA phase just finished
    // reading, issued one instruction at a time between the softmax's steps).
    // Group 1 runs one phase behind group 0 and every phase ends at a
    // workgroup barrier, so on each SIMD one wave issues MFMAs while its
    // partner (same query rows, other key group) runs the softmax and the
    // loads.  Both groups pass 2 * niter + 2 barriers.
    //
    // Loads: every softmax phase issues exactly 8 (4 K, then 4 V; past the
    // last tile they re-read it into buffers no later phase reads), so at the
    // barrier before MFMA phase t, vmcnt(8) completes everything issued
    // before the previous softmax phase -- the K of tile j and V of tile j - 2
    // that this phase reads (loads return in order).  The prologue issues
    // K(j), V(j), K(j + 2): vmcnt(8) there completes K(j).  Page ids run down
    // a chain (V <- K <- next), so each phase reads one new id from LDS, a
    // phase before its use.  No load here is a bare L2 prefetch of a later
    // tile: with in-order completion, the barrier's vmcnt would wait for its
    // HBM latency (a prefetch of tile j + 6 measured 8% slower overall).
    auto load_barrier = [&]() {
      __builtin_amdgcn_sched_barrier(0);
      asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)\n\ts_barrier" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
    };
    auto phase_barrier = [&]() {
      __builtin_amdgcn_sched_barrier(0);
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
    };
    issue_half(tile_page(kg), page_id(tile_page(kg)), 0, 0);
    issue_half(tile_page(kg), page_id(tile_page(kg)), 0, 1);
    issue_half(tile_page(kg + 2), page_id(tile_page(kg + 2)), 1, 0);
    __builtin_amdgcn_sched_barrier(0);
    uint32_t id_v = page_id(tile_page(kg + 2));        // V of tile j + 2
    uint32_t id_k = page_id(tile_page(kg + 4));        // K of tile j + 4
    int32_t next_k = page_slot(tile_page(kg + 6));     // K of tile j + 6
    if (kg == 1) phase_barrier();
    f32x16 sacc[2] = {{}, {}};  // P of tile j - 2: none before the first phase
    bool rescale = false;
    float corr = 1.f;
    for (int t = 0; t <= niter; ++t) {
      const int j = 2 * t + kg;
      const int P = t & 1;
      load_barrier();
      __builtin_amdgcn_s_setprio(1);
      // One site for the whole phase (accumulators updated on two paths would
      // be given two register sets).  At t = 0 the P V half multiplies a
      // zeroed V buffer by P = 0; past the wave's last tile, and at t = niter,
      // the S half's scores are never used.
      if (t == 0 ? active(j) : active(j - 2))
        mfma_phase(std::true_type{}, std::true_type{}, 1 - P, P, sacc, rescale, corr);
      __builtin_amdgcn_s_setprio(0);
      if (t == niter) break;
      phase_barrier();
      const uint32_t id_next = static_cast<uint32_t>(uniform(next_k));
      next_k = page_slot(tile_page(j + 8));
      const StageHalf hk = stage_half(tile_page(j + 4), id_k, P, 0);
      const StageHalf hv = stage_half(tile_page(j + 2), id_v, 1 - P, 1);
      auto stage = [&](int n) __attribute__((always_inline)) {
        __builtin_amdgcn_sched_barrier(0);
        if (n < 4) stage_issue(hk, n);
        else stage_issue(hv, n - 4);
        __builtin_amdgcn_sched_barrier(0);
      };
      if (active(j)) {
        rescale = softmax(j * kBN, sacc, corr, stage);
      } else {
#pragma unroll
        for (int n = 0; n < 8; ++n) stage(n);
      }
      id_v = id_k;
      id_k = id_next;
    }
    if (kg == 0) phase_barrier();
    // Every staging load has landed and every tile read is done before the
    // merge reuses LDS.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  } else {
    // Iteration it computes tile j = 2it + kg from buffer it&1 while tile
    // j + 2 waits in registers; tile j + 2 then goes to the other buffer
    // (whose tile every wave finished before the previous barrier), and one
    // barrier per tile publishes it.
    auto store_tile = [&](int b) {
      uint16_t* kb = group_lds + b * (KT + VT);
      uint16_t* vb = kb + KT;
#pragma unroll
      for (int i = 0; i < PASSES; ++i) {
        const int tok = i * TOKENS_PER_PASS + ld_tok;
        *reinterpret_cast<u32x4*>(&kb[tok * KROW + ld_chunk * 8]) = kreg[i];
        *reinterpret_cast<u32x4*>(&vb[tok * VROW + ld_chunk * 8]) = vreg[i];
      }
    };
    if (kg < ntiles) {
      load_tile(kg);
      store_tile(0);
    }
    if (kg + 2 < ntiles) load_tile(kg + 2);
    __syncthreads();
    for (int it = 0; it < niter; ++it) {
      const int j = 2 * it + kg;
      if (active(j)) {
        f32x16 sacc[2];
        float corr = 1.f;
        scores(it & 1, sacc);
        const bool rescale = softmax(j * kBN, sacc, corr, [](int) {});
        accumulate(it & 1, sacc, rescale, corr);
      }
      if (j + 2 < ntiles) store_tile((it + 1) & 1);
      __syncthreads();
      if (j + 4 < ntiles) load_tile(j + 4);
    }
  }

  // Merge the key groups: group 1 hands (m, l, acc) to group 0 through LDS,
  // laid out [query wave][value][lane] (the last barrier ordered every tile
  // read before these writes).
  float* xs = reinterpret_cast<float*>(lds) + qw * MERGE_FLOATS * 64 + lane;
  if (kg == 1) {
    xs[0] = m;
    xs[64] = lsum;
#pragma unroll
    for (int c = 0; c < DTILES; ++c)
#pragma unroll
      for (int r = 0; r < 16; ++r) xs[(2 + c * 16 + r) * 64] = acc_o[c][r];
  }
  __syncthreads();
  if (kg == 1) return;
  float total;  // the row's sum of P
  {
    const float m1 = xs[0];
    const float mm = fmaxf(m, m1);
    const float c0 = (m == -INFINITY) ? 0.f : fast_exp2(m - mm);
    const float c1 = (m1 == -INFINITY) ? 0.f : fast_exp2(m1 - mm);
    total = lsum * c0 + xs[64] * c1;
    total += __shfl_xor(total, 32, 64);  // the two halves hold the row's two key halves
#pragma unroll
    for (int c = 0; c < DTILES; ++c)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc_o[c][r] = acc_o[c][r] * c0 + xs[(2 + c * 16 + r) * 64] * c1;
  }

  if (!wave_live || !row_valid) return;
  const float inv = total > 0.f ? 1.f / total : 0.f;  // a row that sees no key is written as zeros
  T* orow = static_cast<T*>(a.out) + (row0 + my_row) * a.o_row + static_cast<int64_t>(h) * a.o_head;
#pragma unroll
  for (int c = 0; c < DTILES; ++c)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const u32x2 w2 = {Ops::pack2(acc_o[c][g * 4] * inv, acc_o[c][g * 4 + 1] * inv),
                        Ops::pack2(acc_o[c][g * 4 + 2] * inv, acc_o[c][g * 4 + 3] * inv)};
      *reinterpret_cast<u32x2*>(orow + c * 32 + g * 8 + half * 4) = w2;
    }
}

int64_t expand_bytes(int64_t total_q, int64_t width) {
  const int64_t lens = (total_q * 4 + 255) / 256 * 256;
  const int64_t tables = (total_q * std::max<int64_t>(width, 1) * 4 + 255) / 256 * 256;
  return lens + tables;
}

}  // namespace
}  // namespace rlt

using namespace rlt;

namespace rlt {
namespace {
// Shapes the MFMA kernel takes (it then needs no workspace), given 16-byte
// aligned q / out / cache rows.
bool mfma_shape(int64_t head_dim, int64_t page_size, int dtype) {
  return (dtype == RLT_BFLOAT16 || dtype == RLT_FLOAT16) && (head_dim == 64 || head_dim == 128) && page_size == kPage;
}
int64_t fallback_workspace(int64_t total_q, int64_t width, int64_t hq, int64_t hkv, int64_t d) {
  return expand_bytes(total_q, width) + rlt_paged_decode_workspace_bytes(total_q, hq, hkv, d);
}
}  // namespace
}  // namespace rlt

extern "C" int64_t rlt_paged_prefill_workspace_bytes(int64_t total_q, int64_t num_seqs, int64_t max_table_width,
                                                     int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                                                     int64_t page_size, int dtype) {
  if (total_q <= 0 || num_seqs <= 0) return 0;
  if (mfma_shape(head_dim, page_size, dtype)) return 0;
  return fallback_workspace(total_q, max_table_width, num_q_heads, num_kv_heads, head_dim);
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
  if (!q || !key_cache || !value_cache || !out || !q_strides || !kv_strides || !out_strides)
    return fail(RLT_EINVAL, "rlt_paged_prefill: NULL pointer argument");
  if (num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads)
    return fail(RLT_EINVAL, "rlt_paged_prefill: query heads must be a positive multiple of KV heads");
  if (head_dim <= 0 || page_size <= 0 || num_blocks <= 0)
    return fail(RLT_EINVAL, "rlt_paged_prefill: head_dim, page_size and num_blocks must be positive");
  if (!(scale != 0.f) || !std::isfinite(scale))
    return fail(RLT_EINVAL, "rlt_paged_prefill: scale must be finite and nonzero");

  const int esize = dtype_size(dtype);
  const bool mfma_ok = mfma_shape(head_dim, page_size, dtype) && q_strides[2] == 1 && out_strides[2] == 1 && kv_strides[3] == 1 &&
                       aligned16(q) && aligned16(out) && aligned16(key_cache) && aligned16(value_cache) &&
                       stride16(q_strides[0], esize) && stride16(q_strides[1], esize) &&
                       stride16(out_strides[0], esize) && stride16(out_strides[1], esize) &&
                       stride16(kv_strides[0], esize) && stride16(kv_strides[1], esize) &&
                       stride16(kv_strides[2], esize) && max_table_width > 0 && num_q_heads <= 4096 &&
                       kv_strides[1] >= 0 && kv_strides[1] * esize * page_size < (int64_t(1) << 31);
  if (mfma_ok) {
    PrefillArgs p{};
    p.q = q;
    p.q_row = q_strides[0];
    p.q_head = q_strides[1];
    p.k = key_cache;
    p.v = value_cache;
    p.kv_block = kv_strides[0];
    p.kv_token = kv_strides[1];
    p.kv_head = kv_strides[2];
    p.tables = block_tables;
    p.table_stride = table_stride;
    p.width = max_table_width;
    p.lens = context_lengths;
    p.cu = cu_seqlens_q;
    p.out = out;
    p.o_row = out_strides[0];
    p.o_head = out_strides[1];
    p.num_seqs = static_cast<int>(num_seqs);
    p.hq = static_cast<int>(num_q_heads);
    p.hkv = static_cast<int>(num_kv_heads);
    p.num_blocks = num_blocks;
    // s * scale == (-s) * |scale|: a negative scale negates q exactly (sign bits).
    p.qscale = std::fabs(scale) * kLog2eP;
    p.q_sign = scale < 0.f ? 0x80008000u : 0u;
    // Ranked mode: each XCD's queue holds hq/8 heads of every (sequence,
    // query tile) pair, at most ceil(total_q / kBM) + num_seqs of them.
    const int64_t pairs_bound = (total_q + kBM - 1) / kBM + num_seqs;
    const int64_t max_qt = (max_seqlen_q + kBM - 1) / kBM;
    p.total_q = static_cast<int>(total_q);
    p.ranked = num_seqs <= kRankSeqs && num_q_heads % kXcds == 0;
    if (!p.ranked && max_seqlen_q <= 0)
      return fail(RLT_EINVAL, "rlt_paged_prefill: max_seqlen_q must cover the longest chunk");
    p.max_qt = static_cast<int>(std::min<int64_t>(max_qt, 0x7fffffff));
    const int64_t items = p.ranked ? pairs_bound * num_q_heads : num_seqs * max_qt * num_q_heads;
    if (items > 0x7fffffff) return fail(RLT_EUNSUPPORTED, "rlt_paged_prefill: too many query tiles");
    if (items == 0) return RLT_OK;
    const dim3 grid(static_cast<unsigned>(items));
    hipStream_t st = as_stream(stream);
    // Direct-to-LDS staging needs the key range's page ids to fit in LDS.
    const bool dma = head_dim == 128 && max_table_width <= kTablePages;
    if (dtype == RLT_BFLOAT16) {
      if (dma) hipLaunchKernelGGL((paged_prefill_mfma_kernel<bf16, 128, true>), grid, dim3(512), 0, st, p);
      else if (head_dim == 128) hipLaunchKernelGGL((paged_prefill_mfma_kernel<bf16, 128, false>), grid, dim3(512), 0, st, p);
      else hipLaunchKernelGGL((paged_prefill_mfma_kernel<bf16, 64, false>), grid, dim3(512), 0, st, p);
    } else {
      if (dma) hipLaunchKernelGGL((paged_prefill_mfma_kernel<f16, 128, true>), grid, dim3(512), 0, st, p);
      else if (head_dim == 128) hipLaunchKernelGGL((paged_prefill_mfma_kernel<f16, 128, false>), grid, dim3(512), 0, st, p);
      else hipLaunchKernelGGL((paged_prefill_mfma_kernel<f16, 64, false>), grid, dim3(512), 0, st, p);
    }
    return check_launch("rlt_paged_prefill");
  }

  const int64_t need = fallback_workspace(total_q, max_table_width, num_q_heads, num_kv_heads, head_dim);
  if (!workspace || workspace_bytes < need)
    return fail(RLT_EWORKSPACE,
                "rlt_paged_prefill: workspace of %lld bytes < required %lld (the MFMA path, which needs none, "
                "requires 16-byte aligned q/out/cache rows and head_dim 64/128, page 16, bf16/fp16)",
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
