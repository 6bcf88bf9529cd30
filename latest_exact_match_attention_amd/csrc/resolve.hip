// The prefill latest-match resolver and the value gather (code/lema/attention.py:100-158).
//
// One workgroup (256 threads, 4 wavefronts) owns 1024 consecutive query positions
// [c0, c0 + 1024) of one (b, h) row, four per thread, laid out so that the 64 positions of each
// "word" (o / 64) are the 64 lanes of one wavefront. Query i's answer, the latest key j < i
// with the same code, is found nearest first:
//   (a) earlier lanes of its own word, (b) earlier words of the chunk: every key of the chunk
//       whose code some query of the chunk carries sets its lane bit in a 64-bit mask kept
//       per (code, word) in a sparse LDS map, and its word's bit in a per-code word summary;
//       the answer is then one or two mask lookups and a count-leading-zeros -- O(1) per
//       query, no per-wavefront scan and no ordering pass;
//   (c) before the chunk: every key in [0, c0) is looked up in the LDS hash table of the
//       chunk's query codes and raises that code's latest position with an LDS atomicMax.
// Both LDS tables are bucketized: 4 slots per bucket, read with one 16-byte LDS load, at
// load <= 1/2, so a lookup almost always ends after a single read and the wavefront does not
// wait on its slowest lane's probe chain. The query-code table has 2048 slots for at most
// 1024 codes whatever the code width, so every structure lives in LDS and the kernel needs
// no scratch memory. Step (c) costs O(T^2 / 1024) lookups per row, reading the row's key
// codes from L2 with 16-byte loads one batch ahead; at T = 16k that is 7.5 per query.
//
// With a workspace (the _ws entry points, rows of at least 64 chunks), step (c) of chunks with
// at most 512 distinct query codes instead reads chunk summaries written by summary_kernel
// just before (chunks of more keep the queued scan of resolve_core.h): per full chunk, a 2048-slot table of
// (fingerprint, latest position) per distinct key code. Only the query codes with no earlier
// key in their own chunk (about 300 of 1024 positions' codes on Zipf data) probe the earlier
// chunks' tables, latest first, 8 chunks per round trip, and every candidate is confirmed
// against the key code itself, so the answer stays exact; the LDS work of step (c) drops from
// O(T / 1024) lookups per query to none.
//
// The gather is fused: after resolving, the workgroup copies its 1024 value rows
// v[src] -> y in 16-byte pieces, consecutive threads on consecutive pieces, so both the reads
// of each source row and the (non-temporal) writes of y are coalesced.
#include "resolve_core.h"

#include <atomic>

#ifndef LEMA_GATHER_INFLIGHT
// Rows per thread in flight in the fused gather when a row has at most 256 pieces. With 8, a
// chunk's 1024 rows take 4 full loop trips at 8 pieces a row (256 rows a trip) and 2 at 3
// pieces (680 rows a trip); 12 left a third trip two thirds full (8 pieces) or a second trip
// of 4 rows (3 pieces) and measured 1-3% slower; 4 to 10 came within 1% of 8.
#define LEMA_GATHER_INFLIGHT 8
#endif

namespace lema {
namespace {

// Work item v of the resolver's grid is one (row, chunk). XCD-aware order: item v runs on
// XCD v % 8. When the rows come in whole groups of 64, rows 8g..8g+7 belong to XCD g % 8 and
// its items take one chunk of all 8 rows back to back, latest chunks first: the 8 rows' key
// codes and value rows share that XCD's L2, and where y interleaves the rows (y viewed from
// [B, T, H * dv]) their pieces of each output line are written close together in the same L2
// (measured: 116 -> 112 us on B8 H16 T16384 Zipf codes; 307 -> 172 us, with the filter, on a
// language-model layer of B4 H64 T16384 d 24). Otherwise every chunk of row r runs on XCD
// r % 8, latest chunks first.
// With `alt` every other group of 8 rows takes its chunks earliest first instead. A late
// chunk's backward scan covers more earlier keys, so it costs more, and a persistent
// workgroup b runs items b, b + G, ..., which with G = 8 groups' items (1024 items of 16
// chunks) fall in consecutive groups at the same place: alternating hands it a late chunk and
// then an early one instead of the same late chunk twice. The persistent kernel asks for it
// when each workgroup has two items: on B8 H16 T16384 Zipf codes (d_v 64) the launch after a
// cache eviction went from 111.2-111.7 to 105.9-107.5 us, back to back unchanged. With four
// items (a language-model layer, B4 H64 T16384 d_v 24) alternating, and the pairs c, 15 - c,
// 15 - c, c, both measured 4-6 us slower, so four-item grids keep the latest chunks first.
__device__ __forceinline__ void item_rc(int nchunks, bool group, int v, int64_t& row, int& chunk,
                                        bool alt = false) {
  const int xcd = v % kNumXcd;
  const int k = v / kNumXcd;
  if (group) {
    const int per = kNumXcd * nchunks;
    const int c = (k % per) / kNumXcd;
    chunk = alt && ((k / per) & 1) ? c : nchunks - 1 - c;
    row = (static_cast<int64_t>(k / per) * kNumXcd + xcd) * kNumXcd + (k % per) % kNumXcd;
  } else {
    chunk = nchunks - 1 - (k % nchunks);
    row = static_cast<int64_t>(k / nchunks) * kNumXcd + xcd;
  }
}
__device__ __forceinline__ void item_of(const ResolveArgs& a, int v, int64_t& row, int& chunk,
                                        bool alt = false) {
  item_rc(a.nchunks, a.group != 0, v, row, chunk, alt);
}

// One workgroup (256 threads) per work item: resolve the chunk, then (VEC > 0) copy its value
// rows.
template <typename CodeT, int VEC, bool kSumm>
__global__ __launch_bounds__(kThreads) void resolve_kernel(ResolveArgs a) {
  __shared__ ResolveLds<CodeT> s;
  int64_t row;
  int chunk;
  item_of(a, blockIdx.x, row, chunk);
  if (row >= a.N) return;
  const int t = threadIdx.x;
  int32_t src[kPer];
  auto bar = [] { __syncthreads(); };
  resolve_chunk<CodeT, decltype(bar), kSumm>(s, a, row, chunk, t, bar, src);
  if constexpr (VEC > 0) {
    int32_t* srcs = reinterpret_cast<int32_t*>(s.mbits);  // the masks are dead now
    __syncthreads();
#pragma unroll
    for (int p = 0; p < kPer; ++p) srcs[p * kThreads + t] = src[p];
    __syncthreads();
    const int32_t c0 = chunk * kChunk;
    const int n_here = static_cast<int>(a.T - c0 < kChunk ? a.T - c0 : kChunk);
    gather_rows<VEC, 8, LEMA_GATHER_INFLIGHT>(a.g, row, c0, n_here, t, kThreads,
                                              [&](uint32_t r) -> int64_t { return srcs[r]; });
  }
}

// Persistent form of resolve_kernel with copies. As many workgroups as the GPU holds at once
// take work items blockIdx.x, + gridDim.x, ... (gridDim.x a multiple of 8 keeps every item on
// its XCD). Half of the workgroups (which half: below) copy each chunk one item late: they
// resolve the next chunk first, holding the previous chunk's indices in four registers per
// thread. Launched all at once, workgroups that each resolve and then copy stay in step,
// round after round: the whole chip resolves (HBM idle), and then it copies. With half of
// them a chunk behind, resolving and copying run side by side. Measured on B8 H16 T16384 Zipf
// codes (d_v 64): 84.3 us with one workgroup per item, 77.5 us this way; on a language-model
// layer (B4 H64 T16384, d_v 24): 104.1 and 91.0 us.
// Which half lags (`mode` bit 1): workgroups are dealt to the 8 XCDs in turn, and where each
// XCD spreads its share over its 32 CUs in order, a block of 128 takes one slot on half of
// every XCD's CUs. Lagging every other block of 128 (bid >> 7 odd) then makes whole CUs lag;
// lagging every other block of 256 (bid >> 8 even: slots 0 and 2) lags two of each CU's four
// workgroups instead. Long value rows favour the second (B8 H16 T16384 Zipf codes, d_v 64:
// 78.8-79.2 against 81.2-81.3 us back to back, 100.8 against 104.9-105.0 us after a cache
// eviction; slots 1 and 3 instead: 79.5-81.4 and 100.9-101.7 us), short ones the first
// (language-model layer, d_v 24, y interleaved: 91.8-92.1 against 94.1-94.3 us at B4; after
// an eviction 63.5 against 66.3 us at B2).
// `mode` bit 0 asks item_of for alternating chunk order.
template <typename CodeT, int VEC, bool kSumm>
__global__ __launch_bounds__(kThreads, sizeof(CodeT) == 4 ? 4 : 3) void resolve_lag_kernel(ResolveArgs a, int32_t items,
                                                                                            int32_t mode) {
  static_assert(VEC > 0, "the persistent form exists for copies");
  __shared__ ResolveLds<CodeT> s;
  const int bid = blockIdx.x, G = gridDim.x;
  const bool lagged = (mode & 2) ? !((bid >> 8) & 1) : (bid >> 7) & 1;
  auto bar = [] { __syncthreads(); };
  int32_t* srcs = reinterpret_cast<int32_t*>(s.mbits);  // the masks are dead while copying
  const int n = bid < items ? (items - bid + G - 1) / G : 0;
  int32_t keep[kPer] = {-1, -1, -1, -1};  // the lagged chunk's indices
  int64_t krow = a.N;
  int kch = 0;
#pragma unroll 1
  for (int i = 0; i < n + (lagged ? 1 : 0); ++i) {
    // The thread index through an opaque copy: what the resolver derives from it is formed
    // in each iteration instead of being hoisted out of the loop and held in registers
    // across all of it (4 workgroups per CU leave 128 VGPRs).
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));
    int64_t row = a.N;
    int chunk = 0;
    if (i < n) item_of(a, bid + i * G, row, chunk, (mode & 1) != 0);
    int32_t src[kPer] = {-1, -1, -1, -1};
    const bool resolved = row < a.N;
    if (resolved) {
      resolve_chunk<CodeT, decltype(bar), kSumm>(s, a, row, chunk, t, bar, src);
      bar();  // every wavefront's last table read, before the masks' storage takes indices
    }
    {
      int64_t crow = row;
      int cchunk = chunk;
      int32_t c[kPer];
#pragma unroll
      for (int p = 0; p < kPer; ++p) c[p] = src[p];
      if (lagged) {
        crow = krow;
        cchunk = kch;
#pragma unroll
        for (int p = 0; p < kPer; ++p) {
          c[p] = keep[p];
          keep[p] = src[p];
        }
        krow = resolved ? row : a.N;
        kch = chunk;
      }
      if (crow < a.N) {
#pragma unroll
        for (int p = 0; p < kPer; ++p) srcs[p * kThreads + t] = c[p];
        bar();
        const int32_t c0 = cchunk * kChunk;
        const int n_here = static_cast<int>(a.T - c0 < kChunk ? a.T - c0 : kChunk);
        gather_rows<VEC, 8, LEMA_GATHER_INFLIGHT>(a.g, crow, c0, n_here, t, kThreads,
                                                  [&](uint32_t r) -> int64_t { return srcs[r]; });
        bar();  // the copy's last index read, before the next chunk's tables start over
      }
    }
  }
}

// One workgroup per (row, full chunk except the row's last): the chunk's summary table. The
// LDS table is keyed by the whole code (the all-ones code, its empty marker, is kept apart);
// each key raises its code's latest position with an atomicMax, and the table's image goes
// to HBM with the fingerprints in place of the codes.
// Shorter rows keep the backward scan: its LDS lookups cost O(T) per query, but the summaries'
// extra kernel and the probes' round trips to L2 cost more until about 64 chunks (measured at
// 2M queries: scan 124 vs 146 us at T = 16384, 192 vs 188 us at 65536, 251 vs 227 at 131072).
constexpr int kSummaryMinChunks = 64;

template <typename CodeT>
__global__ __launch_bounds__(kThreads) void summary_kernel(ResolveArgs a) {
  __shared__ __attribute__((aligned(16))) CodeT code[kSumSlots];  // read 4 slots at a time
  __shared__ int32_t last[kSumSlots];
  __shared__ int32_t sent_last;
  const int per = a.nchunks - 1;
  const int bid = blockIdx.x;
  const int xcd = bid % kNumXcd;
  const int k = bid / kNumXcd;
  const int chunk = k % per;
  const int64_t row = static_cast<int64_t>(k / per) * kNumXcd + xcd;
  if (row >= a.N) return;
  const int t = threadIdx.x;
  const CodeT SENT = sentinel<CodeT>();
  const CodeT* krow = static_cast<const CodeT*>(a.kc) + row * a.T + chunk * kChunk;
  CodeT kk[kPer];
  int o[kPer];
  if (a.kvec) {  // 4 consecutive codes per thread, 16-byte aligned
    if constexpr (sizeof(CodeT) == 4) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(krow + 4 * t);
      kk[0] = v.x; kk[1] = v.y; kk[2] = v.z; kk[3] = v.w;
    } else {
      const u32x4 v0 = *reinterpret_cast<const u32x4*>(krow + 4 * t);
      const u32x4 v1 = *reinterpret_cast<const u32x4*>(krow + 4 * t + 2);
      kk[0] = (uint64_t(v0.y) << 32) | v0.x; kk[1] = (uint64_t(v0.w) << 32) | v0.z;
      kk[2] = (uint64_t(v1.y) << 32) | v1.x; kk[3] = (uint64_t(v1.w) << 32) | v1.z;
    }
#pragma unroll
    for (int p = 0; p < kPer; ++p) o[p] = 4 * t + p;
  } else {
#pragma unroll
    for (int p = 0; p < kPer; ++p) {
      o[p] = p * kThreads + t;
      kk[p] = krow[o[p]];
    }
  }
  for (int x = t; x < kSumSlots; x += kThreads) {
    code[x] = SENT;
    last[x] = -1;
  }
  if (t == 0) sent_last = -1;
  __syncthreads();
#pragma unroll
  for (int p = 0; p < kPer; ++p) {
    if (kk[p] == SENT) {
      atomicMax(&sent_last, o[p]);
      continue;
    }
    bool ins;
    const int sl = table_claim<CodeT, kSumBuckets>(code, kk[p], SENT, bucket_of<kSumBuckets>(fold(kk[p])), ins);
    atomicMax(&last[sl], o[p]);
  }
  __syncthreads();
  uint32_t* tab = a.summ_tab + (row * a.nchunks + chunk) * kSumSlots;
  for (int b = t; b < kSumBuckets; b += kThreads) {
    uint32_t e[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const CodeT c = code[4 * b + i];
      e[i] = c == SENT ? kSumEmpty
                       : (fingerprint(fold(c)) << 10) | static_cast<uint32_t>(last[4 * b + i]);
    }
    *reinterpret_cast<u32x4*>(tab + 4 * b) = u32x4{e[0], e[1], e[2], e[3]};
  }
  if (t == 0) a.summ_sent[row * a.nchunks + chunk] = sent_last;
}

// Workspace of the summary path: the tables, then the all-ones code's positions.
struct SummaryLayout {
  int64_t tab_bytes, sent_off, bytes;
};

SummaryLayout summary_layout(int64_t N, int64_t T) {
  SummaryLayout L{0, 0, 0};
  const int64_t nchunks = (T + kChunk - 1) / kChunk;
  if (N <= 0 || nchunks < kSummaryMinChunks) return L;
  L.tab_bytes = N * nchunks * kSumSlots * 4;
  L.sent_off = (L.tab_bytes + 255) / 256 * 256;
  L.bytes = L.sent_off + (N * nchunks * 4 + 255) / 256 * 256;
  return L;
}

// Standalone gather for given indices: one workgroup per (row, 1024 positions).
constexpr int kGatherRows = 1024;

struct GatherOnlyArgs {
  const void* src;
  int32_t src_bytes;
  int64_t N, T;
  int32_t nchunks;
  int32_t group;  // the resolver's grouped order (8 rows of one XCD take a chunk together)
  GatherArgs g;
};

// One workgroup per (row, 1024 positions), in the resolver's order: where y interleaves the
// rows (viewed from [B, T, H * dv]), the 8 rows of one XCD write whole output lines together
// in its L2. (Rows spread over the XCDs wrote each line in parts from several L2s: a
// language-model layer's output, B4 H64 T16384 d_v 24, took 82.5 us that way.)
template <int VEC>
__global__ __launch_bounds__(256) void gather_kernel(GatherOnlyArgs a) {
  __shared__ int32_t ssrc[kGatherRows];
  int64_t row;
  int chunk;
  item_rc(a.nchunks, a.group != 0, blockIdx.x, row, chunk);
  if (row >= a.N) return;
  const int64_t c0 = static_cast<int64_t>(chunk) * kGatherRows;
  const int nrows = static_cast<int>(a.T - c0 < kGatherRows ? a.T - c0 : kGatherRows);
  for (int r = threadIdx.x; r < nrows; r += blockDim.x) {
    const int64_t at = row * a.T + c0 + r;
    ssrc[r] = a.src_bytes == 8 ? static_cast<int32_t>(static_cast<const int64_t*>(a.src)[at])
                               : static_cast<const int32_t*>(a.src)[at];
  }
  __syncthreads();
  gather_rows<VEC, 8, 12>(a.g, row, c0, nrows, threadIdx.x, blockDim.x,
                      [&](uint32_t r) -> int64_t { return ssrc[r]; });
}

// Largest piece size that divides every byte offset the gather forms.
int piece_bytes(int64_t row_bytes, const void* v, const void* y,
                std::initializer_list<int64_t> strides) {
  for (int vec : {16, 8, 4, 2}) {
    bool ok = row_bytes % vec == 0 && aligned(v, vec) && aligned(y, vec);
    for (int64_t s : strides) ok = ok && (s % vec == 0);
    if (ok) return vec;
  }
  return 0;
}

int fill_gather(GatherArgs& g, const void* v, int32_t dtype, int64_t H, int64_t T, int64_t dv,
                int64_t v_sb, int64_t v_sh, int64_t v_st, void* y, int64_t y_sb, int64_t y_sh,
                int64_t y_st, int32_t miss, int* vec_out) {
  const int es = dtype_size(dtype);
  LEMA_REQUIRE(es > 0, "unknown value dtype %d", dtype);
  LEMA_REQUIRE(miss == LEMA_MISS_DENSE || miss == LEMA_MISS_ZERO, "unknown miss mode %d", miss);
  LEMA_REQUIRE(dv >= 1, "value rows must have at least one element (dv = %lld)", (long long)dv);
  LEMA_REQUIRE(v != nullptr && y != nullptr, "v and y must be device pointers");
  const int64_t rb = dv * es;
  const int vec = piece_bytes(rb, v, y, {v_sb * es, v_sh * es, v_st * es, y_sb * es, y_sh * es, y_st * es});
  LEMA_REQUIRE(vec >= es || (vec == 2 && es == 2), "value rows/strides not aligned to the element size");
  LEMA_REQUIRE(rb / vec < (1 << 20), "value rows too long (%lld bytes)", (long long)rb);
  g.v = static_cast<const uint8_t*>(v);
  g.y = static_cast<uint8_t*>(y);
  g.H = H;
  g.T = T;
  g.v_sb = v_sb * es;
  g.v_sh = v_sh * es;
  g.v_st = v_st * es;
  g.y_sb = y_sb * es;
  g.y_sh = y_sh * es;
  g.y_st = y_st * es;
  g.pieces = static_cast<uint32_t>(rb / vec);
  g.pdiv = FastDiv(g.pieces);
  g.miss = miss;
  g.dtype = dtype;
  g.nt = y_st == dv;  // rows of y adjacent: stream them out; else let L2 merge the pieces
  *vec_out = vec;
  return LEMA_OK;
}

template <typename CodeT, bool kSumm>
int launch_vec(ResolveArgs& a, int vec, int64_t grid, hipStream_t st);

template <typename CodeT>
int launch_resolve(ResolveArgs& a, int vec, hipStream_t st) {
  a.kvec = (aligned(a.kc, 16) && (a.T * static_cast<int64_t>(sizeof(CodeT))) % 16 == 0) ? 1 : 0;
  a.group = a.N % 64 == 0;  // 8 whole groups of 8 rows per XCD at least: the grouped order
  const int64_t groups = (a.N + kNumXcd - 1) / kNumXcd;
  const int64_t grid = a.group ? (groups + kNumXcd - 1) / kNumXcd * kNumXcd * kNumXcd * a.nchunks
                               : (a.N + kNumXcd - 1) / kNumXcd * kNumXcd * a.nchunks;
  LEMA_REQUIRE(grid < (int64_t(1) << 31), "too many rows x chunks (%lld)", (long long)grid);
  if (a.summ_tab != nullptr) {
    const int64_t sgrid = (a.N + kNumXcd - 1) / kNumXcd * kNumXcd * (a.nchunks - 1);
    summary_kernel<CodeT><<<dim3(sgrid), dim3(kThreads), 0, st>>>(a);
    if (int rc = launch_status("summary_kernel")) return rc;
    return launch_vec<CodeT, true>(a, vec, grid, st);
  }
  return launch_vec<CodeT, false>(a, vec, grid, st);
}

// Workgroups of `kernel` (256 threads) the current GPU holds at once, 0 if unknown; kept in
// `per_dev` (one array per kernel: every instantiation of a kernel template has the same
// function type) after the first call on a device.
constexpr int kMaxDev = 64;
template <typename K>
int64_t resident_groups(K kernel, std::atomic<int> (&per_dev)[kMaxDev]) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return 0;
  int n = per_dev[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kThreads, 0) != hipSuccess)
      return 0;
    n = cus * per_cu;
    per_dev[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// `items` work items. With copies, and more items than the GPU holds workgroups at once,
// resolve_lag_kernel gives each workgroup k = ceil(items / resident) of them (some k - 1),
// from a grid that is a multiple of 8, when that grid keeps at least 90% of the resident
// slots busy. Otherwise resolve_kernel runs one workgroup per item. Items that do not spread
// evenly would leave some workgroups an extra chunk at the end; with one workgroup per item
// the dispatcher fills the slots as they free up (measured striped: 1152 items on 1024 slots
// 45.8 against 38.6 us one per item; 2048 items of 8-byte codes on 768 slots, 89.0 against
// 75.1 us).
// Value rows of at least this many bytes lag two workgroups of every CU, shorter ones whole
// CUs (resolve_lag_kernel's `mode` bit 1; measured at 128- and 48-byte rows).
constexpr uint32_t kMixedLagRowBytes = 128;

template <typename CodeT, int VEC, bool kSumm>
int launch_items(ResolveArgs& a, int64_t items, hipStream_t st) {
  if constexpr (VEC > 0) {
    const auto lag = resolve_lag_kernel<CodeT, VEC, kSumm>;
    static std::atomic<int> per_dev[kMaxDev];
    const int64_t resident = resident_groups(lag, per_dev) / kNumXcd * kNumXcd;
    if (resident >= kNumXcd && items > resident) {
      const int64_t k = (items + resident - 1) / resident;
      const int64_t g = ((items + k - 1) / k + kNumXcd - 1) / kNumXcd * kNumXcd;
      if (10 * g >= 9 * resident) {
        const int32_t mode = (k == 2 ? 1 : 0) | (a.g.pieces * VEC >= kMixedLagRowBytes ? 2 : 0);
        lag<<<dim3(g), dim3(kThreads), 0, st>>>(a, static_cast<int32_t>(items), mode);
        return launch_status("resolve_lag_kernel");
      }
    }
  }
  resolve_kernel<CodeT, VEC, kSumm><<<dim3(items), dim3(kThreads), 0, st>>>(a);
  return launch_status("resolve_kernel");
}

template <typename CodeT, bool kSumm>
int launch_vec(ResolveArgs& a, int vec, int64_t grid, hipStream_t st) {
  switch (vec) {
    case 0: return launch_items<CodeT, 0, kSumm>(a, grid, st);
    case 16: return launch_items<CodeT, 16, kSumm>(a, grid, st);
    case 8: return launch_items<CodeT, 8, kSumm>(a, grid, st);
    case 4: return launch_items<CodeT, 4, kSumm>(a, grid, st);
    case 2: return launch_items<CodeT, 2, kSumm>(a, grid, st);
    default: set_error("internal: piece size %d", vec); return LEMA_BAD_ARG;
  }
}

int check_rows(const void* qc, const void* kc, int32_t code_bytes, int64_t N, int64_t T) {
  LEMA_REQUIRE(code_bytes == 4 || code_bytes == 8, "code_bytes must be 4 or 8, got %d", code_bytes);
  LEMA_REQUIRE(N >= 0 && T >= 0, "negative shape N=%lld T=%lld", (long long)N, (long long)T);
  LEMA_REQUIRE(T < (int64_t(1) << 30), "T=%lld exceeds the resolver's positions", (long long)T);
  LEMA_REQUIRE(N * T == 0 || (qc != nullptr && kc != nullptr), "null code pointer");
  LEMA_REQUIRE(N * T == 0 || (aligned(qc, code_bytes) && aligned(kc, code_bytes)),
               "code pointers must be aligned to code_bytes");
  return LEMA_OK;
}

}  // namespace
}  // namespace lema

namespace lema {
namespace {

// Points a at the summaries in the caller's workspace when the row length calls for them.
int use_workspace(ResolveArgs& a, void* workspace, int64_t ws_bytes) {
  const SummaryLayout L = summary_layout(a.N, a.T);
  if (L.bytes == 0) return LEMA_OK;
  LEMA_REQUIRE(workspace != nullptr && aligned(workspace, 256) && ws_bytes >= L.bytes,
               "workspace of %lld bytes (256-byte aligned) needed, got %lld", (long long)L.bytes,
               (long long)ws_bytes);
  a.summ_tab = static_cast<uint32_t*>(workspace);
  a.summ_sent = reinterpret_cast<int32_t*>(static_cast<uint8_t*>(workspace) + L.sent_off);
  return LEMA_OK;
}

int latest_prev_match(const void* qc, const void* kc, int32_t code_bytes, int64_t N, int64_t T,
                      void* src, int32_t src_bytes, void* workspace, int64_t ws_bytes,
                      hipStream_t st) {
  if (int rc = check_rows(qc, kc, code_bytes, N, T)) return rc;
  LEMA_REQUIRE(src_bytes == 4 || src_bytes == 8, "src_bytes must be 4 or 8, got %d", src_bytes);
  LEMA_REQUIRE(N * T == 0 || (src != nullptr && aligned(src, src_bytes)), "bad src pointer");
  if (N * T == 0) return LEMA_OK;
  ResolveArgs a{};
  a.qc = qc;
  a.kc = kc;
  a.N = N;
  a.T = T;
  a.nchunks = static_cast<int32_t>((T + kChunk - 1) / kChunk);
  a.src = src;
  a.src_bytes = src_bytes;
  if (workspace != nullptr)
    if (int rc = use_workspace(a, workspace, ws_bytes)) return rc;
  return code_bytes == 4 ? launch_resolve<uint32_t>(a, 0, st) : launch_resolve<uint64_t>(a, 0, st);
}

int hard(const void* qc, const void* kc, int32_t code_bytes, const void* v, int32_t dtype,
         int64_t B, int64_t H, int64_t T, int64_t dv, int64_t v_sb, int64_t v_sh, int64_t v_st,
         void* y, int64_t y_sb, int64_t y_sh, int64_t y_st, int32_t miss, void* src,
         int32_t src_bytes, void* workspace, int64_t ws_bytes, hipStream_t st) {
  LEMA_REQUIRE(B >= 0 && H >= 0, "negative shape B=%lld H=%lld", (long long)B, (long long)H);
  const int64_t N = B * H;
  if (int rc = check_rows(qc, kc, code_bytes, N, T)) return rc;
  if (src != nullptr) {
    LEMA_REQUIRE(src_bytes == 4 || src_bytes == 8, "src_bytes must be 4 or 8, got %d", src_bytes);
    LEMA_REQUIRE(aligned(src, src_bytes), "src pointer not aligned");
  }
  if (N * T == 0) return LEMA_OK;
  ResolveArgs a{};
  int vec = 0;
  if (int rc = fill_gather(a.g, v, dtype, H, T, dv, v_sb, v_sh, v_st, y, y_sb, y_sh, y_st, miss, &vec))
    return rc;
  a.qc = qc;
  a.kc = kc;
  a.N = N;
  a.T = T;
  a.nchunks = static_cast<int32_t>((T + kChunk - 1) / kChunk);
  a.src = src;
  a.src_bytes = src_bytes;
  if (workspace != nullptr)
    if (int rc = use_workspace(a, workspace, ws_bytes)) return rc;
  return code_bytes == 4 ? launch_resolve<uint32_t>(a, vec, st) : launch_resolve<uint64_t>(a, vec, st);
}

}  // namespace
}  // namespace lema

using namespace lema;

extern "C" int lema_latest_prev_match(const void* qc, const void* kc, int32_t code_bytes,
                                      int64_t N, int64_t T, void* src, int32_t src_bytes,
                                      void* stream) {
  clear_error();
  return latest_prev_match(qc, kc, code_bytes, N, T, src, src_bytes, nullptr, 0,
                           static_cast<hipStream_t>(stream));
}

extern "C" int lema_latest_prev_match_ws(const void* qc, const void* kc, int32_t code_bytes,
                                         int64_t N, int64_t T, void* src, int32_t src_bytes,
                                         void* workspace, int64_t workspace_bytes, void* stream) {
  clear_error();
  return latest_prev_match(qc, kc, code_bytes, N, T, src, src_bytes, workspace, workspace_bytes,
                           static_cast<hipStream_t>(stream));
}

extern "C" int64_t lema_resolve_workspace_bytes(int64_t N, int64_t T) {
  return summary_layout(N, T).bytes;
}

extern "C" int lema_hard(const void* qc, const void* kc, int32_t code_bytes, const void* v,
                         int32_t dtype, int64_t B, int64_t H, int64_t T, int64_t dv,
                         int64_t v_sb, int64_t v_sh, int64_t v_st, void* y, int64_t y_sb,
                         int64_t y_sh, int64_t y_st, int32_t miss, void* src,
                         int32_t src_bytes, void* stream) {
  clear_error();
  return hard(qc, kc, code_bytes, v, dtype, B, H, T, dv, v_sb, v_sh, v_st, y, y_sb, y_sh, y_st,
              miss, src, src_bytes, nullptr, 0, static_cast<hipStream_t>(stream));
}

extern "C" int lema_hard_ws(const void* qc, const void* kc, int32_t code_bytes, const void* v,
                            int32_t dtype, int64_t B, int64_t H, int64_t T, int64_t dv,
                            int64_t v_sb, int64_t v_sh, int64_t v_st, void* y, int64_t y_sb,
                            int64_t y_sh, int64_t y_st, int32_t miss, void* src,
                            int32_t src_bytes, void* workspace, int64_t workspace_bytes,
                            void* stream) {
  clear_error();
  return hard(qc, kc, code_bytes, v, dtype, B, H, T, dv, v_sb, v_sh, v_st, y, y_sb, y_sh, y_st,
              miss, src, src_bytes, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

extern "C" int lema_gather(const void* v, int32_t dtype, int64_t B, int64_t H, int64_t T,
                           int64_t dv, int64_t v_sb, int64_t v_sh, int64_t v_st,
                           const void* src, int32_t src_bytes, void* y, int64_t y_sb,
                           int64_t y_sh, int64_t y_st, int32_t miss, void* stream) {
  clear_error();
  LEMA_REQUIRE(B >= 0 && H >= 0 && T >= 0, "negative shape");
  LEMA_REQUIRE(src_bytes == 4 || src_bytes == 8, "src_bytes must be 4 or 8, got %d", src_bytes);
  const int64_t N = B * H;
  if (N * T == 0) return LEMA_OK;
  LEMA_REQUIRE(src != nullptr && aligned(src, src_bytes), "bad src pointer");
  LEMA_REQUIRE(T < (int64_t(1) << 31), "T=%lld exceeds int32 positions", (long long)T);
  GatherOnlyArgs a{};
  int vec = 0;
  if (int rc = fill_gather(a.g, v, dtype, H, T, dv, v_sb, v_sh, v_st, y, y_sb, y_sh, y_st, miss, &vec))
    return rc;
  a.src = src;
  a.src_bytes = src_bytes;
  a.N = N;
  a.T = T;
  a.nchunks = static_cast<int32_t>((T + kGatherRows - 1) / kGatherRows);
  a.group = N % 64 == 0;
  const int64_t groups = (N + kNumXcd - 1) / kNumXcd;
  const int64_t grid = a.group ? (groups + kNumXcd - 1) / kNumXcd * kNumXcd * kNumXcd * a.nchunks
                               : (N + kNumXcd - 1) / kNumXcd * kNumXcd * a.nchunks;
  LEMA_REQUIRE(grid < (int64_t(1) << 31), "too many rows x chunks");
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (vec) {
    case 16: gather_kernel<16><<<dim3(grid), dim3(256), 0, st>>>(a); break;
    case 8: gather_kernel<8><<<dim3(grid), dim3(256), 0, st>>>(a); break;
    case 4: gather_kernel<4><<<dim3(grid), dim3(256), 0, st>>>(a); break;
    case 2: gather_kernel<2><<<dim3(grid), dim3(256), 0, st>>>(a); break;
    default: set_error("internal: piece size %d", vec); return LEMA_BAD_ARG;
  }
  return launch_status("gather_kernel");
}
