// The LEMA retrieval store in HBM: one open-addressing table shared by every (layer, stream,
// head) partition, replacing the reference's host-RAM store (code/lema/csrc/store.cpp,
// driven by code/lema/cache.py:129-302).
//
// Table format -- identical to the reference's, so a table is interchangeable byte for byte:
// slot s is [code u64 | state u64 | value bytes] at s * (16 + vbytes); state 0 = free,
// group + 2 = taken (the reference also passes through 1 while a slot is filled; no completed
// exchange leaves it, and this store never writes it). The home slot of (group, code) is Lemire's fastrange of
// the splitmix64 finaliser of code ^ (group * 2^64/phi) (store.cpp:58-71); probing is linear with
// wrap-around. A zeroed allocation is an empty table.
//
// Exchange semantics (store.cpp:122-162): items i in [0, n) are position i % T of partition
// i / T, group g0 + i / T; in position order within a partition each item looks its query code
// up (value, or zeros) and then inserts its key code -> value (latest write wins); counts[g]
// grows by the newly claimed slots; a key that finds no free slot sets *full.
//
// GPU execution. Partitions run concurrently; the only cross-partition interaction is slot
// claiming: a device-scope CAS of the state word from free straight to the claimer's tag, then
// plain stores of code and value. No reader in the same kernel ever reads a slot it did not
// find before the kernel started -- another partition's slot is skipped on its tag, and a
// partition's own new slots are only probed for "free" -- so the claim needs no intermediate
// state and no fence; the kernel boundary publishes code and value to later exchanges. Every
// slot in front of an entry on its probe path was occupied before the entry was made, so a
// stale read can only show a free slot where someone is claiming: header reads are hints, the
// CAS decides.
//   * T == 1 (a decode step): one kernel; 8 lanes per item read the query's and the key's
//     first 8-slot windows together (one ballot each), look the query up, then update the
//     key's entry or claim a slot for it.
//   * T >= 2: sub-chunks of up to 1024 positions, one launch per sub-chunk (in order), one
//     workgroup per partition: in-chunk matches come from the LDS resolver, other queries from
//     the table; after a workgroup barrier (no query may see a later key) each key code's
//     last occurrence overwrites its existing entry, and after another barrier the codes that
//     had none claim new slots.
#include <mutex>

#include "resolve_core.h"

namespace lema {
namespace {

constexpr uint64_t kStateEmpty = 0;
// Lanes probing one item together, one window of that many slots per round trip: a decode
// step gives each item kStepGroup lanes (wide windows: few items ever need a second one), the
// chunk and bulk kernels kGroup lanes per item (many items in flight, so each window is one
// 128-byte line of two 64-byte slots; measured on B1 H64 calls of 2^20 positions per
// partition: 34.5 ms per call with 8 lanes, 26.1 with 4, 23.6 with 2, 24.6 with 1).
#ifndef LEMA_STORE_GROUP
#define LEMA_STORE_GROUP 2
#endif
#ifndef LEMA_STEP_GROUP
#define LEMA_STEP_GROUP 32
#endif
#ifndef LEMA_STEP_BLOCK
#define LEMA_STEP_BLOCK 128
#endif
constexpr int kGroup = LEMA_STORE_GROUP;
constexpr int kStepGroup = LEMA_STEP_GROUP;
constexpr int kStepBlock = LEMA_STEP_BLOCK;  // threads per decode-step workgroup
static_assert(kGroup == 1 || kGroup == 2 || kGroup == 4 || kGroup == 8 || kGroup == 16 ||
                  kGroup == 32 || kGroup == 64,
              "probe group width");
static_assert(kStepGroup == 8 || kStepGroup == 16 || kStepGroup == 32 || kStepGroup == 64,
              "probe group width");
// A decode step on a table in host memory probes narrower windows: there each step is bound by
// the host link's rate of small requests, not by round trips (1024 partitions at load 0.5:
// 153.7 us per step with 32 lanes, 127.6 with 16, 125.9 with 8).
constexpr int kStepGroupHost = 16;
static_assert(kStepGroupHost == 8 || kStepGroupHost == 16 || kStepGroupHost == 32,
              "probe group width");
static_assert(kStepBlock % 64 == 0 && kStepBlock >= kStepGroup && kStepBlock >= kStepGroupHost,
              "whole wavefronts of groups");

__device__ __forceinline__ uint64_t splitmix_fin(uint64_t x) {
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

__device__ __forceinline__ int64_t home_slot(uint64_t code, uint64_t group, int64_t cap) {
  const uint64_t h = splitmix_fin(code ^ (group * 0x9E3779B97F4A7C15ull));
  return static_cast<int64_t>(__umul64hi(h, static_cast<uint64_t>(cap)));
}

struct StoreArgs {
  uint8_t* table;
  int64_t cap, stride, vbytes;
  const void* qc;  // null: insert only
  const void* kc;
  int32_t code_bytes;
  const uint8_t* values;
  uint8_t* out;  // null when qc is null
  int64_t n, T, g0;
  int64_t s0;   // first position of the sub-chunk (T >= 2)
  int32_t len;  // positions in the sub-chunk
  int32_t piece;   // 16 or 8: value bytes copied per lane
  int32_t pieces;  // vbytes / piece
  bool pre;        // piece 16 and pieces <= kStepGroup: a decode step preloads the value row
  bool spec;       // piece 16 and pieces <= kSpecPieces: its query window reads whole slots
  int32_t cg_log2; // log2 of the lanes that copy one row in wave_copy_rows (pieces, up to 16)
  unsigned long long* counts;
  int32_t* full;
#ifdef LEMA_STEP_STAMPS
  uint64_t* stamps;    // diagnostics build: [step][item][5] realtime clock readings
  int64_t stamp_step;
#endif
};

__device__ __forceinline__ uint64_t code_at(const void* base, int32_t cb, int64_t i) {
  return cb == 4 ? static_cast<uint64_t>(static_cast<const uint32_t*>(base)[i])
                 : static_cast<const uint64_t*>(base)[i];
}

__device__ __forceinline__ uint64_t* state_ptr(const StoreArgs& a, int64_t s) {
  return reinterpret_cast<uint64_t*>(a.table + s * a.stride) + 1;
}

// Copy one value row with the group's lanes (src null: write zeros).
template <int G>
__device__ __forceinline__ void group_copy(const StoreArgs& a, uint8_t* dst, const uint8_t* src,
                                           int gl) {
  const int pieces = static_cast<int>(a.vbytes / a.piece);
  for (int k = gl; k < pieces; k += G) {
    if (a.piece == 16) {
      const u32x4 v = src ? *reinterpret_cast<const u32x4*>(src + 16 * k) : u32x4{0u, 0u, 0u, 0u};
      *reinterpret_cast<u32x4*>(dst + 16 * k) = v;
    } else {
      const u32x2 v = src ? *reinterpret_cast<const u32x2*>(src + 8 * k) : u32x2{0u, 0u};
      *reinterpret_cast<u32x2*>(dst + 8 * k) = v;
    }
  }
}

// Copy the value rows the lanes of a wave name (lane L: dst_L non-null; src_L null writes
// zeros), 2^cg_log2 lanes per row, each lane one piece of a row per instruction: an
// instruction moves whole rows of 64 >> cg_log2 named rows instead of one piece of each of
// 64 scattered rows, so a row costs one or two line requests rather than one per piece.
// Named rows are compacted first (lane r of `order` holds the lane naming the r-th row).
// Every lane of the wave must call it.
__device__ __forceinline__ void wave_copy_rows(const StoreArgs& a, uint8_t* dst, const uint8_t* src) {
  const unsigned long long act = __ballot(dst != nullptr);
  if (act == 0) return;
  const int lane = static_cast<int>(__lane_id());
  const int m = __popcll(act);
  const unsigned long long below = (1ull << lane) - 1ull;
  const int rank = dst != nullptr ? __popcll(act & below) : m + __popcll(~act & below);
  const int order = __builtin_amdgcn_ds_permute(rank << 2, lane);  // a permutation of the lanes
  const int g = 1 << a.cg_log2;
  const int gl = lane & (g - 1);
  const int rows = 64 >> a.cg_log2;  // rows per pass; r0 + lane / g stays below 64
  for (int r0 = 0; r0 < m; r0 += rows) {
    const int r = r0 + (lane >> a.cg_log2);
    const int owner = __shfl(order, r);
    uint8_t* d = reinterpret_cast<uint8_t*>(__shfl(reinterpret_cast<unsigned long long>(dst), owner));
    const uint8_t* sp =
        reinterpret_cast<const uint8_t*>(__shfl(reinterpret_cast<unsigned long long>(src), owner));
    if (r < m) {
      for (int k = gl; k < a.pieces; k += g) {
        if (a.piece == 16) {
          const u32x4 v = sp ? *reinterpret_cast<const u32x4*>(sp + 16 * k) : u32x4{0u, 0u, 0u, 0u};
          *reinterpret_cast<u32x4*>(d + 16 * k) = v;
        } else {
          const u32x2 v = sp ? *reinterpret_cast<const u32x2*>(sp + 8 * k) : u32x2{0u, 0u};
          *reinterpret_cast<u32x2*>(d + 8 * k) = v;
        }
      }
    }
  }
}

// The window of G slots starting at `base` (wrapping); lane gl reads slot base + gl.
// Lanes beyond the `left` slots still to probe report nothing. Returns this group's bits.
struct Window {
  uint64_t match, empty;
};
__device__ __forceinline__ int first_bit(uint64_t x) { return __ffsll(static_cast<unsigned long long>(x)) - 1; }
template <int G>
__device__ __forceinline__ Window window_bits(bool m, bool e, int gbase) {
  const uint64_t mask = G == 64 ? ~0ull : ((1ull << G) - 1);
  return Window{(__ballot(m) >> gbase) & mask, (__ballot(e) >> gbase) & mask};
}
// A lane's slot header of a window (loaded apart from its use, so that other reads can be in
// flight with it).
struct SlotHead {
  uint64_t code, state;
  bool valid;
};
__device__ __forceinline__ SlotHead load_head(const StoreArgs& a, int64_t base, int64_t left,
                                              int gl) {
  SlotHead h{0ull, 0ull, false};
  if (gl < left) {
    int64_t s = base + gl;
    if (s >= a.cap) s -= a.cap;
    const uint64_t* hdr = reinterpret_cast<const uint64_t*>(a.table + s * a.stride);
    h.state = hdr[1];
    h.code = hdr[0];
    h.valid = true;
  }
  return h;
}
template <int G>
__device__ __forceinline__ Window head_window(const SlotHead& h, uint64_t code, uint64_t tag,
                                              int gbase) {
  return window_bits<G>(h.valid && h.state == tag && h.code == code,
                        h.valid && h.state == kStateEmpty, gbase);
}
// Slots in the window at `base` with `left` slots still to probe: G, or with kAligned the slots
// up to the end of base's G-aligned group, so that every window after the first covers one
// whole group (with 64-byte slots and G = 2: one 128-byte line per window, where an unaligned
// pair of slots straddles two lines every other time). The probe order is the same either way.
template <int G, bool kAligned>
__device__ __forceinline__ int64_t window_width(int64_t base, int64_t left) {
  const int64_t w = kAligned ? G - (base & (G - 1)) : G;
  return w < left ? w : left;
}
template <int G, bool kAligned = false>
__device__ __forceinline__ Window read_window(const StoreArgs& a, int64_t base, int64_t left,
                                              uint64_t code, uint64_t tag, int gl, int gbase) {
  return head_window<G>(load_head(a, base, window_width<G, kAligned>(base, left), gl), code, tag,
                        gbase);
}

// The first window read as whole slots (header and value, 16-byte pieces): a hit's value is
// then already in lane `match`'s registers. Needs 16-byte slots and at most kSpecPieces pieces.
constexpr int kSpecPieces = 4;
template <int G>
__device__ __forceinline__ Window read_window_slots(const StoreArgs& a, int64_t base, uint64_t code,
                                                    uint64_t tag, int gl, int gbase,
                                                    u32x4 (&val)[kSpecPieces]) {
  bool m = false, e = false;
  if (gl < a.cap) {
    int64_t s = base + gl;
    if (s >= a.cap) s -= a.cap;
    const uint8_t* slot = a.table + s * a.stride;
    const u32x4 hdr = *reinterpret_cast<const u32x4*>(slot);
#pragma unroll
    for (int k = 0; k < kSpecPieces; ++k)
      if (k < a.pieces) val[k] = *reinterpret_cast<const u32x4*>(slot + 16 + 16 * k);
    const uint64_t c = (static_cast<uint64_t>(hdr[1]) << 32) | hdr[0];
    const uint64_t st = (static_cast<uint64_t>(hdr[3]) << 32) | hdr[2];
    m = st == tag && c == code;
    e = st == kStateEmpty;
  }
  return window_bits<G>(m, e, gbase);
}

// Slot of (tag, code) or -1 (code/lema/csrc/store.cpp:84-93), starting from window w0 read at
// `base` with `left` slots still unprobed. Group-uniform.
template <int G, bool kAligned = false>
__device__ int64_t group_lookup(const StoreArgs& a, uint64_t code, uint64_t tag, int64_t base,
                                int64_t left, Window w0, int gl, int gbase) {
  for (const int64_t left0 = left; left > 0;) {
    const Window w =
        left == left0 ? w0 : read_window<G, kAligned>(a, base, left, code, tag, gl, gbase);
    const int fm = w.match ? first_bit(w.match) : G;
    const int fe = w.empty ? first_bit(w.empty) : G;
    if (fm < fe) {
      const int64_t s = base + fm;
      return s >= a.cap ? s - a.cap : s;
    }
    if (w.empty) return -1;
    const int64_t width = window_width<G, kAligned>(base, left);
    left -= width;
    base += width;
    if (base >= a.cap) base -= a.cap;
  }
  return -1;
}

// Claim the first free slot of window `empty` (bits relative to `base`) for (tag, code):
// the slot index, or -1 when every one of them was taken first by another claimer (a lost
// race just marks that slot taken). The winner's lane writes the code; the caller the value.
__device__ __forceinline__ int64_t claim_in_window(const StoreArgs& a, uint64_t code, uint64_t tag,
                                                   int64_t base, uint64_t empty, int gl, int gbase) {
  while (empty) {
    const int e = first_bit(empty);
    int64_t s = base + e;
    if (s >= a.cap) s -= a.cap;
    unsigned long long old = 0;
    if (gl == e)
      old = atomicCAS(reinterpret_cast<unsigned long long*>(state_ptr(a, s)), kStateEmpty, tag);
    if (__shfl(old == kStateEmpty ? 1 : 0, gbase + e) != 0) {
      if (gl == e) *reinterpret_cast<uint64_t*>(a.table + s * a.stride) = code;
      return s;
    }
    empty &= ~(1ull << e);
  }
  return -1;
}

// Insert (tag, code) -> value (code/lema/csrc/store.cpp:97-117), starting from window w0 read
// at `base` with `left` slots still unprobed: 1 = claimed a new slot, 0 = overwrote the
// partition's own entry, -1 = probed every slot without room. With `claim_only` the key is
// known to be absent and only free slots are looked for. Group-uniform.
template <int G, bool kAligned = false>
__device__ int group_insert(const StoreArgs& a, uint64_t code, uint64_t tag, const uint8_t* value,
                            int64_t base, int64_t left, Window w0, bool claim_only, int gl,
                            int gbase) {
  for (const int64_t left0 = left; left > 0;) {
    const Window w =
        left == left0 ? w0 : read_window<G, kAligned>(a, base, left, code, tag, gl, gbase);
    const int fm = (!claim_only && w.match) ? first_bit(w.match) : G;
    if (fm < G && (!w.empty || fm < first_bit(w.empty))) {
      int64_t s = base + fm;
      if (s >= a.cap) s -= a.cap;
      group_copy<G>(a, a.table + s * a.stride + 16, value, gl);
      return 0;
    }
    const int64_t s = claim_in_window(a, code, tag, base, w.empty, gl, gbase);
    if (s >= 0) {
      group_copy<G>(a, a.table + s * a.stride + 16, value, gl);
      return 1;
    }
    const int64_t width = window_width<G, kAligned>(base, left);
    left -= width;
    base += width;
    if (base >= a.cap) base -= a.cap;
  }
  return -1;
}

// A decode step (T == 1): item i is partition i, G lanes per item. Everything that does
// not depend on the table is loaded up front (both codes, the item's value row when it fits one
// 16-byte piece per lane); the query's first window is read as whole slots when they are small
// enough (`spec`), so a hit needs no further read; after the windows only a claim (one CAS)
// is still a round trip. The query is answered before the key touches the table: a hit's value
// is stored to `out` (its load complete) before any store into the table is issued.
//
// The diagnostics build (LEMA_STEP_STAMPS, `build --stamps`) reads the GPU's constant 100 MHz
// clock at five points of each item -- start, codes loaded, first windows read, claim done,
// value and count written -- each after waiting for the item's memory operations so far,
// into a buffer set with lema_debug_step_stamps. The product build has none of it.
#ifdef LEMA_STEP_STAMPS
#define STEP_STAMP(k)                                                                  \
  do {                                                                                 \
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");                        \
    const uint64_t t_ = __builtin_amdgcn_s_memrealtime();                              \
    if (gl == 0 && a.stamps != nullptr) a.stamps[(a.stamp_step * a.n + i) * 5 + (k)] = t_; \
  } while (0)
#else
#define STEP_STAMP(k) \
  do {                \
  } while (0)
#endif
template <int G>
__global__ __launch_bounds__(kStepBlock) void store_step_kernel(StoreArgs a) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t i = gid / G;
  const int lane = threadIdx.x & 63, gl = lane % G, gbase = lane - gl;
  if (i >= a.n) return;  // whole groups only: n is a count of items, groups are aligned
  STEP_STAMP(0);
  const uint64_t tag = static_cast<uint64_t>(a.g0 + i) + 2;
  const bool has_q = a.qc != nullptr;
  const uint64_t kcode = code_at(a.kc, a.code_bytes, i);
  const uint64_t qcode = has_q ? code_at(a.qc, a.code_bytes, i) : 0;
  const uint8_t* vrow = a.values + i * a.vbytes;
  u32x4 vin = {0u, 0u, 0u, 0u};  // piece gl of the item's value row (`pre`)
  if (a.pre && gl < a.pieces) vin = *reinterpret_cast<const u32x4*>(vrow + 16 * gl);
  const int64_t khome = home_slot(kcode, tag - 2, a.cap);
  const int64_t qhome = has_q ? home_slot(qcode, tag - 2, a.cap) : 0;
  STEP_STAMP(1);
  // the two first windows are independent: their reads are in flight together
  const Window wk = read_window<G>(a, khome, a.cap, kcode, tag, gl, gbase);
  u32x4 qval[kSpecPieces];
  Window wq{0u, 0u};
  if (has_q)
    wq = a.spec ? read_window_slots<G>(a, qhome, qcode, tag, gl, gbase, qval)
                : read_window<G>(a, qhome, a.cap, qcode, tag, gl, gbase);

  if (has_q) {
    uint8_t* dst = a.out + i * a.vbytes;
    const int fm = wq.match ? first_bit(wq.match) : G;
    const int fe = wq.empty ? first_bit(wq.empty) : G;
    if (fm < fe && a.spec) {
      if (gl == fm) {
#pragma unroll
        for (int k = 0; k < kSpecPieces; ++k)
          if (k < a.pieces) *reinterpret_cast<u32x4*>(dst + 16 * k) = qval[k];
      }
    } else {
      const int64_t s = group_lookup<G>(a, qcode, tag, qhome, a.cap, wq, gl, gbase);
      group_copy<G>(a, dst, s >= 0 ? a.table + s * a.stride + 16 : nullptr, gl);
    }
  }

  STEP_STAMP(2);
  int r;
  const int fmk = wk.match ? first_bit(wk.match) : G;
  int64_t s = -1;
  if (fmk < G && (!wk.empty || fmk < first_bit(wk.empty))) {
    s = khome + fmk;  // the partition's entry: overwrite its value
    if (s >= a.cap) s -= a.cap;
    r = 0;
  } else {
    s = claim_in_window(a, kcode, tag, khome, wk.empty, gl, gbase);
    r = 1;
  }
  STEP_STAMP(3);
  if (s >= 0) {
    uint8_t* dst = a.table + s * a.stride + 16;
    if (a.pre) {
      if (gl < a.pieces) *reinterpret_cast<u32x4*>(dst + 16 * gl) = vin;
    } else {
      group_copy<G>(a, dst, vrow, gl);
    }
  } else {  // the first window had no room left: probe on
    int64_t b = khome + G;
    if (b >= a.cap) b -= a.cap;
    const int64_t left = a.cap - G;
    r = left > 0 ? group_insert<G>(a, kcode, tag, vrow, b, left,
                                   read_window<G>(a, b, left, kcode, tag, gl, gbase), false, gl,
                                   gbase)
                 : -1;
  }
  if (gl == 0) {
    if (r > 0) atomicAdd(&a.counts[a.g0 + i], 1ull);
    if (r < 0) atomicOr(a.full, 1);
  }
  STEP_STAMP(4);
}

// One sub-chunk [s0, s0 + len) of every partition, one workgroup (256 threads) per partition.
template <typename CodeT>
__global__ __launch_bounds__(kThreads) void store_chunk_kernel(StoreArgs a) {
  __shared__ ResolveLds<CodeT> s;
  __shared__ int32_t src_in[kChunk];
  __shared__ uint8_t klast[kChunk];
  const int64_t p = blockIdx.x;
  const int t = threadIdx.x, lane = t & 63, gl = lane % kGroup, gbase = lane - gl;
  const int grp = t / kGroup;
  constexpr int kGroups = kThreads / kGroup;
  const int64_t first = p * a.T + a.s0;  // item index of the sub-chunk's position 0
  const uint64_t tag = static_cast<uint64_t>(a.g0 + p) + 2;
  const int n = a.len;
  const CodeT SENT = sentinel<CodeT>();

  // 1. queries answered inside the sub-chunk (latest earlier key with the same code)
  if (a.qc != nullptr) {
    ResolveArgs ra{};
    ra.qc = static_cast<const CodeT*>(a.qc) + first;
    ra.kc = static_cast<const CodeT*>(a.kc) + first;
    ra.N = 1;
    ra.T = n;
    ra.nchunks = 1;
    ra.kvec = 0;
    ra.src = nullptr;
    int32_t src[kPer];
    resolve_chunk(s, ra, 0, 0, t, [] { __syncthreads(); }, src);
#pragma unroll
    for (int q = 0; q < kPer; ++q) src_in[q * kThreads + t] = src[q];
  }
  __syncthreads();

  // 2. the last occurrence of every key code in the sub-chunk (latest wins on insert)
  const CodeT* kr = static_cast<const CodeT*>(a.kc) + first;
  for (int x = t; x < kSlots; x += kThreads) s.code[x] = SENT;
  for (int x = t; x <= kSlots; x += kThreads) s.pos[x] = -1;
  __syncthreads();
  int ks[kPer];
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const int o = q * kThreads + t;
    ks[q] = kSlots;
    if (o >= n) continue;
    const CodeT c = kr[o];
    if (c != SENT) {
      bool ins;
      ks[q] = table_claim<CodeT, kBuckets>(s.code, c, SENT, bucket_of<kBuckets>(fold(c)), ins);
    }
    atomicMax(&s.pos[ks[q]], o);
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const int o = q * kThreads + t;
    if (o < n) klast[o] = s.pos[ks[q]] == o ? 1 : 0;
  }
  __syncthreads();

  // 3. look the queries up: in-chunk matches copy the sub-chunk's own values
  if (a.qc != nullptr) {
    for (int o = grp; o < n; o += kGroups) {
      const int j = src_in[o];
      uint8_t* dst = a.out + (first + o) * a.vbytes;
      if (j >= 0) {
        group_copy<kGroup>(a, dst, a.values + (first + j) * a.vbytes, gl);
      } else {
        const uint64_t c = code_at(a.qc, a.code_bytes, first + o);
        const int64_t h = home_slot(c, tag - 2, a.cap);
        const int64_t sl = group_lookup<kGroup>(a, c, tag, h, a.cap,
                                        read_window<kGroup>(a, h, a.cap, c, tag, gl, gbase), gl, gbase);
        group_copy<kGroup>(a, dst, sl >= 0 ? a.table + sl * a.stride + 16 : nullptr, gl);
      }
    }
  }
  __syncthreads();  // every query of this partition has read the table before any insert

  // 4. each key code's last occurrence overwrites its existing entry; codes without one are
  // marked (klast = 2) and, once no sibling can still be looking entries up, claim a slot
  for (int o = grp; o < n; o += kGroups) {
    if (!klast[o]) continue;
    const uint64_t c = code_at(a.kc, a.code_bytes, first + o);
    const int64_t h = home_slot(c, tag - 2, a.cap);
    const int64_t sl = group_lookup<kGroup>(a, c, tag, h, a.cap,
                                    read_window<kGroup>(a, h, a.cap, c, tag, gl, gbase), gl, gbase);
    if (sl >= 0)
      group_copy<kGroup>(a, a.table + sl * a.stride + 16, a.values + (first + o) * a.vbytes, gl);
    else if (gl == 0)
      klast[o] = 2;
  }
  __syncthreads();
  int added = 0;
  for (int o = grp; o < n; o += kGroups) {
    if (klast[o] != 2) continue;
    const uint64_t c = code_at(a.kc, a.code_bytes, first + o);
    const int64_t h = home_slot(c, tag - 2, a.cap);
    const int r = group_insert<kGroup>(a, c, tag, a.values + (first + o) * a.vbytes, h, a.cap,
                               read_window<kGroup>(a, h, a.cap, c, tag, gl, gbase), true, gl, gbase);
    if (r > 0) ++added;
    if (r < 0 && gl == 0) atomicOr(a.full, 1);
  }
  if (gl == 0 && added > 0) atomicAdd(&a.counts[a.g0 + p], static_cast<unsigned long long>(added));
}

// ------------------------------------------------------------------ one-lane probes
// The bulk kernels give each item one lane, which reads the headers of a line-aligned pair of
// slots itself (window_width<2, true>: the first pair may hold only the home slot): with 64-byte
// slots a probe step is one 128-byte line, and a wave carries 64 items' round trips.
struct PairHead {
  uint64_t c[2], s[2];
  int width;  // slots of the pair on the probe path, 1 or 2
};

__device__ __forceinline__ PairHead load_pair(const StoreArgs& a, int64_t base, int64_t left) {
  PairHead p;
  p.width = static_cast<int>(window_width<2, true>(base, left));
  const uint64_t* h0 = reinterpret_cast<const uint64_t*>(a.table + base * a.stride);
  p.c[0] = h0[0];
  p.s[0] = h0[1];
  p.c[1] = 0;
  p.s[1] = kStateEmpty;
  if (p.width == 2) {
    const int64_t b1 = base + 1 >= a.cap ? base + 1 - a.cap : base + 1;
    const uint64_t* h1 = reinterpret_cast<const uint64_t*>(a.table + b1 * a.stride);
    p.c[1] = h1[0];
    p.s[1] = h1[1];
  }
  return p;
}

// Slot of (tag, code) or -1 (code/lema/csrc/store.cpp:84-93), probing from `base` with the
// first pair already loaded.
__device__ int64_t lane_lookup(const StoreArgs& a, uint64_t code, uint64_t tag, int64_t base,
                               PairHead p) {
  for (int64_t left = a.cap; left > 0;) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      if (k >= p.width) break;
      if (p.s[k] == tag && p.c[k] == code) return base + k >= a.cap ? base + k - a.cap : base + k;
      if (p.s[k] == kStateEmpty) return -1;
    }
    left -= p.width;
    base += p.width;
    if (base >= a.cap) base -= a.cap;
    if (left > 0) p = load_pair(a, base, left);
  }
  return -1;
}

// Insert (tag, code) (code/lema/csrc/store.cpp:97-117) from home slot `base`: 1 = claimed a
// new slot, 0 = found the partition's entry, -1 = probed every slot without room. `slot` is
// the slot whose value the caller writes. No other lane inserts the same key at the same time,
// so a claim lost to a race is another key's slot, and every slot that read free was free
// before the kernel, so the key cannot lie beyond it: the probe goes on to claim.
__device__ int lane_insert(const StoreArgs& a, uint64_t code, uint64_t tag, int64_t base,
                           int64_t& slot) {
  PairHead p = load_pair(a, base, a.cap);
  for (int64_t left = a.cap; left > 0;) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      if (k >= p.width) break;
      const int64_t s = base + k >= a.cap ? base + k - a.cap : base + k;
      if (p.s[k] == tag && p.c[k] == code) {
        slot = s;
        return 0;
      }
      if (p.s[k] == kStateEmpty &&
          atomicCAS(reinterpret_cast<unsigned long long*>(state_ptr(a, s)), kStateEmpty, tag) ==
              kStateEmpty) {
        *reinterpret_cast<uint64_t*>(a.table + s * a.stride) = code;
        slot = s;
        return 1;
      }
    }
    left -= p.width;
    base += p.width;
    if (base >= a.cap) base -= a.cap;
    if (left > 0) p = load_pair(a, base, left);
  }
  slot = -1;
  return -1;
}

// ------------------------------------------------------------------ bulk calls
// A call with many positions per partition runs in sub-calls of up to kBulkSpan positions, each
// as a few kernels over all of its items at once instead of one launch per 1024-position
// sub-chunk:
//   chunks   one workgroup per (partition, 1024-chunk): in-chunk answers of the queries (LDS
//            resolver), the chunk's key summary (code -> latest position, the LDS table
//            written out), and its distinct key codes listed per part of the group table, each
//            with its latest position;
//   table    one workgroup per (partition, part of the code hash space): the part's codes of
//            every chunk entered in an LDS table, code -> mask of the chunks holding keys with
//            it and the latest key of all of them, written out as that part of the
//            partition's group table;
//   queries  a query without an in-chunk answer takes the highest chunk below its own in its
//            code's mask and that chunk's summary gives the key; with no such chunk it looks
//            the store up (the table still holds exactly the keys before the sub-call);
//   insert   every (partition, code) of the sub-call takes its latest key from its group-table
//            entry and writes that value over its existing store entry or claims a slot (code
//            0 in a kernel of its own, see bulk_insert_kernel); the claims are counted per
//            partition on the way.
// The kernel boundary orders every lookup of the sub-call before its inserts. A part with
// more codes than its LDS table takes (only codes chosen to collide in the hash get there) is
// marked spilled: its queries and inserts then search the chunk summaries themselves.
constexpr int kBulkSpan = 32 * kChunk;  // positions per sub-call: chunk masks fit 32 bits
static_assert((kSlots & (kSlots - 1)) == 0, "chunk summaries are probed with a slot mask");
constexpr int kSumPos = kSlots + 4;     // summary positions: kSlots code slots, the sentinel's
constexpr int kTableThreads = 1024;
constexpr int kTableLdsBytes = 131072;  // the table kernel's LDS table
constexpr int kFilterBitsLog2 = 16;     // key-code filter bits per part (8 KB)
constexpr int kFilterWordsQ = (1 << kFilterBitsLog2) / 32;

// Group table per partition: `cap` entries in kParts parts of `sub` entries; a code lives in the
// part given by the top bits of its hash, at the slot given by the low bits, with linear
// probing inside the part. Bit c of an entry's mask: chunk c of the sub-call holds keys with
// the code; beside each entry, its code's latest key in the sub-call (a position below
// kBulkSpan).
//   32-bit codes: 8 parts of up to 8,192 words; a word is code | mask << 32, 0 = free (an
//     entered word always has a mask bit set).
//   64-bit codes: 8 parts of up to 8,192 entries; an entry is a code word (the all-ones code
//     marks a free one) and a 32-bit mask word; the all-ones code's own mask is kept per
//     (partition, part).
template <typename CodeT>
struct GtTraits;
template <>
struct GtTraits<uint32_t> {
  static constexpr int kParts = 8, kPartLog2 = 3, kPartMax = 8192;
};
template <>
struct GtTraits<uint64_t> {
  static constexpr int kParts = 8, kPartLog2 = 3, kPartMax = 8192;
};
// The table kernel's LDS: entries (8 bytes), masks (64-bit codes, 4 bytes) and latest
// positions (4 bytes) of up to kPartMax codes, at fixed offsets for both code widths.
constexpr int kLdsMaskOff = GtTraits<uint64_t>::kPartMax * 8;
constexpr int kLdsPosOff = kLdsMaskOff + GtTraits<uint64_t>::kPartMax * 4;
static_assert(GtTraits<uint32_t>::kPartMax == GtTraits<uint64_t>::kPartMax &&
                  kLdsPosOff + GtTraits<uint64_t>::kPartMax * 4 <= kTableLdsBytes,
              "LDS table");

struct BulkWs {
  unsigned long long* gt;  // P x cap words: code | mask (32-bit codes) or codes (64-bit)
  uint32_t* gmask;         // 64-bit codes: P x cap masks
  uint32_t* smask;         // 64-bit codes: per (partition, part) the all-ones code's mask
  int32_t* spilled;        // per (partition, part): 1 = the part's table was not built
  int64_t* zero_slot;      // per partition: entry of code 0, or -1
  void* sum_code;          // per (partition, chunk): the kSlots key-code slots
  int32_t* sum_pos;        // per (partition, chunk): kSumPos latest positions
  int32_t* src_in;         // per query of the sub-call: in-chunk answer (sub-call position) or -1
  void* qlist;             // per (partition, chunk, part): the chunk's distinct key codes of
                           // the part, up to kChunk
  uint16_t* qlpos;         // beside qlist: each code's latest key as a sub-call position
  int32_t* qcount;         // per (partition, chunk, part): their number
  uint32_t* gpos;          // P x cap: an entry's latest key of the sub-call (sub-call position)
  uint32_t* spos;          // 64-bit codes: per (partition, part) the all-ones code's latest key
  uint32_t* claims;        // per workgroup of bulk_insert_kernel: store slots it claimed
  uint32_t* filter;        // per (partition, part): kFilterWordsQ words, two bits set per key
                           // code of the sub-call (gt_filter_bits)
  int32_t cap;             // entries per partition: a power of two, >= 2 * kBulkSpan or less
  int32_t cap_log2;        // for short calls, >= 256 * kParts
  int32_t sub;             // entries per part: cap / kParts
  int32_t nch;             // chunks per partition in the sub-call
};

template <typename CodeT>
__device__ __forceinline__ int gt_part(uint64_t h) {
  return static_cast<int>(h >> (64 - GtTraits<CodeT>::kPartLog2));
}

// A code's two bits in its part's key-code filter: hash bits that neither the part (at most
// the top three) nor the slot (at most the low 14) uses.
__device__ __forceinline__ void gt_filter_bits(uint64_t h, uint32_t& b1, uint32_t& b2) {
  constexpr uint64_t m = (1u << kFilterBitsLog2) - 1;
  b1 = static_cast<uint32_t>((h >> 20) & m);
  b2 = static_cast<uint32_t>((h >> (20 + kFilterBitsLog2)) & m);
}

__device__ __forceinline__ uint32_t gt_code(unsigned long long word) {
  return static_cast<uint32_t>(word);
}

// The chunk mask of `code` (hash h) in partition r's table, 0 when absent.
template <typename CodeT>
__device__ __forceinline__ uint32_t gt_mask_of(const BulkWs& w, int64_t r, CodeT code, uint64_t h) {
  const int part = gt_part<CodeT>(h);
  const int64_t base = (r << w.cap_log2) + static_cast<int64_t>(part) * w.sub;
  int32_t s = static_cast<int32_t>(h & static_cast<uint64_t>(w.sub - 1));
  if constexpr (sizeof(CodeT) == 4) {
    for (int32_t left = w.sub; left > 0; --left) {
      const unsigned long long k = w.gt[base + s];
      if (k == 0) return 0u;
      if (gt_code(k) == code) return static_cast<uint32_t>(k >> 32);
      s = (s + 1) & (w.sub - 1);
    }
  } else {
    if (code == sentinel<CodeT>()) return w.smask[r * GtTraits<CodeT>::kParts + part];
    for (int32_t left = w.sub; left > 0; --left) {
      const unsigned long long k = w.gt[base + s];
      if (k == code) return w.gmask[base + s];
      if (k == sentinel<CodeT>()) return 0u;
      s = (s + 1) & (w.sub - 1);
    }
  }
  return 0u;
}

// Latest position of `code` in a chunk summary, or -1: the image of the chunk's LDS table
// (4-slot buckets from bucket_of, linear probing), read a bucket at a time; the code's slot
// comes before any free slot on its probe path.
template <typename CodeT>
__device__ __forceinline__ int32_t summary_find(const CodeT* codes, const int32_t* pos, CodeT code) {
  const CodeT SENT = sentinel<CodeT>();
  if (code == SENT) return pos[kSlots];
  int b = bucket_of<kBuckets>(fold(code));
  for (int left = kBuckets; left > 0; --left) {
    CodeT e[4];
    if constexpr (sizeof(CodeT) == 4) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(codes + 4 * b);
      e[0] = v.x; e[1] = v.y; e[2] = v.z; e[3] = v.w;
    } else {
      const u32x4 v0 = *reinterpret_cast<const u32x4*>(codes + 4 * b);
      const u32x4 v1 = *reinterpret_cast<const u32x4*>(codes + 4 * b + 2);
      e[0] = (static_cast<uint64_t>(v0.y) << 32) | v0.x;
      e[1] = (static_cast<uint64_t>(v0.w) << 32) | v0.z;
      e[2] = (static_cast<uint64_t>(v1.y) << 32) | v1.x;
      e[3] = (static_cast<uint64_t>(v1.w) << 32) | v1.z;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (e[i] == code) return pos[4 * b + i];
      if (e[i] == SENT) return -1;
    }
    b = (b + 1) & (kBuckets - 1);
  }
  return -1;
}

template <typename CodeT>
__device__ __forceinline__ int32_t chunk_find(const BulkWs& w, int64_t p, int c, CodeT code) {
  const int64_t sum = p * w.nch + c;
  return summary_find<CodeT>(static_cast<const CodeT*>(w.sum_code) + sum * kSlots,
                             w.sum_pos + sum * kSumPos, code);
}

template <typename CodeT>
__global__ __launch_bounds__(kThreads) void bulk_chunk_kernel(StoreArgs a, BulkWs w) {
  constexpr int kParts = GtTraits<CodeT>::kParts;
  __shared__ ResolveLds<CodeT> s;
  __shared__ int32_t n_in[kParts];
  const int64_t p = blockIdx.x / w.nch;
  const int c = static_cast<int>(blockIdx.x - p * w.nch);
  const int t = threadIdx.x;
  const int64_t first = p * a.T + a.s0 + static_cast<int64_t>(c) * kChunk;
  const int n = a.len - c * kChunk < kChunk ? a.len - c * kChunk : kChunk;
  const CodeT SENT = sentinel<CodeT>();
  const CodeT* qc = static_cast<const CodeT*>(a.qc);
  const CodeT* kc = static_cast<const CodeT*>(a.kc);

  // 1. in-chunk answers of the queries, as positions of the sub-call
  if (qc != nullptr) {
    ResolveArgs ra{};
    ra.qc = qc + first;
    ra.kc = kc + first;
    ra.N = 1;
    ra.T = n;
    ra.nchunks = 1;
    int32_t src[kPer];
    resolve_chunk(s, ra, 0, 0, t, [] { __syncthreads(); }, src);
    int32_t* out = w.src_in + p * a.len + static_cast<int64_t>(c) * kChunk;
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
      const int o = q * kThreads + t;
      if (o < n) out[o] = src[q] >= 0 ? c * kChunk + src[q] : -1;
    }
  }
  __syncthreads();

  // 2. the chunk's key codes with their latest position
  for (int x = t; x < kSlots; x += kThreads) s.code[x] = SENT;
  for (int x = t; x <= kSlots; x += kThreads) s.pos[x] = -1;
  if (t < kParts) n_in[t] = 0;
  __syncthreads();
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const int o = q * kThreads + t;
    if (o >= n) continue;
    const CodeT code = kc[first + o];
    int slot = kSlots;
    if (code != SENT) {
      bool ins;
      slot = table_claim<CodeT, kBuckets>(s.code, code, SENT, bucket_of<kBuckets>(fold(code)), ins);
    }
    atomicMax(&s.pos[slot], o);
  }
  __syncthreads();

  // 3. the summary, and the distinct codes listed per group-table part (a wave takes its
  // places in a list with one LDS atomic)
  const int64_t sum = p * w.nch + c;
  CodeT* scode = static_cast<CodeT*>(w.sum_code) + sum * kSlots;
  int32_t* spos = w.sum_pos + sum * kSumPos;
  for (int x = t; x < kSlots; x += kThreads) scode[x] = s.code[x];
  for (int x = t; x <= kSlots; x += kThreads) spos[x] = s.pos[x];
  // each thread's slots first, then per part one LDS atomic per wave reserves the places of
  // all its codes of that part
  const int lane = t & 63;
  const unsigned long long below = (1ull << lane) - 1;
  CodeT* lists = static_cast<CodeT*>(w.qlist) + sum * kParts * kChunk;
  uint16_t* lpos = w.qlpos + sum * kParts * kChunk;
  constexpr int kRounds = (kSlots + 1 + kThreads - 1) / kThreads;
  CodeT rc[kRounds];
  int rq[kRounds];  // the slot's part, or -1 when the chunk holds no key with its code
  uint16_t rp[kRounds];  // the code's latest key as a sub-call position (< kBulkSpan)
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const int x = r * kThreads + t;
    rc[r] = x < kSlots ? s.code[x] : SENT;
    const int lp = x <= kSlots ? s.pos[x] : -1;
    const bool held = x < kSlots ? rc[r] != SENT : x == kSlots && lp >= 0;
    rq[r] = held ? gt_part<CodeT>(splitmix_fin(rc[r])) : -1;
    rp[r] = static_cast<uint16_t>(held ? c * kChunk + lp : 0);
  }
#pragma unroll
  for (int qq = 0; qq < kParts; ++qq) {
    unsigned long long bal[kRounds];
    int total = 0;
#pragma unroll
    for (int r = 0; r < kRounds; ++r) {
      bal[r] = __ballot(rq[r] == qq);
      total += __popcll(bal[r]);
    }
    if (total == 0) continue;  // wave-uniform
    int at = 0;
    if (lane == 0) at = atomicAdd(&n_in[qq], total);
    at = __shfl(at, 0);
#pragma unroll
    for (int r = 0; r < kRounds; ++r) {
      if (rq[r] == qq) {
        const int i = qq * kChunk + at + __popcll(bal[r] & below);
        lists[i] = rc[r];
        lpos[i] = rp[r];
      }
      at += __popcll(bal[r]);
    }
  }
  __syncthreads();
  if (t < kParts) w.qcount[sum * kParts + t] = n_in[t];
}

// Code slot x (x == kSlots: the sentinel code's own entry) of chunk c's summary: the code, and
// whether the chunk holds keys with it.
template <typename CodeT>
__device__ __forceinline__ bool summary_slot(const BulkWs& w, int64_t p, int c, int x, CodeT& code) {
  const int64_t sum = p * w.nch + c;
  if (x < kSlots) {
    code = static_cast<const CodeT*>(w.sum_code)[sum * kSlots + x];
    return code != sentinel<CodeT>();
  }
  code = sentinel<CodeT>();
  return w.sum_pos[sum * kSumPos + kSlots] >= 0;
}

// One workgroup per (partition, part): the part's table built in LDS from the part's code
// lists of every chunk of the partition, one CAS (new code) or OR (its chunk bit) and one max
// (its latest key) per code and chunk, then written out whole. With more than 3/4 of the part's entries taken the part is
// marked spilled and the table is not written (codes met after that are not entered; one that
// finds no free entry can only do so with the table past that mark).
template <typename CodeT>
__global__ __launch_bounds__(kTableThreads) void bulk_table_kernel(BulkWs w) {
  constexpr int kParts = GtTraits<CodeT>::kParts;
  constexpr bool k32 = sizeof(CodeT) == 4;
  __shared__ __align__(16) unsigned char lds[kTableLdsBytes];
  __shared__ uint32_t bits[kFilterWordsQ];
  __shared__ int32_t start[kBulkSpan / kChunk + 1];  // the part's codes before chunk c
  __shared__ int32_t n_codes, zero_at;
  __shared__ uint32_t sent_mask, sent_pos;
  unsigned long long* tab = reinterpret_cast<unsigned long long*>(lds);  // words or codes
  uint32_t* masks = reinterpret_cast<uint32_t*>(lds + kLdsMaskOff);
  uint32_t* lposs = reinterpret_cast<uint32_t*>(lds + kLdsPosOff);  // latest key per entry
  const CodeT SENT = sentinel<CodeT>();
  const int64_t p = blockIdx.x / kParts;
  const int qt = static_cast<int>(blockIdx.x % kParts);
  const int t = threadIdx.x;
  const int sub = w.sub;
  const int limit = sub / 4 * 3;
  for (int x = t; x < sub; x += kTableThreads) {
    if constexpr (k32) {
      tab[x] = 0ull;
    } else {
      tab[x] = SENT;
      masks[x] = 0u;
    }
    lposs[x] = 0u;
  }
  for (int x = t; x < kFilterWordsQ; x += kTableThreads) bits[x] = 0u;
  if (t == 0) {
    n_codes = 0;
    zero_at = -1;
    sent_mask = 0u;
    sent_pos = 0u;
  }
  if (t < 64) {  // the part's codes before each chunk: one load per lane, scanned in the wave
    const int32_t cnt = t < w.nch ? w.qcount[(p * w.nch + t) * kParts + qt] : 0;
    int32_t incl = cnt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int32_t y = __shfl_up(incl, o);
      if (t >= o) incl += y;
    }
    if (t <= w.nch) start[t] = incl - cnt;  // t == nch: the part's total
  }
  __syncthreads();
  const int total = start[w.nch];
  const CodeT* qlist = static_cast<const CodeT*>(w.qlist);
  constexpr int U = 8;  // codes per thread whose loads are in flight together
  for (int f0 = t; f0 < total; f0 += U * kTableThreads) {
    CodeT code[U];
    int chunk[U];
    uint32_t pos[U];  // the code's latest key in that chunk, as a sub-call position
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int f = f0 + u * kTableThreads;
      int lo = 0, hi = w.nch;  // the chunk c with start[c] <= f < start[c + 1]
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (start[mid] <= f) lo = mid; else hi = mid;
      }
      chunk[u] = f < total ? lo : -1;
      const int64_t li = ((p * w.nch + lo) * kParts + qt) * kChunk + (f - start[lo]);
      code[u] = f < total ? qlist[li] : CodeT(0);
      pos[u] = f < total ? w.qlpos[li] : 0u;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      bool entered = false;
      const uint64_t h = splitmix_fin(code[u]);
      if (chunk[u] >= 0) {  // every code of the part, spilled or not, sets its filter bits
        uint32_t b1, b2;
        gt_filter_bits(h, b1, b2);
        atomicOr(&bits[b1 >> 5], 1u << (b1 & 31));
        atomicOr(&bits[b2 >> 5], 1u << (b2 & 31));
      }
      if (chunk[u] >= 0 &&
          __hip_atomic_load(&n_codes, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) <= limit) {
        int s = static_cast<int>(h & static_cast<uint64_t>(sub - 1));
        if constexpr (k32) {
          const unsigned long long bit = 1ull << (32 + chunk[u]);
          for (int left = sub; left > 0; --left) {
            const unsigned long long k = atomicCAS(&tab[s], 0ull, bit | code[u]);
            if (k == 0) {  // entered
              entered = true;
              atomicMax(&lposs[s], pos[u]);
              if (code[u] == 0) zero_at = s;
              break;
            }
            if (gt_code(k) == code[u]) {
              atomicOr(&tab[s], bit);
              atomicMax(&lposs[s], pos[u]);
              break;
            }
            s = (s + 1) & (sub - 1);
          }
        } else {
          const uint32_t bit = 1u << chunk[u];
          if (code[u] == SENT) {
            atomicOr(&sent_mask, bit);  // kept apart, takes no entry
            atomicMax(&sent_pos, pos[u]);
          } else {
            for (int left = sub; left > 0; --left) {
              const unsigned long long k =
                  atomicCAS(&tab[s], static_cast<unsigned long long>(SENT),
                            static_cast<unsigned long long>(code[u]));
              if (k == SENT || k == code[u]) {  // entered, or the code's entry
                atomicOr(&masks[s], bit);
                atomicMax(&lposs[s], pos[u]);
                entered = k == SENT;
                if (entered && code[u] == 0) zero_at = s;
                break;
              }
              s = (s + 1) & (sub - 1);
            }
          }
        }
      }
      // one count update per wave, by its lowest lane still in the loop
      const unsigned long long b = __ballot(entered);
      if ((t & 63) == __ffsll(__ballot(true)) - 1 && b != 0)
        atomicAdd(&n_codes, static_cast<int32_t>(__popcll(b)));
    }
  }
  __syncthreads();
  const bool spill = n_codes > limit;
  const int64_t base = (p << w.cap_log2) + static_cast<int64_t>(qt) * sub;
  if (t == 0) {
    w.spilled[blockIdx.x] = spill ? 1 : 0;
    if constexpr (!k32) {
      w.smask[blockIdx.x] = sent_mask;
      w.spos[blockIdx.x] = sent_pos;
    }
    if (gt_part<CodeT>(splitmix_fin(CodeT(0))) == qt)
      w.zero_slot[p] = !spill && zero_at >= 0 ? base + zero_at : -1;
  }
  uint32_t* fdst = w.filter + static_cast<int64_t>(blockIdx.x) * kFilterWordsQ;
  for (int x = t; x < kFilterWordsQ; x += kTableThreads) fdst[x] = bits[x];
  if (spill) return;
  for (int x = t; x < sub; x += kTableThreads) {
    w.gt[base + x] = tab[x];
    if constexpr (!k32) w.gmask[base + x] = masks[x];
    w.gpos[base + x] = lposs[x];
  }
}

// One lane per query of the sub-call; the wave then copies its answers' rows together.
template <typename CodeT>
__global__ __launch_bounds__(256) void bulk_query_kernel(StoreArgs a, BulkWs w) {
  constexpr int kParts = GtTraits<CodeT>::kParts;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t n = static_cast<int64_t>(a.n / a.T) * a.len;
  uint8_t* dst = nullptr;  // stays null past the sub-call's queries
  const uint8_t* src = nullptr;
  if (i < n) {  // partition i / len, position i % len
    const int64_t p = i / a.len;
    const int o = static_cast<int>(i - p * a.len);
    const int64_t base = p * a.T + a.s0;  // item of the sub-call's position 0
    dst = a.out + (base + o) * a.vbytes;
    int32_t j = w.src_in[i];
    const CodeT code = static_cast<const CodeT*>(a.qc)[base + o];
    if (j < 0) {
      // the store's first read is in flight while the group table is consulted: most queries
      // without an in-chunk answer end in the store
      const uint64_t tag = static_cast<uint64_t>(a.g0 + p) + 2;
      const int64_t h = home_slot(code, tag - 2, a.cap);
      const PairHead first = load_pair(a, h, a.cap);
      const uint64_t gh = splitmix_fin(code);
      const int c = o / kChunk;
      const int64_t pq = p * kParts + gt_part<CodeT>(gh);
      uint32_t b1, b2;
      gt_filter_bits(gh, b1, b2);
      const uint32_t* f = w.filter + pq * kFilterWordsQ;
      if (!((f[b1 >> 5] >> (b1 & 31)) & (f[b2 >> 5] >> (b2 & 31)) & 1u)) {
        // no key of the sub-call has this code (no false negatives): the store
      } else if (!w.spilled[pq]) {
        const uint32_t m = gt_mask_of<CodeT>(w, p, code, gh) & ((1u << c) - 1u);
        if (m) {
          const int c2 = 31 - __clz(m);
          const int32_t lp = chunk_find<CodeT>(w, p, c2, code);
          j = lp >= 0 ? c2 * kChunk + lp : -1;
        }
      } else {  // spilled part: the summaries of the earlier chunks, latest first
        for (int c2 = c - 1; c2 >= 0 && j < 0; --c2) {
          const int32_t lp = chunk_find<CodeT>(w, p, c2, code);
          if (lp >= 0) j = c2 * kChunk + lp;
        }
      }
      if (j < 0) {
        const int64_t sl = lane_lookup(a, code, tag, h, first);
        src = sl >= 0 ? a.table + sl * a.stride + 16 : nullptr;
      }
    }
    if (j >= 0) src = a.values + (base + j) * a.vbytes;
  }
  wave_copy_rows(a, dst, src);
}

// The key of partition p with `code` at position lp of chunk c (its latest in the sub-call):
// finds the code's existing store entry or claims a slot, and names the copy the caller makes,
// `row` (the slot's value; null when the table is full) from `from` (the key's value). The
// lookups of this sub-call are over (previous kernel), and no other item looks for the same
// key, so the only thing a concurrent claim can be mistaken for is code 0 (a claimed slot
// whose code is not written yet reads as 0): code-0 keys wait for bulk_zero_kernel. Returns 1
// for a claim.
__device__ __forceinline__ int bulk_place_key(const StoreArgs& a, int64_t p, uint64_t code, int c,
                                              int32_t lp, uint8_t*& row, const uint8_t*& from) {
  const uint64_t tag = static_cast<uint64_t>(a.g0 + p) + 2;
  from = a.values + (p * a.T + a.s0 + c * kChunk + lp) * a.vbytes;
  int64_t s;
  const int r = lane_insert(a, code, tag, home_slot(code, tag - 2, a.cap), s);
  if (r < 0) atomicOr(a.full, 1);
  row = s >= 0 ? a.table + s * a.stride + 16 : nullptr;
  return r > 0 ? 1 : 0;
}

// bulk_place_key with the lane's own copy (for lanes that insert on their own).
__device__ __forceinline__ int bulk_insert_key(const StoreArgs& a, int64_t p, uint64_t code, int c,
                                               int32_t lp) {
  uint8_t* row;
  const uint8_t* from;
  const int r = bulk_place_key(a, p, code, c, lp, row, from);
  if (row) group_copy<1>(a, row, from, 0);
  return r;
}

// A code of the group table with its chunk mask and its latest key `pos` (a sub-call
// position, kept by the table kernel), which lies in the highest chunk of the mask. Names the
// copy as bulk_place_key does (`row` null: nothing to copy).
__device__ __forceinline__ int bulk_place_latest(const StoreArgs& a, int64_t p, uint64_t code,
                                                 uint32_t mask, uint32_t pos, uint8_t*& row,
                                                 const uint8_t*& from) {
  const int c2 = static_cast<int>(pos / kChunk);
  if (mask == 0 || c2 != 31 - __clz(mask)) {  // the two always agree; fail loudly if not
    atomicOr(a.full, 2);
    row = nullptr;
    return 0;
  }
  return bulk_place_key(a, p, code, c2, static_cast<int32_t>(pos % kChunk), row, from);
}

// bulk_place_latest with the lane's own copy.
__device__ __forceinline__ int bulk_insert_latest(const StoreArgs& a, int64_t p, uint64_t code,
                                                  uint32_t mask, uint32_t pos) {
  uint8_t* row;
  const uint8_t* from = nullptr;
  const int r = bulk_place_latest(a, p, code, mask, pos, row, from);
  if (row) group_copy<1>(a, row, from, 0);
  return r;
}

// One lane per entry of the group table; a workgroup's 256 entries lie in one part (parts are
// at least 256 entries). With 64-bit codes the first lane of the all-ones code's part also
// inserts that code (it has no entry). A spilled part's workgroups instead take the (chunk,
// summary slot) pairs of the partition whose code falls in the part and insert those whose
// code no later chunk holds. Each workgroup writes its number of claims to `claims`, and
// bulk_zero_kernel adds a partition's numbers to its count once: a partition's workgroups run
// close together in time, so atomics on its count would serialise.
template <typename CodeT>
__global__ __launch_bounds__(256) void bulk_insert_kernel(StoreArgs a, BulkWs w) {
  constexpr int kParts = GtTraits<CodeT>::kParts;
  __shared__ uint32_t n_claims;
  const CodeT SENT = sentinel<CodeT>();
  const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t p = g >> w.cap_log2;
  const int64_t in_p = g & (w.cap - 1);
  const int qt = static_cast<int>(in_p >> (w.cap_log2 - GtTraits<CodeT>::kPartLog2));
  const int64_t in_q = in_p & (w.sub - 1);
  if (threadIdx.x == 0) n_claims = 0;
  __syncthreads();
  int claimed = 0;
  if (!w.spilled[p * kParts + qt]) {  // the same for the whole workgroup
    uint8_t* row = nullptr;
    const uint8_t* from = nullptr;
    if constexpr (sizeof(CodeT) == 4) {
      const unsigned long long word = w.gt[g];
      if (word != 0 && gt_code(word) != 0)
        claimed = bulk_place_latest(a, p, gt_code(word), static_cast<uint32_t>(word >> 32),
                                    w.gpos[g], row, from);
    } else {
      const CodeT code = w.gt[g];
      if (code != SENT && code != 0)
        claimed = bulk_place_latest(a, p, code, w.gmask[g], w.gpos[g], row, from);
      if (in_q == 0 && gt_part<CodeT>(splitmix_fin(SENT)) == qt) {
        const uint32_t m = w.smask[p * kParts + qt];
        if (m) claimed += bulk_insert_latest(a, p, SENT, m, w.spos[p * kParts + qt]);
      }
    }
    wave_copy_rows(a, row, from);
  } else {
    const int per_chunk = kSlots + 1;
    for (int64_t q = in_q; q < static_cast<int64_t>(w.nch) * per_chunk; q += w.sub) {
      const int c = static_cast<int>(q / per_chunk);
      const int x = static_cast<int>(q - static_cast<int64_t>(c) * per_chunk);
      CodeT code;
      if (!summary_slot<CodeT>(w, p, c, x, code) || code == 0 ||
          gt_part<CodeT>(splitmix_fin(code)) != qt)
        continue;
      bool later = false;
      for (int c2 = c + 1; c2 < w.nch && !later; ++c2) later = chunk_find<CodeT>(w, p, c2, code) >= 0;
      if (later) continue;
      const int64_t sum = p * w.nch + c;
      claimed += bulk_insert_key(a, p, code, c, w.sum_pos[sum * kSumPos + x]);
    }
  }
  const unsigned long long b = __ballot(claimed != 0);
  uint32_t mine = claimed;
  for (int d = 32; d > 0; d >>= 1) mine += __shfl_xor(mine, d);  // claims of the wave
  if ((threadIdx.x & 63) == 0 && b != 0) atomicAdd(&n_claims, mine);
  __syncthreads();
  if (threadIdx.x == 0) w.claims[blockIdx.x] = n_claims;
}

// One workgroup per partition: the insert of code 0, then the partition's claims of the
// sub-call (its workgroup numbers, and code 0's) added to its count.
template <typename CodeT>
__global__ __launch_bounds__(256) void bulk_zero_kernel(StoreArgs a, BulkWs w, int32_t blocks_per_part) {
  constexpr int kParts = GtTraits<CodeT>::kParts;
  __shared__ uint32_t total;
  const int64_t p = blockIdx.x;
  const int t = threadIdx.x;
  if (t == 0) total = 0;
  __syncthreads();
  if (t == 0) {
    int r = 0;
    if (!w.spilled[p * kParts + gt_part<CodeT>(splitmix_fin(CodeT(0)))]) {
      const int64_t g = w.zero_slot[p];
      if (g >= 0) {
        const uint32_t m = sizeof(CodeT) == 4 ? static_cast<uint32_t>(w.gt[g] >> 32) : w.gmask[g];
        r = bulk_insert_latest(a, p, 0ull, m, w.gpos[g]);
      }
    } else {  // spilled part: code 0's latest chunk from the summaries
      for (int c = w.nch - 1; c >= 0; --c) {
        const int32_t lp = chunk_find<CodeT>(w, p, c, CodeT(0));
        if (lp >= 0) {
          r = bulk_insert_key(a, p, 0ull, c, lp);
          break;
        }
      }
    }
    if (r) atomicAdd(&total, 1u);
  }
  uint32_t sum = 0;
  for (int i = t; i < blocks_per_part; i += blockDim.x) sum += w.claims[p * blocks_per_part + i];
  if (sum) atomicAdd(&total, sum);
  __syncthreads();
  if (t == 0 && total) atomicAdd(&a.counts[a.g0 + p], static_cast<unsigned long long>(total));
}

// Workspace layout of a bulk call of P partitions (sub-calls of S positions).
struct BulkLayout {
  int64_t cap, cap_log2, nch, off_gmask, off_smask, off_spill, off_zero, off_scode, off_spos,
      off_src, off_qlist, off_qlpos, off_qcount, off_gpos, off_sposq, off_claims, off_filter,
      bytes;
};

int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }

BulkLayout bulk_layout(int64_t P, int64_t T, int32_t code_bytes) {
  BulkLayout L{};
  const int64_t parts = code_bytes == 4 ? GtTraits<uint32_t>::kParts : GtTraits<uint64_t>::kParts;
  const int64_t S = T < kBulkSpan ? T : kBulkSpan;
  L.cap = 256 * parts;
  L.cap_log2 = 8 + (parts == 8 ? 3 : 2);
  while (L.cap < 2 * S) {
    L.cap <<= 1;
    ++L.cap_log2;
  }
  L.nch = (S + kChunk - 1) / kChunk;
  int64_t o = align256(P * L.cap * 8);
  L.off_gmask = o;
  o += code_bytes == 8 ? align256(P * L.cap * 4) : 0;
  L.off_smask = o;
  o += align256(P * parts * 4);
  L.off_spill = o;
  o += align256(P * parts * 4);
  L.off_zero = o;
  o += align256(P * 8);
  L.off_scode = o;
  o += align256(P * L.nch * kSlots * code_bytes);
  L.off_spos = o;
  o += align256(P * L.nch * kSumPos * 4);
  L.off_src = o;
  o += align256(P * S * 4);
  L.off_qlist = o;
  o += align256(P * L.nch * parts * kChunk * code_bytes);
  L.off_qlpos = o;
  o += align256(P * L.nch * parts * kChunk * 2);
  L.off_qcount = o;
  o += align256(P * L.nch * parts * 4);
  L.off_gpos = o;
  o += align256(P * L.cap * 4);
  L.off_sposq = o;
  o += align256(P * parts * 4);
  L.off_claims = o;
  o += align256(P * L.cap / 256 * 4);
  L.off_filter = o;
  o += align256(P * parts * kFilterWordsQ * 4);
  L.bytes = o;
  return L;
}
static_assert(2 * kBulkSpan / GtTraits<uint32_t>::kParts <= GtTraits<uint32_t>::kPartMax &&
                  2 * kBulkSpan / GtTraits<uint64_t>::kParts <= GtTraits<uint64_t>::kPartMax,
              "a part fits the LDS table");

}  // namespace
}  // namespace lema

using namespace lema;

namespace {

// Bulk or chunked, by partitions P and positions T per call. A chunked launch runs one
// workgroup per partition, so with few partitions most of the chip idles through the T/1024
// launches in order, while the bulk kernels' costs per sub-call and per partition only pay
// off over long enough calls. Measured on one MI355X with 64-bit codes and 48- and 128-byte
// value rows, microseconds chunked / bulk, on a fresh table (every key claims a slot, as in a
// prefill) and on one already holding the keys (overwrites only):
//   T = 1024: claims 107 / 91 at 128 partitions, 274 / 383 at 1024; overwrites 42 / 49 at 24;
//   T = 2048: claims 205 / 116 at 128, 205 / 164 at 256, 241 / 335 and 427 / 401 at 512;
//             overwrites 85 / 56 at 24, 115 / 147 at 256;
//   T = 4096: claims 597 / 558 and 846 / 659 at 512, 1236 / 1032 and 1859 / 1300 at 1024;
//             overwrites 740 / 872 at 1024;
//   T = 16384: bulk ahead everywhere (overwrites at 1024 partitions: 3169 / 3011).
#ifdef LEMA_STEP_STAMPS
uint64_t* g_stamps = nullptr;  // where the decode steps of the diagnostics build write
int64_t g_stamp_step = 0;      // the next T == 1 exchange's row of that buffer
#endif

bool bulk_applies(int64_t P, int64_t T) {
  if (T <= 1024) return false;
  return P <= 128 || T > 2048;
}

template <typename CodeT>
int run_bulk(StoreArgs a, void* workspace, int64_t ws_bytes, hipStream_t st) {
  constexpr int kParts = GtTraits<CodeT>::kParts;
  const int64_t P = a.n / a.T;
  const BulkLayout L = bulk_layout(P, a.T, sizeof(CodeT));
  LEMA_REQUIRE(workspace != nullptr && ws_bytes >= L.bytes && aligned(workspace, 256),
               "workspace of %lld bytes (256-byte aligned) needed, got %lld", (long long)L.bytes,
               (long long)ws_bytes);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  BulkWs w{};
  w.gt = reinterpret_cast<unsigned long long*>(ws);
  w.gmask = reinterpret_cast<uint32_t*>(ws + L.off_gmask);
  w.smask = reinterpret_cast<uint32_t*>(ws + L.off_smask);
  w.spilled = reinterpret_cast<int32_t*>(ws + L.off_spill);
  w.zero_slot = reinterpret_cast<int64_t*>(ws + L.off_zero);
  w.sum_code = ws + L.off_scode;
  w.sum_pos = reinterpret_cast<int32_t*>(ws + L.off_spos);
  w.src_in = reinterpret_cast<int32_t*>(ws + L.off_src);
  w.qlist = ws + L.off_qlist;
  w.qlpos = reinterpret_cast<uint16_t*>(ws + L.off_qlpos);
  w.qcount = reinterpret_cast<int32_t*>(ws + L.off_qcount);
  w.gpos = reinterpret_cast<uint32_t*>(ws + L.off_gpos);
  w.spos = reinterpret_cast<uint32_t*>(ws + L.off_sposq);
  w.claims = reinterpret_cast<uint32_t*>(ws + L.off_claims);
  w.filter = reinterpret_cast<uint32_t*>(ws + L.off_filter);
  w.cap = static_cast<int32_t>(L.cap);
  w.cap_log2 = static_cast<int32_t>(L.cap_log2);
  w.sub = static_cast<int32_t>(L.cap / kParts);
  const int32_t blocks_per_part = static_cast<int32_t>(L.cap / 256);  // whole: cap >= 256 * kParts
  for (int64_t s0 = 0; s0 < a.T; s0 += kBulkSpan) {
    a.s0 = s0;
    a.len = static_cast<int32_t>(a.T - s0 < kBulkSpan ? a.T - s0 : kBulkSpan);
    w.nch = (a.len + kChunk - 1) / kChunk;
    bulk_chunk_kernel<CodeT><<<dim3(P * w.nch), dim3(kThreads), 0, st>>>(a, w);
    if (int rc = launch_status("bulk_chunk_kernel")) return rc;
    bulk_table_kernel<CodeT><<<dim3(P * kParts), dim3(kTableThreads), 0, st>>>(w);
    if (int rc = launch_status("bulk_table_kernel")) return rc;
    if (a.qc != nullptr) {
      bulk_query_kernel<CodeT><<<dim3((P * a.len + 255) / 256), dim3(256), 0, st>>>(a, w);
      if (int rc = launch_status("bulk_query_kernel")) return rc;
    }
    bulk_insert_kernel<CodeT><<<dim3(P * blocks_per_part), dim3(256), 0, st>>>(a, w);
    if (int rc = launch_status("bulk_insert_kernel")) return rc;
    bulk_zero_kernel<CodeT><<<dim3(P), dim3(256), 0, st>>>(a, w, blocks_per_part);
    if (int rc = launch_status("bulk_zero_kernel")) return rc;
  }
  return LEMA_OK;
}

// Whether `table` is host memory (a pinned table the kernels reach over the host link). The
// answer for the calling thread's last table is kept, so a run of decode steps asks HIP once;
// a table freed and another allocated at the same address could only get the other window
// width, never a wrong result. A pointer HIP does not know counts as device memory, and the
// error the query leaves is cleared so that it is not reported for the next launch.
bool table_in_host_memory(const void* table) {
  static thread_local const void* last = nullptr;
  static thread_local bool last_host = false;
  if (table != last) {
    hipPointerAttribute_t at{};
    const hipError_t e = hipPointerGetAttributes(&at, table);
    if (e != hipSuccess) (void)hipGetLastError();
    last_host = e == hipSuccess && at.type == hipMemoryTypeHost;
    last = table;
  }
  return last_host;
}

int store_exchange(void* table, int64_t cap, int64_t vbytes, const void* qc, const void* kc,
                   int32_t code_bytes, const void* values, void* out, int64_t n, int64_t T,
                   int64_t g0, int64_t* counts, int32_t* full, void* workspace, int64_t ws_bytes,
                   void* stream) {
  clear_error();
  LEMA_REQUIRE(cap >= 1, "capacity must be positive, got %lld", (long long)cap);
  LEMA_REQUIRE(vbytes > 0 && vbytes % 8 == 0,
               "value row of %lld bytes breaks slot alignment (must be a multiple of 8)",
               (long long)vbytes);
  LEMA_REQUIRE(code_bytes == 4 || code_bytes == 8, "code_bytes must be 4 or 8, got %d", code_bytes);
  LEMA_REQUIRE(T > 0 && n >= 0 && n % T == 0, "items must be partitions x T (n=%lld, T=%lld)",
               (long long)n, (long long)T);
  LEMA_REQUIRE(g0 >= 0, "negative group offset");
  if (n == 0) return LEMA_OK;
  LEMA_REQUIRE(table != nullptr && kc != nullptr && values != nullptr && counts != nullptr &&
                   full != nullptr, "null pointer");
  LEMA_REQUIRE(qc == nullptr || out != nullptr, "queries need an output buffer");
  LEMA_REQUIRE(aligned(table, 8) && aligned(kc, code_bytes) && aligned(values, 8) &&
                   aligned(counts, 8) && aligned(full, 4) &&
                   (qc == nullptr || (aligned(qc, code_bytes) && aligned(out, 8))),
               "misaligned pointer");
  StoreArgs a{};
  a.table = static_cast<uint8_t*>(table);
  a.cap = cap;
  a.stride = 16 + vbytes;
  a.vbytes = vbytes;
  a.qc = qc;
  a.kc = kc;
  a.code_bytes = code_bytes;
  a.values = static_cast<const uint8_t*>(values);
  a.out = static_cast<uint8_t*>(out);
  a.n = n;
  a.T = T;
  a.g0 = g0;
  a.counts = reinterpret_cast<unsigned long long*>(counts);
  a.full = full;
#ifdef LEMA_STEP_STAMPS
  a.stamps = T == 1 ? g_stamps : nullptr;
  a.stamp_step = a.stamps != nullptr ? g_stamp_step++ : 0;
#endif
  const bool p16 = vbytes % 16 == 0 && aligned(table, 16) && aligned(values, 16) &&
                   (out == nullptr || aligned(out, 16));
  a.piece = p16 ? 16 : 8;
  a.pieces = static_cast<int32_t>(vbytes / a.piece);
  a.pre = false;  // set for a decode step below
  a.spec = p16 && a.pieces <= kSpecPieces;
  a.cg_log2 = 0;
  while ((1 << a.cg_log2) < a.pieces && a.cg_log2 < 4) ++a.cg_log2;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t P = n / T;
  if (T == 1) {
    const bool host = table_in_host_memory(table);
    const int G = host ? kStepGroupHost : kStepGroup;
    a.pre = p16 && a.pieces <= G;
    const int64_t threads = n * G;
    const int64_t grid = (threads + kStepBlock - 1) / kStepBlock;
    LEMA_REQUIRE(grid < (int64_t(1) << 31), "too many items (%lld)", (long long)n);
    if (host)
      store_step_kernel<kStepGroupHost><<<dim3(grid), dim3(kStepBlock), 0, st>>>(a);
    else
      store_step_kernel<kStepGroup><<<dim3(grid), dim3(kStepBlock), 0, st>>>(a);
    return launch_status("store_step_kernel");
  }
  LEMA_REQUIRE(P < (int64_t(1) << 31), "too many partitions (%lld)", (long long)P);
  if (workspace != nullptr && bulk_applies(P, T)) {
    LEMA_REQUIRE(P < (int64_t(1) << 31) - 1 && P * (T < kBulkSpan ? T : kBulkSpan) < (int64_t(1) << 31),
                 "too many items per sub-call (%lld partitions)", (long long)P);
    return code_bytes == 4 ? run_bulk<uint32_t>(a, workspace, ws_bytes, st)
                           : run_bulk<uint64_t>(a, workspace, ws_bytes, st);
  }
  for (int64_t s0 = 0; s0 < T; s0 += kChunk) {
    a.s0 = s0;
    a.len = static_cast<int32_t>(T - s0 < kChunk ? T - s0 : kChunk);
    if (code_bytes == 4)
      store_chunk_kernel<uint32_t><<<dim3(P), dim3(kThreads), 0, st>>>(a);
    else
      store_chunk_kernel<uint64_t><<<dim3(P), dim3(kThreads), 0, st>>>(a);
    if (int rc = launch_status("store_chunk_kernel")) return rc;
  }
  return LEMA_OK;
}

}  // namespace

extern "C" int lema_store_exchange(void* table, int64_t cap, int64_t vbytes, const void* qc,
                                   const void* kc, int32_t code_bytes, const void* values,
                                   void* out, int64_t n, int64_t T, int64_t g0, int64_t* counts,
                                   int32_t* full, void* stream) {
  return store_exchange(table, cap, vbytes, qc, kc, code_bytes, values, out, n, T, g0, counts,
                        full, nullptr, 0, stream);
}

extern "C" int64_t lema_store_workspace_bytes(int64_t n, int64_t T, int32_t code_bytes) {
  if (T <= 0 || n <= 0 || n % T != 0 || (code_bytes != 4 && code_bytes != 8) ||
      !bulk_applies(n / T, T))
    return 0;
  return bulk_layout(n / T, T, code_bytes).bytes;
}

extern "C" int lema_store_exchange_ws(void* table, int64_t cap, int64_t vbytes, const void* qc,
                                      const void* kc, int32_t code_bytes, const void* values,
                                      void* out, int64_t n, int64_t T, int64_t g0, int64_t* counts,
                                      int32_t* full, void* workspace, int64_t workspace_bytes,
                                      void* stream) {
  return store_exchange(table, cap, vbytes, qc, kc, code_bytes, values, out, n, T, g0, counts,
                        full, workspace, workspace_bytes, stream);
}

// ---- the exchange without a workspace argument and without allocation ----
//
// The bulk path's workspace lives in `scratch`, one file-scope device array per GPU, held
// until the process ends. Host code never passes `scratch` itself (in host code the name is a
// host-side stand-in, not a device address): its address on a device is looked up once per
// device with hipGetSymbolAddress, with that device current, and kept in scratch_ptr[].
// Every call on a device shares its array and no call clears it (the bulk kernels rewrite
// every word they read within a sub-call), so calls that overlap on one device -- on two
// streams, or from two threads -- race; calls in one stream's order do not.
constexpr int64_t kNoAllocScratchBytes = LEMA_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
uint8_t* scratch_ptr[kMaxDevices];
std::mutex scratch_mutex;

// The device-side address of `scratch` on the device `stream` belongs to (the current device
// for the null stream), looked up on the first call for that device.
int scratch_address(hipStream_t st, uint8_t** out) {
  int dev = 0;
  if (st != nullptr) {
    LEMA_HIP_CHECK(hipStreamGetDevice(st, &dev));
  } else {
    LEMA_HIP_CHECK(hipGetDevice(&dev));
  }
  LEMA_REQUIRE(dev >= 0 && dev < kMaxDevices, "device %d beyond the %d this library tracks",
               dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(scratch_mutex);
  if (scratch_ptr[dev] == nullptr) {
    int cur = 0;
    LEMA_HIP_CHECK(hipGetDevice(&cur));
    if (cur != dev) LEMA_HIP_CHECK(hipSetDevice(dev));
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) LEMA_HIP_CHECK(hipSetDevice(cur));
    LEMA_HIP_CHECK(e);
    LEMA_REQUIRE(p != nullptr && aligned(p, 256), "scratch of device %d is misaligned", dev);
    scratch_ptr[dev] = static_cast<uint8_t*>(p);
  }
  *out = scratch_ptr[dev];
  return LEMA_OK;
}

}  // namespace

extern "C" int lema_store_exchange_noalloc(void* table, int64_t cap, int64_t vbytes,
                                           const void* qc, const void* kc, int32_t code_bytes,
                                           const void* values, void* out, int64_t n, int64_t T,
                                           int64_t g0, int64_t* counts, int32_t* full,
                                           void* stream) {
  clear_error();
  LEMA_REQUIRE(code_bytes == 4 || code_bytes == 8, "code_bytes must be 4 or 8, got %d", code_bytes);
  LEMA_REQUIRE(T > 0 && n >= 0 && n % T == 0, "items must be partitions x T (n=%lld, T=%lld)",
               (long long)n, (long long)T);
  LEMA_REQUIRE(vbytes > 0 && vbytes % 8 == 0,
               "value row of %lld bytes breaks slot alignment (must be a multiple of 8)",
               (long long)vbytes);
  const int64_t P = n / T;
  if (n == 0 || !bulk_applies(P, T))      // decode steps and chunked calls use no scratch
    return store_exchange(table, cap, vbytes, qc, kc, code_bytes, values, out, n, T, g0, counts,
                          full, nullptr, 0, stream);
  // Partitions never read one another's entries, so a call may run as consecutive slices of
  // its partitions, each small enough for the scratch (bulk_applies holds for every slice:
  // a slice is never longer and never has more partitions than the call).
  const int64_t one = bulk_layout(1, T, code_bytes).bytes;
  LEMA_REQUIRE(one <= kNoAllocScratchBytes,
               "a partition of %lld positions needs %lld bytes of scratch, more than the %lld "
               "this entry point has", (long long)T, (long long)one,
               (long long)kNoAllocScratchBytes);
  int64_t most = kNoAllocScratchBytes / one;
  if (most > P) most = P;
  while (bulk_layout(most, T, code_bytes).bytes > kNoAllocScratchBytes) --most;
  const int64_t slices = (P + most - 1) / most;
  const int64_t per = (P + slices - 1) / slices;
  uint8_t* ws = nullptr;
  if (int rc = scratch_address(static_cast<hipStream_t>(stream), &ws)) return rc;
  for (int64_t p0 = 0; p0 < P; p0 += per) {
    const int64_t ps = P - p0 < per ? P - p0 : per;
    const int64_t i0 = p0 * T;
    const void* q = qc != nullptr ? static_cast<const uint8_t*>(qc) + i0 * code_bytes : nullptr;
    void* o = out != nullptr ? static_cast<uint8_t*>(out) + i0 * vbytes : nullptr;
    if (int rc = store_exchange(table, cap, vbytes, q, static_cast<const uint8_t*>(kc) +
                                    i0 * code_bytes, code_bytes,
                                static_cast<const uint8_t*>(values) + i0 * vbytes, o, ps * T, T,
                                g0 + p0, counts, full, ws, kNoAllocScratchBytes, stream))
      return rc;
  }
  return LEMA_OK;
}

#ifdef LEMA_STEP_STAMPS
// ---- diagnostics build only: decode-step timestamps and the graph-node floor ----
// Every T == 1 exchange enqueued after this call (a graph capture included) writes its
// items' five clock readings to row k of `stamps` ([steps][n][5] uint64, device memory), k
// counting those exchanges from 0; NULL stops it.
extern "C" void lema_debug_step_stamps(void* stamps) {
  g_stamps = static_cast<uint64_t*>(stamps);
  g_stamp_step = 0;
}

__global__ __launch_bounds__(kStepBlock) void empty_step_kernel(int64_t n) {
  (void)n;
}

// A kernel with a decode step's grid for n items that does nothing: the cost of a graph node.
extern "C" int lema_debug_empty_step(int64_t n, void* stream) {
  const int64_t grid = (n * kStepGroup + kStepBlock - 1) / kStepBlock;
  empty_step_kernel<<<dim3(grid), dim3(kStepBlock), 0, static_cast<hipStream_t>(stream)>>>(n);
  return launch_status("empty_step_kernel");
}
#endif
