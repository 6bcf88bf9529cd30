// Device building blocks of the latest-match resolver, shared by the prefill kernels
// (resolve.hip) and the store's in-chunk resolution (store.hip). The design is described at the
// top of resolve.hip.
#pragma once
#include <type_traits>

#include "lema_internal.h"

namespace lema {
namespace {

template <typename CodeT>
__device__ __forceinline__ CodeT sentinel() {
  return static_cast<CodeT>(~static_cast<CodeT>(0));
}

__device__ __forceinline__ uint32_t lds_cas(uint32_t* p, uint32_t cmp, uint32_t val) {
  return atomicCAS(p, cmp, val);
}
__device__ __forceinline__ uint64_t lds_cas(uint64_t* p, uint64_t cmp, uint64_t val) {
  return atomicCAS(reinterpret_cast<unsigned long long*>(p),
                   static_cast<unsigned long long>(cmp), static_cast<unsigned long long>(val));
}

// 32 bits of a code for hashing (equality always compares the whole code).
__device__ __forceinline__ uint32_t fold(uint32_t c) { return c; }
__device__ __forceinline__ uint32_t fold(uint64_t c) {
  return static_cast<uint32_t>(c) ^ static_cast<uint32_t>(c >> 32);
}

// Fibonacci hashing, then Lemire's fastrange into [0, n) (n need not be a power of two).
template <int N>
__device__ __forceinline__ int bucket_of(uint32_t x) {
  return static_cast<int>(__umulhi(x * 0x9E3779B1u, static_cast<uint32_t>(N)));
}

// Resolver geometry: 256 threads (4 wavefronts) own a chunk of 1024 query positions, 4 per
// thread. Position o of the chunk is handled by thread o % 256 as its (o / 256)-th position,
// so the 64 positions of a "word" o / 64 are the 64 lanes of one wavefront.
constexpr int kThreads = 256;
constexpr int kPer = 4;
constexpr int kChunk = kThreads * kPer;
#ifndef LEMA_RESOLVE_SLOTS
#define LEMA_RESOLVE_SLOTS 2048
#endif
#ifndef LEMA_RESOLVE_PREFETCH
#define LEMA_RESOLVE_PREFETCH 1
#endif
#ifndef LEMA_RESOLVE_MAP_SLOTS
#define LEMA_RESOLVE_MAP_SLOTS 1536
#endif
constexpr int kPrefetch = LEMA_RESOLVE_PREFETCH;  // key batches loaded ahead of the lookups
constexpr int kSlots = LEMA_RESOLVE_SLOTS;  // query-code table: at most kChunk codes
constexpr int kBuckets = kSlots / 4;
constexpr int kMapSlots = LEMA_RESOLVE_MAP_SLOTS;  // (code slot, word) -> lane mask: at most
constexpr int kMapBuckets = kMapSlots / 4;          // kChunk keys
static_assert(kSlots > kChunk && kSlots % 4 == 0 && kMapSlots > kChunk && kMapSlots % 4 == 0,
              "tables must keep free slots");
constexpr uint32_t kMapEmpty = 0xFFFFFFFFu;
static_assert(kChunk / 64 <= 16, "word summary is a 16-bit mask");

// A one-hash bit filter of the chunk's query codes (8192 bits for at most 1024 codes): a key
// whose bit is clear carries no query code, and skips the table lookup. Keys of codes that
// seldom repeat (pre-activation codes of a language model) then cost one 4-byte LDS read
// each. LEMA_RESOLVE_FILTER: 0 never, 1 always, 2 in chunks of more than kFilterMinCodes
// distinct query codes (on Zipf-distributed codes, ~370 per chunk, the filter passes most
// keys and only adds a read). Chunks with the filter scan their earlier keys through the
// wider filter below, use that one for their own keys too, and do not build this one.
#ifndef LEMA_RESOLVE_FILTER
#define LEMA_RESOLVE_FILTER 2
#endif
constexpr int kFilterWords = 256;
constexpr int kFilterMinCodes = 512;  // used by chunks with more distinct query codes than this
__device__ __forceinline__ uint32_t filter_hash(uint32_t h) { return (h * 0x2C1B3C6Du) >> 19; }
// The wider filter of the queued scan (one bit per code among 32768: about 3% of the keys of
// codes no query of the chunk carries pass it, against 12% for the 8192 bits above), and the
// capacity of a wavefront's queue: a batch adds at most 4 * 64 keys, so a queue is looked up
// once it holds more than kQueueCap - 256.
constexpr int kWideBits = 32768;
constexpr int kQueueCap = 384;
constexpr int kScanGroup = 4;  // key batches whose loads the queued scan issues together
// With chunk summaries, a chunk with the filter still scans through the queue, ignoring the
// summaries, when more than this many of its codes are distinct. Codes that nearly never repeat
// (uniform codes: 1014-1024 distinct per chunk) leave almost every query without an in-chunk
// answer and without an early hit in the summaries, and probing every earlier chunk's summary
// for each of them cost 5-6.5x the queued scan (32 rows x T = 65536: 701 against 129 us;
// 16 x 262144: 3431 against 526 us). Zipf codes over 4096 values (585-668 distinct per chunk)
// find their latest key a few chunks back, where the summaries win (16 x 262144: 441 against
// 879 us).
constexpr int kQueueSummMinCodes = 896;
// The scan tests every earlier key with it, so it avoids the quarter-rate 32-bit multiply:
// the high half is folded into the low 24 bits, which a full-rate 24-bit multiply mixes.
// (__umul24 is declared to return int: the product is shifted as unsigned.)
__device__ __forceinline__ uint32_t wide_hash(uint32_t h) {
  return static_cast<uint32_t>(__umul24((h ^ (h >> 16)) & 0xFFFFFFu, 0x9E3779u)) >> 17;
}

template <typename CodeT>
struct ResolveLds {
  alignas(16) uint64_t mbits[kMapSlots];  // lanes of that word whose key carries that code
  alignas(16) CodeT code[kSlots];         // query code of a slot, sentinel() = free
  alignas(16) uint32_t mkey[kMapSlots];   // code slot << 4 | word, kMapEmpty = free
  alignas(16) int32_t pos[kSlots + 1];  // latest key position before the chunk, -1 = none;
                                        // the entry [kSlots] here and in summ belongs to the
                                        // sentinel code itself
  alignas(16) uint16_t summ[kSlots + 2];  // bit w: word w of the chunk holds a key with this
                                          // code; updated as 32-bit pairs
  alignas(16) uint32_t qbits[kFilterWords];  // bit filter_hash(c) set for every query code c of
                                             // the chunk
  int32_t sent_used;
  int32_t nq;     // distinct query codes of the chunk (the all-ones code aside)
  int32_t nneed;  // query codes that need their latest key before the chunk (summary path)
  int32_t khit;   // some key of the chunk carries a query code of the chunk (queued scan)
};
// The queued scan borrows the map (each wavefront's queue: codes in mbits, positions in mkey)
// and the word summaries (the wide filter) before the chunk's keys fill them.
static_assert(kMapSlots * 8 >= (kThreads / 64) * kQueueCap * 8 &&
                  kMapSlots * 4 >= (kThreads / 64) * kQueueCap * 4 &&
                  (kSlots + 1) * 2 >= kWideBits / 8,
              "the queued scan's borrowed LDS");

// The 4 slots of bucket b, one (u32 codes) or two (u64 codes) 16-byte LDS reads.
template <typename CodeT>
__device__ __forceinline__ void read_bucket(const CodeT* base, int b, CodeT (&x)[4]) {
  if constexpr (sizeof(CodeT) == 4) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(base + 4 * b);
    x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
  } else {
    const u32x4 v0 = *reinterpret_cast<const u32x4*>(base + 4 * b);
    const u32x4 v1 = *reinterpret_cast<const u32x4*>(base + 4 * b + 2);
    x[0] = (uint64_t(v0.y) << 32) | v0.x; x[1] = (uint64_t(v0.w) << 32) | v0.z;
    x[2] = (uint64_t(v1.y) << 32) | v1.x; x[3] = (uint64_t(v1.w) << 32) | v1.z;
  }
}

// The filled slots of a bucket are always a prefix of its 4: an insert claims the first free
// slot it saw, slots are never freed, and a claim that loses its slot reads the bucket again.
// So a bucket whose last slot is free has room (a probe sequence ends there), and its first
// free slot is the number of filled ones. A key is in at most one slot.
// Slot of `key` among the bucket's 4, or -1, without branches; `open` gets whether the bucket
// has room.
template <typename KeyT>
__device__ __forceinline__ int match4(const KeyT (&x)[4], KeyT key, KeyT empty, bool& open) {
  open = x[3] == empty;
  const bool m1 = x[1] == key, m2 = x[2] == key, m3 = x[3] == key;
  const int e = (m1 ? 1 : 0) | (m2 ? 2 : 0) | (m3 ? 3 : 0);
  return x[0] == key || m1 || m2 || m3 ? e : -1;
}

// Insert `key` into a table of NB buckets (or find it), probing from bucket b: returns its
// slot; `inserted` tells whether this call put it there. The table must have an empty slot
// somewhere (load < 1 here). Torn 8-byte reads are re-checked atomically.
template <typename KeyT, int NB>
__device__ __forceinline__ int table_claim_loop(KeyT* base, KeyT key, KeyT empty, int b,
                                                bool& inserted) {
  inserted = false;
  for (;;) {
    KeyT x[4];
    read_bucket(base, b, x);
    bool open;
    const int e = match4(x, key, empty, open);
    if (e >= 0) {
      if (sizeof(KeyT) == 4 || lds_cas(&base[4 * b + e], key, key) == key) return 4 * b + e;
      continue;  // a torn read of a slot being written: read the bucket again
    }
    if (!open) {
      b = b + 1 == NB ? 0 : b + 1;
      continue;
    }
    const int f = (x[0] != empty ? 1 : 0) + (x[1] != empty ? 1 : 0) + (x[2] != empty ? 1 : 0);
    const KeyT old = lds_cas(&base[4 * b + f], empty, key);
    if (old == empty) inserted = true;
    if (old == empty || old == key) return 4 * b + f;
    // another key took that slot first: read the same bucket again
  }
}

// table_claim_loop with its first round written out: one bucket read, then either the key's
// slot or one CAS at the bucket's first free slot, without the loop's branches. Lanes that
// meet a full bucket, a lost CAS or (8-byte keys) a torn read go on in the loop, behind a
// branch that is uniform across the lanes taking part.
template <typename KeyT, int NB>
__device__ __forceinline__ int table_claim(KeyT* base, KeyT key, KeyT empty, int b,
                                           bool& inserted) {
  KeyT x[4];
  read_bucket(base, b, x);
  bool open;
  const int e = match4(x, key, empty, open);
  const int f = (x[0] != empty ? 1 : 0) + (x[1] != empty ? 1 : 0) + (x[2] != empty ? 1 : 0);
  int slot = -1;
  inserted = false;
  if (e >= 0) {
    if (sizeof(KeyT) == 4 || lds_cas(&base[4 * b + e], key, key) == key) slot = 4 * b + e;
  } else if (open) {
    const KeyT old = lds_cas(&base[4 * b + f], empty, key);
    inserted = old == empty;
    if (old == empty || old == key) slot = 4 * b + f;
  }
  if (__ballot(slot < 0) != 0 && slot < 0) slot = table_claim_loop<KeyT, NB>(base, key, empty, b, inserted);
  return slot;
}

// Finish a lookup whose first bucket b was read into x: slot of key, or -1 (no concurrent
// writers: the table is read only after the barrier that ends its construction).
template <typename KeyT, int NB>
__device__ __forceinline__ int table_find(const KeyT* base, KeyT key, KeyT empty, int b,
                                          KeyT (&x)[4]) {
  for (;;) {
    bool open;
    const int e = match4(x, key, empty, open);
    if (e >= 0) return 4 * b + e;
    if (open) return -1;
    b = b + 1 == NB ? 0 : b + 1;
    read_bucket(base, b, x);
  }
}

// Arguments of the gather half. Strides and row sizes are in BYTES.
struct GatherArgs {
  const uint8_t* v;
  uint8_t* y;
  int64_t H, T;
  int64_t v_sb, v_sh, v_st;
  int64_t y_sb, y_sh, y_st;
  uint32_t pieces;  // 16/8/4/2-byte pieces per value row
  FastDiv pdiv;     // division by `pieces`
  int32_t miss;
  int32_t dtype;
  int32_t nt;  // non-temporal stores of y (rows of y adjacent); plain stores let L2 merge the
               // pieces of interleaved rows (y viewed from [B, T, H * dv]) into whole lines
};

struct ResolveArgs {
  const void* qc;
  const void* kc;
  int64_t N, T;
  int32_t nchunks;
  int32_t kvec;  // key rows allow 16-byte loads of 4 consecutive codes
  void* src;     // optional
  int32_t src_bytes;
  // Chunk summaries (optional): per (row, chunk) a table of kSumSlots entries, one per
  // distinct key code of the chunk, and the latest position of the all-ones code. With them,
  // keys before a chunk are found by probing the summaries of earlier chunks instead of
  // scanning every earlier key.
  uint32_t* summ_tab;
  int32_t* summ_sent;
  int32_t group;  // workgroup order: 8 consecutive rows per XCD, one chunk of all 8 in a row
  GatherArgs g;
};

// ------------------------------------------------------------------ chunk summaries
// Entry of a summary table: (fingerprint << 10) | position in the chunk, kSumEmpty = free.
// The table is the image of an LDS table keyed by the whole code (4-slot buckets from
// bucket_of, linear probing), so a lookup visits the code's slot before any free slot. The
// fingerprint only filters: every candidate is confirmed against the key code itself.
constexpr int kSumSlots = 2048;
constexpr int kSumBuckets = kSumSlots / 4;
constexpr uint32_t kSumEmpty = 0xFFFFFFFFu;
static_assert(kSumSlots > 1024, "a summary table keeps free slots");

// 22-bit fingerprint: the MurmurHash3 32-bit finaliser of the folded code, top bits; never
// the all-ones value (that entry would read as free).
__device__ __forceinline__ uint32_t fingerprint(uint32_t h) {
  h ^= h >> 16;
  h *= 0x85EBCA6Bu;
  h ^= h >> 13;
  h *= 0xC2B2AE35u;
  h ^= h >> 16;
  const uint32_t f = h >> 10;
  return f == 0x3FFFFFu ? 0x3FFFFEu : f;
}

// Latest position of code x in full chunk cc of a row (krow = the row's keys), or -1, from
// the chunk's summary table tab, whose bucket b0 is already in e.
template <typename CodeT>
__device__ __forceinline__ int32_t summary_probe(const uint32_t* tab, const CodeT* krow, int cc,
                                                 CodeT x, uint32_t fp, int b0, u32x4 e) {
  int b = b0;
  for (;;) {
    const uint32_t ent[4] = {e.x, e.y, e.z, e.w};
    bool open = false;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (ent[i] == kSumEmpty) {
        open = true;
      } else if ((ent[i] >> 10) == fp) {
        const int32_t j = cc * 1024 + static_cast<int32_t>(ent[i] & 1023u);
        if (krow[j] == x) return j;
      }
    }
    if (open) return -1;
    b = b + 1 == kSumBuckets ? 0 : b + 1;
    e = *reinterpret_cast<const u32x4*>(tab + 4 * b);
  }
}

// Latest key position before chunk `chunk` of row `row` for code x (sent: x is the all-ones
// code), or -1: the summaries of the earlier chunks are probed latest first, 8 at a time
// with their first buckets loaded together.
template <typename CodeT>
__device__ __forceinline__ int32_t before_chunk(const ResolveArgs& a, int64_t row, int chunk, CodeT x, bool sent) {
  constexpr int kAhead = 8;
  const int64_t rc = row * a.nchunks;
  if (sent) {
    for (int cb = chunk - 1; cb >= 0; cb -= kAhead) {
      int32_t v[kAhead];
#pragma unroll
      for (int i = 0; i < kAhead; ++i) v[i] = cb - i >= 0 ? a.summ_sent[rc + cb - i] : -1;
#pragma unroll
      for (int i = 0; i < kAhead; ++i)
        if (v[i] >= 0) return (cb - i) * 1024 + v[i];
    }
    return -1;
  }
  const CodeT* krow = static_cast<const CodeT*>(a.kc) + row * a.T;
  const uint32_t fp = fingerprint(fold(x));
  const int b0 = bucket_of<kSumBuckets>(fold(x));
  for (int cb = chunk - 1; cb >= 0; cb -= kAhead) {
    u32x4 e[kAhead];
#pragma unroll
    for (int i = 0; i < kAhead; ++i)
      e[i] = cb - i >= 0 ? *reinterpret_cast<const u32x4*>(a.summ_tab + (rc + cb - i) * kSumSlots + 4 * b0)
                         : u32x4{kSumEmpty, kSumEmpty, kSumEmpty, kSumEmpty};
#pragma unroll
    for (int i = 0; i < kAhead; ++i) {
      if (cb - i < 0) break;
      const int32_t j = summary_probe(a.summ_tab + (rc + cb - i) * kSumSlots, krow, cb - i, x,
                                      fp, b0, e[i]);
      if (j >= 0) return j;
    }
  }
  return -1;
}

// ------------------------------------------------------------------ miss fill (dense path)
// y = v[row, 0] * 0 in the value dtype: a zero with v's sign, a quiet NaN for NaN (payload
// kept) and the default NaN for +-inf.
__device__ __forceinline__ uint32_t miss_half(uint32_t h, uint32_t e, uint32_t m, uint32_t q,
                                              uint32_t nan) {
  if ((h & e) == e) return (h & m) ? (h | q) : nan;
  return h & 0x8000u;
}

__device__ __forceinline__ uint32_t miss_word(uint32_t w, int32_t dtype) {
  if (dtype == LEMA_F32) {
    if ((w & 0x7F800000u) == 0x7F800000u) return (w & 0x007FFFFFu) ? (w | 0x00400000u) : 0x7FC00000u;
    return w & 0x80000000u;
  }
  const uint32_t e = dtype == LEMA_BF16 ? 0x7F80u : 0x7C00u;
  const uint32_t m = dtype == LEMA_BF16 ? 0x007Fu : 0x03FFu;
  const uint32_t q = dtype == LEMA_BF16 ? 0x0040u : 0x0200u;
  const uint32_t nan = dtype == LEMA_BF16 ? 0x7FC0u : 0x7E00u;
  return miss_half(w & 0xFFFFu, e, m, q, nan) | (miss_half(w >> 16, e, m, q, nan) << 16);
}

template <int VEC>
struct Piece;
template <>
struct Piece<16> {
  typedef u32x4 T;
  static __device__ __forceinline__ T load(const uint8_t* p) { return *reinterpret_cast<const T*>(p); }
  template <bool NT>
  static __device__ __forceinline__ void store(uint8_t* p, T v) {
    if constexpr (NT)
      __builtin_nontemporal_store(v, reinterpret_cast<T*>(p));
    else
      *reinterpret_cast<T*>(p) = v;
  }
  static __device__ __forceinline__ T zero() { return T{0u, 0u, 0u, 0u}; }
  static __device__ __forceinline__ T miss(T v, int32_t d) {
    return T{miss_word(v.x, d), miss_word(v.y, d), miss_word(v.z, d), miss_word(v.w, d)};
  }
};
template <>
struct Piece<8> {
  typedef u32x2 T;
  static __device__ __forceinline__ T load(const uint8_t* p) { return *reinterpret_cast<const T*>(p); }
  template <bool NT>
  static __device__ __forceinline__ void store(uint8_t* p, T v) {
    if constexpr (NT)
      __builtin_nontemporal_store(v, reinterpret_cast<T*>(p));
    else
      *reinterpret_cast<T*>(p) = v;
  }
  static __device__ __forceinline__ T zero() { return T{0u, 0u}; }
  static __device__ __forceinline__ T miss(T v, int32_t d) { return T{miss_word(v.x, d), miss_word(v.y, d)}; }
};
template <>
struct Piece<4> {
  typedef uint32_t T;
  static __device__ __forceinline__ T load(const uint8_t* p) { return *reinterpret_cast<const T*>(p); }
  template <bool NT>
  static __device__ __forceinline__ void store(uint8_t* p, T v) {
    if constexpr (NT)
      __builtin_nontemporal_store(v, reinterpret_cast<T*>(p));
    else
      *reinterpret_cast<T*>(p) = v;
  }
  static __device__ __forceinline__ T zero() { return 0u; }
  static __device__ __forceinline__ T miss(T v, int32_t d) { return miss_word(v, d); }
};
template <>
struct Piece<2> {
  typedef uint16_t T;
  static __device__ __forceinline__ T load(const uint8_t* p) { return *reinterpret_cast<const T*>(p); }
  template <bool NT>
  static __device__ __forceinline__ void store(uint8_t* p, T v) {
    if constexpr (NT)
      __builtin_nontemporal_store(v, reinterpret_cast<T*>(p));
    else
      *reinterpret_cast<T*>(p) = v;
  }
  static __device__ __forceinline__ T zero() { return 0; }
  static __device__ __forceinline__ T miss(T v, int32_t d) {
    return static_cast<T>(miss_word(v, d) & 0xFFFFu);  // 2-byte pieces only for 16-bit dtypes
  }
};

// Copy the value rows of `nrows` consecutive positions starting at c0 of row (b, h): y[c0 + r]
// = v[src_of(r)]. An index outside [0, T) is filled like a miss, so no index can make the
// kernel read outside v.
// Rows of at most nthreads pieces: thread t always copies piece t % pieces of rows
// t / pieces + k * (nthreads / pieces) (consecutive threads on consecutive pieces of
// consecutive rows), so its miss value (from v's first row, or zero) is formed once, and each
// piece is one conditional load and one store, kInFlightP2 loads issued before the first
// store. (A miss must not load into the same registers as a copy: the two loads would then be
// waited for one by one.) Longer rows: thread t takes pieces t, t + nthreads, ..., with
// kInFlight independent loads issued before the first store.
template <int VEC, int kInFlight, int kInFlightP2, bool NT, typename SrcFn>
__device__ __forceinline__ void gather_rows_as(const GatherArgs& g, int64_t row, int64_t c0,
                                               int nrows, int t, int nthreads, SrcFn src_of) {
  typedef Piece<VEC> P;
  const int64_t b = row / g.H, h = row - (row / g.H) * g.H;
  const uint8_t* vbase = g.v + b * g.v_sb + h * g.v_sh;
  uint8_t* ybase = g.y + b * g.y_sb + h * g.y_sh + c0 * g.y_st;
  if (g.pieces <= static_cast<uint32_t>(nthreads)) {
    const int pieces = static_cast<int>(g.pieces);
    const int rpp = static_cast<int>(g.pdiv.div(static_cast<uint32_t>(nthreads)));
    const int r0 = static_cast<int>(g.pdiv.div(static_cast<uint32_t>(t)));
    if (r0 >= rpp) return;  // the threads past rpp * pieces
    const int pc = t - r0 * pieces;
    const uint8_t* vp = vbase + pc * VEC;
    uint8_t* yp = ybase + pc * VEC;
    const typename P::T missv = g.miss == LEMA_MISS_ZERO ? P::zero() : P::miss(P::load(vp), g.dtype);
    for (int rb = r0; rb < nrows; rb += kInFlightP2 * rpp) {
      typename P::T val[kInFlightP2];
      int32_t sv[kInFlightP2];  // source position, -1 a miss, -2 past the chunk's rows
      int64_t x[kInFlightP2];  // read for every u (a row inside the chunk stands in), so
                               // the reads are issued together
#pragma unroll
      for (int u = 0; u < kInFlightP2; ++u) {
        const int r = rb + u * rpp;
        x[u] = src_of(r < nrows ? r : nrows - 1);
      }
#pragma unroll
      for (int u = 0; u < kInFlightP2; ++u)
        sv[u] = rb + u * rpp >= nrows ? -2 : (x[u] >= 0 && x[u] < g.T ? static_cast<int32_t>(x[u]) : -1);
#pragma unroll
      for (int u = 0; u < kInFlightP2; ++u)
        if (sv[u] >= 0) val[u] = P::load(vp + static_cast<int64_t>(sv[u]) * g.v_st);
#pragma unroll
      for (int u = 0; u < kInFlightP2; ++u)
        if (sv[u] != -2)
          P::template store<NT>(yp + static_cast<int64_t>(rb + u * rpp) * g.y_st, sv[u] >= 0 ? val[u] : missv);
    }
    return;
  }
  const uint32_t total = static_cast<uint32_t>(nrows) * g.pieces;
  for (uint32_t base = t; base < total; base += kInFlight * nthreads) {
    typename P::T val[kInFlight];
    const uint8_t* from[kInFlight];
    uint8_t* to[kInFlight];
    int kind[kInFlight];  // 0 none, 1 copy, 2 miss from v[0], 3 zero
#pragma unroll
    for (int u = 0; u < kInFlight; ++u) {
      const uint32_t idx = base + u * nthreads;
      kind[u] = 0;
      if (idx >= total) continue;
      const uint32_t r = g.pdiv.div(idx);
      const uint32_t pc = idx - r * g.pieces;
      const int64_t s = src_of(r);
      to[u] = ybase + static_cast<int64_t>(r) * g.y_st + pc * VEC;
      if (s >= 0 && s < g.T) {
        kind[u] = 1;
        from[u] = vbase + s * g.v_st + pc * VEC;
      } else {
        kind[u] = g.miss == LEMA_MISS_ZERO ? 3 : 2;
        from[u] = vbase + pc * VEC;
      }
    }
#pragma unroll
    for (int u = 0; u < kInFlight; ++u)
      if (kind[u] == 1 || kind[u] == 2) val[u] = P::load(from[u]);
#pragma unroll
    for (int u = 0; u < kInFlight; ++u) {
      if (kind[u] == 0) continue;
      const typename P::T out =
          kind[u] == 1 ? val[u] : (kind[u] == 2 ? P::miss(val[u], g.dtype) : P::zero());
      P::template store<NT>(to[u], out);
    }
  }
}

// The store kind is chosen once, outside the copy loops.
template <int VEC, int kInFlight, int kInFlightP2, typename SrcFn>
__device__ __forceinline__ void gather_rows(const GatherArgs& g, int64_t row, int64_t c0,
                                            int nrows, int t, int nthreads, SrcFn src_of) {
  if (g.nt)
    gather_rows_as<VEC, kInFlight, kInFlightP2, true>(g, row, c0, nrows, t, nthreads, src_of);
  else
    gather_rows_as<VEC, kInFlight, kInFlightP2, false>(g, row, c0, nrows, t, nthreads, src_of);
}

// find4 for the keys with pass[i] set (the others get -1 without touching the table).
template <typename KeyT, int NB>
__device__ __forceinline__ void find4_masked(const KeyT* base, const KeyT (&key)[4], KeyT empty,
                                             const bool (&pass)[4], int (&slot)[4]) {
  int b[4];
  KeyT x[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    b[i] = bucket_of<NB>(fold(key[i]));
    if (pass[i]) read_bucket(base, b[i], x[i]);
  }
  // The first bucket answers almost every lookup: matched without branches; a full bucket
  // without the key sends the wavefront on to the next buckets (rarely).
  bool more[4];
  bool any = false;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    bool open;
    const int e = match4(x[i], key[i], empty, open);
    slot[i] = pass[i] && e >= 0 ? 4 * b[i] + e : -1;
    more[i] = pass[i] && e < 0 && !open;
    any = any || more[i];
  }
  if (__ballot(any) != 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (!more[i]) continue;
      const int nb = b[i] + 1 == NB ? 0 : b[i] + 1;
      read_bucket(base, nb, x[i]);
      slot[i] = table_find<KeyT, NB>(base, key[i], empty, nb, x[i]);
    }
  }
}

// Find 4 keys at once (first bucket reads issued together); -1 where absent or inactive.
template <typename KeyT, int NB>
__device__ __forceinline__ void find4(const KeyT* base, const KeyT (&key)[4], KeyT empty,
                                      int (&slot)[4]) {
  const bool all[4] = {true, true, true, true};
  find4_masked<KeyT, NB>(base, key, empty, all, slot);
}

// Resolve the 1024 queries of chunk `chunk` of row `row` with the 256 threads t = 0..255
// (four wavefronts), synchronising them with `bar`; leaves each thread's answers in src[p]
// for positions p * 256 + t, and stores them to a.src when that is given. Every phase issues
// the LDS reads (or CASes) of a thread's four positions together before waiting on any.
template <typename CodeT, typename Bar, bool kSumm = false>
__device__ __forceinline__ void resolve_chunk(ResolveLds<CodeT>& s, const ResolveArgs& a,
                                              int64_t row, int chunk, int t, Bar bar,
                                              int32_t (&src)[kPer]) {
  const int lane = t & 63;
  const CodeT SENT = sentinel<CodeT>();
  const CodeT* qrow = static_cast<const CodeT*>(a.qc) + row * a.T;
  const CodeT* krow = static_cast<const CodeT*>(a.kc) + row * a.T;
  const int32_t c0 = chunk * kChunk;
  const int n_here = static_cast<int>(a.T - c0 < kChunk ? a.T - c0 : kChunk);

  CodeT q[kPer], kk[kPer];
  bool act[kPer];
#pragma unroll
  for (int p = 0; p < kPer; ++p) {
    const int o = p * kThreads + t;
    act[p] = o < n_here;
    q[p] = act[p] ? qrow[c0 + o] : CodeT(0);
    kk[p] = act[p] ? krow[c0 + o] : CodeT(0);
  }
  // Keys before the chunk stream in batches of 1024 (4 per thread), latest batch first, the
  // next kPrefetch batches loaded while the current one is looked up; c0 is a multiple of the
  // batch.
  constexpr int kBatch = 4 * kThreads;
  CodeT nxt[kPrefetch][4];
  auto load_batch = [&](CodeT (&dst)[4], int32_t j0) {
    if (a.kvec) {  // 4 consecutive codes per thread, 16-byte aligned
      const CodeT* p = krow + j0 + 4 * t;
      if constexpr (sizeof(CodeT) == 4) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(p);
        dst[0] = v.x; dst[1] = v.y; dst[2] = v.z; dst[3] = v.w;
      } else {
        const u32x4 v0 = *reinterpret_cast<const u32x4*>(p);
        const u32x4 v1 = *reinterpret_cast<const u32x4*>(p + 2);
        dst[0] = (uint64_t(v0.y) << 32) | v0.x; dst[1] = (uint64_t(v0.w) << 32) | v0.z;
        dst[2] = (uint64_t(v1.y) << 32) | v1.x; dst[3] = (uint64_t(v1.w) << 32) | v1.z;
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) dst[e] = krow[j0 + e * kThreads + t];
    }
  };
  if constexpr (!kSumm) {
#pragma unroll
    for (int d = 0; d < kPrefetch; ++d)
      if (c0 - (d + 1) * kBatch >= 0) load_batch(nxt[d], c0 - (d + 1) * kBatch);
  }

  // the tables are cleared with 16-byte stores (the sentinel, -1 and kMapEmpty are all ones)
  static_assert(kSlots % 8 == 0 && kMapSlots % 4 == 0 && kFilterWords % 4 == 0 &&
                    kMapEmpty == 0xFFFFFFFFu,
                "16-byte clears");
  const u32x4 ones = {~0u, ~0u, ~0u, ~0u}, zero = {0u, 0u, 0u, 0u};
  auto fill = [&](void* base, int n16, u32x4 v) {
    u32x4* q4 = reinterpret_cast<u32x4*>(base);
    for (int x = t; x < n16; x += kThreads) q4[x] = v;
  };
  {
    fill(s.code, kSlots * static_cast<int>(sizeof(CodeT)) / 16, ones);
    fill(s.pos, kSlots / 4, ones);
    fill(s.summ, kSlots / 8, zero);
    fill(s.mkey, kMapSlots / 4, ones);
    fill(s.mbits, kMapSlots / 2, zero);
    fill(s.qbits, kFilterWords / 4, zero);
  }
  if (t == 0) {
    s.pos[kSlots] = -1;
    s.summ[kSlots] = 0;
    s.summ[kSlots + 1] = 0;
    s.sent_used = 0;
    s.nq = 0;
    s.nneed = 0;
    s.khit = 0;
  }
  bar();

  // 1. the chunk's query codes -> table slots; the sentinel code has its own slot kSlots
  // One position after another: a code inserted for an earlier position is usually found
  // by a plain read, which keeps CAS traffic on popular codes low.
  int qs[kPer];
#pragma unroll
  for (int p = 0; p < kPer; ++p) {
    qs[p] = kSlots;
    bool ins = false;
    if (act[p]) {
      if (q[p] == SENT)
        s.sent_used = 1;
      else
        qs[p] = table_claim<CodeT, kBuckets>(s.code, q[p], SENT, bucket_of<kBuckets>(fold(q[p])), ins);
    }
    if (LEMA_RESOLVE_FILTER == 2) {  // every lane of the wavefront takes part in the count
      const int n = __popcll(__ballot(ins));
      if (lane == 0 && n) atomicAdd(&s.nq, n);
    }
  }
  bar();
  // the filter, when the chunk's query codes are many (few keys then carry one)
  const bool filt = LEMA_RESOLVE_FILTER == 1 || (LEMA_RESOLVE_FILTER == 2 && s.nq > kFilterMinCodes);
  // The rest is compiled twice, with and without the filter, so that chunks without it run
  // the code they ran before it existed.
  auto rest = [&](auto filter_on, auto queue_on) {
    constexpr bool kFilt = decltype(filter_on)::value;
    // Chunks with the filter scan the earlier keys first, through a wider filter, queueing the
    // few keys that pass (see below); the map and word summaries lend it their LDS meanwhile.
    // Where chunk summaries exist, only chunks of nearly all distinct codes do (see
    // kQueueSummMinCodes).
    constexpr bool kQueue = decltype(queue_on)::value;
    static_assert(kFilt || !kQueue, "the queued scan needs the filter's chunk");
    uint32_t* wide = reinterpret_cast<uint32_t*>(s.summ);  // kWideBits, while kQueue scans
    if constexpr (kFilt) {
#pragma unroll
      for (int p = 0; p < kPer; ++p) {
        if (!act[p] || q[p] == SENT) continue;
        if constexpr (kQueue) {  // the wide filter serves the chunk's own keys too
          const uint32_t w = wide_hash(fold(q[p]));
          atomicOr(&wide[w >> 5], 1u << (w & 31));
        } else {
          const uint32_t h = filter_hash(fold(q[p]));
          atomicOr(&s.qbits[h >> 5], 1u << (h & 31));
        }
      }
      bar();
    }

    const bool sent_used = s.sent_used != 0;
    // slots among the query codes of 4 key codes (-1 = no query of the chunk asks for it)
    auto find_codes = [&](const CodeT (&c)[4], int (&sl)[4]) {
      if constexpr (kFilt) {
        bool pass[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if constexpr (kQueue) {  // only before the map takes the wide filter's storage back
            const uint32_t w = wide_hash(fold(c[i]));
            pass[i] = (wide[w >> 5] >> (w & 31)) & 1u;
          } else {
            const uint32_t h = filter_hash(fold(c[i]));
            pass[i] = (s.qbits[h >> 5] >> (h & 31)) & 1u;
          }
        }
        find4_masked<CodeT, kBuckets>(s.code, c, SENT, pass, sl);
      } else {
        find4<CodeT, kBuckets>(s.code, c, SENT, sl);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (c[i] == SENT) sl[i] = sent_used ? kSlots : -1;
    };

    // 2a. keys inside the chunk: each sets its lane in its (code, word) mask; the key that
    // creates a (code, word) entry also sets the word's bit in the code's summary
    auto keys_in_chunk = [&](const int (&sl)[kPer]) {
#pragma unroll
      for (int p = 0; p < kPer; ++p) {
        if (!act[p] || sl[p] < 0) continue;
        const int wd = (p * kThreads + t) >> 6;
        const uint32_t key = (static_cast<uint32_t>(sl[p]) << 4) | wd;
        bool ins;
        const int m = table_claim<uint32_t, kMapBuckets>(s.mkey, key, kMapEmpty,
                                                         bucket_of<kMapBuckets>(key), ins);
        atomicOr(reinterpret_cast<unsigned long long*>(&s.mbits[m]), 1ull << lane);
        if (ins)
          atomicOr(reinterpret_cast<uint32_t*>(&s.summ[sl[p] & ~1]), (1u << wd) << (16 * (sl[p] & 1)));
      }
    };
    auto key_pos = [&](int32_t j0, int e) -> int32_t {
      return a.kvec ? j0 + 4 * t + e : j0 + e * kThreads + t;
    };

    bool fast = false;  // (queued scan) no key of the chunk carries a query code of it
    if constexpr (kQueue) {
      // 2b (filter on). The chunk's query codes seldom repeat (more than kFilterMinCodes
      // distinct), so few earlier keys carry one. Each earlier key is tested against a
      // kWideBits filter of the chunk's query codes (one LDS read); the keys that pass go to
      // their wavefront's queue, which is looked up in the query-code table in bulk, 4 keys
      // per lane with their reads in flight together, whenever it could not take another
      // batch and at the end. A batch then costs its loads and filter reads, and the table's
      // dependent lookups are paid per queue rather than per batch whenever a single key of
      // the wavefront passes. The queues live in the map's storage (codes in mbits, positions
      // in mkey), which the in-chunk keys fill only after this scan.
      CodeT* qcode = reinterpret_cast<CodeT*>(s.mbits) + (t >> 6) * kQueueCap;
      int32_t* qpos = reinterpret_cast<int32_t*>(s.mkey) + (t >> 6) * kQueueCap;
      const unsigned long long below = (1ull << lane) - 1ull;
      int cnt = 0;  // entries in this wavefront's queue (uniform across the wavefront)
      auto flush = [&]() {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        for (int b0 = 0; b0 < cnt; b0 += 4 * 64) {
          CodeT c[4];
          int32_t jj[4];
          bool in[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int b = b0 + i * 64 + lane;
            in[i] = b < cnt;
            c[i] = in[i] ? qcode[b] : SENT;
            jj[i] = in[i] ? qpos[b] : -1;
          }
          int sl[4];
          find4_masked<CodeT, kBuckets>(s.code, c, SENT, in, sl);
          int32_t known[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) known[i] = sl[i] >= 0 ? s.pos[sl[i]] : 0x7FFFFFFF;
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (sl[i] >= 0 && known[i] < jj[i]) atomicMax(&s.pos[sl[i]], jj[i]);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        cnt = 0;
      };
      // kScanGroup batches' loads are issued together and then filtered one batch after
      // another: the filtering is too short to hide a load's latency behind one batch.
      for (int32_t jb = c0 - kBatch; jb >= 0; jb -= kScanGroup * kBatch) {
        CodeT grp[kScanGroup][4];
#pragma unroll
        for (int g = 0; g < kScanGroup; ++g)
          if (jb - g * kBatch >= 0) load_batch(grp[g], jb - g * kBatch);
#pragma unroll
        for (int g = 0; g < kScanGroup; ++g) {
          const int32_t j0 = jb - g * kBatch;
          if (j0 < 0) break;
          CodeT cur[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) cur[e] = grp[g][e];
          bool pass[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t w = wide_hash(fold(cur[e]));
            pass[e] = (wide[w >> 5] >> (w & 31)) & 1u;
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (cur[e] == SENT) {  // the all-ones code has its own slot, never queued
              pass[e] = false;
              if (sent_used && s.pos[kSlots] < key_pos(j0, e)) atomicMax(&s.pos[kSlots], key_pos(j0, e));
            }
            const unsigned long long bal = __ballot(pass[e]);
            if (pass[e]) {
              const int at = cnt + __popcll(bal & below);
              qcode[at] = cur[e];
              qpos[at] = key_pos(j0, e);
            }
            cnt += __popcll(bal);
          }
          if (cnt > kQueueCap - 4 * 64) flush();
        }
      }
      flush();
      // Does some key of the chunk carry a query code of the chunk? Codes that seldom repeat
      // usually give none (a 64-head language model's 24-bit codes at 16K tokens: 90-97% of
      // chunks), and then no query has an in-chunk match: every answer is the code's latest
      // position before the chunk, and the map, the chunk's own keys and the per-query map
      // lookups are skipped.
      int sl[kPer];
      find_codes(kk, sl);
      bool hit = false;
#pragma unroll
      for (int p = 0; p < kPer; ++p) hit = hit || (act[p] && sl[p] >= 0);
      if (__ballot(hit) != 0 && lane == 0) s.khit = 1;
      bar();
      fast = s.khit == 0;
      if (!fast) {
        // the map and the word summaries start over for the keys inside the chunk
        fill(s.mkey, kMapSlots / 4, ones);
        fill(s.mbits, kMapSlots / 2, zero);
        fill(s.summ, kSlots / 8, zero);
        if (t == 0) s.summ[kSlots] = 0;
        bar();
        keys_in_chunk(sl);
      }
    } else {
      {
        int sl[kPer];
        find_codes(kk, sl);
        keys_in_chunk(sl);
      }
      // 2b. keys before the chunk raise their code's latest position. Walking backwards, a
      // code whose latest position is already known skips the atomic, so only the first batch
      // that holds a popular code contends on its slot.
      for (int32_t jb = kSumm ? -1 : c0 - kBatch; jb >= 0; jb -= kPrefetch * kBatch) {
#pragma unroll
        for (int d = 0; d < kPrefetch; ++d) {
          const int32_t j0 = jb - d * kBatch;
          if (j0 < 0) break;
          CodeT cur[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) cur[e] = nxt[d][e];
          if (j0 - kPrefetch * kBatch >= 0) load_batch(nxt[d], j0 - kPrefetch * kBatch);
          int sl[4];
          find_codes(cur, sl);
          int32_t known[4];  // read for every key (slot kSlots stands in for the others, which
                             // raise nothing), so the reads need no branches
#pragma unroll
          for (int e = 0; e < 4; ++e) known[e] = s.pos[sl[e] >= 0 ? sl[e] : kSlots];
#pragma unroll
          for (int e = 0; e < 4; ++e) known[e] = sl[e] >= 0 ? known[e] : 0x7FFFFFFF;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int32_t j = key_pos(j0, e);
            if (sl[e] >= 0 && known[e] < j) atomicMax(&s.pos[sl[e]], j);
          }
        }
      }
    }
    if (!fast) bar();

    // 3. resolve: the latest earlier lane of the own word, else the latest earlier word of the
    // chunk holding the code, else the latest position before the chunk
    bool nb[kPer];  // the answer is the code's latest position before the chunk
    if (fast) {
#pragma unroll
      for (int p = 0; p < kPer; ++p) {
        nb[p] = act[p];
        src[p] = act[p] ? s.pos[qs[p]] : -1;
      }
    } else {
      int m[kPer];
      uint32_t key[kPer];
#pragma unroll
      for (int p = 0; p < kPer; ++p)
        key[p] = (static_cast<uint32_t>(qs[p]) << 4) | ((p * kThreads + t) >> 6);
      uint64_t bits[kPer];
      uint32_t words[kPer];
      int32_t before[kPer];
      if constexpr (kFilt) {
        // Codes that seldom repeat: most queries' codes have no key in the chunk, which
        // their word summary (read first) shows; only the others look up their lane mask.
        bool own[kPer];
#pragma unroll
        for (int p = 0; p < kPer; ++p) {
          words[p] = s.summ[qs[p]];
          before[p] = s.pos[qs[p]];
        }
#pragma unroll
        for (int p = 0; p < kPer; ++p)
          own[p] = act[p] && ((words[p] >> ((p * kThreads + t) >> 6)) & 1u);
        find4_masked<uint32_t, kMapBuckets>(s.mkey, key, kMapEmpty, own, m);
#pragma unroll
        for (int p = 0; p < kPer; ++p) bits[p] = m[p] >= 0 ? s.mbits[m[p]] : 0;
      } else {
        find4<uint32_t, kMapBuckets>(s.mkey, key, kMapEmpty, m);
#pragma unroll
        for (int p = 0; p < kPer; ++p) {  // every read a position may need, issued together
          bits[p] = s.mbits[m[p] >= 0 ? m[p] : 0];
          words[p] = s.summ[qs[p]];
          before[p] = s.pos[qs[p]];
        }
      }
      uint32_t key2[kPer];
      bool second[kPer];
#pragma unroll
      for (int p = 0; p < kPer; ++p) {
        const int wd = (p * kThreads + t) >> 6;
        const uint64_t below = m[p] >= 0 ? (bits[p] & ((1ull << lane) - 1)) : 0;
        const uint32_t w_below = words[p] & ((1u << wd) - 1);
        second[p] = false;
        nb[p] = false;
        key2[p] = kMapEmpty;
        if (!act[p]) {
          src[p] = -1;
        } else if (below) {
          src[p] = c0 + (wd << 6) + 63 - __clzll(below);
        } else if (w_below) {
          const int w2 = 31 - __clz(w_below);
          second[p] = true;
          key2[p] = (static_cast<uint32_t>(qs[p]) << 4) | w2;
          src[p] = c0 + (w2 << 6);
        } else {
          src[p] = before[p];
          nb[p] = true;
        }
      }
      int m2[kPer];
      find4_masked<uint32_t, kMapBuckets>(s.mkey, key2, kMapEmpty, second, m2);
#pragma unroll
      for (int p = 0; p < kPer; ++p)
        if (second[p]) src[p] += 63 - __clzll(s.mbits[m2[p]]);
    }
    if (kSumm && !kQueue && chunk > 0) {
      // Summary path: the codes some query needs from before the chunk are listed (in the key
      // map's storage, dead by now) and each is looked up in the earlier chunks' summaries.
#pragma unroll
      for (int p = 0; p < kPer; ++p)
        if (nb[p]) s.pos[qs[p]] = -2;
      bar();
      int32_t* need = reinterpret_cast<int32_t*>(s.mkey);
      for (int x = t; x <= kSlots; x += kThreads)
        if (s.pos[x] == -2) need[atomicAdd(&s.nneed, 1)] = x;
      bar();
      const int nneed = s.nneed;
      for (int i = t; i < nneed; i += kThreads) {
        const int x = need[i];
        s.pos[x] = before_chunk<CodeT>(a, row, chunk, x == kSlots ? SENT : s.code[x], x == kSlots);
      }
      bar();
#pragma unroll
      for (int p = 0; p < kPer; ++p)
        if (nb[p]) src[p] = s.pos[qs[p]];
    }
    if (a.src != nullptr) {
#pragma unroll
      for (int p = 0; p < kPer; ++p) {
        const int o = p * kThreads + t;
        if (o >= n_here) continue;
        if (a.src_bytes == 8)
          static_cast<int64_t*>(a.src)[row * a.T + c0 + o] = src[p];
        else
          static_cast<int32_t*>(a.src)[row * a.T + c0 + o] = src[p];
      }
    }
  };
  if (!filt) {
    rest(std::false_type{}, std::false_type{});
  } else if constexpr (kSumm) {
    if (s.nq > kQueueSummMinCodes)
      rest(std::true_type{}, std::true_type{});
    else
      rest(std::true_type{}, std::false_type{});
  } else {
    rest(std::true_type{}, std::true_type{});
  }
}

}  // namespace
}  // namespace lema
