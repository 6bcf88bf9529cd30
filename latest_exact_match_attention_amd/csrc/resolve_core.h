// Device building blocks of the latest-match resolver, shared by the prefill kernels
// (resolve.hip) and the store's in-chunk resolution (store.hip). The design is described at the
// top of resolve.hip.
#pragma once
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
#ifndef LEMA_RESOLVE_MAP_SLOTS
#define LEMA_RESOLVE_MAP_SLOTS 1536
#endif
constexpr int kSlots = LEMA_RESOLVE_SLOTS;  // query-code table: at most kChunk codes
constexpr int kBuckets = kSlots / 4;
constexpr int kMapSlots = LEMA_RESOLVE_MAP_SLOTS;  // (code slot, word) -> lane mask: at most
constexpr int kMapBuckets = kMapSlots / 4;          // kChunk keys
static_assert(kSlots > kChunk && kSlots % 4 == 0 && kMapSlots > kChunk && kMapSlots % 4 == 0,
              "tables must keep free slots");
constexpr uint32_t kMapEmpty = 0xFFFFFFFFu;
static_assert(kChunk / 64 <= 16, "word summary is a 16-bit mask");

template <typename CodeT>
struct ResolveLds {
  alignas(16) uint64_t mbits[kMapSlots];  // lanes of that word whose key carries that code
  alignas(16) CodeT code[kSlots];         // query code of a slot, sentinel() = free
  alignas(16) uint32_t mkey[kMapSlots];   // code slot << 4 | word, kMapEmpty = free
  int32_t pos[kSlots + 1];    // latest key position before the chunk, -1 = none; the entry
                              // [kSlots] here and in summ belongs to the sentinel code itself
  alignas(4) uint16_t summ[kSlots + 2];  // bit w: word w of the chunk holds a key with this
                                         // code; updated as 32-bit pairs
  int32_t sent_used;
};

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

// Slot of `key` among the bucket's 4 (first match), or -1; `open` gets whether an empty slot
// was seen, which ends a probe sequence.
template <typename KeyT>
__device__ __forceinline__ int match4(const KeyT (&x)[4], KeyT key, KeyT empty, bool& open) {
  open = x[0] == empty || x[1] == empty || x[2] == empty || x[3] == empty;
  return x[0] == key ? 0 : x[1] == key ? 1 : x[2] == key ? 2 : x[3] == key ? 3 : -1;
}

// Insert `key` into a table of NB buckets (or find it): returns its slot; `inserted` tells
// whether this call put it there. The table must have an empty slot somewhere (load < 1
// here). Torn 8-byte reads are re-checked atomically.
template <typename KeyT, int NB>
__device__ __forceinline__ int table_claim(KeyT* base, KeyT key, KeyT empty, int b,
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
    const int f = x[0] == empty ? 0 : x[1] == empty ? 1 : x[2] == empty ? 2 : 3;
    const KeyT old = lds_cas(&base[4 * b + f], empty, key);
    if (old == empty) inserted = true;
    if (old == empty || old == key) return 4 * b + f;
    // another key took that slot first: read the same bucket again
  }
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
  int32_t plog;     // log2(pieces) when pieces is a power of two <= 64, else -1
  int32_t miss;
  int32_t dtype;
};

struct ResolveArgs {
  const void* qc;
  const void* kc;
  int64_t N, T;
  int32_t nchunks;
  int32_t kvec;  // key rows allow 16-byte loads of 4 consecutive codes
  void* src;     // optional
  int32_t src_bytes;
  GatherArgs g;
};

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
  static __device__ __forceinline__ void store(uint8_t* p, T v) {
    __builtin_nontemporal_store(v, reinterpret_cast<T*>(p));
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
  static __device__ __forceinline__ void store(uint8_t* p, T v) {
    __builtin_nontemporal_store(v, reinterpret_cast<T*>(p));
  }
  static __device__ __forceinline__ T zero() { return T{0u, 0u}; }
  static __device__ __forceinline__ T miss(T v, int32_t d) { return T{miss_word(v.x, d), miss_word(v.y, d)}; }
};
template <>
struct Piece<4> {
  typedef uint32_t T;
  static __device__ __forceinline__ T load(const uint8_t* p) { return *reinterpret_cast<const T*>(p); }
  static __device__ __forceinline__ void store(uint8_t* p, T v) {
    __builtin_nontemporal_store(v, reinterpret_cast<T*>(p));
  }
  static __device__ __forceinline__ T zero() { return 0u; }
  static __device__ __forceinline__ T miss(T v, int32_t d) { return miss_word(v, d); }
};
template <>
struct Piece<2> {
  typedef uint16_t T;
  static __device__ __forceinline__ T load(const uint8_t* p) { return *reinterpret_cast<const T*>(p); }
  static __device__ __forceinline__ void store(uint8_t* p, T v) {
    __builtin_nontemporal_store(v, reinterpret_cast<T*>(p));
  }
  static __device__ __forceinline__ T zero() { return 0; }
  static __device__ __forceinline__ T miss(T v, int32_t d) {
    return static_cast<T>(miss_word(v, d) & 0xFFFFu);  // 2-byte pieces only for 16-bit dtypes
  }
};

// Copy the value rows of `nrows` consecutive positions starting at c0 of row (b, h): y[c0 + r]
// = v[src_of(r)]. Thread `t` of `nthreads` takes pieces t, t + nthreads, ..., with kInFlight
// independent loads issued before the first store. An index outside [0, T) is filled like a
// miss, so no index can make the kernel read outside v.
template <int VEC, int kInFlight, int kInFlightP2, typename SrcFn>
__device__ __forceinline__ void gather_rows(const GatherArgs& g, int64_t row, int64_t c0,
                                            int nrows, int t, int nthreads, SrcFn src_of) {
  typedef Piece<VEC> P;
  const int64_t b = row / g.H, h = row - (row / g.H) * g.H;
  const uint8_t* vbase = g.v + b * g.v_sb + h * g.v_sh;
  uint8_t* ybase = g.y + b * g.y_sb + h * g.y_sh + c0 * g.y_st;
  if (g.plog >= 0) {
    // pieces = 2^plog divides the block: thread t always copies piece t % pieces of rows
    // t / pieces + k * (nthreads / pieces), with kInFlight of them loaded before storing
    const int rpp = nthreads >> g.plog;
    const int r0 = t >> g.plog, pc = t & ((1 << g.plog) - 1);
    const uint8_t* vp = vbase + pc * VEC;
    uint8_t* yp = ybase + pc * VEC;
    for (int rb = r0; rb < nrows; rb += kInFlightP2 * rpp) {
      typename P::T val[kInFlightP2];
      int32_t sv[kInFlightP2];
#pragma unroll
      for (int u = 0; u < kInFlightP2; ++u) {
        const int r = rb + u * rpp;
        const int64_t x = r < nrows ? src_of(r) : -2;
        sv[u] = r >= nrows ? -2 : (x >= 0 && x < g.T ? static_cast<int32_t>(x) : -1);
      }
#pragma unroll
      for (int u = 0; u < kInFlightP2; ++u) {
        if (sv[u] >= 0)
          val[u] = P::load(vp + sv[u] * g.v_st);
        else if (sv[u] == -1 && g.miss != LEMA_MISS_ZERO)
          val[u] = P::load(vp);
      }
#pragma unroll
      for (int u = 0; u < kInFlightP2; ++u) {
        if (sv[u] == -2) continue;
        const typename P::T out = sv[u] >= 0 ? val[u]
                                  : (g.miss == LEMA_MISS_ZERO ? P::zero() : P::miss(val[u], g.dtype));
        P::store(yp + static_cast<int64_t>(rb + u * rpp) * g.y_st, out);
      }
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
      P::store(to[u], out);
    }
  }
}

// Find 4 keys at once (first bucket reads issued together); -1 where absent or inactive.
template <typename KeyT, int NB>
__device__ __forceinline__ void find4(const KeyT* base, const KeyT (&key)[4], KeyT empty,
                                      int (&slot)[4]) {
  int b[4];
  KeyT x[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    b[i] = bucket_of<NB>(fold(key[i]));
    read_bucket(base, b[i], x[i]);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) slot[i] = table_find<KeyT, NB>(base, key[i], empty, b[i], x[i]);
}

// Resolve the 1024 queries of chunk `chunk` of row `row` with the 256 threads t = 0..255
// (four wavefronts), synchronising them with `bar`; leaves each thread's answers in src[p]
// for positions p * 256 + t, and stores them to a.src when that is given. Every phase issues
// the LDS reads (or CASes) of a thread's four positions together before waiting on any.
template <typename CodeT, typename Bar>
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
  // next batch loaded while the current one is looked up; c0 is a multiple of the batch.
  constexpr int kBatch = 4 * kThreads;
  CodeT nxt[4];
  auto load_batch = [&](int32_t j0) {
    if (a.kvec) {  // 4 consecutive codes per thread, 16-byte aligned
      const CodeT* p = krow + j0 + 4 * t;
      if constexpr (sizeof(CodeT) == 4) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(p);
        nxt[0] = v.x; nxt[1] = v.y; nxt[2] = v.z; nxt[3] = v.w;
      } else {
        const u32x4 v0 = *reinterpret_cast<const u32x4*>(p);
        const u32x4 v1 = *reinterpret_cast<const u32x4*>(p + 2);
        nxt[0] = (uint64_t(v0.y) << 32) | v0.x; nxt[1] = (uint64_t(v0.w) << 32) | v0.z;
        nxt[2] = (uint64_t(v1.y) << 32) | v1.x; nxt[3] = (uint64_t(v1.w) << 32) | v1.z;
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) nxt[e] = krow[j0 + e * kThreads + t];
    }
  };
  if (c0 > 0) load_batch(c0 - kBatch);

  for (int x = t; x < kSlots; x += kThreads) s.code[x] = SENT;
  for (int x = t; x <= kSlots; x += kThreads) {
    s.pos[x] = -1;
    s.summ[x] = 0;
  }
  for (int x = t; x < kMapSlots; x += kThreads) {
    s.mkey[x] = kMapEmpty;
    s.mbits[x] = 0;
  }
  if (t == 0) s.sent_used = 0;
  bar();

  // 1. the chunk's query codes -> table slots; the sentinel code has its own slot kSlots
  // One position after another: a code inserted for an earlier position is usually found
  // by a plain read, which keeps CAS traffic on popular codes low.
  int qs[kPer];
#pragma unroll
  for (int p = 0; p < kPer; ++p) {
    qs[p] = kSlots;
    if (!act[p]) continue;
    if (q[p] == SENT) {
      s.sent_used = 1;
      continue;
    }
    bool ins;
    qs[p] = table_claim<CodeT, kBuckets>(s.code, q[p], SENT, bucket_of<kBuckets>(fold(q[p])), ins);
  }
  bar();

  const bool sent_used = s.sent_used != 0;
  // slots among the query codes of 4 key codes (-1 = no query of the chunk asks for it)
  auto find_codes = [&](const CodeT (&c)[4], int (&sl)[4]) {
    find4<CodeT, kBuckets>(s.code, c, SENT, sl);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (c[i] == SENT) sl[i] = sent_used ? kSlots : -1;
  };

  // 2a. keys inside the chunk: each sets its lane in its (code, word) mask; the key that
  // creates a (code, word) entry also sets the word's bit in the code's summary
  {
    int sl[kPer];
    find_codes(kk, sl);
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
  }
  // 2b. keys before the chunk raise their code's latest position. Walking backwards, a code
  // whose latest position is already known skips the atomic, so only the first batch that
  // holds a popular code contends on its slot.
  for (int32_t j0 = c0 - kBatch; j0 >= 0; j0 -= kBatch) {
    CodeT cur[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) cur[e] = nxt[e];
    if (j0 > 0) load_batch(j0 - kBatch);
    int sl[4];
    find_codes(cur, sl);
    int32_t known[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) known[e] = s.pos[sl[e] >= 0 ? sl[e] : kSlots];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int32_t j = a.kvec ? j0 + 4 * t + e : j0 + e * kThreads + t;
      if (sl[e] >= 0 && known[e] < j) atomicMax(&s.pos[sl[e]], j);
    }
  }
  bar();

  // 3. resolve: the latest earlier lane of the own word, else the latest earlier word of the
  // chunk holding the code, else the latest position before the chunk
  {
    int m[kPer];
    uint32_t key[kPer];
#pragma unroll
    for (int p = 0; p < kPer; ++p)
      key[p] = (static_cast<uint32_t>(qs[p]) << 4) | ((p * kThreads + t) >> 6);
    find4<uint32_t, kMapBuckets>(s.mkey, key, kMapEmpty, m);
    uint64_t bits[kPer];
    uint32_t words[kPer];
    int32_t before[kPer];
#pragma unroll
    for (int p = 0; p < kPer; ++p) {  // every read a position may need, issued together
      bits[p] = s.mbits[m[p] >= 0 ? m[p] : 0];
      words[p] = s.summ[qs[p]];
      before[p] = s.pos[qs[p]];
    }
    uint32_t key2[kPer];
    bool second[kPer];
#pragma unroll
    for (int p = 0; p < kPer; ++p) {
      const int wd = (p * kThreads + t) >> 6;
      const uint64_t below = m[p] >= 0 ? (bits[p] & ((1ull << lane) - 1)) : 0;
      const uint32_t w_below = words[p] & ((1u << wd) - 1);
      second[p] = false;
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
      }
    }
    int m2[kPer];
    find4<uint32_t, kMapBuckets>(s.mkey, key2, kMapEmpty, m2);
#pragma unroll
    for (int p = 0; p < kPer; ++p)
      if (second[p]) src[p] += 63 - __clzll(s.mbits[m2[p]]);
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
}

}  // namespace
}  // namespace lema
