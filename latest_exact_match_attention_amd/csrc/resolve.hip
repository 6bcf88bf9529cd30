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
// The gather is fused: after resolving, the workgroup copies its 1024 value rows
// v[src] -> y in 16-byte pieces, consecutive threads on consecutive pieces, so both the reads
// of each source row and the (non-temporal) writes of y are coalesced.
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

// Fibonacci hashing into [0, 2^LOG).
template <int LOG>
__device__ __forceinline__ int hash32(uint32_t x) {
  return static_cast<int>((x * 0x9E3779B1u) >> (32 - LOG));
}

// Resolver geometry: 256 threads (4 wavefronts) own a chunk of 1024 query positions, 4 per
// thread. Position o of the chunk is handled by thread o % 256 as its (o / 256)-th position,
// so the 64 positions of a "word" o / 64 are the 64 lanes of one wavefront.
constexpr int kThreads = 256;
constexpr int kPer = 4;
constexpr int kChunk = kThreads * kPer;
constexpr int kSlots = 2 * kChunk;  // query-code table: at most kChunk codes, load <= 1/2
constexpr int kBucketLog = 9;       // 512 buckets of 4 slots
constexpr int kMapSlots = 2 * kChunk;  // (code slot, word) -> lane mask: at most kChunk keys
constexpr int kMapBucketLog = 9;
constexpr uint32_t kMapEmpty = 0xFFFFFFFFu;
static_assert(kSlots == 4 << kBucketLog && kMapSlots == 4 << kMapBucketLog, "table sizes");
static_assert(kChunk / 64 <= 32, "word summary is a 32-bit mask");

template <typename CodeT>
struct ResolveLds {
  alignas(16) uint64_t mbits[kMapSlots];  // lanes of that word whose key carries that code
  alignas(16) CodeT code[kSlots];         // query code of a slot, sentinel() = free
  alignas(16) uint32_t mkey[kMapSlots];   // code slot << 5 | word, kMapEmpty = free
  int32_t pos[kSlots + 1];    // latest key position before the chunk, -1 = none; the entry
  uint32_t summ[kSlots + 1];  // bit w: word w of the chunk holds a key with this code
                              // [kSlots] of both belongs to the sentinel code itself
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

// Insert `key` into a bucketized table (or find it): returns its slot. The table must have an
// empty slot somewhere (load <= 1/2 here). Torn 8-byte reads are re-checked atomically.
template <typename KeyT, int BLOG>
__device__ __forceinline__ int table_claim(KeyT* base, KeyT key, KeyT empty, int b) {
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
      b = (b + 1) & ((1 << BLOG) - 1);
      continue;
    }
    const int f = x[0] == empty ? 0 : x[1] == empty ? 1 : x[2] == empty ? 2 : 3;
    const KeyT old = lds_cas(&base[4 * b + f], empty, key);
    if (old == empty || old == key) return 4 * b + f;
    // another key took that slot first: read the same bucket again
  }
}

// Finish a lookup whose first bucket b was read into x: slot of key, or -1 (no concurrent
// writers: the table is read only after the barrier that ends its construction).
template <typename KeyT, int BLOG>
__device__ __forceinline__ int table_find(const KeyT* base, KeyT key, KeyT empty, int b,
                                          KeyT (&x)[4]) {
  for (;;) {
    bool open;
    const int e = match4(x, key, empty, open);
    if (e >= 0) return 4 * b + e;
    if (open) return -1;
    b = (b + 1) & ((1 << BLOG) - 1);
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
template <int VEC, int kInFlight, typename SrcFn>
__device__ __forceinline__ void gather_rows(const GatherArgs& g, int64_t row, int64_t c0,
                                            int nrows, int t, int nthreads, SrcFn src_of) {
  typedef Piece<VEC> P;
  const int64_t b = row / g.H, h = row - (row / g.H) * g.H;
  const uint8_t* vbase = g.v + b * g.v_sb + h * g.v_sh;
  uint8_t* ybase = g.y + b * g.y_sb + h * g.y_sh + c0 * g.y_st;
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

template <typename CodeT, int VEC>
__global__ __launch_bounds__(kThreads) void resolve_kernel(ResolveArgs a) {
  __shared__ ResolveLds<CodeT> s;

  // XCD-aware work mapping: every chunk of row r runs on XCD r % 8, which then keeps that
  // row's key codes and value rows in its own L2; the heaviest chunks (latest) go first.
  const int bid = blockIdx.x;
  const int xcd = bid % kNumXcd;
  const int k = bid / kNumXcd;
  const int chunk = a.nchunks - 1 - (k % a.nchunks);
  const int64_t row = static_cast<int64_t>(k / a.nchunks) * kNumXcd + xcd;
  if (row >= a.N) return;

  const int t = threadIdx.x, lane = t & 63;
  const CodeT SENT = sentinel<CodeT>();
  const CodeT* qrow = static_cast<const CodeT*>(a.qc) + row * a.T;
  const CodeT* krow = static_cast<const CodeT*>(a.kc) + row * a.T;
  const int32_t c0 = chunk * kChunk;
  const int n_here = static_cast<int>(a.T - c0 < kChunk ? a.T - c0 : kChunk);

  CodeT q[kPer], kk[kPer];
#pragma unroll
  for (int p = 0; p < kPer; ++p) {
    const int o = p * kThreads + t;
    q[p] = o < n_here ? qrow[c0 + o] : CodeT(0);
    kk[p] = o < n_here ? krow[c0 + o] : CodeT(0);
  }
  // Keys before the chunk stream in batches of 1024 (4 per thread), the next batch loaded
  // while the current one is looked up; c0 is a multiple of the batch.
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
  if (c0 > 0) load_batch(0);

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
  __syncthreads();

  // 1. the chunk's query codes -> table slots; the sentinel code has its own slot kSlots
  int qs[kPer];
#pragma unroll
  for (int p = 0; p < kPer; ++p) {
    qs[p] = kSlots;
    if (p * kThreads + t >= n_here) continue;
    if (q[p] == SENT) {
      s.sent_used = 1;
      continue;
    }
    qs[p] = table_claim<CodeT, kBucketLog>(s.code, q[p], SENT, hash32<kBucketLog>(fold(q[p])));
  }
  __syncthreads();

  const bool sent_used = s.sent_used != 0;
  // slot of key code c (first bucket b already read into x) among the query codes, or -1
  auto find_code = [&](CodeT c, int b, CodeT (&x)[4]) -> int {
    if (c == SENT) return sent_used ? kSlots : -1;
    return table_find<CodeT, kBucketLog>(s.code, c, SENT, b, x);
  };

  // 2a. keys inside the chunk: each sets its lane in its (code, word) mask
  {
    int b[kPer];
    CodeT x[kPer][4];
#pragma unroll
    for (int p = 0; p < kPer; ++p) {  // first bucket reads of all 4 positions together
      b[p] = hash32<kBucketLog>(fold(kk[p]));
      read_bucket(s.code, b[p], x[p]);
    }
#pragma unroll
    for (int p = 0; p < kPer; ++p) {
      const int o = p * kThreads + t;
      if (o >= n_here) continue;
      const int sl = find_code(kk[p], b[p], x[p]);
      if (sl < 0) continue;
      const int wd = o >> 6;
      const uint32_t key = (static_cast<uint32_t>(sl) << 5) | wd;
      const int m = table_claim<uint32_t, kMapBucketLog>(s.mkey, key, kMapEmpty,
                                                         hash32<kMapBucketLog>(key));
      atomicOr(reinterpret_cast<unsigned long long*>(&s.mbits[m]), 1ull << lane);
      atomicOr(&s.summ[sl], 1u << wd);
    }
  }
  // 2b. keys before the chunk raise their code's latest position
  for (int32_t j0 = 0; j0 < c0; j0 += kBatch) {
    CodeT cur[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) cur[e] = nxt[e];
    if (j0 + kBatch < c0) load_batch(j0 + kBatch);
    int b[4];
    CodeT x[4][4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      b[e] = hash32<kBucketLog>(fold(cur[e]));
      read_bucket(s.code, b[e], x[e]);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int sl = find_code(cur[e], b[e], x[e]);
      if (sl >= 0) atomicMax(&s.pos[sl], a.kvec ? j0 + 4 * t + e : j0 + e * kThreads + t);
    }
  }
  __syncthreads();

  // 3. resolve: the latest earlier lane of the own word, else the latest earlier word of the
  // chunk holding the code, else the latest position before the chunk
  int32_t src[kPer];
  {
    int mb[kPer];
    uint32_t mx[kPer][4], key0[kPer];
#pragma unroll
    for (int p = 0; p < kPer; ++p) {  // first map reads of every position's own (code, word)
      key0[p] = (static_cast<uint32_t>(qs[p]) << 5) | ((p * kThreads + t) >> 6);
      mb[p] = hash32<kMapBucketLog>(key0[p]);
      read_bucket(s.mkey, mb[p], mx[p]);
    }
#pragma unroll
    for (int p = 0; p < kPer; ++p) {
      const int o = p * kThreads + t;
      src[p] = -1;
      if (o >= n_here) continue;
      const uint32_t sl = static_cast<uint32_t>(qs[p]);
      const int wd = o >> 6;
      const int m = table_find<uint32_t, kMapBucketLog>(s.mkey, key0[p], kMapEmpty, mb[p], mx[p]);
      const uint64_t below = m >= 0 ? (s.mbits[m] & ((1ull << lane) - 1)) : 0;
      if (below) {
        src[p] = c0 + (wd << 6) + 63 - __clzll(below);
        continue;
      }
      const uint32_t words = s.summ[sl] & ((1u << wd) - 1);
      if (words) {
        const int w2 = 31 - __clz(words);
        const uint32_t key2 = (sl << 5) | w2;
        uint32_t y2[4];
        const int b2 = hash32<kMapBucketLog>(key2);
        read_bucket(s.mkey, b2, y2);
        const int m2 = table_find<uint32_t, kMapBucketLog>(s.mkey, key2, kMapEmpty, b2, y2);
        src[p] = c0 + (w2 << 6) + 63 - __clzll(s.mbits[m2]);
      } else {
        src[p] = s.pos[sl];
      }
    }
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

  if constexpr (VEC > 0) {
    int32_t* srcs = reinterpret_cast<int32_t*>(s.mbits);  // the masks are dead now
    __syncthreads();
#pragma unroll
    for (int p = 0; p < kPer; ++p) srcs[p * kThreads + t] = src[p];
    __syncthreads();
    gather_rows<VEC, 8>(a.g, row, c0, n_here, t, kThreads,
                        [&](uint32_t r) -> int64_t { return srcs[r]; });
  }
}

// Standalone gather for given indices: one workgroup per (row, 1024 positions).
constexpr int kGatherRows = 1024;

struct GatherOnlyArgs {
  const void* src;
  int32_t src_bytes;
  int64_t N, T;
  int32_t nchunks;
  GatherArgs g;
};

template <int VEC>
__global__ __launch_bounds__(256) void gather_kernel(GatherOnlyArgs a) {
  __shared__ int32_t ssrc[kGatherRows];
  const int bid = blockIdx.x;
  const int xcd = bid % kNumXcd;
  const int k = bid / kNumXcd;
  const int chunk = k % a.nchunks;
  const int64_t row = static_cast<int64_t>(k / a.nchunks) * kNumXcd + xcd;
  if (row >= a.N) return;
  const int64_t c0 = static_cast<int64_t>(chunk) * kGatherRows;
  const int nrows = static_cast<int>(a.T - c0 < kGatherRows ? a.T - c0 : kGatherRows);
  for (int r = threadIdx.x; r < nrows; r += blockDim.x) {
    const int64_t at = row * a.T + c0 + r;
    ssrc[r] = a.src_bytes == 8 ? static_cast<int32_t>(static_cast<const int64_t*>(a.src)[at])
                               : static_cast<const int32_t*>(a.src)[at];
  }
  __syncthreads();
  gather_rows<VEC, 8>(a.g, row, c0, nrows, threadIdx.x, blockDim.x,
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
  *vec_out = vec;
  return LEMA_OK;
}

template <typename CodeT>
int launch_resolve(ResolveArgs& a, int vec, hipStream_t st) {
  const int64_t groups = (a.N + kNumXcd - 1) / kNumXcd;
  const int64_t grid = groups * kNumXcd * a.nchunks;
  LEMA_REQUIRE(grid < (int64_t(1) << 31), "too many rows x chunks (%lld)", (long long)grid);
  a.kvec = (aligned(a.kc, 16) && (a.T * static_cast<int64_t>(sizeof(CodeT))) % 16 == 0) ? 1 : 0;
  switch (vec) {
    case 0: resolve_kernel<CodeT, 0><<<dim3(grid), dim3(kThreads), 0, st>>>(a); break;
    case 16: resolve_kernel<CodeT, 16><<<dim3(grid), dim3(kThreads), 0, st>>>(a); break;
    case 8: resolve_kernel<CodeT, 8><<<dim3(grid), dim3(kThreads), 0, st>>>(a); break;
    case 4: resolve_kernel<CodeT, 4><<<dim3(grid), dim3(kThreads), 0, st>>>(a); break;
    case 2: resolve_kernel<CodeT, 2><<<dim3(grid), dim3(kThreads), 0, st>>>(a); break;
    default: set_error("internal: piece size %d", vec); return LEMA_BAD_ARG;
  }
  return launch_status("resolve_kernel");
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

using namespace lema;

extern "C" int lema_latest_prev_match(const void* qc, const void* kc, int32_t code_bytes,
                                      int64_t N, int64_t T, void* src, int32_t src_bytes,
                                      void* stream) {
  clear_error();
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
  hipStream_t st = static_cast<hipStream_t>(stream);
  return code_bytes == 4 ? launch_resolve<uint32_t>(a, 0, st) : launch_resolve<uint64_t>(a, 0, st);
}

extern "C" int lema_hard(const void* qc, const void* kc, int32_t code_bytes, const void* v,
                         int32_t dtype, int64_t B, int64_t H, int64_t T, int64_t dv,
                         int64_t v_sb, int64_t v_sh, int64_t v_st, void* y, int64_t y_sb,
                         int64_t y_sh, int64_t y_st, int32_t miss, void* src,
                         int32_t src_bytes, void* stream) {
  clear_error();
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
  hipStream_t st = static_cast<hipStream_t>(stream);
  return code_bytes == 4 ? launch_resolve<uint32_t>(a, vec, st) : launch_resolve<uint64_t>(a, vec, st);
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
  const int64_t grid = (N + kNumXcd - 1) / kNumXcd * kNumXcd * a.nchunks;
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
