// The prefill latest-match resolver and the value gather (code/lema/attention.py:100-158).
//
// One workgroup owns CHUNK consecutive query positions [c0, c0 + CHUNK) of one (b, h) row,
// one position per thread. Its answer for query i is the latest key j < i with the same code,
// found in three places, nearest first:
//   (a) the same wavefront (64 positions): a 64-step register scan with readlane;
//   (b) earlier wavefronts of the chunk: for every (sub-block, query code) the chunk offset of
//       the sub-block's latest such key, turned into an exclusive running max over sub-blocks;
//   (c) before the chunk: every key in [0, c0) is looked up in an LDS hash table of the
//       chunk's query codes and raises that code's position with an LDS atomicMax.
// Only keys whose code some query of the chunk carries matter, so the LDS table has 2*CHUNK
// slots (load <= 1/2) whatever the code width, and every structure lives in LDS: the kernel
// needs no scratch memory. Its cost is O(T^2 / CHUNK) table lookups per row for (c), reading
// the row's key codes from L2; that is cheap next to the gather at the T this path serves
// (16k: 15 lookups per query), and long rows go through the store instead.
//
// The gather is fused: after resolving, the workgroup copies its CHUNK value rows
// v[src] -> y in 16-byte pieces, consecutive threads on consecutive pieces, so both the
// reads of each source row and the (non-temporal) writes of y are coalesced.
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

// Fibonacci hashing of the code into [0, 2^LOG).
template <int LOG, typename CodeT>
__device__ __forceinline__ int slot_hash(CodeT c) {
  return static_cast<int>((static_cast<uint64_t>(c) * 0x9E3779B97F4A7C15ull) >> (64 - LOG));
}

template <int CHUNK>
struct Log2 {
  static constexpr int value = CHUNK <= 1 ? 0 : 1 + Log2<CHUNK / 2>::value;
};
template <>
struct Log2<1> {
  static constexpr int value = 0;
};

template <typename CodeT, int CHUNK>
struct ResolveLds {
  static constexpr int kSlots = 2 * CHUNK;
  static constexpr int kSub = CHUNK / 64;
  CodeT code[kSlots + 1];     // slot key, sentinel() = free; [kSlots] stands for the sentinel code
  int32_t pos[kSlots + 1];    // latest key position before the chunk, -1 = none
  int16_t id[kSlots + 1];     // dense id (< CHUNK) of an occupied slot
  int16_t last[kSub][CHUNK];  // [sub-block][id]: chunk offset of the latest key, -1 = none
  int32_t src[CHUNK];
  int32_t nid;
  int32_t sent_used;
};

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
  void* src;  // optional
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
// = v[src_of(r)]. Thread `t` of `nthreads` takes pieces t, t + nthreads, ... An index outside
// [0, T) is filled like a miss, so no index can make the kernel read outside v.
template <int VEC, typename SrcFn>
__device__ __forceinline__ void gather_rows(const GatherArgs& g, int64_t row, int64_t c0,
                                            int nrows, int t, int nthreads, SrcFn src_of) {
  typedef Piece<VEC> P;
  const int64_t b = row / g.H, h = row - (row / g.H) * g.H;
  const uint8_t* vbase = g.v + b * g.v_sb + h * g.v_sh;
  uint8_t* ybase = g.y + b * g.y_sb + h * g.y_sh + c0 * g.y_st;
  const uint32_t total = static_cast<uint32_t>(nrows) * g.pieces;
  for (uint32_t idx = t; idx < total; idx += nthreads) {
    const uint32_t r = g.pdiv.div(idx);
    const uint32_t pc = idx - r * g.pieces;
    const int64_t s = src_of(r);
    typename P::T val;
    if (s >= 0 && s < g.T) {
      val = P::load(vbase + s * g.v_st + pc * VEC);
    } else if (g.miss == LEMA_MISS_ZERO) {
      val = P::zero();
    } else {
      val = P::miss(P::load(vbase + pc * VEC), g.dtype);
    }
    P::store(ybase + static_cast<int64_t>(r) * g.y_st + pc * VEC, val);
  }
}

template <typename CodeT, int CHUNK, int VEC>
__global__ __launch_bounds__(CHUNK) void resolve_kernel(ResolveArgs a) {
  typedef ResolveLds<CodeT, CHUNK> L;
  constexpr int kSlots = L::kSlots, kMask = kSlots - 1, kSub = L::kSub;
  constexpr int kLog = Log2<kSlots>::value;
  __shared__ L s;

  // XCD-aware work mapping: every chunk of row r runs on XCD r % 8, which then keeps that
  // row's key codes and value rows in its own L2; the heaviest chunks (latest) go first.
  const int bid = blockIdx.x;
  const int xcd = bid % kNumXcd;
  const int k = bid / kNumXcd;
  const int chunk = a.nchunks - 1 - (k % a.nchunks);
  const int64_t row = static_cast<int64_t>(k / a.nchunks) * kNumXcd + xcd;
  if (row >= a.N) return;

  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const CodeT SENT = sentinel<CodeT>();
  const CodeT* qrow = static_cast<const CodeT*>(a.qc) + row * a.T;
  const CodeT* krow = static_cast<const CodeT*>(a.kc) + row * a.T;
  const int64_t c0 = static_cast<int64_t>(chunk) * CHUNK;
  const int64_t i = c0 + t;
  const bool active = i < a.T;
  const CodeT q = active ? qrow[i] : CodeT(0);
  const CodeT kk = active ? krow[i] : CodeT(0);

  for (int x = t; x <= kSlots; x += CHUNK) {
    s.code[x] = SENT;
    s.pos[x] = -1;
  }
  {
    uint32_t* lw = reinterpret_cast<uint32_t*>(&s.last[0][0]);
    for (int x = t; x < kSub * CHUNK / 2; x += CHUNK) lw[x] = 0xFFFFFFFFu;
  }
  if (t == 0) {
    s.nid = 0;
    s.sent_used = 0;
  }
  __syncthreads();

  // 1. the chunk's query codes -> slots; the first claimant of a slot gives it a dense id
  int qs = kSlots;
  if (active) {
    if (q == SENT) {
      if (atomicCAS(&s.sent_used, 0, 1) == 0) s.id[kSlots] = static_cast<int16_t>(atomicAdd(&s.nid, 1));
    } else {
      int h = slot_hash<kLog>(q);
      for (;;) {
        const CodeT old = lds_cas(&s.code[h], SENT, q);
        if (old == SENT) {
          s.id[h] = static_cast<int16_t>(atomicAdd(&s.nid, 1));
          break;
        }
        if (old == q) break;
        h = (h + 1) & kMask;
      }
      qs = h;
    }
  }
  __syncthreads();

  // the slot of code c among the chunk's query codes, or -1
  auto find = [&](CodeT c) -> int {
    if (c == SENT) return s.sent_used ? kSlots : -1;
    int h = slot_hash<kLog>(c);
    for (;;) {
      const CodeT x = s.code[h];
      if (x == c) return h;
      if (x == SENT) return -1;
      h = (h + 1) & kMask;
    }
  };

  // 2. (c) keys before the chunk raise their code's latest position
  for (int64_t j0 = 0; j0 < c0; j0 += 4 * CHUNK) {
    CodeT kj[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t j = j0 + e * CHUNK + t;
      kj[e] = j < c0 ? krow[j] : CodeT(0);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t j = j0 + e * CHUNK + t;
      if (j < c0) {
        const int sl = find(kj[e]);
        if (sl >= 0) atomicMax(&s.pos[sl], static_cast<int32_t>(j));
      }
    }
  }

  // 3. (a) + (b) keys inside the chunk
  int kid = -1;
  if (active) {
    const int sl = find(kk);
    if (sl >= 0) kid = s.id[sl];
  }
  const int qid = active ? static_cast<int>(s.id[qs]) : -2;
  int qbest = -1;
  bool klast = true;
#pragma unroll
  for (int l2 = 0; l2 < 64; ++l2) {
    const int o = __builtin_amdgcn_readlane(kid, l2);
    if (o == qid && l2 < lane) qbest = l2;
    if (o == kid && l2 > lane) klast = false;
  }
  if (kid >= 0 && klast) s.last[w][kid] = static_cast<int16_t>(t);
  __syncthreads();

  const int nid = s.nid;
  for (int x = t; x < nid; x += CHUNK) {
    int run = -1;
#pragma unroll
    for (int ww = 0; ww < kSub; ++ww) {
      const int m = s.last[ww][x];
      s.last[ww][x] = static_cast<int16_t>(run);
      run = m > run ? m : run;
    }
  }
  __syncthreads();

  int32_t src = -1;
  if (active) {
    if (qbest >= 0) {
      src = static_cast<int32_t>(c0 + w * 64 + qbest);
    } else {
      const int m = s.last[w][qid];
      src = m >= 0 ? static_cast<int32_t>(c0 + m) : s.pos[qs];
    }
    if (a.src != nullptr) {
      if (a.src_bytes == 8)
        static_cast<int64_t*>(a.src)[row * a.T + i] = src;
      else
        static_cast<int32_t*>(a.src)[row * a.T + i] = src;
    }
  }

  if constexpr (VEC > 0) {
    s.src[t] = src;
    __syncthreads();
    const int nrows = static_cast<int>(a.T - c0 < CHUNK ? a.T - c0 : CHUNK);
    gather_rows<VEC>(a.g, row, c0, nrows, t, CHUNK,
                     [&](uint32_t r) -> int64_t { return s.src[r]; });
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
  gather_rows<VEC>(a.g, row, c0, nrows, threadIdx.x, blockDim.x,
                   [&](uint32_t r) -> int64_t { return ssrc[r]; });
}

constexpr int kChunk = 1024;

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
  switch (vec) {
    case 0: resolve_kernel<CodeT, kChunk, 0><<<dim3(grid), dim3(kChunk), 0, st>>>(a); break;
    case 16: resolve_kernel<CodeT, kChunk, 16><<<dim3(grid), dim3(kChunk), 0, st>>>(a); break;
    case 8: resolve_kernel<CodeT, kChunk, 8><<<dim3(grid), dim3(kChunk), 0, st>>>(a); break;
    case 4: resolve_kernel<CodeT, kChunk, 4><<<dim3(grid), dim3(kChunk), 0, st>>>(a); break;
    case 2: resolve_kernel<CodeT, kChunk, 2><<<dim3(grid), dim3(kChunk), 0, st>>>(a); break;
    default: set_error("internal: piece size %d", vec); return LEMA_BAD_ARG;
  }
  return launch_status("resolve_kernel");
}

int check_rows(const void* qc, const void* kc, int32_t code_bytes, int64_t N, int64_t T) {
  LEMA_REQUIRE(code_bytes == 4 || code_bytes == 8, "code_bytes must be 4 or 8, got %d", code_bytes);
  LEMA_REQUIRE(N >= 0 && T >= 0, "negative shape N=%lld T=%lld", (long long)N, (long long)T);
  LEMA_REQUIRE(T < (int64_t(1) << 31), "T=%lld exceeds int32 positions", (long long)T);
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
