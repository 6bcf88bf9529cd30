// Skinny bf16 GEMMs on the matrix cores for decoding: Y[M, N] = X[M, K] . W[N, K]^T with few
// rows (M <= 32: one token of each of a batch of streams), the shape of every projection of a
// decode step (code/lema/model.py:168-179, 85-94, the head). Such a product reads W once and is
// bound by that read; a workgroup streams a block of 16 * CT rows of W with its 8 wavefronts
// splitting K, each wavefront running v_mfma_f32_16x16x32_bf16 on 16-byte fragments loaded
// straight from memory (no LDS staging: X is a few KB and stays in L2), and the partial sums
// are reduced through LDS.
//
// Epilogues:
//   plain  Y rounded to bf16;
//   pack   the q or k projection straight to codes (code/lema/attention.py:82-97): the block
//          covers whole heads of d columns, and bit j of a head's code is (bf16(z_j) >= 0),
//          the sign of the value the unfused path would have stored -- the projection's
//          output never goes to HBM.
//
// Operand layout of v_mfma_f32_16x16x32_bf16 (checked on the device): lane l holds A row l%16
// and B column l%16, k = 8 * (l / 16) + j, j < 8; the result's register r of lane l is row
// 4 * (l / 16) + r, column l % 16.
#include "lema_internal.h"

namespace lema {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kSkThreads = 512;
constexpr int kSkWaves = kSkThreads / 64;
constexpr int kSkUnroll = 4;  // K-steps of 32 with loads in flight per wavefront

struct SkinnyArgs {
  const uint16_t* x;
  int64_t ldx;
  const uint16_t* w;
  int64_t ldw;
  uint16_t* y;
  int64_t ldy;
  void* codes;
  int32_t code_bytes;
  int32_t M, N, K;
  int32_t d;      // pack: bits per code (one head's columns)
  int32_t H, T;   // pack: heads per row of Y, positions per stream: row m = (b, t)
};

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  const uint32_t b = __float_as_uint(f);
  if ((b & 0x7F800000u) == 0x7F800000u && (b & 0x007FFFFFu) != 0) return 0x7FC0u;
  return (b + 0x7FFFu + ((b >> 16) & 1u)) >> 16;
}

// (bf16(z) >= 0) as a float comparison: -0 -> true, NaN -> false.
__device__ __forceinline__ bool bf16_nonneg(float z) {
  return __uint_as_float(f32_to_bf16_bits(z) << 16) >= 0.0f;
}

template <int MT, int CT, bool PACK>
__global__ __launch_bounds__(kSkThreads) void skinny_kernel(SkinnyArgs a) {
  __shared__ float part[kSkWaves][MT * 16][CT * 16 + 1];
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int n0 = blockIdx.x * (CT * 16);
  const int ksteps = a.K / 32;
  const int per = (ksteps + kSkWaves - 1) / kSkWaves;
  const int s0 = wave * per;
  const int s1 = s0 + per < ksteps ? s0 + per : ksteps;
  const int r16 = l & 15, kg = (l >> 4) * 8;

  const uint16_t* wp[CT];
  bool wok[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    const int n = n0 + 16 * ct + r16;
    wok[ct] = n < a.N;
    wp[ct] = a.w + static_cast<int64_t>(wok[ct] ? n : 0) * a.ldw + kg;
  }
  const uint16_t* xp[MT];
  bool xok[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = 16 * mt + r16;
    xok[mt] = m < a.M;
    xp[mt] = a.x + static_cast<int64_t>(xok[mt] ? m : 0) * a.ldx + kg;
  }

  f32x4 acc[MT][CT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) acc[mt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
  const bf16x8 zero8 = {};
  for (int s = s0; s < s1; s += kSkUnroll) {
    bf16x8 wf[kSkUnroll][CT], xf[kSkUnroll][MT];
#pragma unroll
    for (int u = 0; u < kSkUnroll; ++u) {
      const bool in = s + u < s1;
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
        wf[u][ct] = (in && wok[ct]) ? *reinterpret_cast<const bf16x8*>(wp[ct] + (s + u) * 32) : zero8;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        xf[u][mt] = (in && xok[mt]) ? *reinterpret_cast<const bf16x8*>(xp[mt] + (s + u) * 32) : zero8;
    }
#pragma unroll
    for (int u = 0; u < kSkUnroll; ++u)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
          acc[mt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf[u][mt], wf[u][ct], acc[mt][ct], 0, 0, 0);
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
      for (int r = 0; r < 4; ++r) part[wave][16 * mt + 4 * (l >> 4) + r][16 * ct + r16] = acc[mt][ct][r];
  __syncthreads();

  constexpr int kRows = MT * 16, kCols = CT * 16;
  if constexpr (!PACK) {
    for (int e = threadIdx.x; e < kRows * kCols; e += kSkThreads) {
      const int row = e / kCols, col = e - (e / kCols) * kCols;
      float v = 0.f;
#pragma unroll
      for (int wv = 0; wv < kSkWaves; ++wv) v += part[wv][row][col];
      if (row < a.M && n0 + col < a.N)
        a.y[static_cast<int64_t>(row) * a.ldy + n0 + col] = static_cast<uint16_t>(f32_to_bf16_bits(v));
    }
  } else {
    float sums[(kRows * kCols + kSkThreads - 1) / kSkThreads];
#pragma unroll
    for (int i = 0; i < (kRows * kCols + kSkThreads - 1) / kSkThreads; ++i) {
      const int e = threadIdx.x + i * kSkThreads;
      sums[i] = 0.f;
      if (e < kRows * kCols) {
        const int row = e / kCols, col = e - (e / kCols) * kCols;
#pragma unroll
        for (int wv = 0; wv < kSkWaves; ++wv) sums[i] += part[wv][row][col];
      }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < (kRows * kCols + kSkThreads - 1) / kSkThreads; ++i) {
      const int e = threadIdx.x + i * kSkThreads;
      if (e < kRows * kCols) part[0][e / kCols][e - (e / kCols) * kCols] = sums[i];
    }
    __syncthreads();
    const int heads = kCols / a.d;  // whole heads per block (checked on the host)
    for (int e = threadIdx.x; e < kRows * heads; e += kSkThreads) {
      const int row = e / heads, hh = e - (e / heads) * heads;
      const int h = n0 / a.d + hh;
      if (row >= a.M || h >= a.H) continue;
      uint64_t code = 0;
      for (int j = 0; j < a.d; ++j)
        if (bf16_nonneg(part[0][row][hh * a.d + j])) code |= uint64_t(1) << j;
      const int64_t b = row / a.T, t = row - (row / a.T) * a.T;
      const int64_t at = (b * a.H + h) * a.T + t;
      if (a.code_bytes == 4)
        static_cast<uint32_t*>(a.codes)[at] = static_cast<uint32_t>(code);
      else
        static_cast<uint64_t*>(a.codes)[at] = code;
    }
  }
}

template <int MT, bool PACK>
int launch_mt(const SkinnyArgs& a, int ct, hipStream_t st) {
  const int cols = 16 * ct;
  const dim3 grid((a.N + cols - 1) / cols), block(kSkThreads);
  switch (ct) {
    case 1: skinny_kernel<MT, 1, PACK><<<grid, block, 0, st>>>(a); break;
    case 2: skinny_kernel<MT, 2, PACK><<<grid, block, 0, st>>>(a); break;
    case 3: skinny_kernel<MT, 3, PACK><<<grid, block, 0, st>>>(a); break;
    default: skinny_kernel<MT, 4, PACK><<<grid, block, 0, st>>>(a); break;
  }
  return launch_status("skinny_kernel");
}

template <bool PACK>
int launch_skinny(const SkinnyArgs& a, int ct, hipStream_t st) {
  return a.M <= 16 ? launch_mt<1, PACK>(a, ct, st) : launch_mt<2, PACK>(a, ct, st);
}

int check_skinny(const void* x, int64_t ldx, const void* w, int64_t ldw, int64_t M, int64_t N,
                 int64_t K) {
  LEMA_REQUIRE(M >= 1 && M <= 32, "skinny products take 1..32 rows, got %lld", (long long)M);
  LEMA_REQUIRE(N >= 1 && N < (int64_t(1) << 30) && K >= 32 && K % 32 == 0 && K < (int64_t(1) << 30),
               "N=%lld, K=%lld (K a multiple of 32)", (long long)N, (long long)K);
  LEMA_REQUIRE(ldx >= K && ldw >= K && ldx % 8 == 0 && ldw % 8 == 0,
               "row strides must be >= K and multiples of 8");
  LEMA_REQUIRE(x != nullptr && w != nullptr && aligned(x, 16) && aligned(w, 16),
               "x and w must be 16-byte aligned device pointers");
  return LEMA_OK;
}

}  // namespace
}  // namespace lema

using namespace lema;

extern "C" int lema_skinny_gemm_bf16(const void* x, int64_t ldx, const void* w, int64_t ldw,
                                     void* y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                                     void* stream) {
  clear_error();
  if (int rc = check_skinny(x, ldx, w, ldw, M, N, K)) return rc;
  LEMA_REQUIRE(y != nullptr && ldy >= N, "bad output");
  SkinnyArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.ldx = ldx;
  a.w = static_cast<const uint16_t*>(w);
  a.ldw = ldw;
  a.y = static_cast<uint16_t*>(y);
  a.ldy = ldy;
  a.M = static_cast<int32_t>(M);
  a.N = static_cast<int32_t>(N);
  a.K = static_cast<int32_t>(K);
  return launch_skinny<false>(a, 1, static_cast<hipStream_t>(stream));
}

extern "C" int lema_skinny_pack_bf16(const void* x, int64_t ldx, const void* w, int64_t ldw,
                                     int64_t M, int64_t N, int64_t K, int32_t d, int64_t T,
                                     void* codes, int32_t code_bytes, void* stream) {
  clear_error();
  if (int rc = check_skinny(x, ldx, w, ldw, M, N, K)) return rc;
  LEMA_REQUIRE(d >= 1 && d <= 64 && N % d == 0, "head width %d must divide N=%lld", d, (long long)N);
  LEMA_REQUIRE(code_bytes == 8 || (code_bytes == 4 && d <= 32), "code_bytes %d for %d-bit codes",
               code_bytes, d);
  LEMA_REQUIRE(T >= 1 && M % T == 0, "rows %lld are not streams x %lld positions", (long long)M,
               (long long)T);
  LEMA_REQUIRE(codes != nullptr && aligned(codes, code_bytes), "bad code pointer");
  int ct = 0;
  for (int c = 1; c <= 4 && !ct; ++c)
    if ((16 * c) % d == 0) ct = c;
  LEMA_REQUIRE(ct > 0, "head width %d does not tile 16..64 columns", d);
  SkinnyArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.ldx = ldx;
  a.w = static_cast<const uint16_t*>(w);
  a.ldw = ldw;
  a.codes = codes;
  a.code_bytes = code_bytes;
  a.M = static_cast<int32_t>(M);
  a.N = static_cast<int32_t>(N);
  a.K = static_cast<int32_t>(K);
  a.d = d;
  a.H = static_cast<int32_t>(N / d);
  a.T = static_cast<int32_t>(T);
  return launch_skinny<true>(a, ct, static_cast<hipStream_t>(stream));
}
