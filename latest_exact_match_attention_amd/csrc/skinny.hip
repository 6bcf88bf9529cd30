// Skinny bf16 GEMMs on the matrix cores for decoding: Y[M, N] = X[M, K] . W[N, K]^T with few
// rows (M <= 32: one token of each of a batch of streams), the shape of every projection of a
// decode step (code/lema/model.py:168-179, 85-94, the head). Such a product reads W once and is
// bound by that read; a workgroup streams a block of 16 * CT rows of W with its 8 wavefronts
// splitting K, each wavefront running v_mfma_f32_16x16x32_bf16 on 16-byte fragments loaded
// straight from memory (no LDS staging: X is a few KB and stays in L2), and the partial sums
// are reduced through LDS.
//
// Epilogues (a launch can hold up to three weight segments over the same x, e.g. a layer's q,
// k and v projections):
//   plain   Y rounded to bf16, optionally added to a bf16 residual (the MLP's down projection
//           and the residual add of Block.forward, code/lema/model.py:229-232);
//   pack    the q or k projection straight to codes (code/lema/attention.py:82-97): bit j of a
//           head's code is (bf16(z_j) >= 0), the sign of the value the unfused path would have
//           stored -- the projection's output never goes to HBM. A block covers 16 columns and
//           writes the bytes of each code its columns hold (d a multiple of 8), or whole heads;
//   swiglu  silu(x . gate^T) * (x . up^T) with the same bf16 roundings as SwiGLU.forward's
//           ops (code/lema/model.py:85-94): the block computes 16 columns of both.
// A swiglu launch can also take the MLP's pre-norm (Block.forward's norm2 with the attention's
// residual add, code/lema/model.py:229-232): every block then forms the normalised rows
// itself, with the stand-alone norm kernel's arithmetic (norm_row.h), into LDS and multiplies
// those; block 0 also writes x + d, the MLP's residual. That saves the norm's launch. A q/k/v
// launch takes the attention's pre-norm the same way (norm1, no addend): batch-16 decode steps
// of the 24-layer LM went 1.428 -> 1.391 ms.
//
// Operand layout of v_mfma_f32_16x16x32_bf16 (checked on the device): lane l holds A row l%16
// and B column l%16, k = 8 * (l / 16) + j, j < 8; the result's register r of lane l is row
// 4 * (l / 16) + r, column l % 16.
#include "lema_internal.h"
#include "norm_row.h"

namespace lema {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kSkThreads = 512;
constexpr int kSkWaves = kSkThreads / 64;
constexpr int kSkUnroll = 4;  // K-steps of 32 with loads in flight per wavefront
constexpr int kSkNormSteps = 4;  // a fused pre-norm's rows: up to 4 * 512 elements in registers

// One weight segment of a launch: its blocks cover N output columns of x . w^T with one
// epilogue. A launch holds up to three segments sharing x (the q, k and v projections of a
// layer in one launch).
enum SkMode : int32_t { kSkPlain = 0, kSkPack = 1, kSkSwiglu = 2 };

struct SkSegment {
  const uint16_t* w;   // [N, K]
  const uint16_t* w2;  // swiglu: the up projection [N, K] (w is the gate)
  void* out;           // plain / swiglu: bf16 [M, ldy]; pack: codes
  const uint16_t* res; // plain: optional bf16 [M, ldy] residual, out = bf16(res + bf16(sum))
  int64_t ldy;
  int32_t N, mode, blocks, code_bytes;
  int32_t cols;        // output columns per block (set at launch; swiglu: of the gate and of up)
};

// A product on few blocks leaves CUs idle, and each block's weight read is bound by what its
// CU keeps in flight (measured at M = 1, K = 1536: 96 and 192 blocks of 16 columns both take
// 3.9 us). A launch of plain segments only (16-column tiles) with at most kNarrowMaxN columns
// therefore takes blocks of 8 columns, the other half of each matrix-core tile idle. A launch
// with packed segments (q/k/v) already has three segments' blocks and keeps 16 columns.
constexpr int kNarrowCols = 8;
constexpr int kNarrowMaxN = 256 * kNarrowCols;

struct SkinnyArgs {
  const uint16_t* x;
  int64_t ldx, ldw;
  int32_t M, K;
  int32_t d, T;  // pack: bits per code (one head), positions per stream (row m = (b, t))
  int32_t nseg;
  SkSegment seg[3];
  // fused pre-norm (nw non-null): x is the residual stream, nd the addend (or null), rows of
  // K; the product's input is norm(x + nd) * nw, and ns receives x + nd (rows of K)
  const uint16_t* nd;
  const uint16_t* nw;
  uint16_t* ns;
  float eps;
};

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  const uint32_t b = __float_as_uint(f);
  if ((b & 0x7F800000u) == 0x7F800000u && (b & 0x007FFFFFu) != 0) return 0x7FC0u;
  return (b + 0x7FFFu + ((b >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// (bf16(z) >= 0) as a float comparison: -0 -> true, NaN -> false.
__device__ __forceinline__ bool bf16_nonneg(float z) {
  return bf16_bits_to_f32(f32_to_bf16_bits(z)) >= 0.0f;
}

// A block owns `cols` columns: 16 * CT, or 8 for a narrow plain segment (swiglu: 16 columns
// of the gate and the same 16 of up).
template <int MT, int CT, bool kNorm>
__global__ __launch_bounds__(kSkThreads) void skinny_kernel(SkinnyArgs a) {
  __shared__ float part[kSkWaves][MT * 16][CT * 16 + 1];
  extern __shared__ __align__(16) uint16_t xs[];  // kNorm: the normalised rows, stride K + 8
  int bid = blockIdx.x, si = 0;
  while (si + 1 < a.nseg && bid >= a.seg[si].blocks) {
    bid -= a.seg[si].blocks;
    ++si;
  }
  const SkSegment& sg = a.seg[si];
  const bool glu = sg.mode == kSkSwiglu;
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int cols = sg.cols;
  const int n0 = bid * cols;
  const int ksteps = a.K / 32;
  const int per = (ksteps + kSkWaves - 1) / kSkWaves;
  const int s0 = wave * per;
  const int s1 = s0 + per < ksteps ? s0 + per : ksteps;
  const int r16 = l & 15, kg = (l >> 4) * 8;

  const uint16_t* wp[CT];
  bool wok[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    const int c = glu ? r16 : 16 * ct + r16;  // column of the block
    const int n = n0 + c;
    wok[ct] = c < cols && n < sg.N && (!glu || ct < 2);
    const uint16_t* base = (glu && ct == 1) ? sg.w2 : sg.w;
    wp[ct] = base + static_cast<int64_t>(wok[ct] ? n : 0) * a.ldw + kg;
  }
  const uint16_t* xp[MT];
  bool xok[MT];
  if constexpr (kNorm) {
    // rows m and m + 8 of x by wavefront m, into LDS (a stride of K + 8 puts the 16 rows a
    // fragment load reads in different banks)
    const int xst = a.K + 8;
    for (int m = wave; m < a.M; m += 2 * kSkWaves) {
      const int n = m + kSkWaves < a.M ? 2 : 1;
      const uint16_t* xr[2];
      const uint16_t* dr[2];
      uint16_t* sr[2];
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int64_t mr = m + r * kSkWaves < a.M ? m + r * kSkWaves : m;
        xr[r] = a.x + mr * a.ldx;
        dr[r] = a.nd != nullptr ? a.nd + mr * a.K : nullptr;
        sr[r] = blockIdx.x == 0 && a.ns != nullptr ? a.ns + mr * a.K : nullptr;
      }
      norm_rows<2, kSkNormSteps>(xr, dr, n, a.nw, a.eps, a.K, l, sr, [&](int r, int e, u32x4 h) {
        *reinterpret_cast<u32x4*>(xs + (m + r * kSkWaves) * xst + e) = h;
      });
    }
    __syncthreads();
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = 16 * mt + r16;
      xok[mt] = m < a.M;
      xp[mt] = xs + (xok[mt] ? m : 0) * xst + kg;
    }
  } else {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = 16 * mt + r16;
      xok[mt] = m < a.M;
      xp[mt] = a.x + static_cast<int64_t>(xok[mt] ? m : 0) * a.ldx + kg;
    }
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
  constexpr int kPer = (kRows * kCols + kSkThreads - 1) / kSkThreads;
  float sums[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int e = threadIdx.x + i * kSkThreads;
    sums[i] = 0.f;
    if (e < kRows * kCols) {
      const int row = e / kCols, col = e - (e / kCols) * kCols;
#pragma unroll
      for (int wv = 0; wv < kSkWaves; ++wv) sums[i] += part[wv][row][col];
    }
  }
  if (sg.mode == kSkPlain) {
    uint16_t* y = static_cast<uint16_t*>(sg.out);
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int e = threadIdx.x + i * kSkThreads;
      const int row = e / kCols, col = e - (e / kCols) * kCols;
      if (e < kRows * kCols && row < a.M && col < cols && n0 + col < sg.N) {
        const int64_t at = static_cast<int64_t>(row) * sg.ldy + n0 + col;
        uint32_t out = f32_to_bf16_bits(sums[i]);
        if (sg.res != nullptr) out = f32_to_bf16_bits(bf16_bits_to_f32(sg.res[at]) + bf16_bits_to_f32(out));
        y[at] = static_cast<uint16_t>(out);
      }
    }
    return;
  }
  __syncthreads();  // every partial is read: the block's sums go to part[0]
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int e = threadIdx.x + i * kSkThreads;
    if (e < kRows * kCols) part[0][e / kCols][e - (e / kCols) * kCols] = sums[i];
  }
  __syncthreads();
  if (glu) {  // out = silu(gate) * up, the silu rounded to bf16 first
    uint16_t* y = static_cast<uint16_t*>(sg.out);
    for (int e = threadIdx.x; e < kRows * 16; e += kSkThreads) {
      const int row = e >> 4, c = e & 15;
      if (row >= a.M || c >= cols || n0 + c >= sg.N) continue;
      const float g = bf16_bits_to_f32(f32_to_bf16_bits(part[0][row][c]));
      const float u = bf16_bits_to_f32(f32_to_bf16_bits(part[0][row][16 + c]));
      const float sl = bf16_bits_to_f32(f32_to_bf16_bits(g / (1.0f + expf(-g))));
      y[static_cast<int64_t>(row) * sg.ldy + n0 + c] = static_cast<uint16_t>(f32_to_bf16_bits(sl * u));
    }
    return;
  }
  // the heads this block's columns [n0, n0 + cols) touch; a head split over blocks gets its
  // byte-aligned bit range written by each (d is a multiple of 8 then, checked on the host),
  // the block with its last bit also clearing the code's bytes above d
  const int H = sg.N / a.d;
  const int h0 = n0 / a.d;
  const int h1 = min((n0 + cols - 1) / a.d, H - 1);
  const int nh = h1 - h0 + 1;
  for (int e = threadIdx.x; e < kRows * nh; e += kSkThreads) {
    const int row = e / nh, h = h0 + (e - (e / nh) * nh);
    if (row >= a.M) continue;
    const int c_lo = max(n0, h * a.d), c_hi = min(n0 + cols, (h + 1) * a.d);
    uint64_t code = 0;
    for (int n = c_lo; n < c_hi; ++n)
      if (bf16_nonneg(part[0][row][n - n0])) code |= uint64_t(1) << (n - h * a.d);
    const int64_t b = row / a.T, t = row - (row / a.T) * a.T;
    const int64_t at = (b * H + h) * a.T + t;
    const int j_lo = c_lo - h * a.d, j_hi = c_hi - h * a.d;  // bits [j_lo, j_hi) of the code
    if (j_lo == 0 && j_hi == a.d) {
      if (sg.code_bytes == 4)
        static_cast<uint32_t*>(sg.out)[at] = static_cast<uint32_t>(code);
      else
        static_cast<uint64_t*>(sg.out)[at] = code;
    } else {
      uint8_t* w8 = static_cast<uint8_t*>(sg.out) + at * sg.code_bytes;
      for (int k = j_lo / 8; k < j_hi / 8; ++k) w8[k] = static_cast<uint8_t>(code >> (8 * k));
      if (j_hi == a.d)
        for (int k = a.d / 8; k < sg.code_bytes; ++k) w8[k] = 0;
    }
  }
}

template <int CT>
int launch_skinny(SkinnyArgs& a, hipStream_t st) {
  int blocks = 0;
  for (int i = 0; i < a.nseg; ++i) {
    SkSegment& sg = a.seg[i];
    bool all_plain = true;
    for (int j = 0; j < a.nseg; ++j) all_plain = all_plain && a.seg[j].mode == kSkPlain;
    sg.cols = sg.mode == kSkSwiglu ? 16
              : CT == 1 && all_plain && sg.N <= kNarrowMaxN ? kNarrowCols
                                                           : 16 * CT;
    sg.blocks = (sg.N + sg.cols - 1) / sg.cols;
    blocks += sg.blocks;
  }
  const dim3 grid(blocks), block(kSkThreads);
  if (a.nw != nullptr) {  // the normalised rows in LDS (checked to fit by the entry point)
    const size_t lds = static_cast<size_t>(a.M) * (a.K + 8) * sizeof(uint16_t);
    if (a.M <= 16)
      skinny_kernel<1, CT, true><<<grid, block, lds, st>>>(a);
    else
      skinny_kernel<2, CT, true><<<grid, block, lds, st>>>(a);
  } else if (a.M <= 16) {
    skinny_kernel<1, CT, false><<<grid, block, 0, st>>>(a);
  } else {
    skinny_kernel<2, CT, false><<<grid, block, 0, st>>>(a);
  }
  return launch_status("skinny_kernel");
}

int launch_ct(SkinnyArgs& a, int ct, hipStream_t st) {
  switch (ct) {
    case 1: return launch_skinny<1>(a, st);
    case 2: return launch_skinny<2>(a, st);
    case 3: return launch_skinny<3>(a, st);
    default: return launch_skinny<4>(a, st);
  }
}

int check_skinny(const void* x, int64_t ldx, int64_t ldw, int64_t M, int64_t K) {
  LEMA_REQUIRE(M >= 1 && M <= 32, "skinny products take 1..32 rows, got %lld", (long long)M);
  LEMA_REQUIRE(K >= 32 && K % 32 == 0 && K < (int64_t(1) << 30), "K=%lld must be a multiple of 32",
               (long long)K);
  LEMA_REQUIRE(ldx >= K && ldw >= K && ldx % 8 == 0 && ldw % 8 == 0,
               "row strides must be >= K and multiples of 8");
  LEMA_REQUIRE(x != nullptr && aligned(x, 16), "x must be a 16-byte aligned device pointer");
  return LEMA_OK;
}

int check_weight(const void* w, int64_t N) {
  LEMA_REQUIRE(w != nullptr && aligned(w, 16), "weights must be 16-byte aligned device pointers");
  LEMA_REQUIRE(N >= 1 && N < (int64_t(1) << 30), "N=%lld", (long long)N);
  return LEMA_OK;
}

// Column tiles per block for codes of d bits: one (16 columns, a head split over blocks
// writes its bytes from each) when d is a multiple of 8, else the least multiple of 16 (up to
// 64) holding whole heads, or 0. More blocks of fewer weight rows: the q and k projections of
// 64-bit heads ran on 24 blocks of 64 rows each.
int pack_ct(int32_t d) {
  if (d % 8 == 0) return 1;
  for (int c = 1; c <= 4; ++c)
    if ((16 * c) % d == 0) return c;
  return 0;
}

}  // namespace
}  // namespace lema

using namespace lema;

extern "C" int lema_skinny_gemm_bf16(const void* x, int64_t ldx, const void* w, int64_t ldw,
                                     void* y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                                     void* stream) {
  clear_error();
  if (int rc = check_skinny(x, ldx, ldw, M, K)) return rc;
  if (int rc = check_weight(w, N)) return rc;
  LEMA_REQUIRE(y != nullptr && ldy >= N, "bad output");
  SkinnyArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.ldx = ldx;
  a.ldw = ldw;
  a.M = static_cast<int32_t>(M);
  a.K = static_cast<int32_t>(K);
  a.nseg = 1;
  a.seg[0] = SkSegment{static_cast<const uint16_t*>(w), nullptr, y, nullptr, ldy,
                       static_cast<int32_t>(N), kSkPlain, 0, 0};
  return launch_ct(a, 1, static_cast<hipStream_t>(stream));
}

extern "C" int lema_skinny_gemm_add_bf16(const void* x, int64_t ldx, const void* w, int64_t ldw,
                                         const void* r, void* y, int64_t ldy, int64_t M, int64_t N,
                                         int64_t K, void* stream) {
  clear_error();
  if (int rc = check_skinny(x, ldx, ldw, M, K)) return rc;
  if (int rc = check_weight(w, N)) return rc;
  LEMA_REQUIRE(y != nullptr && r != nullptr && ldy >= N, "bad output or residual");
  SkinnyArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.ldx = ldx;
  a.ldw = ldw;
  a.M = static_cast<int32_t>(M);
  a.K = static_cast<int32_t>(K);
  a.nseg = 1;
  a.seg[0] = SkSegment{static_cast<const uint16_t*>(w), nullptr, y,
                       static_cast<const uint16_t*>(r), ldy, static_cast<int32_t>(N), kSkPlain, 0,
                       0};
  return launch_ct(a, 1, static_cast<hipStream_t>(stream));
}

extern "C" int lema_skinny_pack_bf16(const void* x, int64_t ldx, const void* w, int64_t ldw,
                                     int64_t M, int64_t N, int64_t K, int32_t d, int64_t T,
                                     void* codes, int32_t code_bytes, void* stream) {
  clear_error();
  if (int rc = check_skinny(x, ldx, ldw, M, K)) return rc;
  if (int rc = check_weight(w, N)) return rc;
  LEMA_REQUIRE(d >= 1 && d <= 64 && N % d == 0, "head width %d must divide N=%lld", d, (long long)N);
  LEMA_REQUIRE(code_bytes == 8 || (code_bytes == 4 && d <= 32), "code_bytes %d for %d-bit codes",
               code_bytes, d);
  LEMA_REQUIRE(T >= 1 && M % T == 0, "rows %lld are not streams x %lld positions", (long long)M,
               (long long)T);
  LEMA_REQUIRE(codes != nullptr && aligned(codes, code_bytes), "bad code pointer");
  const int ct = pack_ct(d);
  LEMA_REQUIRE(ct > 0, "head width %d does not tile 16..64 columns", d);
  SkinnyArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.ldx = ldx;
  a.ldw = ldw;
  a.M = static_cast<int32_t>(M);
  a.K = static_cast<int32_t>(K);
  a.d = d;
  a.T = static_cast<int32_t>(T);
  a.nseg = 1;
  a.seg[0] = SkSegment{static_cast<const uint16_t*>(w), nullptr, codes, nullptr, 0,
                       static_cast<int32_t>(N), kSkPack, 0, code_bytes};
  return launch_ct(a, ct, static_cast<hipStream_t>(stream));
}

namespace lema {
namespace {

// The checks and the three segments of a q/k/v launch; `ct` receives its block width.
int qkv_args(SkinnyArgs& a, int& ct, const void* x, int64_t ldx, const void* wq, const void* wk,
             const void* wv, int64_t ldw, int64_t M, int64_t Nqk, int64_t Nv, int64_t K,
             int32_t d, int64_t T, void* qcodes, void* kcodes, int32_t code_bytes, void* v) {
  if (int rc = check_skinny(x, ldx, ldw, M, K)) return rc;
  if (int rc = check_weight(wq, Nqk)) return rc;
  if (int rc = check_weight(wk, Nqk)) return rc;
  if (int rc = check_weight(wv, Nv)) return rc;
  LEMA_REQUIRE(d >= 1 && d <= 64 && Nqk % d == 0, "head width %d must divide %lld", d,
               (long long)Nqk);
  LEMA_REQUIRE(code_bytes == 8 || (code_bytes == 4 && d <= 32), "code_bytes %d for %d-bit codes",
               code_bytes, d);
  LEMA_REQUIRE(T >= 1 && M % T == 0, "rows %lld are not streams x %lld positions", (long long)M,
               (long long)T);
  LEMA_REQUIRE(qcodes && kcodes && aligned(qcodes, code_bytes) && aligned(kcodes, code_bytes) &&
                   v != nullptr, "bad output pointer");
  ct = pack_ct(d);
  LEMA_REQUIRE(ct > 0, "head width %d does not tile 16..64 columns", d);
  a.x = static_cast<const uint16_t*>(x);
  a.ldx = ldx;
  a.ldw = ldw;
  a.M = static_cast<int32_t>(M);
  a.K = static_cast<int32_t>(K);
  a.d = d;
  a.T = static_cast<int32_t>(T);
  a.nseg = 3;
  a.seg[0] = SkSegment{static_cast<const uint16_t*>(wq), nullptr, qcodes, nullptr, 0,
                       static_cast<int32_t>(Nqk), kSkPack, 0, code_bytes};
  a.seg[1] = SkSegment{static_cast<const uint16_t*>(wk), nullptr, kcodes, nullptr, 0,
                       static_cast<int32_t>(Nqk), kSkPack, 0, code_bytes};
  a.seg[2] = SkSegment{static_cast<const uint16_t*>(wv), nullptr, v, nullptr, Nv,
                       static_cast<int32_t>(Nv), kSkPlain, 0, 0};
  return LEMA_OK;
}

}  // namespace
}  // namespace lema

extern "C" int lema_skinny_qkv_bf16(const void* x, int64_t ldx, const void* wq, const void* wk,
                                    const void* wv, int64_t ldw, int64_t M, int64_t Nqk,
                                    int64_t Nv, int64_t K, int32_t d, int64_t T, void* qcodes,
                                    void* kcodes, int32_t code_bytes, void* v, void* stream) {
  clear_error();
  SkinnyArgs a{};
  int ct = 0;
  if (int rc = qkv_args(a, ct, x, ldx, wq, wk, wv, ldw, M, Nqk, Nv, K, d, T, qcodes, kcodes,
                        code_bytes, v))
    return rc;
  return launch_ct(a, ct, static_cast<hipStream_t>(stream));
}

// The attention's pre-norm inside the q/k/v launch (Block.gpu_pre: norm1, then the
// projections, code/lema/model.py:224-227): every block normalises the rows of x (contiguous,
// K elements) into LDS with the stand-alone norm kernel's arithmetic and multiplies those, so
// the codes and v equal lema_rmsnorm_bf16 followed by lema_skinny_qkv_bf16 with one launch
// fewer.
extern "C" int lema_skinny_norm_qkv_bf16(const void* x, const void* nw, float eps,
                                         const void* wq, const void* wk, const void* wv,
                                         int64_t ldw, int64_t M, int64_t Nqk, int64_t Nv,
                                         int64_t K, int32_t d, int64_t T, void* qcodes,
                                         void* kcodes, int32_t code_bytes, void* v,
                                         void* stream) {
  clear_error();
  SkinnyArgs a{};
  int ct = 0;
  if (int rc = qkv_args(a, ct, x, K, wq, wk, wv, ldw, M, Nqk, Nv, K, d, T, qcodes, kcodes,
                        code_bytes, v))
    return rc;
  LEMA_REQUIRE(K <= 512 * kSkNormSteps, "the fused norm takes rows of at most %d elements, got K=%lld",
               512 * kSkNormSteps, (long long)K);
  // LDS: the rows (M x (K + 8) bf16) next to the partial sums (8 x 16 or 32 rows x 16 ct + 1)
  const int64_t lds = M * (K + 8) * 2 + kSkWaves * (M <= 16 ? 16 : 32) * (16 * ct + 1) * 4;
  LEMA_REQUIRE(lds <= 160 * 1024, "%lld rows of %lld do not fit the LDS of a workgroup",
               (long long)M, (long long)K);
  LEMA_REQUIRE(nw != nullptr && aligned(nw, 16), "norm weight must be a 16-byte aligned device pointer");
  a.nd = nullptr;
  a.nw = static_cast<const uint16_t*>(nw);
  a.ns = nullptr;
  a.eps = eps;
  return launch_ct(a, ct, static_cast<hipStream_t>(stream));
}

extern "C" int lema_skinny_swiglu_bf16(const void* x, int64_t ldx, const void* wg, const void* wu,
                                       int64_t ldw, int64_t M, int64_t N, int64_t K, void* out,
                                       void* stream) {
  clear_error();
  if (int rc = check_skinny(x, ldx, ldw, M, K)) return rc;
  if (int rc = check_weight(wg, N)) return rc;
  if (int rc = check_weight(wu, N)) return rc;
  LEMA_REQUIRE(out != nullptr, "bad output pointer");
  SkinnyArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.ldx = ldx;
  a.ldw = ldw;
  a.M = static_cast<int32_t>(M);
  a.K = static_cast<int32_t>(K);
  a.nseg = 1;
  a.seg[0] = SkSegment{static_cast<const uint16_t*>(wg), static_cast<const uint16_t*>(wu), out,
                       nullptr, N, static_cast<int32_t>(N), kSkSwiglu, 0, 0};
  return launch_ct(a, 2, static_cast<hipStream_t>(stream));
}

extern "C" int lema_skinny_norm_swiglu_bf16(const void* x, const void* d, const void* nw,
                                            float eps, void* x_out, const void* wg,
                                            const void* wu, int64_t ldw, int64_t M, int64_t N,
                                            int64_t K, void* out, void* stream) {
  clear_error();
  if (int rc = check_skinny(x, K, ldw, M, K)) return rc;
  if (int rc = check_weight(wg, N)) return rc;
  if (int rc = check_weight(wu, N)) return rc;
  LEMA_REQUIRE(out != nullptr, "bad output pointer");
  LEMA_REQUIRE(K <= 512 * kSkNormSteps, "the fused norm takes rows of at most %d elements, got K=%lld",
               512 * kSkNormSteps, (long long)K);
  // LDS: the rows (M x (K + 8) bf16) next to the partial sums (8 x 16 or 32 rows x 33 floats)
  const int64_t lds = M * (K + 8) * 2 + kSkWaves * (M <= 16 ? 16 : 32) * 33 * 4;
  LEMA_REQUIRE(lds <= 160 * 1024, "%lld rows of %lld do not fit the LDS of a workgroup",
               (long long)M, (long long)K);
  LEMA_REQUIRE(nw != nullptr && aligned(nw, 16), "norm weight must be a 16-byte aligned device pointer");
  LEMA_REQUIRE(d == nullptr || (aligned(d, 16) && x_out != nullptr && aligned(x_out, 16) &&
                                x_out != x && x_out != d),
               "the addend needs a 16-byte aligned output for x + d that is neither input");
  SkinnyArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.ldx = K;
  a.ldw = ldw;
  a.M = static_cast<int32_t>(M);
  a.K = static_cast<int32_t>(K);
  a.nseg = 1;
  a.seg[0] = SkSegment{static_cast<const uint16_t*>(wg), static_cast<const uint16_t*>(wu), out,
                       nullptr, N, static_cast<int32_t>(N), kSkSwiglu, 0, 0};
  a.nd = static_cast<const uint16_t*>(d);
  a.nw = static_cast<const uint16_t*>(nw);
  a.ns = static_cast<uint16_t*>(x_out);
  a.eps = eps;
  return launch_ct(a, 2, static_cast<hipStream_t>(stream));
}
