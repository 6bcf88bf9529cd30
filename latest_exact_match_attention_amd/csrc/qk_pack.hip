// The query and key projections of a prefill straight to codes: codes of x . Wq^T and
// x . Wk^T (code/lema/model.py:168-175 followed by pack_codes, code/lema/attention.py:82-97),
// bit j of a head's code being (bf16(z_j) >= 0), with z never written to HBM. The unfused path
// writes zq and zk (2 x 201 MB of bf16 per layer of the language model at B4 T16384) and the
// pack kernel reads them back.
//
// A persistent bf16 MFMA GEMM on the concatenated columns [q | k] (2N), 256 x 256 tiles, one
// 512-thread workgroup per CU walking its tiles in XCD-local order (the row tiles of XCD x are
// [x, x + 1) * tiles_m / 8, taken GM at a time across every column tile). Waves w and w + 4
// share a SIMD; group g = w / 4 computes rows [128 g, 128 g + 128) of a tile, a wave 64 x 128
// as 2 x 4 v_mfma_f32_32x32x16_bf16 tiles. The groups alternate, one phase apart, between a
// memory phase (all fragments of a 64-deep stage read from LDS into registers; group 0 also
// issues the next stage's global -> LDS loads, buffer_load ... lds, into the other of two
// 64 KB stages) and a compute phase (32 MFMAs), so each SIMD always has one wave in MFMA. The
// epilogue turns each row's 32 column signs of an MFMA tile into one word (two instructions
// per sign; the lane pair holding the row combines its halves) and stores the code bytes: d is
// a multiple of 8, so a byte of a code never straddles a tile, and the writer of a code's last
// byte clears the bytes above d. The epilogue runs while the other group computes, so its
// instruction count sets what it costs: ~500 VALU instructions per tile and wave.
//
// Measured on the language model's shape (x [65536, 1536], Wq and Wk [1536, 1536], 64 heads
// of 24 bits, the model's layer-0 input), alternating with the unfused path on one device:
// 494.5 us (1.25 PFLOP/s) against 526 us for two hipBLASLt GEMMs and two packs, codes
// identical; 523 us with an epilogue of ~1230 instructions (a bf16 conversion and two compares
// per pair of signs, 64-bit divisions for the addresses).
#include "lema_internal.h"

namespace lema {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kQkBM = 256, kQkBN = 256, kQkBK = 64, kQkThreads = 512;
constexpr int kQkA = kQkBM * kQkBK * 2;      // one stage's A slab: 32 KB
constexpr int kQkStage = kQkA + kQkBN * kQkBK * 2;

// s_waitcnt vmcnt(0) alone; lgkmcnt(0) alone
#define QK_WAIT_VM0() __builtin_amdgcn_s_waitcnt(0x0F70)
#define QK_WAIT_LGKM0() __builtin_amdgcn_s_waitcnt(0xC07F)
#define QK_BARRIER()                   \
  do {                                 \
    __builtin_amdgcn_sched_barrier(0); \
    __builtin_amdgcn_s_barrier();      \
    __builtin_amdgcn_sched_barrier(0); \
  } while (0)

struct QkArgs {
  const uint16_t* x;
  const uint16_t* wq;
  const uint16_t* wk;
  void* qc;
  void* kc;
  int32_t M, N, K, ldx, ldw;
  int32_t d, T, H, code_bytes;
  int32_t tiles_m, tiles_n, gm;
  int32_t db, hstride;  // code bytes in use (d / 8); T * code_bytes
  float inv_db;
  int64_t bstride;      // one stream's codes: H * T * code_bytes
};

// w * 2 + (bf16(z) >= 0): for every fp32 z, NaN included, bf16(z) >= 0 under round to nearest
// even is z >= -2^-134 (a tie at 2^-134 rounds to -0, and fp32 denormals are kept), so one
// compare into VCC and an add that takes VCC as its carry in push the bit
__device__ __forceinline__ uint32_t push_sign(uint32_t w, float z, uint32_t thr) {
  uint32_t r;
  asm("v_cmp_le_f32_e32 vcc, %2, %1\n\tv_addc_co_u32_e32 %0, vcc, %3, %3, vcc"
      : "=v"(r)
      : "v"(z), "s"(thr), "v"(w)
      : "vcc");
  return r;
}

__global__ __launch_bounds__(kQkThreads, 1) void qk_pack_kernel(QkArgs g) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int t = threadIdx.x, l = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int grp = wave >> 2, wq = wave & 3;
  const int wr = grp * 128 + (wq >> 1) * 64;  // the wave's rows in the tile
  const int wc = (wq & 1) * 128;              // the wave's columns in the tile

  const int bid = blockIdx.x, nwg = gridDim.x;
  const int xcd = bid % 8, k8 = bid / 8, g8 = nwg / 8;
  const int per_x = g.tiles_m / 8;
  const int GM = g.gm;
  const int gsz = GM * g.tiles_n;
  const int my_tiles = (per_x * g.tiles_n - k8 + g8 - 1) / g8;
  auto tile_of = [&](int it, int& m0, int& n0) __attribute__((always_inline)) {
    const int li = k8 + it * g8;
    m0 = (xcd * per_x + (li / gsz) * GM + li % GM) * kQkBM;
    n0 = ((li % gsz) / GM) * kQkBN;
  };
  const int nk = g.K / kQkBK;
  const int total = my_tiles * nk;
  if (total <= 0) return;

  // global -> LDS (group 0): a stage is 64 blocks of 8 rows x 128 B, 16 per wave (blocks
  // wq + 4 x: x < 8 of A, x >= 8 of W). Row r keeps its 16-byte chunk c in slot
  // c ^ (r % 8) ^ ((r / 8) % 2) (conflict-free fragment reads); lane l writes row l / 8 of its
  // block, slot l % 8.
  const int lr = l >> 3, lc = (l & 7) ^ lr ^ (wq & 1);
  const uint32_t la = static_cast<uint32_t>(lr * g.ldx * 2 + lc * 16);
  const uint32_t lb = static_cast<uint32_t>(lr * g.ldw * 2 + lc * 16);
  auto dma_stage = [&](int s) __attribute__((always_inline)) {
    const int it = s / nk, kb = s - it * nk;
    int m0, n0;
    tile_of(it, m0, n0);
    const bool isq = n0 < g.N;
    const uint16_t* w = isq ? g.wq : g.wk;
    const int wrow = isq ? n0 : n0 - g.N;
    uint8_t* sa = smem + (s & 1) * kQkStage;
    const uint8_t* pa = reinterpret_cast<const uint8_t*>(g.x) +
                        static_cast<int64_t>(m0 + wq * 8) * g.ldx * 2 + kb * kQkBK * 2;
    const uint8_t* pb = reinterpret_cast<const uint8_t*>(w) +
                        static_cast<int64_t>(wrow + wq * 8) * g.ldw * 2 + kb * kQkBK * 2;
    const __amdgpu_buffer_rsrc_t ra =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(pa), 0, 0x7FFFFFFF, 0x00020000);
    const __amdgpu_buffer_rsrc_t rb =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(pb), 0, 0x7FFFFFFF, 0x00020000);
#pragma unroll
    for (int x = 0; x < 8; ++x)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, sa + (wq + 4 * x) * 1024, 16, la,
                                               x * 32 * g.ldx * 2, 0, 0);
#pragma unroll
    for (int x = 0; x < 8; ++x)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, sa + kQkA + (wq + 4 * x) * 1024, 16, lb,
                                               x * 32 * g.ldw * 2, 0, 0);
  };

  const int fr = l & 31;
  const int fsw = (fr & 7) ^ ((fr >> 3) & 1);
  bf16x8_t fa[4][2], fb[4][4];
  f32x16_t acc[2][4];
  auto zero_acc = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  };
  // memory phase: every fragment of stage s (buffer s & 1); group 0 first issues stage s + 1
  auto mphase = [&](int s) __attribute__((always_inline)) {
    if (grp == 0 && s + 1 < total) dma_stage(s + 1);
    const uint8_t* sb = smem + (s & 1) * kQkStage;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int ch = ((2 * kk + (l >> 5)) ^ fsw) << 4;
#pragma unroll
      for (int i = 0; i < 2; ++i)
        fa[kk][i] = *reinterpret_cast<const bf16x8_t*>(sb + (wr + i * 32 + fr) * 128 + ch);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        fb[kk][j] = *reinterpret_cast<const bf16x8_t*>(sb + kQkA + (wc + j * 32 + fr) * 128 + ch);
    }
    QK_WAIT_LGKM0();
  };
  // compute phase: with the W fragment first, lane l holds row l % 32 of an MFMA tile and its
  // columns 8 q + 4 (l / 32) + e in acc[i][j][4 q + e]
  auto cphase = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[kk][j], fa[kk][i], acc[i][j], 0, 0, 0);
  };
  const int h = l >> 5;
  const uint32_t thr = __builtin_amdgcn_readfirstlane(0x80008000u);
  auto epilogue = [&](int it) __attribute__((always_inline)) {
    int m0, n0;
    tile_of(it, m0, n0);
    const bool isq = n0 < g.N;
    uint8_t* codes = static_cast<uint8_t*>(isq ? g.qc : g.kc);
    // the byte of 8 columns gi = (this lane's first) + 4 j + y is byte gi % db of head gi / db
    // ((gi + 0.5) / db in fp32 is exact for gi < 2^13)
    const int gb = (((isq ? n0 : n0 - g.N) + wc) >> 3) + 2 * h;
    int coff[4][2];
    bool last[4][2];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int y = 0; y < 2; ++y) {
        const int gi = gb + 4 * j + y;
        const int head = static_cast<int>((static_cast<float>(gi) + 0.5f) * g.inv_db);
        const int kb = gi - head * g.db;
        coff[j][y] = head * g.hstride + kb;
        last[j][y] = kb == g.db - 1;
      }
    const __amdgpu_buffer_rsrc_t rc =
        __builtin_amdgcn_make_buffer_rsrc(codes, 0, 0x7FFFFFFF, 0x00020000);
    uint32_t roff[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t row = static_cast<uint32_t>(m0 + wr + i * 32 + fr);
      const uint32_t b = row / static_cast<uint32_t>(g.T);
      roff[i] = b * static_cast<uint32_t>(g.bstride) + (row - b * g.T) * g.code_bytes;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // column 8 q + 4 h + e of the row (acc[i][j][4 q + e]) lands in bit 8 q + 4 h + e
        uint32_t w = 0;
#pragma unroll
        for (int q = 3; q >= 0; --q) {
#pragma unroll
          for (int e = 3; e >= 0; --e) w = push_sign(w, acc[i][j][4 * q + e], thr);
          if (q) w <<= 4;
        }
        w <<= 4 * h;
        const uint32_t m = w | static_cast<uint32_t>(__shfl_xor(static_cast<int>(w), 32));
#pragma unroll
        for (int y = 0; y < 2; ++y) {
          const uint32_t o = roff[i] + coff[j][y];
          __builtin_amdgcn_raw_buffer_store_b8(static_cast<uint8_t>(m >> (8 * (2 * h + y))), rc, o, 0, 0);
          if (last[j][y])
            for (int z = 1; z < g.code_bytes - g.db + 1; ++z)
              __builtin_amdgcn_raw_buffer_store_b8(static_cast<uint8_t>(0), rc, o + z, 0, 0);
        }
      }
  };

  // Group 0 runs M(0) C(0) M(1) C(1) ..., group 1 the same one phase later. Stage s + 1 goes
  // into the buffer stage s - 1 held, after both groups read it (the barrier before M(s));
  // group 0 waits for those loads at the end of C(s), before group 0's M(s + 1).
  if (grp == 0) {
    dma_stage(0);
    QK_WAIT_VM0();
  }
  QK_BARRIER();                 // stage 0 landed
  if (grp == 1) QK_BARRIER();   // one phase behind group 0
  zero_acc();
  for (int s = 0; s < total; ++s) {
    mphase(s);
    QK_BARRIER();
    cphase();
    if (grp == 0) QK_WAIT_VM0();
    QK_BARRIER();
    if (s % nk == nk - 1) {
      epilogue(s / nk);
      zero_acc();
    }
  }
  if (grp == 0) QK_BARRIER();   // the same barrier count in both groups
  QK_WAIT_VM0();                // no load still writing this workgroup's LDS at its end
}

int num_cus() {
  static int n = 0;
  if (n == 0) {
    int dev = 0;
    (void)hipGetDevice(&dev);
    (void)hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
  }
  return n;
}

}  // namespace
}  // namespace lema

using namespace lema;

extern "C" int lema_qk_pack_bf16(const void* x, int64_t ldx, const void* wq, const void* wk,
                                 int64_t ldw, int64_t M, int64_t N, int64_t K, int32_t d,
                                 int64_t T, void* qcodes, void* kcodes, int32_t code_bytes,
                                 void* stream) {
  clear_error();
  LEMA_REQUIRE(M > 0 && M % (8 * kQkBM) == 0 && M < (int64_t(1) << 31),
               "rows %lld must be a positive multiple of %d", (long long)M, 8 * kQkBM);
  LEMA_REQUIRE(N > 0 && N % kQkBN == 0 && N <= 65536,
               "columns per projection %lld must be a positive multiple of %d, at most 65536",
               (long long)N, kQkBN);
  LEMA_REQUIRE(K >= kQkBK && K % kQkBK == 0 && K < (int64_t(1) << 20),
               "K=%lld must be a multiple of %d", (long long)K, kQkBK);
  LEMA_REQUIRE(d > 0 && d <= 64 && d % 8 == 0 && N % d == 0,
               "code width %d must be a multiple of 8 up to 64 dividing N", d);
  LEMA_REQUIRE(code_bytes == (d <= 32 ? 4 : 8), "codes of %d bits take %d-byte words", d,
               d <= 32 ? 4 : 8);
  LEMA_REQUIRE(T > 0 && M % T == 0, "rows %lld must be whole streams of %lld", (long long)M,
               (long long)T);
  LEMA_REQUIRE(M * (N / d) * code_bytes < (int64_t(1) << 31), "codes of %lld bytes: at most 2 GiB",
               (long long)(M * (N / d) * code_bytes));
  LEMA_REQUIRE(ldx >= K && ldw >= K && ldx % 8 == 0 && ldw % 8 == 0 && ldx < (1 << 20) &&
                   ldw < (1 << 20),
               "row strides must be >= K and multiples of 8");
  LEMA_REQUIRE(x && wq && wk && qcodes && kcodes && aligned(x, 16) && aligned(wq, 16) &&
                   aligned(wk, 16) && aligned(qcodes, 4) && aligned(kcodes, 4),
               "operands must be aligned device pointers");
  QkArgs g{};
  g.x = static_cast<const uint16_t*>(x);
  g.wq = static_cast<const uint16_t*>(wq);
  g.wk = static_cast<const uint16_t*>(wk);
  g.qc = qcodes;
  g.kc = kcodes;
  g.M = static_cast<int32_t>(M);
  g.N = static_cast<int32_t>(N);
  g.K = static_cast<int32_t>(K);
  g.ldx = static_cast<int32_t>(ldx);
  g.ldw = static_cast<int32_t>(ldw);
  g.d = d;
  g.T = static_cast<int32_t>(T);
  g.H = static_cast<int32_t>(N / d);
  g.code_bytes = code_bytes;
  g.tiles_m = static_cast<int32_t>(M / kQkBM);
  g.tiles_n = static_cast<int32_t>(2 * N / kQkBN);
  const int per_x = g.tiles_m / 8;
  g.gm = per_x % 4 == 0 ? 4 : per_x % 2 == 0 ? 2 : 1;
  g.db = d / 8;
  g.inv_db = 1.0f / static_cast<float>(g.db);
  g.hstride = static_cast<int32_t>(T * code_bytes);
  g.bstride = static_cast<int64_t>(N / d) * T * code_bytes;
  const int cus = num_cus();
  LEMA_REQUIRE(cus >= 8 && cus % 8 == 0, "%d compute units: the tile order needs whole XCDs", cus);
  hipStream_t st = static_cast<hipStream_t>(stream);
  LEMA_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(qk_pack_kernel),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, 2 * kQkStage));
  const int tiles = g.tiles_m * g.tiles_n;
  const int grid = tiles < cus ? (tiles + 7) / 8 * 8 : cus;
  qk_pack_kernel<<<dim3(grid), dim3(kQkThreads), 2 * kQkStage, st>>>(g);
  return launch_status("qk_pack_kernel");
}
