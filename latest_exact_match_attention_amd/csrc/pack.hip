// Sign-packing of projected queries/keys into integer codes (code/lema/attention.py:82-97).
//
// Bit j of the code of a row is (z_j >= 0) as a float compare: -0.0 -> 1, NaN -> 0, LSB = dim 0.
//
// Dense path (the rows form one packed array in some order of (b, h, t), as for both a
// contiguous [B, H, T, D] tensor and the transposed [B, T, H, D] projection view, 16-byte
// aligned): a wavefront takes 64 consecutive rows in MEMORY order, i.e. 64*D consecutive
// elements; each lane turns 8 consecutive elements (one 16-byte load) into one byte of the
// rows' concatenated bit string in LDS, and lane l then cuts its row's D bits out of it and
// writes the code to its (b, h, t) slot -- or, when 64 heads are innermost in memory and the
// codes run along positions, a workgroup stages 32 positions x 64 heads and writes runs.
// Generic path (any strides, last dim contiguous): one thread per row.
#include "lema_internal.h"

namespace lema {
namespace {

template <int DTYPE>
__device__ __forceinline__ bool nonneg(const void* z, int64_t e) {
  if constexpr (DTYPE == LEMA_F32) {
    return static_cast<const float*>(z)[e] >= 0.0f;
  } else if constexpr (DTYPE == LEMA_BF16) {
    const uint32_t b = static_cast<uint32_t>(static_cast<const uint16_t*>(z)[e]) << 16;
    return __uint_as_float(b) >= 0.0f;
  } else {  // IEEE half, tested on its bits: NaN -> false, -0 -> true
    const uint32_t h = static_cast<const uint16_t*>(z)[e];
    if ((h & 0x7C00u) == 0x7C00u && (h & 0x03FFu) != 0) return false;
    return (h & 0x8000u) == 0 || (h & 0x7FFFu) == 0;
  }
}

// Memory order of the rows: m = i0 * E1 * E2 + i1 * E2 + i2, output index sum(i_k * os_k).
struct DenseArgs {
  const void* z;
  void* codes;
  int64_t R;            // rows
  int64_t E1, E2;       // extents of the two inner memory-order dims
  int64_t os0, os1, os2;  // output strides (codes) of the memory-order dims
  int32_t D;
};

constexpr int kPackThreads = 256;

// One lane's 8 consecutive elements: 16 bytes (32 for fp32), loaded before any is tested.
template <int DTYPE>
struct Raw8 {
  u32x4 v[DTYPE == LEMA_F32 ? 2 : 1];
};

template <int DTYPE>
__device__ __forceinline__ Raw8<DTYPE> load8(const void* z, int64_t e) {
  Raw8<DTYPE> r;
  if constexpr (DTYPE == LEMA_F32) {
    r.v[0] = *reinterpret_cast<const u32x4*>(static_cast<const float*>(z) + e);
    r.v[1] = *reinterpret_cast<const u32x4*>(static_cast<const float*>(z) + e + 4);
  } else {
    r.v[0] = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(z) + e);
  }
  return r;
}

// Sign bits of the 8 elements, bit k = element k.
template <int DTYPE>
__device__ __forceinline__ uint32_t sign_byte(const Raw8<DTYPE>& r) {
  uint32_t m = 0;
  if constexpr (DTYPE == LEMA_F32) {
    const uint32_t w[8] = {r.v[0].x, r.v[0].y, r.v[0].z, r.v[0].w,
                           r.v[1].x, r.v[1].y, r.v[1].z, r.v[1].w};
#pragma unroll
    for (int k = 0; k < 8; ++k) m |= (__uint_as_float(w[k]) >= 0.0f ? 1u : 0u) << k;
  } else {
    const uint32_t w[4] = {r.v[0].x, r.v[0].y, r.v[0].z, r.v[0].w};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t h = (w[k >> 1] >> (16 * (k & 1))) & 0xFFFFu;
      bool b;
      if constexpr (DTYPE == LEMA_BF16) {
        b = __uint_as_float(h << 16) >= 0.0f;
      } else {  // IEEE half on its bits: NaN -> false, -0 -> true
        b = !((h & 0x7C00u) == 0x7C00u && (h & 0x03FFu) != 0) &&
            ((h & 0x8000u) == 0 || (h & 0x7FFFu) == 0);
      }
      m |= (b ? 1u : 0u) << k;
    }
  }
  return m;
}

// Dense path: a wavefront owns 64 consecutive rows in memory order, i.e. 64*D consecutive
// elements. Each lane reads 16 (32 for fp32) bytes per step -- 8 elements, their 8 sign bits
// one byte of the rows' concatenated bit string, staged in LDS -- so the wavefront covers
// the string in ceil(D / 8) coalesced steps; lane l then cuts row l's D bits out of it.
template <int DTYPE>
__device__ __forceinline__ uint64_t row_code(const DenseArgs& a, uint64_t* words, int64_t m0,
                                             int lane) {
  const int64_t e0 = m0 * a.D, eend = a.R * a.D;
  uint8_t* bytes = reinterpret_cast<uint8_t*>(words);
  const int steps = (a.D + 7) / 8;  // 8 * D bytes of bit string, 64 bytes per step
  const bool whole = e0 + 64 * static_cast<int64_t>(a.D) <= eend;  // no array end inside
  if (whole) {
    Raw8<DTYPE> raw[8];  // every load of the lane in flight before the first test
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int b = it * 64 + lane;
      if (it < steps && b < 8 * a.D) raw[it] = load8<DTYPE>(a.z, e0 + static_cast<int64_t>(b) * 8);
    }
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int b = it * 64 + lane;
      if (it < steps && b < 8 * a.D) bytes[b] = static_cast<uint8_t>(sign_byte<DTYPE>(raw[it]));
    }
  } else {  // the array's last rows: element by element
    for (int it = 0; it < steps; ++it) {
      const int b = it * 64 + lane;
      if (b >= 8 * a.D) continue;
      const int64_t e = e0 + static_cast<int64_t>(b) * 8;
      uint32_t m = 0;
      for (int k = 0; k < 8; ++k)
        if (e + k < eend && nonneg<DTYPE>(a.z, e + k)) m |= 1u << k;
      bytes[b] = static_cast<uint8_t>(m);
    }
  }
  if (lane == 0) words[a.D] = 0;
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const int bitpos = lane * a.D;
  const int wi = bitpos >> 6, off = bitpos & 63;
  uint64_t code = words[wi] >> off;
  if (off != 0 && off + a.D > 64) code |= words[wi + 1] << (64 - off);
  if (a.D < 64) code &= (uint64_t(1) << a.D) - 1;
  __builtin_amdgcn_wave_barrier();  // the bit string is read before the next row group's
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  return code;
}

__device__ __forceinline__ int64_t out_index(const DenseArgs& a, int64_t m) {
  const int64_t i2 = m % a.E2;
  const int64_t r = m / a.E2;
  const int64_t i1 = r % a.E1, i0 = r / a.E1;
  return i0 * a.os0 + i1 * a.os1 + i2 * a.os2;
}

template <int DTYPE, typename CodeT>
__global__ __launch_bounds__(kPackThreads) void pack_dense_kernel(DenseArgs a) {
  __shared__ uint64_t words[kPackThreads / 64][64 + 1];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t m0 = (static_cast<int64_t>(blockIdx.x) * (kPackThreads / 64) + w) * 64;
  if (m0 >= a.R) return;
  const uint64_t code = row_code<DTYPE>(a, words[w], m0, lane);
  const int64_t m = m0 + lane;
  if (m >= a.R) return;
  static_cast<CodeT*>(a.codes)[out_index(a, m)] = static_cast<CodeT>(code);
}

// Rows of 64 heads innermost in memory (the [B, T, H * D] projection viewed as [B, H, T, D])
// whose codes go to [B, H, T]: a wavefront's 64 codes would land T apart. A workgroup packs
// G consecutive row groups (positions) instead, G / 4 per wavefront, stages the [G][64] codes
// in LDS and writes each head's G positions as one contiguous run. G = 16 on inputs of 2^21
// rows or more, 8 below, so that smaller inputs still spread over the whole GPU (one LM layer,
// B4 H64 T16384 d 24: 36-37 us with 8 or 16, 37.9 with 32; B1 H64 T1000: 4.3 us with 8,
// 6.0 with 16, 10.0 with 32; a read of the same bytes alone takes 33.3 and 4.4 us).
template <int DTYPE, typename CodeT, int G>
__global__ __launch_bounds__(kPackThreads) void pack_tile_kernel(DenseArgs a) {
  __shared__ uint64_t words[kPackThreads / 64][64 + 1];
  __shared__ CodeT tile[G][64 + 1];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * G * 64;
  for (int g = w; g < G; g += kPackThreads / 64) {
    const int64_t m0 = base + static_cast<int64_t>(g) * 64;
    if (m0 < a.R) tile[g][lane] = static_cast<CodeT>(row_code<DTYPE>(a, words[w], m0, lane));
  }
  __syncthreads();
  for (int idx = t; idx < G * 64; idx += kPackThreads) {
    const int h = idx / G, g = idx % G;  // consecutive threads: positions
    const int64_t m = base + static_cast<int64_t>(g) * 64 + h;
    if (m < a.R) static_cast<CodeT*>(a.codes)[out_index(a, m)] = tile[g][h];
  }
}

struct StridedArgs {
  const void* z;
  void* codes;
  int64_t B, H, T;
  int64_t sb, sh, st;
  int32_t D;
};

template <int DTYPE, typename CodeT>
__global__ __launch_bounds__(kPackThreads) void pack_strided_kernel(StridedArgs a) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * kPackThreads + threadIdx.x;
  if (r >= a.B * a.H * a.T) return;
  const int64_t t = r % a.T;
  const int64_t bh = r / a.T;
  const int64_t h = bh % a.H, b = bh / a.H;
  const int64_t base = b * a.sb + h * a.sh + t * a.st;
  uint64_t code = 0;
  for (int j = 0; j < a.D; ++j)
    if (nonneg<DTYPE>(a.z, base + j)) code |= uint64_t(1) << j;
  static_cast<CodeT*>(a.codes)[r] = static_cast<CodeT>(code);
}

template <typename CodeT, int G>
int launch_tile(int32_t dtype, const DenseArgs& a, hipStream_t st) {
  const int64_t grid = (a.R + G * 64 - 1) / (G * 64);
  LEMA_REQUIRE(grid < (int64_t(1) << 31), "too many rows to pack");
  switch (dtype) {
    case LEMA_F32: pack_tile_kernel<LEMA_F32, CodeT, G><<<dim3(grid), dim3(kPackThreads), 0, st>>>(a); break;
    case LEMA_F16: pack_tile_kernel<LEMA_F16, CodeT, G><<<dim3(grid), dim3(kPackThreads), 0, st>>>(a); break;
    default: pack_tile_kernel<LEMA_BF16, CodeT, G><<<dim3(grid), dim3(kPackThreads), 0, st>>>(a); break;
  }
  return launch_status("pack_tile_kernel");
}

template <typename CodeT>
int launch_dense(int32_t dtype, const DenseArgs& a, hipStream_t st) {
  if (a.E2 == 64 && a.os1 == 1 && a.os2 != 1)  // 64 heads innermost, positions contiguous out
    return a.R >= (int64_t(1) << 21) ? launch_tile<CodeT, 16>(dtype, a, st)
                                     : launch_tile<CodeT, 8>(dtype, a, st);
  const int64_t grid = (a.R + kPackThreads - 1) / kPackThreads;
  LEMA_REQUIRE(grid < (int64_t(1) << 31), "too many rows to pack");
  switch (dtype) {
    case LEMA_F32: pack_dense_kernel<LEMA_F32, CodeT><<<dim3(grid), dim3(kPackThreads), 0, st>>>(a); break;
    case LEMA_F16: pack_dense_kernel<LEMA_F16, CodeT><<<dim3(grid), dim3(kPackThreads), 0, st>>>(a); break;
    default: pack_dense_kernel<LEMA_BF16, CodeT><<<dim3(grid), dim3(kPackThreads), 0, st>>>(a); break;
  }
  return launch_status("pack_dense_kernel");
}

template <typename CodeT>
int launch_strided(int32_t dtype, const StridedArgs& a, hipStream_t st) {
  const int64_t grid = (a.B * a.H * a.T + kPackThreads - 1) / kPackThreads;
  LEMA_REQUIRE(grid < (int64_t(1) << 31), "too many rows to pack");
  switch (dtype) {
    case LEMA_F32: pack_strided_kernel<LEMA_F32, CodeT><<<dim3(grid), dim3(kPackThreads), 0, st>>>(a); break;
    case LEMA_F16: pack_strided_kernel<LEMA_F16, CodeT><<<dim3(grid), dim3(kPackThreads), 0, st>>>(a); break;
    default: pack_strided_kernel<LEMA_BF16, CodeT><<<dim3(grid), dim3(kPackThreads), 0, st>>>(a); break;
  }
  return launch_status("pack_strided_kernel");
}

}  // namespace
}  // namespace lema

using namespace lema;

extern "C" int lema_pack_codes(const void* z, int32_t dtype, int64_t B, int64_t H, int64_t T,
                               int32_t D, int64_t z_sb, int64_t z_sh, int64_t z_st, void* codes,
                               int32_t code_bytes, void* stream) {
  clear_error();
  const int es = dtype_size(dtype);
  LEMA_REQUIRE(es > 0, "unknown value dtype %d", dtype);
  LEMA_REQUIRE(D >= 1 && D <= 64, "d_qk %d > 64 cannot pack into a uint64", D);
  LEMA_REQUIRE(code_bytes == 8 || (code_bytes == 4 && D <= 32),
               "code_bytes %d cannot hold %d-bit codes", code_bytes, D);
  LEMA_REQUIRE(B >= 0 && H >= 0 && T >= 0, "negative shape");
  const int64_t R = B * H * T;
  if (R == 0) return LEMA_OK;
  LEMA_REQUIRE(z != nullptr && codes != nullptr, "null pointer");
  LEMA_REQUIRE(aligned(z, es) && aligned(codes, code_bytes), "misaligned pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);

  // Are the rows one packed array? Drop unit dims, order the rest by stride (outermost
  // first) and check that each stride is the product of the inner extents times D.
  struct Dim { int64_t e, s, os; };
  Dim dims[3] = {{B, z_sb, H * T}, {H, z_sh, T}, {T, z_st, 1}};
  Dim kept[3];
  int nk = 0;
  for (const Dim& d : dims)
    if (d.e > 1) kept[nk++] = d;
  for (int i = 0; i < nk; ++i)
    for (int j = i + 1; j < nk; ++j)
      if (kept[j].s > kept[i].s) { Dim x = kept[i]; kept[i] = kept[j]; kept[j] = x; }
  bool dense = true;
  int64_t need = D;
  for (int i = nk - 1; i >= 0; --i) {
    dense = dense && kept[i].s == need;
    need *= kept[i].e;
  }
  if (dense && aligned(z, 16)) {
    Dim full[3] = {{1, 0, 0}, {1, 0, 0}, {1, 0, 0}};
    for (int i = 0; i < nk; ++i) full[3 - nk + i] = kept[i];
    DenseArgs a{z, codes, R, full[1].e, full[2].e, full[0].os, full[1].os, full[2].os, D};
    return code_bytes == 4 ? launch_dense<uint32_t>(dtype, a, st) : launch_dense<uint64_t>(dtype, a, st);
  }
  StridedArgs a{z, codes, B, H, T, z_sb, z_sh, z_st, D};
  return code_bytes == 4 ? launch_strided<uint32_t>(dtype, a, st) : launch_strided<uint64_t>(dtype, a, st);
}
