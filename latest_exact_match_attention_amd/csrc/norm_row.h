// One row of the LEMA model's RMS norm in bf16 (nn.RMSNorm over bf16 tensors,
// code/lema/model.py:212-255), shared by the stand-alone norm kernel and the skinny products
// that normalise their own input, so both round every element identically:
//   s = x (+ d), each sum rounded to bf16;
//   h = bf16(s * rsqrt(mean(s^2) + eps) * w), the mean's sum in fp32, one rounding at the end:
//   torch's nn.RMSNorm on bf16 tensors rounds the same way (on this GPU and on the CPU), so
//   only the order of the mean's sum can differ.
// One wavefront per row of D elements (D % 8 == 0, D <= kNormMaxD); lane `lane` takes the
// 8 elements at (k * 64 + lane) * 8 for each step k, and the sum of squares is added up in that
// order and then across the wavefront.
#pragma once
#include "lema_internal.h"

namespace lema {

constexpr int kNormMaxSteps = 8;
constexpr int kNormMaxD = 64 * 8 * kNormMaxSteps;  // 4096

__device__ __forceinline__ float nr_bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }
// Round to nearest even, NaN to the canonical quiet NaN (as torch's bfloat16 conversion).
__device__ __forceinline__ uint32_t nr_f32_to_bf16(float f) {
  const uint32_t b = __float_as_uint(f);
  if ((b & 0x7F800000u) == 0x7F800000u && (b & 0x007FFFFFu) != 0) return 0x7FC0u;
  return (b + 0x7FFFu + ((b >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ float nr_wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Up to R rows (`n` of them, n <= R) at once by one wavefront, each exactly as alone: rows r
// start at x[r] (and d[r], null: no addend); s goes to s_out[r] when d[r] and s_out[r] are
// given, and h's 8 elements at each offset e to put_h(r, e, h8). Every global read (the rows'
// x and d and the weight) is issued before the first reduction, so the rows cost one round
// trip. S (at most kNormMaxSteps) bounds the steps, D <= 512 * S: it sizes the registers that
// hold the rows.
template <int R, int S, typename PutH>
__device__ __forceinline__ void norm_rows(const uint16_t* const (&x)[R], const uint16_t* const (&d)[R],
                                          int n, const uint16_t* w, float eps, int D, int lane,
                                          uint16_t* const (&s_out)[R], PutH put_h) {
  const int steps = D / 512 + (D % 512 ? 1 : 0);
  static_assert(S >= 1 && S <= kNormMaxSteps, "steps of 512 elements");
  u32x4 xv[R][S], dv[R][S], wv[S];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const int e = (s * 64 + lane) * 8;
    if (s >= steps || e >= D) continue;
    wv[s] = *reinterpret_cast<const u32x4*>(w + e);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (r >= n) continue;
      xv[r][s] = *reinterpret_cast<const u32x4*>(x[r] + e);
      if (d[r] != nullptr) dv[r][s] = *reinterpret_cast<const u32x4*>(d[r] + e);
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (r >= n) continue;
    float ss = 0.0f;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int e = (s * 64 + lane) * 8;
      if (s >= steps || e >= D) continue;
      u32x4 v = xv[r][s];
      if (d[r] != nullptr) {
        uint32_t* pv = reinterpret_cast<uint32_t*>(&v);
        const uint32_t* pd = reinterpret_cast<const uint32_t*>(&dv[r][s]);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t lo =
              nr_f32_to_bf16(nr_bf16_to_f32(pv[k] & 0xFFFFu) + nr_bf16_to_f32(pd[k] & 0xFFFFu));
          const uint32_t hi =
              nr_f32_to_bf16(nr_bf16_to_f32(pv[k] >> 16) + nr_bf16_to_f32(pd[k] >> 16));
          pv[k] = lo | (hi << 16);
        }
        if (s_out[r] != nullptr) *reinterpret_cast<u32x4*>(s_out[r] + e) = v;
      }
      xv[r][s] = v;
      const uint32_t* pv = reinterpret_cast<const uint32_t*>(&v);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float a = nr_bf16_to_f32(pv[k] & 0xFFFFu), b = nr_bf16_to_f32(pv[k] >> 16);
        ss += a * a + b * b;
      }
    }
    const float rstd = rsqrtf(nr_wave_sum(ss) / static_cast<float>(D) + eps);
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int e = (s * 64 + lane) * 8;
      if (s >= steps || e >= D) continue;
      const uint32_t* pv = reinterpret_cast<const uint32_t*>(&xv[r][s]);
      const uint32_t* pw = reinterpret_cast<const uint32_t*>(&wv[s]);
      u32x4 o;
      uint32_t* po = reinterpret_cast<uint32_t*>(&o);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t lo =
            nr_f32_to_bf16(nr_bf16_to_f32(pv[k] & 0xFFFFu) * rstd * nr_bf16_to_f32(pw[k] & 0xFFFFu));
        const uint32_t hi =
            nr_f32_to_bf16(nr_bf16_to_f32(pv[k] >> 16) * rstd * nr_bf16_to_f32(pw[k] >> 16));
        po[k] = lo | (hi << 16);
      }
      put_h(r, e, o);
    }
  }
}

}  // namespace lema
