// Fused elementwise and normalisation kernels of the LEMA language model's forward in bf16
// (code/lema/model.py:85-94, 212-255, code/lema/train.py:131-152). The reference compiles
// these segments with torch.compile; here each is one hand-written pass over HBM:
//   swiglu      out = silu(gate) * up, with the intermediate rounded to bf16 as the two torch
//               ops round it (SwiGLU.forward);
//   rmsnorm     x_out = x + d (optional residual, rounded to bf16), h = x_out * rsqrt(mean(
//               x_out^2) + eps) * w (Block's pre-norms, the final norm);
//   xent        per row, logsumexp(logits) - logits[target] from bf16 logits in fp32, one read
//               of the row (online max and rescaled sum), instead of a fp32 copy plus a
//               softmax pass;
//   argmax      a decode step's greedy pick, written straight into the token buffer;
//   embedding   the token embedding rows of a decode step, one workgroup per row.
#include "lema_internal.h"
#include "norm_row.h"

namespace lema {
namespace {

__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// Round to nearest even, NaN to the canonical quiet NaN (as torch's bfloat16 conversion).
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  const uint32_t b = __float_as_uint(f);
  if ((b & 0x7F800000u) == 0x7F800000u && (b & 0x007FFFFFu) != 0) return 0x7FC0u;
  return (b + 0x7FFFu + ((b >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ uint32_t swiglu_pair(uint32_t g2, uint32_t u2) {
  uint32_t out = 0;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const float g = bf16_to_f32((g2 >> (16 * k)) & 0xFFFFu);
    const float u = bf16_to_f32((u2 >> (16 * k)) & 0xFFFFu);
    const float s = bf16_to_f32(f32_to_bf16(g / (1.0f + expf(-g))));
    out |= f32_to_bf16(s * u) << (16 * k);
  }
  return out;
}

// Two 16-byte pieces of gate and of up per thread and trip, all four loads in flight before
// the first product (one piece per trip: 447-522 us on [65536, 6144] over two GPUs; two:
// 428-461 us, the same bits).
__global__ __launch_bounds__(256) void swiglu_kernel(const u32x4* gate, const u32x4* up,
                                                     u32x4* out, int64_t n8) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i0 = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i0 < n8;
       i0 += 2 * stride) {
    const int64_t i1 = i0 + stride;
    const bool two = i1 < n8;
    const u32x4 g0 = gate[i0], u0 = up[i0];
    u32x4 g1 = g0, u1 = u0;
    if (two) {
      g1 = gate[i1];
      u1 = up[i1];
    }
    out[i0] = u32x4{swiglu_pair(g0.x, u0.x), swiglu_pair(g0.y, u0.y), swiglu_pair(g0.z, u0.z),
                    swiglu_pair(g0.w, u0.w)};
    if (two)
      out[i1] = u32x4{swiglu_pair(g1.x, u1.x), swiglu_pair(g1.y, u1.y), swiglu_pair(g1.z, u1.z),
                      swiglu_pair(g1.w, u1.w)};
  }
}

// One wavefront per row of D bf16 (D % 8 == 0, D <= 512 * S).
template <int S>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint16_t* x, const uint16_t* d,
                                                      const uint16_t* w, float eps, int64_t rows,
                                                      int D, uint16_t* x_out, uint16_t* h_out) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (blockDim.x / 64) + (threadIdx.x >> 6);
  if (row >= rows) return;
  uint16_t* h = h_out + row * D;
  const uint16_t* const xr[1] = {x + row * D};
  const uint16_t* const dr[1] = {d != nullptr ? d + row * D : nullptr};
  uint16_t* const sr[1] = {d != nullptr ? x_out + row * D : nullptr};
  norm_rows<1, S>(xr, dr, 1, w, eps, D, lane, sr,
               [h](int, int e, u32x4 v) { *reinterpret_cast<u32x4*>(h + e) = v; });
}

// One workgroup (256 threads) per row of V bf16 logits (V % 8 == 0, rows 16-byte aligned):
// each thread keeps a running max and a sum rescaled to it, then the workgroup combines them.
// Each trip loads two 16-byte pieces (both in flight), and e^(x - m) is 2^(x log2 e - m log2 e):
// one FMA and the hardware base-2 exponential per logit. With expf per logit and one load per
// trip the kernel was bound by VALU issue: 4096 x 50304 logits took 114-133 us, now 75 us
// (5.4 TB/s), at the same error against an fp32 cross-entropy (about 2e-7 per row).
__global__ __launch_bounds__(256) void xent_kernel(const uint16_t* logits, int64_t V, int64_t ld,
                                                   const int64_t* target, float* loss) {
  __shared__ float smax[4], ssum[4];
  constexpr float kLog2e = 1.4426950408889634f;
  const int64_t row = blockIdx.x;
  const uint16_t* r = logits + row * ld;
  float m = -INFINITY, s = 0.0f;
  for (int64_t e0 = static_cast<int64_t>(threadIdx.x) * 8; e0 < V; e0 += 2 * 256 * 8) {
    const int64_t e1 = e0 + 256 * 8;
    const bool two = e1 < V;
    const u32x4 va = *reinterpret_cast<const u32x4*>(r + e0);
    u32x4 vb = va;  // a repeat of the first piece when the second lies past the row
    if (two) vb = *reinterpret_cast<const u32x4*>(r + e1);
    const uint32_t pv[8] = {va.x, va.y, va.z, va.w, vb.x, vb.y, vb.z, vb.w};
    float x[16];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      x[2 * k] = bf16_to_f32(pv[k] & 0xFFFFu);
      x[2 * k + 1] = bf16_to_f32(pv[k] >> 16);
    }
    float bm = x[0];
#pragma unroll
    for (int k = 1; k < 16; ++k) bm = fmaxf(bm, x[k]);
    if (bm > m) {
      s *= __builtin_amdgcn_exp2f((m - bm) * kLog2e);
      m = bm;
    }
    const float mb = m * kLog2e;
    float sa = 0.0f, sb = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) sa += __builtin_amdgcn_exp2f(fmaf(x[k], kLog2e, -mb));
#pragma unroll
    for (int k = 8; k < 16; ++k) sb += __builtin_amdgcn_exp2f(fmaf(x[k], kLog2e, -mb));
    // while every logit so far is -inf, m is -inf and each term is exp2(-inf + inf) = NaN:
    // such a trip adds nothing (e^-inf = 0), as in the combine below
    if (m != -INFINITY) s += two ? sa + sb : sa;
  }
  // combine: wavefront, then the 4 wavefronts
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float om = __shfl_xor(m, o), os = __shfl_xor(s, o);
    const float nm = fmaxf(m, om);
    s = (m == -INFINITY ? 0.0f : s * expf(m - nm)) + (om == -INFINITY ? 0.0f : os * expf(om - nm));
    m = nm;
  }
  const int wv = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    smax[wv] = m;
    ssum[wv] = s;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float M = smax[0];
    for (int k = 1; k < 4; ++k) M = fmaxf(M, smax[k]);
    float S = 0.0f;
    for (int k = 0; k < 4; ++k) S += smax[k] == -INFINITY ? 0.0f : ssum[k] * expf(smax[k] - M);
    const int64_t t = target[row];
    const float xt = (t >= 0 && t < V) ? bf16_to_f32(r[t]) : NAN;
    loss[row] = logf(S) + M - xt;
  }
}

}  // namespace
}  // namespace lema

using namespace lema;

extern "C" int lema_swiglu_bf16(const void* gate, const void* up, void* out, int64_t n,
                                void* stream) {
  clear_error();
  LEMA_REQUIRE(n >= 0 && n % 8 == 0, "element count %lld must be a multiple of 8", (long long)n);
  if (n == 0) return LEMA_OK;
  LEMA_REQUIRE(gate && up && out && aligned(gate, 16) && aligned(up, 16) && aligned(out, 16),
               "gate, up and out must be 16-byte aligned device pointers");
  const int64_t n8 = n / 8;
  int64_t grid = (n8 + 255) / 256;
  if (grid > 65536) grid = 65536;
  swiglu_kernel<<<dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const u32x4*>(gate), static_cast<const u32x4*>(up), static_cast<u32x4*>(out), n8);
  return launch_status("swiglu_kernel");
}

extern "C" int lema_rmsnorm_bf16(const void* x, const void* d, const void* w, float eps,
                                 int64_t rows, int64_t D, void* x_out, void* h_out, void* stream) {
  clear_error();
  LEMA_REQUIRE(rows >= 0 && D > 0 && D % 8 == 0 && D <= 64 * 8 * kNormMaxSteps,
               "row length %lld must be a multiple of 8 and at most %d", (long long)D,
               64 * 8 * kNormMaxSteps);
  if (rows == 0) return LEMA_OK;
  LEMA_REQUIRE(x && w && h_out && (d == nullptr || x_out != nullptr), "null pointer");
  LEMA_REQUIRE(aligned(x, 16) && aligned(w, 16) && aligned(h_out, 16) &&
                   (d == nullptr || (aligned(d, 16) && aligned(x_out, 16))),
               "pointers must be 16-byte aligned");
  const int64_t grid = (rows + 3) / 4;
  LEMA_REQUIRE(grid < (int64_t(1) << 31), "too many rows");
  // rows of up to 2048 (the models' widths) hold 4 steps in registers, longer ones 8
  auto kernel = D <= 2048 ? rmsnorm_kernel<4> : rmsnorm_kernel<kNormMaxSteps>;
  kernel<<<dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(d),
      static_cast<const uint16_t*>(w), eps, rows, static_cast<int>(D),
      static_cast<uint16_t*>(x_out), static_cast<uint16_t*>(h_out));
  return launch_status("rmsnorm_kernel");
}

// Is (a, ia) ahead of (b, ib) for torch.argmax: NaN above every number, then the larger value,
// then the lower index.
__device__ __forceinline__ bool argmax_ahead(float a, int64_t ia, float b, int64_t ib) {
  const bool an = a != a, bn = b != b;
  if (an || bn) return an && (!bn || ia < ib);
  return a > b || (a == b && ia < ib);
}

// One workgroup (1024 threads) per row of V bf16 values (V % 8 == 0, rows 16-byte aligned):
// out[row * out_stride] = the row's argmax (code/lema/decode.py:71-93, the greedy pick).
__global__ __launch_bounds__(1024) void argmax_kernel(const uint16_t* x, int64_t V, int64_t ld,
                                                      int64_t* out, int64_t out_stride) {
  __shared__ float sv[16];
  __shared__ int64_t si[16];
  const int64_t row = blockIdx.x;
  const uint16_t* r = x + row * ld;
  float bv = 0.0f;
  int64_t bi = -1;  // none yet
  for (int64_t e = static_cast<int64_t>(threadIdx.x) * 8; e < V; e += 1024 * 8) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(r + e);
    const uint32_t* pv = reinterpret_cast<const uint32_t*>(&v);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float f = bf16_to_f32((pv[k >> 1] >> (16 * (k & 1))) & 0xFFFFu);
      if (bi < 0 || argmax_ahead(f, e + k, bv, bi)) {
        bv = f;
        bi = e + k;
      }
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const int64_t oi = __shfl_xor(bi, o);
    if (oi >= 0 && (bi < 0 || argmax_ahead(ov, oi, bv, bi))) {
      bv = ov;
      bi = oi;
    }
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sv[wave] = bv;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 16; ++w)
      if (si[w] >= 0 && (bi < 0 || argmax_ahead(sv[w], si[w], bv, bi))) {
        bv = sv[w];
        bi = si[w];
      }
    out[row * out_stride] = bi;
  }
}

// One workgroup per id: out row i = table row ids[i] (D bf16, D % 8 == 0, 16-byte aligned
// rows), or zeros for an id outside [0, vocab).
__global__ __launch_bounds__(256) void embedding_kernel(const uint16_t* table, int64_t vocab,
                                                        int64_t D, const int64_t* ids,
                                                        uint16_t* out) {
  const int64_t i = blockIdx.x;
  const int64_t id = ids[i];
  const bool ok = id >= 0 && id < vocab;
  const u32x4* src = reinterpret_cast<const u32x4*>(table + (ok ? id : 0) * D);
  u32x4* dst = reinterpret_cast<u32x4*>(out + i * D);
  for (int64_t k = threadIdx.x; k < D / 8; k += blockDim.x)
    dst[k] = ok ? src[k] : u32x4{0u, 0u, 0u, 0u};
}

extern "C" int lema_cross_entropy_bf16(const void* logits, int64_t rows, int64_t V, int64_t ld,
                                       const int64_t* target, float* loss, void* stream) {
  clear_error();
  LEMA_REQUIRE(rows >= 0 && V > 0 && V % 8 == 0 && ld >= V && ld % 8 == 0,
               "vocabulary %lld and row stride %lld must be multiples of 8", (long long)V,
               (long long)ld);
  if (rows == 0) return LEMA_OK;
  LEMA_REQUIRE(logits && target && loss && aligned(logits, 16) && aligned(target, 8) &&
                   aligned(loss, 4), "bad pointer");
  LEMA_REQUIRE(rows < (int64_t(1) << 31), "too many rows");
  xent_kernel<<<dim3(rows), dim3(256), 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(logits), V, ld, target, loss);
  return launch_status("xent_kernel");
}

extern "C" int lema_argmax_bf16(const void* x, int64_t rows, int64_t V, int64_t ld, int64_t* out,
                                int64_t out_stride, void* stream) {
  clear_error();
  LEMA_REQUIRE(rows >= 0 && V > 0 && V % 8 == 0 && ld >= V && ld % 8 == 0,
               "row length %lld and stride %lld must be multiples of 8", (long long)V,
               (long long)ld);
  if (rows == 0) return LEMA_OK;
  LEMA_REQUIRE(x && out && aligned(x, 16) && aligned(out, 8) && out_stride >= 1, "bad pointer");
  LEMA_REQUIRE(rows < (int64_t(1) << 31), "too many rows");
  argmax_kernel<<<dim3(rows), dim3(1024), 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(x), V, ld, out, out_stride);
  return launch_status("argmax_kernel");
}

extern "C" int lema_embedding_bf16(const void* table, int64_t vocab, int64_t D, const int64_t* ids,
                                   int64_t n, void* out, void* stream) {
  clear_error();
  LEMA_REQUIRE(vocab >= 1 && D > 0 && D % 8 == 0, "rows of %lld must be a multiple of 8",
               (long long)D);
  if (n == 0) return LEMA_OK;
  LEMA_REQUIRE(n > 0 && n < (int64_t(1) << 31), "bad id count %lld", (long long)n);
  LEMA_REQUIRE(table && ids && out && aligned(table, 16) && aligned(ids, 8) && aligned(out, 16),
               "bad pointer");
  embedding_kernel<<<dim3(n), dim3(256), 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(table), vocab, D, ids, static_cast<uint16_t*>(out));
  return launch_status("embedding_kernel");
}
