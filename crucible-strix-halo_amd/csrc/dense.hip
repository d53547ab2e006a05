// Dense fp16-weight linear y[r][o] = W[o] . x[r] (the MoE router: W = [E + 1][H] with the
// shared-expert gate as row E).  Two kernels, as in the reference's router launch
// (engine/engine.hip:1824-1870):
//   * up to 8 rows of fp32 x: one wave per output row, fp32 products and sums
//     (DenseGemvKernel, engine/layers/ops.h:30-61);
//   * more rows, or fp16 x: x rounded to fp16 (the reference packs it first,
//     PrefillPackKernel), v_mfma_f32_16x16x32_f16 tiles of 64 rows x 64 outputs.
#include "internal.hpp"

namespace cx {

// One wave per output o; lane l covers inputs [8 l + 512 c, 8 l + 512 c + 8) for chunks c.
// R rows of x, fp32; the per-lane partial sums are reduced across the wave by DPP.
template <int R>
__global__ void __launch_bounds__(256) DenseGemvKernel(const __half* __restrict__ W, int O, int I,
                                                       const float* __restrict__ x, int ldx, float* __restrict__ y,
                                                       int ldy) {
  const int o = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (o >= O) return;  // whole waves
  const int lane = threadIdx.x & 63;
  const __half* w = W + (size_t)o * I;
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
  for (int k0 = lane * 8; k0 < I; k0 += 512) {
    float wf[8];
    LoadH8(w + k0, wf);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float xv[8];
      LoadF8(x + (size_t)r * ldx + k0, xv);
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) s += wf[i] * xv[i];
      acc[r] += s;
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float v = acc[r];
    v += Dpp<kDppQuadSwap1>(v);
    v += Dpp<kDppQuadSwap2>(v);
    v += Dpp<kDppRowHalfMirror>(v);
    v += Dpp<kDppRowMirror>(v);
    v = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0)) +
        __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16)) +
        __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32)) +
        __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    if (lane == 0) y[(size_t)r * ldy + o] = v;
  }
}

// MFMA tile: a 256-thread workgroup computes rows [64 bx, 64 bx + 64) x outputs
// [64 by, 64 by + 64); wave w owns rows 16 w .. 16 w + 15 and all 64 outputs.  Per
// 32-wide k step a lane loads 8 consecutive k of its x row (A operand) and of 4 W rows
// (B operands: W is [O][I], so B = W^T has consecutive k contiguous).  Rows >= M and
// outputs >= O read zeros (buffer bounds) and are not stored.  XF32: x is fp32 and is
// rounded to fp16 on load.
template <bool XF32>
__global__ void __launch_bounds__(256) DenseMfmaKernel(const __half* __restrict__ W, int O, int I,
                                                       const void* __restrict__ x, int ldx, int M,
                                                       float* __restrict__ y, int ldy) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int m0 = blockIdx.x * 64 + wave * 16, o0 = blockIdx.y * 64;
  const int kq = 8 * (lane >> 4), ln = lane & 15;
  const int esz = XF32 ? 4 : 2;
  const int rows = max(0, min(16, M - m0));
  const __amdgpu_buffer_rsrc_t rx =
      MakeRsrc(static_cast<const char*>(x) + (size_t)m0 * ldx * esz, (uint32_t)((size_t)rows * ldx * esz));
  const int outs = max(0, min(64, O - o0));
  const __amdgpu_buffer_rsrc_t rw = MakeRsrc(W + (size_t)o0 * I, (uint32_t)((size_t)outs * I * 2));
  const uint32_t xoff = (uint32_t)((ln * ldx + kq) * esz);
  float4_t acc[4];
#pragma unroll
  for (int n = 0; n < 4; ++n) acc[n] = float4_t{0.f, 0.f, 0.f, 0.f};
  for (int k = 0; k < I; k += 32) {
    half8_t a;
    if constexpr (XF32) {
      // Whole-vector casts: element-wise bit casts of ext-vector elements are miscompiled
      // by this toolchain (every element reads element 0).
      const float4_t lo = __builtin_bit_cast(float4_t, BufLoad128(rx, xoff, (uint32_t)k * 4));
      const float4_t hi = __builtin_bit_cast(float4_t, BufLoad128(rx, xoff + 16, (uint32_t)k * 4));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        a[i] = (_Float16)lo[i];
        a[4 + i] = (_Float16)hi[i];
      }
    } else {
      a = __builtin_bit_cast(half8_t, BufLoad128(rx, xoff, (uint32_t)k * 2));
    }
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      const half8_t b = __builtin_bit_cast(half8_t, BufLoad128(rw, (uint32_t)(((n * 16 + ln) * I + kq) * 2), (uint32_t)k * 2));
      acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[n], 0, 0, 0);
    }
  }
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    const int o = o0 + n * 16 + ln;
    if (o >= O) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = m0 + 4 * (lane >> 4) + i;
      if (r < M) y[(size_t)r * ldy + o] = acc[n][i];
    }
  }
}

}  // namespace cx

using namespace cx;

extern "C" {

int cx_dense_linear(const uint16_t* W, int32_t O, int32_t I, const void* x, int32_t x_dtype, int32_t ldx, int32_t M,
                    float* y, int32_t ldy, cx_stream_t stream) {
  if (!W || !x || !y) return CX_E_ARG;
  if (x_dtype != CX_F16 && x_dtype != CX_F32) return CX_E_ARG;
  if (O <= 0 || I <= 0 || M <= 0 || I % 32 || ldx < I || ldy < O) return CX_E_SHAPE;
  // Buffer descriptors address at most 4 GiB per operand.
  if ((size_t)O * I * 2 >= (1ull << 32) || (size_t)M * ldx * (x_dtype == CX_F32 ? 4 : 2) >= (1ull << 32))
    return CX_E_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  const __half* w = reinterpret_cast<const __half*>(W);
  if (x_dtype == CX_F32 && M <= 8) {
    if (ldx % 4) return CX_E_SHAPE;  // 16-byte row chunks
    const float* xf = static_cast<const float*>(x);
    const dim3 grid((O + 3) / 4);
    switch (M) {
      case 1: hipLaunchKernelGGL(DenseGemvKernel<1>, grid, dim3(256), 0, s, w, O, I, xf, ldx, y, ldy); break;
      case 2: hipLaunchKernelGGL(DenseGemvKernel<2>, grid, dim3(256), 0, s, w, O, I, xf, ldx, y, ldy); break;
      case 3: hipLaunchKernelGGL(DenseGemvKernel<3>, grid, dim3(256), 0, s, w, O, I, xf, ldx, y, ldy); break;
      case 4: hipLaunchKernelGGL(DenseGemvKernel<4>, grid, dim3(256), 0, s, w, O, I, xf, ldx, y, ldy); break;
      case 5: hipLaunchKernelGGL(DenseGemvKernel<5>, grid, dim3(256), 0, s, w, O, I, xf, ldx, y, ldy); break;
      case 6: hipLaunchKernelGGL(DenseGemvKernel<6>, grid, dim3(256), 0, s, w, O, I, xf, ldx, y, ldy); break;
      case 7: hipLaunchKernelGGL(DenseGemvKernel<7>, grid, dim3(256), 0, s, w, O, I, xf, ldx, y, ldy); break;
      default: hipLaunchKernelGGL(DenseGemvKernel<8>, grid, dim3(256), 0, s, w, O, I, xf, ldx, y, ldy); break;
    }
    return LaunchStatus();
  }
  const dim3 grid((M + 63) / 64, (O + 63) / 64);
  if (x_dtype == CX_F32)
    hipLaunchKernelGGL(DenseMfmaKernel<true>, grid, dim3(256), 0, s, w, O, I, x, ldx, M, y, ldy);
  else
    hipLaunchKernelGGL(DenseMfmaKernel<false>, grid, dim3(256), 0, s, w, O, I, x, ldx, M, y, ldy);
  return LaunchStatus();
}

}  // extern "C"
