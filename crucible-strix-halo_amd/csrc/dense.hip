// Dense fp16-weight linear y[r][o] = W[o] . x[r] (the MoE router: W = [E + 1][H] with the
// shared-expert gate as row E).  Two kernels, as in the reference's router launch
// (engine/engine.hip:1824-1870):
//   * up to 8 rows of fp32 x: one wave per output row, fp32 products and sums
//     (DenseGemvKernel, engine/layers/ops.h:30-61);
//   * more rows, or fp16 x: x rounded to fp16 (the reference packs it first,
//     PrefillPackKernel) and v_mfma_f32_16x16x32_f16 with fp32 sums: up to 64 rows one
//     workgroup per 16 outputs with K split over its 8 waves (DenseSplitKernel), above
//     that tiles of 64 rows x 64 outputs (DenseMfmaKernel).
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
// [16 NB by, 16 NB (by + 1)); wave w owns rows 16 w .. 16 w + 15 and all 16 NB outputs
// (x, the larger operand at prefill sizes, is read once per 16 NB outputs).  Per
// 32-wide k step a lane loads 8 consecutive k of its x row (A operand) and of 4 W rows
// (B operands: W is [O][I], so B = W^T has consecutive k contiguous).  Rows >= M and
// outputs >= O read zeros (buffer bounds) and are not stored.  XF32: x is fp32 and is
// rounded to fp16 on load.
template <bool XF32, int NB>
__global__ void __launch_bounds__(256) DenseMfmaKernel(const __half* __restrict__ W, int O, int I,
                                                       const void* __restrict__ x, int ldx, int M,
                                                       float* __restrict__ y, int ldy) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int m0 = blockIdx.x * 64 + wave * 16, o0 = blockIdx.y * 16 * NB;
  const int kq = 8 * (lane >> 4), ln = lane & 15;
  const int esz = XF32 ? 4 : 2;
  const int rows = max(0, min(16, M - m0));
  const __amdgpu_buffer_rsrc_t rx =
      MakeRsrc(static_cast<const char*>(x) + (size_t)m0 * ldx * esz, (uint32_t)((size_t)rows * ldx * esz));
  const int outs = max(0, min(16 * NB, O - o0));
  const __amdgpu_buffer_rsrc_t rw = MakeRsrc(W + (size_t)o0 * I, (uint32_t)((size_t)outs * I * 2));
  const uint32_t xoff = (uint32_t)((ln * ldx + kq) * esz);
  float4_t acc[NB];
#pragma unroll
  for (int n = 0; n < NB; ++n) acc[n] = float4_t{0.f, 0.f, 0.f, 0.f};
  // PF steps of loads in flight ahead of the MFMAs (loads past the last step read other
  // columns or fall outside the buffers; their results are not used).
  struct Step {
    u32x4_t a[XF32 ? 2 : 1];
    u32x4_t b[NB];
  };
  auto load = [&](Step& st, int k) {
    st.a[0] = BufLoad128(rx, xoff, (uint32_t)k * esz);
    if constexpr (XF32) st.a[1] = BufLoad128(rx, xoff + 16, (uint32_t)k * 4);
#pragma unroll
    for (int n = 0; n < NB; ++n) st.b[n] = BufLoad128(rw, (uint32_t)(((n * 16 + ln) * I + kq) * 2), (uint32_t)k * 2);
  };
  auto mma = [&](const Step& st) {
    half8_t a;
    if constexpr (XF32) {
      // Whole-vector casts: element-wise bit casts of ext-vector elements are miscompiled
      // by this toolchain (every element reads element 0).
      const float4_t lo = __builtin_bit_cast(float4_t, st.a[0]);
      const float4_t hi = __builtin_bit_cast(float4_t, st.a[1]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        a[i] = (_Float16)lo[i];
        a[4 + i] = (_Float16)hi[i];
      }
    } else {
      a = __builtin_bit_cast(half8_t, st.a[0]);
    }
#pragma unroll
    for (int n = 0; n < NB; ++n)
      acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, __builtin_bit_cast(half8_t, st.b[n]), acc[n], 0, 0, 0);
  };
  // Two groups of U steps: the next group's loads are issued before the current group's
  // MFMAs.  The main loop has no branch (a conditional MFMA there makes the compiler wait
  // for every load in flight at each iteration); the last I % (64 U) inputs follow it.
  constexpr int U = 2;
  Step ga[U], gb[U];
#pragma unroll
  for (int u = 0; u < U; ++u) load(ga[u], 32 * u);
  const int kmain = I - I % (64 * U);
  for (int k = 0; k < kmain; k += 64 * U) {
#pragma unroll
    for (int u = 0; u < U; ++u) load(gb[u], k + 32 * (U + u));
#pragma unroll
    for (int u = 0; u < U; ++u) mma(ga[u]);
#pragma unroll
    for (int u = 0; u < U; ++u) load(ga[u], k + 32 * (2 * U + u));
#pragma unroll
    for (int u = 0; u < U; ++u) mma(gb[u]);
  }
  // Tail: at most 2 U - 1 steps; ga holds the first U of them.
  if (kmain < I) {
#pragma unroll
    for (int u = 0; u < U; ++u) load(gb[u], kmain + 32 * (U + u));
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (kmain + 32 * u < I) mma(ga[u]);
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (kmain + 32 * (U + u) < I) mma(gb[u]);
  }
#pragma unroll
  for (int n = 0; n < NB; ++n) {
    const int o = o0 + n * 16 + ln;
    if (o >= O) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = m0 + 4 * (lane >> 4) + i;
      if (r < M) y[(size_t)r * ldy + o] = acc[n][i];
    }
  }
}

// Up to 64 rows (NRB 16-row blocks): a 512-thread workgroup owns outputs [16 bx, 16 bx +
// 16) and wave w the k range [w I / 8, (w + 1) I / 8) (I a multiple of 256), all NRB row
// blocks; the weight and activation loads of the next two 2-step groups are in flight
// while a group's MFMAs run.  The 8 waves' sums are added in wave order through LDS (the
// result does not depend on the number of rows beyond the block count).  Rows >= M and
// outputs >= O read zeros (buffer bounds) and are not stored.
template <bool XF32, int NRB>
__global__ void __launch_bounds__(512) DenseSplitKernel(const __half* __restrict__ W, int O, int I,
                                                        const void* __restrict__ x, int ldx, int M,
                                                        float* __restrict__ y, int ldy) {
  constexpr int NW = 8, U = 2;
  __shared__ float4_t red[NW - 1][NRB][64];
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int o0 = blockIdx.x * 16, kq = 8 * (lane >> 4), ln = lane & 15;
  const int kw = I / NW, k0 = wave * kw, steps = kw / 32;
  const int esz = XF32 ? 4 : 2;
  const int outs = max(0, min(16, O - o0));
  const __amdgpu_buffer_rsrc_t rw = MakeRsrc(W + (size_t)o0 * I, (uint32_t)((size_t)outs * I * 2));
  const __amdgpu_buffer_rsrc_t rx = MakeRsrc(x, (uint32_t)((size_t)M * ldx * esz));
  const uint32_t woff = (uint32_t)((ln * I + k0 + kq) * 2);
  uint32_t xoff[NRB];
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb) {
    const int r = rb * 16 + ln;
    xoff[rb] = r < M ? (uint32_t)((r * ldx + k0 + kq) * esz) : 0xF0000000u;  // past M: outside the buffer
  }
  struct Step {
    u32x4_t b;
    u32x4_t a[NRB][XF32 ? 2 : 1];
  };
  auto load = [&](Step& st, int s) {
    st.b = BufLoad128(rw, woff, (uint32_t)s * 64);
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
      st.a[rb][0] = BufLoad128(rx, xoff[rb], (uint32_t)s * 32 * esz);
      if constexpr (XF32) st.a[rb][1] = BufLoad128(rx, xoff[rb] + 16, (uint32_t)s * 128);
    }
  };
  float4_t acc[NRB];
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb) acc[rb] = float4_t{0.f, 0.f, 0.f, 0.f};
  auto mma = [&](const Step& st) {
    const half8_t b = __builtin_bit_cast(half8_t, st.b);
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
      half8_t a;
      if constexpr (XF32) {
        // Whole-vector casts (element-wise bit casts of ext-vector elements read element 0).
        const float4_t lo = __builtin_bit_cast(float4_t, st.a[rb][0]);
        const float4_t hi = __builtin_bit_cast(float4_t, st.a[rb][1]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          a[i] = (_Float16)lo[i];
          a[4 + i] = (_Float16)hi[i];
        }
      } else {
        a = __builtin_bit_cast(half8_t, st.a[rb][0]);
      }
      acc[rb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[rb], 0, 0, 0);
    }
  };
  // Loads are unconditional, also past the last step (outside the wave's k range they read
  // other waves' columns or fall outside the buffer; the results are not used).
  Step ga[U], gb[U];
#pragma unroll
  for (int u = 0; u < U; ++u) load(ga[u], u);
  for (int s = 0; s < steps; s += 2 * U) {
#pragma unroll
    for (int u = 0; u < U; ++u) load(gb[u], s + U + u);
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (s + u < steps) mma(ga[u]);
#pragma unroll
    for (int u = 0; u < U; ++u) load(ga[u], s + 2 * U + u);
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (s + U + u < steps) mma(gb[u]);
  }
  if (wave > 0) {
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) red[wave - 1][rb][lane] = acc[rb];
  }
  __syncthreads();
  if (wave > 0) return;
#pragma unroll
  for (int w = 0; w < NW - 1; ++w)
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) acc[rb] += red[w][rb][lane];
  const int o = o0 + ln;
  if (o >= O) return;
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = rb * 16 + 4 * (lane >> 4) + i;
      if (r < M) y[(size_t)r * ldy + o] = acc[rb][i];
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
  if (M <= 64 && I % 256 == 0 && (x_dtype == CX_F16 || ldx % 4 == 0)) {
    const dim3 grid((O + 15) / 16);
    const bool f32 = x_dtype == CX_F32;
    switch ((M + 15) / 16) {
      case 1:
        if (f32) hipLaunchKernelGGL((DenseSplitKernel<true, 1>), grid, dim3(512), 0, s, w, O, I, x, ldx, M, y, ldy);
        else hipLaunchKernelGGL((DenseSplitKernel<false, 1>), grid, dim3(512), 0, s, w, O, I, x, ldx, M, y, ldy);
        break;
      case 2:
        if (f32) hipLaunchKernelGGL((DenseSplitKernel<true, 2>), grid, dim3(512), 0, s, w, O, I, x, ldx, M, y, ldy);
        else hipLaunchKernelGGL((DenseSplitKernel<false, 2>), grid, dim3(512), 0, s, w, O, I, x, ldx, M, y, ldy);
        break;
      case 3:
        if (f32) hipLaunchKernelGGL((DenseSplitKernel<true, 3>), grid, dim3(512), 0, s, w, O, I, x, ldx, M, y, ldy);
        else hipLaunchKernelGGL((DenseSplitKernel<false, 3>), grid, dim3(512), 0, s, w, O, I, x, ldx, M, y, ldy);
        break;
      default:
        if (f32) hipLaunchKernelGGL((DenseSplitKernel<true, 4>), grid, dim3(512), 0, s, w, O, I, x, ldx, M, y, ldy);
        else hipLaunchKernelGGL((DenseSplitKernel<false, 4>), grid, dim3(512), 0, s, w, O, I, x, ldx, M, y, ldy);
        break;
    }
    return LaunchStatus();
  }
  constexpr int NB = 4;  // 64 outputs per workgroup
  const dim3 grid((M + 63) / 64, (O + 16 * NB - 1) / (16 * NB));
  if (x_dtype == CX_F32)
    hipLaunchKernelGGL((DenseMfmaKernel<true, NB>), grid, dim3(256), 0, s, w, O, I, x, ldx, M, y, ldy);
  else
    hipLaunchKernelGGL((DenseMfmaKernel<false, NB>), grid, dim3(256), 0, s, w, O, I, x, ldx, M, y, ldy);
  return LaunchStatus();
}

}  // extern "C"
