// Sustained MFMA throughput of the fp16 matrix instructions on this GPU (gfx950): each
// wave issues chains of independent MFMAs on register operands (no memory traffic), over
// 2, 4 and 8 waves per SIMD.  The prefill GEMMs' fraction of peak is read against these
// rates as well as against the published dense peak (2.5 PFLOP/s fp16).
//   make -C crucible-strix-halo_amd probes && crucible-strix-halo_amd/probes/mfma_rate
#include <hip/hip_runtime.h>

#include <cstdio>

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));

// MODE 0: v_mfma_f32_16x16x32_f16, 1: v_mfma_f32_32x32x16_f16, 2: 16x16x16, 3: 32x32x8.
template <int MODE, int NACC>
__global__ void __launch_bounds__(256) Chain(float* out, int iters) {
  half8_t a, b;
  half4_t a4, b4;
  for (int i = 0; i < 8; ++i) {
    a[i] = (_Float16)(threadIdx.x * 0.001f + i);
    b[i] = (_Float16)(i * 0.5f);
  }
  for (int i = 0; i < 4; ++i) {
    a4[i] = a[i];
    b4[i] = b[i];
  }
  float s = 0.f;
  if constexpr (MODE == 0 || MODE == 2) {
    float4_t acc[NACC];
    for (int j = 0; j < NACC; ++j) acc[j] = float4_t{0.f, 0.f, 0.f, 0.f};
    for (int it = 0; it < iters; ++it)
#pragma unroll
      for (int j = 0; j < NACC; ++j) {
        if constexpr (MODE == 0) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[j], 0, 0, 0);
        else acc[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(a4, b4, acc[j], 0, 0, 0);
      }
    for (int j = 0; j < NACC; ++j) s += acc[j][0] + acc[j][3];
  } else {
    float16_t acc[NACC];
    for (int j = 0; j < NACC; ++j)
      for (int e = 0; e < 16; ++e) acc[j][e] = 0.f;
    for (int it = 0; it < iters; ++it)
#pragma unroll
      for (int j = 0; j < NACC; ++j) {
        if constexpr (MODE == 1) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[j], 0, 0, 0);
        else acc[j] = __builtin_amdgcn_mfma_f32_32x32x8f16(a4, b4, acc[j], 0, 0, 0);
      }
    for (int j = 0; j < NACC; ++j) s += acc[j][0] + acc[j][15];
  }
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

template <int MODE, int NACC>
static void Run(const char* name, double flops_per, float* out, int cus) {
  hipEvent_t e0, e1;
  (void)hipEventCreate(&e0);
  (void)hipEventCreate(&e1);
  const int iters = 2000;
  for (int per_simd : {2, 4, 8}) {
    const int wgs = cus * per_simd;  // 4 waves per workgroup = one per SIMD
    hipLaunchKernelGGL((Chain<MODE, NACC>), dim3(wgs), dim3(256), 0, 0, out, iters);
    (void)hipEventRecord(e0);
    hipLaunchKernelGGL((Chain<MODE, NACC>), dim3(wgs), dim3(256), 0, 0, out, iters);
    (void)hipEventRecord(e1);
    (void)hipEventSynchronize(e1);
    float ms = 0.f;
    (void)hipEventElapsedTime(&ms, e0, e1);
    const double flops = (double)wgs * 4 * iters * NACC * flops_per;
    std::printf("%-28s %d waves/SIMD: %8.3f ms  %7.1f TFLOP/s\n", name, per_simd, ms, flops / ms / 1e9);
  }
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
}

int main() {
  hipDeviceProp_t p;
  if (hipGetDeviceProperties(&p, 0) != hipSuccess) return 1;
  std::printf("device %s, %d CUs, clock %d MHz\n", p.gcnArchName, p.multiProcessorCount, p.clockRate / 1000);
  float* out = nullptr;
  if (hipMalloc(&out, (size_t)p.multiProcessorCount * 8 * 256 * sizeof(float)) != hipSuccess) return 1;
  Run<0, 8>("v_mfma_f32_16x16x32_f16", 16384.0, out, p.multiProcessorCount);
  Run<1, 4>("v_mfma_f32_32x32x16_f16", 32768.0, out, p.multiProcessorCount);
  Run<2, 8>("v_mfma_f32_16x16x16_f16", 8192.0, out, p.multiProcessorCount);
  Run<3, 4>("v_mfma_f32_32x32x8_f16", 16384.0, out, p.multiProcessorCount);
  (void)hipFree(out);
  return 0;
}
