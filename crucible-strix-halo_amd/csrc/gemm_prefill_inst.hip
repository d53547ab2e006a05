// Exl3GemmPrefillKernel instantiations for one rate (compiled once per rate with
// -DCX_RATE=K2).  Built with MFMA accumulators in VGPRs (-amdgpu-mfma-vgpr-form): with
// accumulator VGPRs the register allocator otherwise copies accumulators between the
// two register files inside the decode loop.
#include "internal.hpp"

#ifndef CX_RATE
#error "compile with -DCX_RATE=<2 x bits per weight>"
#endif

namespace cx {

#define CX_CAT2(a, b) a##b
#define CX_CAT(a, b) CX_CAT2(a, b)

bool CX_CAT(LaunchGemmPrefillRate, CX_RATE)(int cb, int nrbt, int wpg, bool mid, dim3 grid, const GemmArgs& g,
                                           hipStream_t s) {
  constexpr int K2 = CX_RATE;
  auto go = [&](auto cbc, auto nc, auto wc) {
    constexpr int CB = decltype(cbc)::value, NRBT = decltype(nc)::value, WPG = decltype(wc)::value;
    hipLaunchKernelGGL((Exl3GemmPrefillKernel<K2, CB, NRBT, 1, WPG>), grid, dim3(64 * WPG), 0, s, g);
    return true;
  };
  auto shape = [&](auto cbc) {
    if (mid) {  // gate and up in one workgroup, the mid in the epilogue
      if (nrbt != 4 || wpg != 4) return false;
      hipLaunchKernelGGL((Exl3GemmPrefillKernel<K2, decltype(cbc)::value, 4, 1, 4, true>), grid, dim3(512), 0, s, g);
      return true;
    }
    if (nrbt == 4 && wpg == 4) return go(cbc, IC<4>{}, IC<4>{});
    if (nrbt == 4 && wpg == 8) return go(cbc, IC<4>{}, IC<8>{});
    if (nrbt == 4 && wpg == 16) return go(cbc, IC<4>{}, IC<16>{});
    if (nrbt == 8 && wpg == 4) return go(cbc, IC<8>{}, IC<4>{});
    if (nrbt == 8 && wpg == 8) return go(cbc, IC<8>{}, IC<8>{});
    return false;
  };
  if (cb == kCbMul1) return shape(IC<kCbMul1>{});
  if constexpr (K2 % 2 == 0) {
    if (cb == kCbMcg) return shape(IC<kCbMcg>{});
    if (cb == kCb3Inst) return shape(IC<kCb3Inst>{});
  }
  return false;
}

}  // namespace cx

namespace cx {

bool CX_CAT(LaunchGemmTallRate, CX_RATE)(int cb, dim3 grid, const GemmArgs& g, hipStream_t s) {
  constexpr int K2 = CX_RATE;
  auto go = [&](auto cbc) {
    hipLaunchKernelGGL((Exl3GemmTallKernel<K2, decltype(cbc)::value, kTallRowBlocksPerWave>), grid, dim3(256), 0, s, g);
    return true;
  };
  if (cb == kCbMul1) return go(IC<kCbMul1>{});
  if constexpr (K2 % 2 == 0) {
    if (cb == kCbMcg) return go(IC<kCbMcg>{});
    if (cb == kCb3Inst) return go(IC<kCb3Inst>{});
  }
  return false;
}

}  // namespace cx

