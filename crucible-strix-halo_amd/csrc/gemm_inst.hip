// Exl3GemmKernel instantiations for one rate (compiled once per rate with -DCX_RATE=K2).
#include "internal.hpp"

#ifndef CX_RATE
#error "compile with -DCX_RATE=<2 x bits per weight>"
#endif

namespace cx {

#define CX_CAT2(a, b) a##b
#define CX_CAT(a, b) CX_CAT2(a, b)

bool CX_CAT(LaunchGemmRate, CX_RATE)(int cb, int nrb, int ksw, dim3 grid, const GemmArgs& g, hipStream_t s) {
  constexpr int K2 = CX_RATE;
  constexpr int U = 2;  // step groups in flight per wave (fewer registers, more waves)
  auto go = [&](auto cbc, auto nrbc, auto kswc) {
    constexpr int CB = decltype(cbc)::value, NRB = decltype(nrbc)::value, KSW = decltype(kswc)::value;
    if constexpr (NRB == 1 && KSW == 1) {
      if (g.mid_yg) {  // the decode down projection with the mid in its prologue
        // 16 rows of I + 8 halves, the up to 3 U - 1 steps (4 units each) the loop reads
        // past the last one (results unused), and at least the epilogue's 16 x 132 floats
        // it aliases
        const size_t lds = std::max((size_t)(16 * (g.A * 2 + 1) + 12 * U) * 16, (size_t)16 * 132 * 4);
        hipLaunchKernelGGL((Exl3GemmKernel<K2, CB, NRB, KSW, U, true>), grid, dim3(256), lds, s, g);
        return true;
      }
    } else if (g.mid_yg) {
      return false;  // the prologue mid exists for one row block per wave and no K split only
    }
    hipLaunchKernelGGL((Exl3GemmKernel<K2, CB, NRB, KSW, U>), grid, dim3(256), 0, s, g);
    return true;
  };
  auto rows = [&](auto cbc, auto kswc) {
    switch (nrb) {
      case 1: return go(cbc, IC<1>{}, kswc);
      case 2: return go(cbc, IC<2>{}, kswc);
      case 3: return go(cbc, IC<3>{}, kswc);
      case 4: return go(cbc, IC<4>{}, kswc);
      default: return false;
    }
  };
  auto split = [&](auto cbc) {
    if (ksw == 1) return rows(cbc, IC<1>{});
    if (ksw == 4) return rows(cbc, IC<4>{});
    return false;
  };
  if (cb == kCbMul1) return split(IC<kCbMul1>{});
  if constexpr (K2 % 2 == 0) {  // the mcg and 3inst codebooks exist at whole bit rates only
    if (cb == kCbMcg) return split(IC<kCbMcg>{});
    if (cb == kCb3Inst) return split(IC<kCb3Inst>{});
  }
  return false;
}

bool CX_CAT(LaunchGemmMultiRate, CX_RATE)(int cb, int nrb, const GemmMulti& gm, hipStream_t s) {
  constexpr int K2 = CX_RATE;
  constexpr int U = 2;
  auto go = [&](auto cbc, auto nrbc) {
    constexpr int CB = decltype(cbc)::value, NRB = decltype(nrbc)::value;
    hipLaunchKernelGGL((Exl3GemmMultiKernel<K2, CB, NRB, 4, U>), dim3((unsigned)gm.start[gm.n]), dim3(256), 0, s, gm);
    return true;
  };
  auto rows = [&](auto cbc) {
    switch (nrb) {
      case 1: return go(cbc, IC<1>{});
      case 2: return go(cbc, IC<2>{});
      case 3: return go(cbc, IC<3>{});
      case 4: return go(cbc, IC<4>{});
      default: return false;
    }
  };
  if (cb == kCbMul1) return rows(IC<kCbMul1>{});
  if constexpr (K2 % 2 == 0) {
    if (cb == kCbMcg) return rows(IC<kCbMcg>{});
    if (cb == kCb3Inst) return rows(IC<kCb3Inst>{});
  }
  return false;
}

// The down rates a stage launch of gate/up rate K2 takes: K2 itself (every codebook), and
// for mul1 layers the next two rates up (K2 + 2, K2 + 4: e.g. 3 bpw gate/up with 4 or 5 bpw
// down).
constexpr bool StageDownRate(int k2d) { return (k2d >= 2 && k2d <= 16 && k2d % 2 == 0) || k2d == 3 || k2d == 5 || k2d == 7; }

bool CX_CAT(LaunchDecodeStageRate, CX_RATE)(int cb, int k2d, const GemmArgs& gu, const GemmArgs& dn, int nyp,
                                             hipStream_t s) {
  constexpr int K2 = CX_RATE;
  const unsigned blocks = (unsigned)((2 * gu.ncp + dn.ncp / 4) * nyp);
  auto go = [&](auto cbc) {
    constexpr int CB = decltype(cbc)::value;
    hipLaunchKernelGGL((Exl3DecodeStageKernel<K2, K2, CB>), dim3(blocks), dim3(256), 0, s, gu, dn, nyp);
    return true;
  };
  auto mixed = [&](auto k2dc) {
    constexpr int K2D = decltype(k2dc)::value;
    if constexpr (StageDownRate(K2D))
      hipLaunchKernelGGL((Exl3DecodeStageKernel<K2, K2D, kCbMul1>), dim3(blocks), dim3(256), 0, s, gu, dn, nyp);
    return StageDownRate(K2D);
  };
  if (k2d != K2) {
    if (cb != kCbMul1) return false;
    if (k2d == K2 + 2) return mixed(IC<K2 + 2>{});
    if (k2d == K2 + 4) return mixed(IC<K2 + 4>{});
    return false;
  }
  if (cb == kCbMul1) return go(IC<kCbMul1>{});
  if constexpr (K2 % 2 == 0) {
    if (cb == kCbMcg) return go(IC<kCbMcg>{});
    if (cb == kCb3Inst) return go(IC<kCb3Inst>{});
  }
  return false;
}

}  // namespace cx
