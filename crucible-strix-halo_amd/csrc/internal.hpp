// Host-side internals shared by the library's translation units.
#pragma once

#include <algorithm>
#include <cstddef>
#include <type_traits>

#include "../../include/crucible_exl3.h"
#include "gemm.hpp"

namespace cx {

inline bool ValidK2(int k2) { return (k2 >= 2 && k2 <= 16 && !(k2 & 1)) || k2 == 3 || k2 == 5 || k2 == 7; }
inline size_t AlignUp(size_t v, size_t a) { return (v + a - 1) / a * a; }
// Workspaces are carved into 256-byte aligned pieces (device tables, 16-byte rows).
inline bool WorkspaceAligned(const void* p) { return reinterpret_cast<uintptr_t>(p) % 256 == 0; }

inline int LaunchStatus() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? CX_OK : (int)e;
}

template <int V>
using IC = std::integral_constant<int, V>;

// Calls f(IC<K2>, IC<CB>) for a supported (rate, codebook); false otherwise.
template <class F>
bool DispatchK2Cb(int k2, int cb, F&& f) {
  auto with_cb = [&](auto k2c) {
    constexpr int K2 = decltype(k2c)::value;
    if (cb == kCbMul1) { f(k2c, IC<kCbMul1>{}); return true; }
    if constexpr (K2 % 2 == 0) {
      if (cb == kCbMcg) { f(k2c, IC<kCbMcg>{}); return true; }
      if (cb == kCb3Inst) { f(k2c, IC<kCb3Inst>{}); return true; }
    }
    return false;
  };
  switch (k2) {
    case 2: return with_cb(IC<2>{});
    case 3: return with_cb(IC<3>{});
    case 4: return with_cb(IC<4>{});
    case 5: return with_cb(IC<5>{});
    case 6: return with_cb(IC<6>{});
    case 7: return with_cb(IC<7>{});
    case 8: return with_cb(IC<8>{});
    case 10: return with_cb(IC<10>{});
    case 12: return with_cb(IC<12>{});
    case 14: return with_cb(IC<14>{});
    case 16: return with_cb(IC<16>{});
    default: return false;
  }
}

// Kernel-argument tables of the grouped activation transforms (no device-side tables).
constexpr int kMaxGroupJobs = 16;
struct XfIn {
  const void* x;
  const __half* suh;
  __half* xp;
  int ldx, I, xf32, item0;
};
struct XfInTable {
  XfIn job[kMaxGroupJobs];
  int n, M;
};
struct XfOut {
  const float* part;
  long long seg_stride;
  const __half* svh;
  void* y;
  int S, ldy, O, f16, item0;
};
struct XfOutTable {
  XfOut job[kMaxGroupJobs];
  int n, M;
};

struct LinearPlan {
  int A, ncp;     // k-tiles, column pairs
  int nrb;        // 16-row blocks per wave
  int chunk;      // rows per entry (16 * nrb)
  int n_entries;  // row entries
  int ksw;        // K splits inside a workgroup (waves per column pair)
  int S;          // K segments across workgroups
  int u;          // unused (kept for plan printing)
};

int CheckMatrix(const cx_exl3_matrix* m);
int RowOffsetsCheck(const int32_t* row_offsets, int32_t n_sessions, int32_t M);
LinearPlan PlanLinear(int I, int O, int M);
size_t LinearWorkspace(const LinearPlan& p, int I, int O, int M);

// Launches Exl3GemmKernel for a runtime (rate, codebook, rows per wave, waves per
// column pair).  Returns false for an unsupported combination.
bool LaunchGemm(int k2, int cb, int nrb, int ksw, int u, dim3 grid, const GemmArgs& g, hipStream_t s);
// The prefill GEMM (Exl3GemmPrefillKernel): grid (O / (32 wpg), entries padded to 8, planes);
// mid: gate and up in one workgroup with the mid fused (grid (O / 128, entries padded, 1)).
bool LaunchGemmPrefill(int k2, int cb, int nrbt, int wpg, bool mid, dim3 grid, const GemmArgs& g, hipStream_t s);
// The tall prefill GEMM (Exl3GemmTallKernel): entries of up to 64 kTallRowBlocksPerWave
// rows, grid (O / 128, entries padded to 8, planes).
constexpr int kTallRowBlocksPerWave = 3;
bool LaunchGemmTall(int k2, int cb, dim3 grid, const GemmArgs& g, hipStream_t s);
// Gate/up, mid and down of a decode call in one launch (Exl3DecodeStageKernel), all four
// matrices of every expert at rate k2 and codebook cb; nyp entries (a multiple of 8).
bool LaunchDecodeStage(int k2, int k2d, int cb, const GemmArgs& gu, const GemmArgs& dn, int nyp, hipStream_t s);
// Exl3GemmMultiKernel: gm.n jobs (K split over 4 waves) at rate k2, codebook cb, nrb row
// blocks; gm.start[gm.n] workgroups.
bool LaunchGemmMulti(int k2, int cb, int nrb, const GemmMulti& gm, hipStream_t s);
// Per-rate launchers (one translation unit per rate, gemm_inst.hip).
#define CX_DECLARE_RATE(K2)                                                                          \
  bool LaunchGemmRate##K2(int cb, int nrb, int ksw, dim3 grid, const GemmArgs& g, hipStream_t s); \
  bool LaunchGemmPrefillRate##K2(int cb, int nrbt, int wpg, bool mid, dim3 grid, const GemmArgs& g, \
                                 hipStream_t s);                                                         \
  bool LaunchGemmTallRate##K2(int cb, dim3 grid, const GemmArgs& g, hipStream_t s);                         \
  bool LaunchDecodeStageRate##K2(int cb, int k2d, const GemmArgs& gu, const GemmArgs& dn, int nyp, hipStream_t s); \
  bool LaunchGemmMultiRate##K2(int cb, int nrb, const GemmMulti& gm, hipStream_t s);
CX_DECLARE_RATE(2)
CX_DECLARE_RATE(3)
CX_DECLARE_RATE(4)
CX_DECLARE_RATE(5)
CX_DECLARE_RATE(6)
CX_DECLARE_RATE(7)
CX_DECLARE_RATE(8)
CX_DECLARE_RATE(10)
CX_DECLARE_RATE(12)
CX_DECLARE_RATE(14)
CX_DECLARE_RATE(16)
#undef CX_DECLARE_RATE

}  // namespace cx
