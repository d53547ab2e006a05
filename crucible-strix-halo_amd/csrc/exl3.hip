// EXL3 linear op on MI355X: loader repack, bit-exact dequant, and the linear
// (input transform -> fused decode/MFMA GEMM -> fixed-order split sum + output transform).
#include <vector>

#include "internal.hpp"

namespace cx {

// ---- loader repack ------------------------------------------------------------------

// Checkpoint tile (a, b) -> column-pair-major index ((b/2) A + a) 2 + b % 2.  The 8K
// dwords of a tile are its 16K little-endian int16 words unchanged.
__global__ void RepackKernel(const uint32_t* __restrict__ src, uint32_t* __restrict__ dst, int A, int B, int T) {
  const size_t total = (size_t)A * B * T;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const size_t tile = i / T;
    const int w = (int)(i % T);
    const int a = (int)(tile / B), b = (int)(tile % B);
    const size_t d = (((size_t)(b >> 1) * A + a) * 2 + (b & 1)) * T + w;
    dst[d] = src[i];
  }
}

// ---- dequant ------------------------------------------------------------------------

// One wave per tile pair: the GEMM's own decode (same lanes, same arithmetic), written
// out as W_hat[16a + r][16b + c].
template <int K2, int CB>
__global__ void __launch_bounds__(256) DequantKernel(const uint32_t* __restrict__ tiles, __half* __restrict__ w,
                                                     int A, int ncp) {
  constexpr int T = TileDwords(K2);
  constexpr int ND = WindowDwords(K2);
  const int pair = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (pair >= A * ncp) return;
  const int lane = threadIdx.x & 63;
  const int cp = pair / A, a = pair % A;
  const uint32_t* base = tiles + (size_t)pair * 2 * T;
  const LaneRun<K2> lr(lane);
  uint32_t win[3] = {0, 0, 0};
#pragma unroll
  for (int i = 0; i < ND; ++i) win[i] = base[lr.ByteOffset(i) / 4];
  half4_t lo, hi;
  DecodeRun<K2, CB>(win[0], win[1], ND > 2 ? win[2] : win[1], lr.shift, lo, hi);
  const int O = ncp * 32;
  const int q = lane >> 4, c = (lane & 7), b = 2 * cp + ((lane & 15) >> 3);
  // (Elements go through scalar locals: bit-casting a vector element lvalue directly
  // is miscompiled by this toolchain into element 0 for every index.)
  unsigned short* wu = reinterpret_cast<unsigned short*>(w);
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int r = 16 * a + PermRow16(4 * q + s);
    const _Float16 vlo = lo[s], vhi = hi[s];
    wu[(size_t)r * O + b * 16 + c] = __builtin_bit_cast(unsigned short, vlo);
    wu[(size_t)r * O + b * 16 + c + 8] = __builtin_bit_cast(unsigned short, vhi);
  }
}

// ---- activation transforms ----------------------------------------------------------

// Input transforms of a group of linears over the same M rows: RoundH(RoundH(x) * suh)
// -> WHT128 -> * norm -> fp16, stored in MFMA row order.  One 128-block per 16 lanes; job
// j owns the 16-lane items [item0, item0 + M I / 128).  ref/exl3_ref.py:140-152;
// engine/exl3/exl3.h:48-65 (fp32 sources are rounded to fp16 first, as LinInLane does).
__global__ void __launch_bounds__(256) InputTransformKernel(XfInTable t) {
  const int item = (blockIdx.x * blockDim.x + threadIdx.x) >> 4;
  int jb = 0;
  while (jb + 1 < t.n && item >= t.job[jb + 1].item0) ++jb;
  const XfIn& J = t.job[jb];
  const int nb = J.I / 128, local = item - J.item0;
  if (local >= t.M * nb) return;  // whole 16-lane groups
  const int r = local / nb, blk = local % nb, j = threadIdx.x & 15;
  const int c0 = blk * 128 + 8 * j;
  // x as 4 packed fp16 pairs (fp32 sources rounded), times suh in fp16 (the fp16
  // product is RoundH of the exact fp32 product), into the transform's first stage.
  uint32_t h[4];
  if (J.xf32) {
    float f[8];
    LoadF8(static_cast<const float*>(J.x) + (size_t)r * J.ldx + c0, f);
#pragma unroll
    for (int k = 0; k < 4; ++k) h[k] = __builtin_bit_cast(uint32_t, __floats2half2_rn(f[2 * k], f[2 * k + 1]));
  } else {
    const uint4 u = *reinterpret_cast<const uint4*>(static_cast<const __half*>(J.x) + (size_t)r * J.ldx + c0);
    h[0] = u.x;
    h[1] = u.y;
    h[2] = u.z;
    h[3] = u.w;
  }
  const uint4 su = *reinterpret_cast<const uint4*>(J.suh + c0);
  const uint32_t hs[4] = {su.x, su.y, su.z, su.w};
#pragma unroll
  for (int k = 0; k < 4; ++k)
    h[k] = __builtin_bit_cast(uint32_t, __hmul2(__builtin_bit_cast(__half2, h[k]), __builtin_bit_cast(__half2, hs[k])));
  float v[8];
  Wht128x8SignedH(h, v);
  StorePerm32x8(J.xp + (size_t)r * J.I + blk * 128, v, kHadNorm * WhtLaneSign());
}

// Fixed-order sum of S K-segment partials, then the output transform, for a group of
// linears.  f16 = 0: WHT in fp32, * (norm * svh) (engine LinOutBlock,
// engine/exl3/exl3.h:69-82).  f16 = 1: y_h rounded to fp16, WHT, * norm -> fp16, * svh
// -> fp16 (ref/exl3_ref.py:153-156).
__global__ void __launch_bounds__(256) OutputTransformKernel(XfOutTable t) {
  const int item = (blockIdx.x * blockDim.x + threadIdx.x) >> 4;
  int jb = 0;
  while (jb + 1 < t.n && item >= t.job[jb + 1].item0) ++jb;
  const XfOut& J = t.job[jb];
  const int nb = J.O / 128, local = item - J.item0;
  if (local >= t.M * nb) return;
  const int r = local / nb, blk = local % nb, j = threadIdx.x & 15;
  const int c0 = blk * 128 + 8 * j;
  float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, p[8], sv[8];
  for (int s = 0; s < J.S; ++s) {
    LoadF8(J.part + s * J.seg_stride + (size_t)r * J.O + c0, p);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] += p[i];
  }
  if (J.f16) {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = RoundH(v[i]);
  }
  Wht128x8Signed(v);
  LoadH8(J.svh + c0, sv);
  const float sg = WhtLaneSign();
  if (J.f16) {
    __half* d = static_cast<__half*>(J.y) + (size_t)r * J.ldy + c0;
#pragma unroll
    for (int i = 0; i < 8; ++i) d[i] = __float2half(RoundH(v[i] * (sg * kHadNorm)) * sv[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] *= sg * (kHadNorm * sv[i]);
    StoreF8(static_cast<float*>(J.y) + (size_t)r * J.ldy + c0, v);
  }
}

// ---- host side ------------------------------------------------------------------------

int CheckMatrix(const cx_exl3_matrix* m) {
  if (!m || !m->tiles || !m->suh || !m->svh) return CX_E_ARG;
  if (m->in_features <= 0 || m->out_features <= 0 || m->in_features % 128 || m->out_features % 128) return CX_E_SHAPE;
  if (!ValidK2(m->k2)) return CX_E_BITRATE;
  if (m->codebook < 0 || m->codebook > 2) return CX_E_ARG;
  if ((m->k2 & 1) && m->codebook != CX_CB_MUL1) return CX_E_BITRATE;  // half rates require mul1
  return CX_OK;
}

int RowOffsetsCheck(const int32_t* row_offsets, int32_t n_sessions, int32_t M) {
  if (!row_offsets) return CX_OK;
  if (n_sessions < 1 || row_offsets[0] != 0) return CX_E_SHAPE;
  for (int s = 0; s < n_sessions; ++s)
    if (row_offsets[s + 1] < row_offsets[s]) return CX_E_SHAPE;
  return row_offsets[n_sessions] == M ? CX_OK : CX_E_SHAPE;
}

LinearPlan PlanLinear(int I, int O, int M) {
  LinearPlan p;
  p.A = I / 16;
  p.ncp = O / 32;
  p.nrb = M >= 64 ? 4 : (M + 15) / 16;
  if (p.nrb < 1) p.nrb = 1;
  p.chunk = 16 * p.nrb;
  p.n_entries = (M + p.chunk - 1) / p.chunk;
  p.ksw = 4;
  // Grow the cross-workgroup K split until ~512 workgroups or 4 steps per wave.  The
  // split depends on the matrix only, never on M, so a row's result is bitwise the same
  // whatever other rows share the call.
  p.S = 1;
  const int wgs = p.ncp;
  // Steps are two k-tiles; keep at least 8 steps per wave (measured: config-2 GEMVs at 8
  // steps per wave 13.3 us per call against 14.5 us at 4, 19 us at 2).
  while (wgs * p.S < 512 && (p.A / 2) / (p.ksw * p.S * 2) >= 8) p.S *= 2;
  const int steps = p.A / 2 / (p.ksw * p.S);
  p.u = steps % 4 == 0 ? 4 : steps % 2 == 0 ? 2 : 1;
  return p;
}

bool LaunchGemm(int k2, int cb, int nrb, int ksw, int u, dim3 grid, const GemmArgs& g, hipStream_t s) {
  (void)u;
  switch (k2) {
    case 2: return LaunchGemmRate2(cb, nrb, ksw, grid, g, s);
    case 3: return LaunchGemmRate3(cb, nrb, ksw, grid, g, s);
    case 4: return LaunchGemmRate4(cb, nrb, ksw, grid, g, s);
    case 5: return LaunchGemmRate5(cb, nrb, ksw, grid, g, s);
    case 6: return LaunchGemmRate6(cb, nrb, ksw, grid, g, s);
    case 7: return LaunchGemmRate7(cb, nrb, ksw, grid, g, s);
    case 8: return LaunchGemmRate8(cb, nrb, ksw, grid, g, s);
    case 10: return LaunchGemmRate10(cb, nrb, ksw, grid, g, s);
    case 12: return LaunchGemmRate12(cb, nrb, ksw, grid, g, s);
    case 14: return LaunchGemmRate14(cb, nrb, ksw, grid, g, s);
    case 16: return LaunchGemmRate16(cb, nrb, ksw, grid, g, s);
    default: return false;
  }
}

bool LaunchGemmPrefill(int k2, int cb, int nrbt, int wpg, bool mid, dim3 grid, const GemmArgs& g, hipStream_t s) {
  switch (k2) {
    case 2: return LaunchGemmPrefillRate2(cb, nrbt, wpg, mid, grid, g, s);
    case 3: return LaunchGemmPrefillRate3(cb, nrbt, wpg, mid, grid, g, s);
    case 4: return LaunchGemmPrefillRate4(cb, nrbt, wpg, mid, grid, g, s);
    case 5: return LaunchGemmPrefillRate5(cb, nrbt, wpg, mid, grid, g, s);
    case 6: return LaunchGemmPrefillRate6(cb, nrbt, wpg, mid, grid, g, s);
    case 7: return LaunchGemmPrefillRate7(cb, nrbt, wpg, mid, grid, g, s);
    case 8: return LaunchGemmPrefillRate8(cb, nrbt, wpg, mid, grid, g, s);
    case 10: return LaunchGemmPrefillRate10(cb, nrbt, wpg, mid, grid, g, s);
    case 12: return LaunchGemmPrefillRate12(cb, nrbt, wpg, mid, grid, g, s);
    case 14: return LaunchGemmPrefillRate14(cb, nrbt, wpg, mid, grid, g, s);
    case 16: return LaunchGemmPrefillRate16(cb, nrbt, wpg, mid, grid, g, s);
    default: return false;
  }
}

bool LaunchDecodeStage(int k2, int k2d, int cb, const GemmArgs& gu, const GemmArgs& dn, int nyp, hipStream_t s) {
  switch (k2) {
    case 2: return LaunchDecodeStageRate2(cb, k2d, gu, dn, nyp, s);
    case 3: return LaunchDecodeStageRate3(cb, k2d, gu, dn, nyp, s);
    case 4: return LaunchDecodeStageRate4(cb, k2d, gu, dn, nyp, s);
    case 5: return LaunchDecodeStageRate5(cb, k2d, gu, dn, nyp, s);
    case 6: return LaunchDecodeStageRate6(cb, k2d, gu, dn, nyp, s);
    case 7: return LaunchDecodeStageRate7(cb, k2d, gu, dn, nyp, s);
    case 8: return LaunchDecodeStageRate8(cb, k2d, gu, dn, nyp, s);
    case 10: return LaunchDecodeStageRate10(cb, k2d, gu, dn, nyp, s);
    case 12: return LaunchDecodeStageRate12(cb, k2d, gu, dn, nyp, s);
    case 14: return LaunchDecodeStageRate14(cb, k2d, gu, dn, nyp, s);
    case 16: return LaunchDecodeStageRate16(cb, k2d, gu, dn, nyp, s);
    default: return false;
  }
}

bool LaunchGemmMulti(int k2, int cb, int nrb, const GemmMulti& gm, hipStream_t s) {
  switch (k2) {
    case 2: return LaunchGemmMultiRate2(cb, nrb, gm, s);
    case 3: return LaunchGemmMultiRate3(cb, nrb, gm, s);
    case 4: return LaunchGemmMultiRate4(cb, nrb, gm, s);
    case 5: return LaunchGemmMultiRate5(cb, nrb, gm, s);
    case 6: return LaunchGemmMultiRate6(cb, nrb, gm, s);
    case 7: return LaunchGemmMultiRate7(cb, nrb, gm, s);
    case 8: return LaunchGemmMultiRate8(cb, nrb, gm, s);
    case 10: return LaunchGemmMultiRate10(cb, nrb, gm, s);
    case 12: return LaunchGemmMultiRate12(cb, nrb, gm, s);
    case 14: return LaunchGemmMultiRate14(cb, nrb, gm, s);
    case 16: return LaunchGemmMultiRate16(cb, nrb, gm, s);
    default: return false;
  }
}

bool LaunchGemmTall(int k2, int cb, dim3 grid, const GemmArgs& g, hipStream_t s) {
  switch (k2) {
    case 2: return LaunchGemmTallRate2(cb, grid, g, s);
    case 3: return LaunchGemmTallRate3(cb, grid, g, s);
    case 4: return LaunchGemmTallRate4(cb, grid, g, s);
    case 5: return LaunchGemmTallRate5(cb, grid, g, s);
    case 6: return LaunchGemmTallRate6(cb, grid, g, s);
    case 7: return LaunchGemmTallRate7(cb, grid, g, s);
    case 8: return LaunchGemmTallRate8(cb, grid, g, s);
    case 10: return LaunchGemmTallRate10(cb, grid, g, s);
    case 12: return LaunchGemmTallRate12(cb, grid, g, s);
    case 14: return LaunchGemmTallRate14(cb, grid, g, s);
    case 16: return LaunchGemmTallRate16(cb, grid, g, s);
    default: return false;
  }
}

size_t LinearWorkspace(const LinearPlan& p, int I, int O, int M) {
  return AlignUp((size_t)M * I * 2, 256) + AlignUp((size_t)p.S * M * O * 4, 256);
}

// One group of linears over the same M rows: the grouped input transform, the GEMMs (dense
// row entries, no device tables; the jobs of one rate and codebook in one launch, up to
// kMaxMultiJobs a launch), the grouped output transform.  Jobs are checked by the caller;
// ws holds each job's transformed input and partials.
int RunGroup(const cx_exl3_job* jobs, int n, int M, char* ws, hipStream_t s) {
  XfInTable tin{};
  XfOutTable tout{};
  tin.n = tout.n = n;
  tin.M = tout.M = M;
  int in_items = 0, out_items = 0;
  std::vector<GemmArgs> gs(n);
  std::vector<LinearPlan> ps(n);
  for (int j = 0; j < n; ++j) {
    const cx_exl3_matrix* m = &jobs[j].m;
    const int I = m->in_features, O = m->out_features;
    const LinearPlan p = PlanLinear(I, O, M);
    __half* xp = reinterpret_cast<__half*>(ws);
    ws += AlignUp((size_t)M * I * 2, 256);
    float* part = reinterpret_cast<float*>(ws);
    ws += AlignUp((size_t)p.S * M * O * 4, 256);
    tin.job[j] = XfIn{jobs[j].x, reinterpret_cast<const __half*>(m->suh), xp, jobs[j].ldx, I,
                      jobs[j].x_dtype == CX_F32 ? 1 : 0, in_items};
    in_items += M * (I / 128);
    tout.job[j] = XfOut{part, (long long)M * O, reinterpret_cast<const __half*>(m->svh), jobs[j].y, p.S, jobs[j].ldy, O,
                        jobs[j].y_dtype == CX_F16 ? 1 : 0, out_items};
    out_items += M * (O / 128);
    GemmArgs& g = gs[j];
    g = GemmArgs{};
    g.plane[0] = GemmPlane{nullptr, xp, part, I, O, (long long)M * O, 0, nullptr};
    g.plane[1] = g.plane[0];
    g.entries = nullptr;
    g.n_entries = nullptr;
    g.n_entries_host = p.n_entries;
    g.A = p.A;
    g.ncp = p.ncp;
    g.S = p.S;
    g.mat = MatPtr{m->tiles, reinterpret_cast<const __half*>(m->suh), reinterpret_cast<const __half*>(m->svh)};
    g.rows = M;
    g.chunk = p.chunk;
    ps[j] = p;
  }
  hipLaunchKernelGGL(InputTransformKernel, dim3((unsigned)((in_items * 16 + 255) / 256)), dim3(256), 0, s, tin);
  // Every job has the same row count, so the same row-block count, and the same in-workgroup
  // K split (4): jobs of one rate and codebook can share a launch.
  std::vector<bool> done(n, false);
  for (int j = 0; j < n; ++j) {
    if (done[j]) continue;
    GemmMulti gm{};
    for (int i = j; i < n && gm.n < kMaxMultiJobs; ++i) {
      if (done[i] || jobs[i].m.k2 != jobs[j].m.k2 || jobs[i].m.codebook != jobs[j].m.codebook) continue;
      const LinearPlan& p = ps[i];
      gm.gx[gm.n] = p.ncp / (4 / p.ksw) * p.S;
      gm.g[gm.n] = gs[i];
      gm.start[gm.n + 1] = gm.start[gm.n] + gm.gx[gm.n] * p.n_entries;
      ++gm.n;
      done[i] = true;
    }
    if (gm.n == 1) {
      const LinearPlan& p = ps[j];
      const dim3 grid(p.ncp / (4 / p.ksw) * p.S, p.n_entries, 1);
      if (!LaunchGemm(jobs[j].m.k2, jobs[j].m.codebook, p.nrb, p.ksw, p.u, grid, gs[j], s)) return CX_E_UNSUPPORTED;
    } else if (!LaunchGemmMulti(jobs[j].m.k2, jobs[j].m.codebook, ps[j].nrb, gm, s)) {
      return CX_E_UNSUPPORTED;
    }
  }
  hipLaunchKernelGGL(OutputTransformKernel, dim3((unsigned)((out_items * 16 + 255) / 256)), dim3(256), 0, s, tout);
  return LaunchStatus();
}

int CheckJob(const cx_exl3_job& j) {
  int rc = CheckMatrix(&j.m);
  if (rc) return rc;
  if (!j.x || !j.y) return CX_E_ARG;
  if ((j.x_dtype != CX_F16 && j.x_dtype != CX_F32) || (j.y_dtype != CX_F16 && j.y_dtype != CX_F32)) return CX_E_ARG;
  // Rows are read and written in 16- / 32-byte pieces.
  if (j.ldx < j.m.in_features || j.ldy < j.m.out_features || j.ldx % 8 || j.ldy % 8) return CX_E_SHAPE;
  if (reinterpret_cast<uintptr_t>(j.x) % 16 || reinterpret_cast<uintptr_t>(j.y) % 16) return CX_E_SHAPE;
  return CX_OK;
}

size_t GroupWorkspace(const cx_exl3_job* jobs, int n, int M) {
  size_t t = 0;
  for (int j = 0; j < n; ++j) {
    const LinearPlan p = PlanLinear(jobs[j].m.in_features, jobs[j].m.out_features, M);
    t += LinearWorkspace(p, jobs[j].m.in_features, jobs[j].m.out_features, M);
  }
  return t;
}

}  // namespace cx

using namespace cx;

extern "C" {

size_t cx_exl3_tile_bytes(int32_t in_features, int32_t out_features, int32_t k2) {
  return (size_t)in_features * out_features * k2 / 16;
}

int cx_exl3_repack(const int16_t* trellis, int32_t in_features, int32_t out_features, int32_t k2, uint32_t* tiles,
                   cx_stream_t stream) {
  if (!trellis || !tiles) return CX_E_ARG;
  if (in_features <= 0 || out_features <= 0 || in_features % 128 || out_features % 128) return CX_E_SHAPE;
  if (!ValidK2(k2)) return CX_E_BITRATE;
  const int A = in_features / 16, B = out_features / 16, T = TileDwords(k2);
  const size_t total = (size_t)A * B * T;
  const int grid = (int)std::min<size_t>((total + 255) / 256, 65536);
  hipLaunchKernelGGL(RepackKernel, dim3(grid), dim3(256), 0, (hipStream_t)stream,
                     reinterpret_cast<const uint32_t*>(trellis), tiles, A, B, T);
  return LaunchStatus();
}

int cx_exl3_dequant(const cx_exl3_matrix* m, uint16_t* w_hat, cx_stream_t stream) {
  int rc = CheckMatrix(m);
  if (rc) return rc;
  if (!w_hat) return CX_E_ARG;
  const int A = m->in_features / 16, ncp = m->out_features / 32;
  const dim3 grid((A * ncp + 3) / 4);
  auto* w = reinterpret_cast<__half*>(w_hat);
  bool ok = DispatchK2Cb(m->k2, m->codebook, [&](auto k2c, auto cbc) {
    constexpr int K2 = decltype(k2c)::value, CB = decltype(cbc)::value;
    hipLaunchKernelGGL((DequantKernel<K2, CB>), grid, dim3(256), 0, (hipStream_t)stream, m->tiles, w, A, ncp);
  });
  if (!ok) return CX_E_BITRATE;
  return LaunchStatus();
}

int cx_exl3_input_transform(const cx_exl3_matrix* m, const void* x, int32_t x_dtype, int32_t ldx, int32_t M,
                            uint16_t* xh, cx_stream_t stream) {
  int rc = CheckMatrix(m);
  if (rc) return rc;
  if (!x || !xh) return CX_E_ARG;
  if (x_dtype != CX_F16 && x_dtype != CX_F32) return CX_E_ARG;
  if (M <= 0 || ldx < m->in_features || ldx % 8) return CX_E_SHAPE;
  XfInTable t{};
  t.n = 1;
  t.M = M;
  t.job[0] = XfIn{x, reinterpret_cast<const __half*>(m->suh), reinterpret_cast<__half*>(xh), ldx, m->in_features,
                  x_dtype == CX_F32 ? 1 : 0, 0};
  const long items = (long)M * (m->in_features / 128);
  hipLaunchKernelGGL(InputTransformKernel, dim3((unsigned)((items * 16 + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, t);
  return LaunchStatus();
}

int cx_exl3_output_transform(const cx_exl3_matrix* m, const float* y_raw, int32_t M, void* y, int32_t y_dtype,
                             cx_stream_t stream) {
  int rc = CheckMatrix(m);
  if (rc) return rc;
  if (!y_raw || !y) return CX_E_ARG;
  if (y_dtype != CX_F16 && y_dtype != CX_F32) return CX_E_ARG;
  if (M <= 0) return CX_E_SHAPE;
  const int O = m->out_features;
  XfOutTable t{};
  t.n = 1;
  t.M = M;
  t.job[0] = XfOut{y_raw, (long long)M * O, reinterpret_cast<const __half*>(m->svh), y, 1, O, O,
                   y_dtype == CX_F16 ? 1 : 0, 0};
  const long items = (long)M * (O / 128);
  hipLaunchKernelGGL(OutputTransformKernel, dim3((unsigned)((items * 16 + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, t);
  return LaunchStatus();
}

size_t cx_exl3_linear_workspace_size(const cx_exl3_matrix* m, int32_t M) {
  if (CheckMatrix(m) || M <= 0) return 0;
  const LinearPlan p = PlanLinear(m->in_features, m->out_features, M);
  return LinearWorkspace(p, m->in_features, m->out_features, M);
}

int cx_exl3_linear(const cx_exl3_matrix* m, const void* x, int32_t x_dtype, int32_t ldx, int32_t M,
                   const int32_t* row_offsets, int32_t n_sessions, void* y, int32_t y_dtype, void* workspace,
                   size_t workspace_bytes, cx_stream_t stream) {
  int rc = CheckMatrix(m);
  if (rc) return rc;
  if (!x || !y || !workspace) return CX_E_ARG;
  if (M <= 0 || !WorkspaceAligned(workspace)) return CX_E_SHAPE;
  if ((rc = RowOffsetsCheck(row_offsets, n_sessions, M))) return rc;
  const cx_exl3_job job{*m, x, x_dtype, ldx, y, y_dtype, m->out_features};
  if ((rc = CheckJob(job))) return rc;
  if (workspace_bytes < GroupWorkspace(&job, 1, M)) return CX_E_WORKSPACE;
  return RunGroup(&job, 1, M, static_cast<char*>(workspace), (hipStream_t)stream);
}

size_t cx_exl3_group_workspace_size(const cx_exl3_job* jobs, int32_t n_jobs, int32_t M) {
  if (!jobs || n_jobs <= 0 || n_jobs > kMaxGroupJobs || M <= 0) return 0;
  for (int j = 0; j < n_jobs; ++j)
    if (CheckMatrix(&jobs[j].m)) return 0;
  return GroupWorkspace(jobs, n_jobs, M);
}

int cx_exl3_group(const cx_exl3_job* jobs, int32_t n_jobs, int32_t M, const int32_t* row_offsets, int32_t n_sessions,
                  void* workspace, size_t workspace_bytes, cx_stream_t stream) {
  if (!jobs || !workspace) return CX_E_ARG;
  if (n_jobs <= 0 || n_jobs > kMaxGroupJobs || M <= 0 || !WorkspaceAligned(workspace)) return CX_E_SHAPE;
  int rc;
  for (int j = 0; j < n_jobs; ++j)
    if ((rc = CheckJob(jobs[j]))) return rc;
  if ((rc = RowOffsetsCheck(row_offsets, n_sessions, M))) return rc;
  if (workspace_bytes < GroupWorkspace(jobs, n_jobs, M)) return CX_E_WORKSPACE;
  return RunGroup(jobs, n_jobs, M, static_cast<char*>(workspace), (hipStream_t)stream);
}

const char* cx_version(void) { return "crucible-exl3-mi355x 0.1 (gfx950)"; }

}  // extern "C"
