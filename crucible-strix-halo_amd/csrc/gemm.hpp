// Fused EXL3 decode + MFMA GEMM over compact activation rows (decode GEMV and prefill
// GEMM share this body; they differ in rows per wave and in how K is split).
//
// Tile layout in HBM ("column-pair-major"): the two tiles of column pair cp at k-tile
// a are adjacent, and consecutive k-tiles of one column pair are adjacent:
//   tile (a, b) -> tile index ((b / 2) * A + a) * 2 + (b % 2),  8K dwords per tile.
// A wave walks one column pair down K, so every wave's weight stream is contiguous.
//
// Work item (one 256-thread workgroup = 4 waves):
//   blockIdx.x -> (column-pair group, K segment), blockIdx.y -> row entry
//   {matrix, first row, rows}, blockIdx.z -> plane (e.g. gate / up).
//   Each wave owns one column pair and one K split; KSW waves split a column pair's K
//   inside the workgroup and are summed in LDS in fixed wave order.  Rows: NRB blocks
//   of 16 rows per wave, all fed by the same decoded weights.
#pragma once

#include "decode.hpp"

namespace cx {

struct MatPtr {
  const uint32_t* tiles;  // column-pair-major tiles
  const __half* suh;      // [I] input scales
  const __half* svh;      // [O] output scales
};

struct GemmPlane {
  const MatPtr* mats;  // indexed by the entry's matrix id
  const __half* x;     // MFMA-ordered activations; row r at x + r * ldx
  float* y;            // fp32 raw outputs; row r at y + r * ldy (+ K segment * seg_stride)
  int ldx, ldy;
  long long seg_stride;
};

struct GemmArgs {
  GemmPlane plane[2];
  const int4* entries;   // {matrix, row0, nrows, unused}
  const int* n_entries;  // device-side count (nullptr: use n_entries_host)
  int n_entries_host;
  int A;    // k-tiles (I / 16)
  int ncp;  // column pairs (O / 32)
  int S;    // K segments across workgroups
};

template <int K2, int CB, int NRB, int KSW, int U>
__global__ void __launch_bounds__(256) Exl3GemmKernel(GemmArgs g) {
  constexpr int CPW = 4 / KSW;
  constexpr int T = TileDwords(K2);
  constexpr int ND = WindowDwords(K2);
  const int n_entries = g.n_entries ? *g.n_entries : g.n_entries_host;
  if ((int)blockIdx.y >= n_entries) return;
  const int4 ent = g.entries[blockIdx.y];
  const GemmPlane& pl = g.plane[blockIdx.z];
  const int ncpg = g.ncp / CPW;
  const int cpg = blockIdx.x % ncpg, kseg = blockIdx.x / ncpg;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int cp = cpg * CPW + wave / KSW, ks = wave % KSW;
  const int nsplit = g.S * KSW, split = kseg * KSW + ks;
  const int a0 = g.A * split / nsplit, a1 = g.A * (split + 1) / nsplit;
  const int steps = a1 - a0;
  const int row0 = ent.y, nrows = ent.z;
  const MatPtr m = pl.mats[ent.x];

  const __amdgpu_buffer_rsrc_t rw = MakeRsrc(m.tiles + ((size_t)cp * g.A + a0) * 2 * T, (uint32_t)steps * 2 * T * 4);
  const __amdgpu_buffer_rsrc_t rx = MakeRsrc(pl.x + (size_t)row0 * pl.ldx, (uint32_t)nrows * pl.ldx * 2);
  const LaneRun<K2> lr(lane);
  uint32_t woff[ND];
#pragma unroll
  for (int i = 0; i < ND; ++i) woff[i] = lr.ByteOffset(i);
  uint32_t xoff[NRB];
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb) xoff[rb] = (uint32_t)(((rb * 16 + (lane & 15)) * pl.ldx + a0 * 16 + 4 * (lane >> 4)) * 2);

  float4_t acc[NRB][2];
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb) acc[rb][0] = acc[rb][1] = float4_t{0.f, 0.f, 0.f, 0.f};

  uint32_t wa[U][ND], wb[U][ND];
  u32x2_t xa[U][NRB], xb[U][NRB];
  auto load = [&](uint32_t (&w)[U][ND], u32x2_t (&x)[U][NRB], int s0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t sw = (uint32_t)(s0 + u) * 2 * T * 4, sx = (uint32_t)(s0 + u) * 32;
#pragma unroll
      for (int i = 0; i < ND; ++i) w[u][i] = BufLoad32(rw, woff[i], sw);
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb) x[u][rb] = BufLoad64(rx, xoff[rb], sx);
    }
  };
  auto compute = [&](uint32_t (&w)[U][ND], u32x2_t (&x)[U][NRB]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      half4_t blo, bhi;
      DecodeRun<K2, CB>(w[u][0], w[u][1], ND > 2 ? w[u][ND - 1] : 0u, lr.shift, blo, bhi);
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb) {
        const half4_t av = __builtin_bit_cast(half4_t, x[u][rb]);
        acc[rb][0] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, blo, acc[rb][0], 0, 0, 0);
        acc[rb][1] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, bhi, acc[rb][1], 0, 0, 0);
      }
    }
  };
  // Two register sets: decode one group of U steps while the next is in flight, then
  // the remaining (< U) steps one at a time.
  int s = 0;
  if (steps >= U) load(wa, xa, 0);
  while (s + U <= steps) {
    const bool more = s + 2 * U <= steps;
    if (more) load(wb, xb, s + U);
    compute(wa, xa);
    s += U;
    if (!more) break;
    const bool more2 = s + 2 * U <= steps;
    if (more2) load(wa, xa, s + U);
    compute(wb, xb);
    s += U;
    if (!more2) break;
  }
  for (; s < steps; ++s) {
    uint32_t w1[1][ND];
    u32x2_t x1[1][NRB];
    const uint32_t sw = (uint32_t)s * 2 * T * 4, sx = (uint32_t)s * 32;
#pragma unroll
    for (int i = 0; i < ND; ++i) w1[0][i] = BufLoad32(rw, woff[i], sw);
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) x1[0][rb] = BufLoad64(rx, xoff[rb], sx);
    half4_t blo, bhi;
    DecodeRun<K2, CB>(w1[0][0], w1[0][1], ND > 2 ? w1[0][ND - 1] : 0u, lr.shift, blo, bhi);
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
      const half4_t av = __builtin_bit_cast(half4_t, x1[0][rb]);
      acc[rb][0] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, blo, acc[rb][0], 0, 0, 0);
      acc[rb][1] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, bhi, acc[rb][1], 0, 0, 0);
    }
  }

  if constexpr (KSW > 1) {
    // Fixed-order reduction of the K splits of each column pair.
    __shared__ float4_t red[CPW][KSW - 1][NRB * 2][64];
    const int c = wave / KSW;
    if (ks > 0) {
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb) {
        red[c][ks - 1][rb * 2][lane] = acc[rb][0];
        red[c][ks - 1][rb * 2 + 1][lane] = acc[rb][1];
      }
    }
    __syncthreads();
    if (ks > 0) return;
#pragma unroll
    for (int k = 0; k < KSW - 1; ++k)
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb) {
        acc[rb][0] += red[c][k][rb * 2][lane];
        acc[rb][1] += red[c][k][rb * 2 + 1][lane];
      }
  }
  float* y = pl.y + (size_t)kseg * pl.seg_stride;
  const int col = (2 * cp + ((lane & 15) >> 3)) * 16 + (lane & 7);
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = rb * 16 + 4 * (lane >> 4) + i;
      if (r < nrows) {
        float* yr = y + (size_t)(row0 + r) * pl.ldy;
        yr[col] = acc[rb][0][i];
        yr[col + 8] = acc[rb][1][i];
      }
    }
}

}  // namespace cx
