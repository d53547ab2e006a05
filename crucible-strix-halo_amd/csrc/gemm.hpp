// Fused EXL3 decode + MFMA GEMM over compact activation rows (decode GEMV and prefill
// GEMM share this body; they differ in rows per wave and in how K is split).
//
// Tile layout in HBM ("column-pair-major"): the two tiles of column pair cp at k-tile
// a are adjacent, and consecutive k-tiles of one column pair are adjacent:
//   tile (a, b) -> tile index ((b / 2) * A + a) * 2 + (b % 2),  8K dwords per tile.
// A wave walks one column pair down K, so every wave's weight stream is contiguous.
//
// A step is two k-tiles of one column pair: 4 tiles, contiguous in HBM.  Each lane
// loads a contiguous slice of the step (coalesced, no lane reads a byte twice) into the
// wave's LDS slot; each lane then reads the window dwords of its two runs (run t of the
// step's first and second k-tile) back from LDS, decodes 16 weights and feeds two
// v_mfma_f32_16x16x32_f16 (columns c and c + 8 of its tile).  Activations are stored
// in the matching 32-row order (PermPos32), one 16-byte load per lane and 16-row block.
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
  float* y;            // fp32 outputs; row r at y + r * ldy (+ K segment * seg_stride)
  int ldx, ldy;
  long long seg_stride;
  int epi;  // 0: raw sums y_h; 1: output transform WHT128(y_h) * norm * svh (needs KSW = 1, S = 1)
};

struct GemmArgs {
  GemmPlane plane[2];
  const int4* entries;   // {matrix, row0, nrows, unused}
  const int* n_entries;  // device-side count (nullptr: use n_entries_host)
  int n_entries_host;
  int entry_base;        // blockIdx.y + entry_base indexes entries
  int A;    // k-tiles (I / 16)
  int ncp;  // column pairs (O / 32)
  int S;    // K segments across workgroups
};

template <int K2, int CB, int NRB, int KSW, int U>
__global__ void __launch_bounds__(256) Exl3GemmKernel(GemmArgs g) {
  constexpr int CPW = 4 / KSW;
  constexpr int T = TileDwords(K2);    // dwords per tile
  constexpr int SD = 4 * T;            // dwords per step
  constexpr int DPL = (SD + 63) / 64;  // dwords each lane loads per step
  constexpr int ND = WindowDwords(K2);
  __shared__ uint32_t stage[4][64 * DPL];
  const int n_entries = g.n_entries ? *g.n_entries : g.n_entries_host;
  const int ei = (int)blockIdx.y + g.entry_base;
  if (ei >= n_entries) return;
  const int4 ent = g.entries[ei];
  const GemmPlane& pl = g.plane[blockIdx.z];
  const int ncpg = g.ncp / CPW;
  const int cpg = blockIdx.x % ncpg, kseg = blockIdx.x / ncpg;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int cp = cpg * CPW + wave / KSW, ks = wave % KSW;
  const int nsplit = g.S * KSW, split = kseg * KSW + ks;
  const int A2 = g.A / 2;
  const int s0 = A2 * split / nsplit, s1 = A2 * (split + 1) / nsplit;
  const int steps = s1 - s0, a0 = 2 * s0;
  const int row0 = ent.y, nrows = ent.z;
  const MatPtr m = pl.mats[ent.x];

  const __amdgpu_buffer_rsrc_t rw = MakeRsrc(m.tiles + ((size_t)cp * g.A + a0) * 2 * T, (uint32_t)steps * SD * 4);
  const __amdgpu_buffer_rsrc_t rx = MakeRsrc(pl.x + (size_t)row0 * pl.ldx, (uint32_t)nrows * pl.ldx * 2);
  const LaneRun<K2> lr(lane);
  // LDS dword offsets of the lane's windows: run t of tile (k-tile j, column tile tau).
  uint32_t woff[2][ND];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int i = 0; i < ND; ++i) woff[j][i] = (uint32_t)((2 * j + lr.tile) * T + (lr.d0 + i) % T);
  const uint32_t loff = (uint32_t)lane * DPL * 4;
  uint32_t xoff[NRB];
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb) xoff[rb] = (uint32_t)(((rb * 16 + (lane & 15)) * pl.ldx + a0 * 16 + 8 * (lane >> 4)) * 2);
  uint32_t* slot = stage[wave];

  float4_t acc[NRB][2];
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb) acc[rb][0] = acc[rb][1] = float4_t{0.f, 0.f, 0.f, 0.f};

  auto load_w = [&](int s) { return BufLoadN<DPL>(rw, loff, (uint32_t)s * SD * 4); };
  auto load_x = [&](int s, int rb) { return BufLoad128(rx, xoff[rb], (uint32_t)s * 64); };
  auto step = [&](const Dwords<DPL>& w, const u32x4_t (&x)[NRB]) {
    // Stage the step in the wave's slot; LDS executes a wave's operations in order, so
    // the window reads below see these writes and the next step's writes follow them.
#pragma unroll
    for (int i = 0; i < DPL; ++i) slot[lane * DPL + i] = w.v[i];
    __builtin_amdgcn_wave_barrier();
    uint32_t v[2][3];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int i = 0; i < ND; ++i) v[j][i] = slot[woff[j][i]];
      if constexpr (ND == 2) v[j][2] = 0u;
    }
    __builtin_amdgcn_wave_barrier();
    half4_t lo0, hi0, lo1, hi1;
    DecodeRun<K2, CB>(v[0][0], v[0][1], v[0][2], lr.shift, lo0, hi0);
    DecodeRun<K2, CB>(v[1][0], v[1][1], v[1][2], lr.shift, lo1, hi1);
    const half8_t b0 = {lo0[0], lo0[1], lo0[2], lo0[3], lo1[0], lo1[1], lo1[2], lo1[3]};
    const half8_t b1 = {hi0[0], hi0[1], hi0[2], hi0[3], hi1[0], hi1[1], hi1[2], hi1[3]};
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
      const half8_t av = __builtin_bit_cast(half8_t, x[rb]);
      acc[rb][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, b0, acc[rb][0], 0, 0, 0);
      acc[rb][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, b1, acc[rb][1], 0, 0, 0);
    }
  };

  // Register double buffering: the loads of the next U steps are in flight while the
  // current U steps are decoded; then the remaining (< U) steps one at a time.
  Dwords<DPL> wa[U], wb[U];
  u32x4_t xa[U][NRB], xb[U][NRB];
  auto load_group = [&](Dwords<DPL> (&w)[U], u32x4_t (&x)[U][NRB], int sb) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      w[u] = load_w(sb + u);
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb) x[u][rb] = load_x(sb + u, rb);
    }
  };
  int s = 0;
  if (steps >= U) load_group(wa, xa, 0);
  while (s + U <= steps) {
    const bool more = s + 2 * U <= steps;
    if (more) load_group(wb, xb, s + U);
#pragma unroll
    for (int u = 0; u < U; ++u) step(wa[u], xa[u]);
    s += U;
    if (!more) break;
    const bool more2 = s + 2 * U <= steps;
    if (more2) load_group(wa, xa, s + U);
#pragma unroll
    for (int u = 0; u < U; ++u) step(wb[u], xb[u]);
    s += U;
    if (!more2) break;
  }
  for (; s < steps; ++s) {
    const Dwords<DPL> w1 = load_w(s);
    u32x4_t x1[NRB];
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) x1[rb] = load_x(s, rb);
    step(w1, x1);
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
  if constexpr (KSW == 1) {
    if (pl.epi == 1) {
      // The workgroup holds columns [128 cpg, 128 cpg + 128): one whole output Hadamard
      // block.  Stage y_h in LDS, then WHT128 * norm * svh per row (engine LinOutBlock,
      // engine/exl3/exl3.h:69-82), fp32.
      __shared__ float ebuf[16 * NRB][132];
      const int cl = wave * 32 + ((lane & 15) >> 3) * 16 + (lane & 7);
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = rb * 16 + 4 * (lane >> 4) + i;
          ebuf[r][cl] = acc[rb][0][i];
          ebuf[r][cl + 8] = acc[rb][1][i];
        }
      __syncthreads();
      const int j = threadIdx.x & 15, c0 = cpg * 128 + 8 * j;
      float sv[8];
      LoadH8(m.svh + c0, sv);
      for (int r = threadIdx.x >> 4; r < nrows; r += 16) {
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = 0.f + ebuf[r][8 * j + i];
        Wht128x8(v);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] *= kHadNorm * sv[i];
        StoreF8(pl.y + (size_t)(row0 + r) * pl.ldy + c0, v);
      }
      return;
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
