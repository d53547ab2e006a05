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

#include <utility>

#include "decode.hpp"


namespace cx {

// Per-wave LDS staging of one step.  At most rates dword d of the step lives at
// d + 2 (d / 32), so the two column tiles of a step (T = 8K dwords apart) do not map their
// equal dword offsets onto one bank, and 8-byte lane slices stay 8-byte aligned.  At
// K2 = 6, 10 and 12 (3, 5, 6 bpw) the windows of a half wave spread over the banks better
// without padding: a model of the 32-bank mapping of the window reads and staging writes
// gives 4 / 12 / 12 extra cycles per step unpadded against 8 / 36 / 36 padded (the measured
// conflict cycles per LDS instruction of the 6-bpw decode GEMM were 3.9 padded), and the
// same count as now (0 at 4 bpw) at every other rate.
template <int K2>
__host__ __device__ constexpr int StagePad(int d) {
  return K2 == 6 || K2 == 10 || K2 == 12 ? d : d + 2 * (d / 32);
}
template <int K2, int DPL>
__host__ __device__ constexpr int StageDwords() { return StagePad<K2>(64 * DPL) + 2; }
// Writes a lane's DPL dwords of a step into the staging slot.  Slices of 1, 2 or 4 dwords
// never straddle a 32-dword boundary; 3-dword slices are written one by one.
template <int K2, int DPL>
__device__ __forceinline__ void StageWrite(uint32_t* slot, int lane, const uint32_t* v) {
  if constexpr (DPL == 3) {
#pragma unroll
    for (int i = 0; i < 3; ++i) slot[StagePad<K2>(3 * lane + i)] = v[i];
  } else {
    const int o = StagePad<K2>(lane * DPL);
#pragma unroll
    for (int i = 0; i < DPL; ++i) slot[o + i] = v[i];
  }
}

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
  // 0: raw sums y_h; 1: output transform WHT128(y_h) * norm * svh, fp32 (needs KSW = 1,
  // S = 1); 2: the same transform stored as fp16 with a power-of-two scale per (row,
  // 128-column block): y as __half rows of ldy halves, the scales in ysc [row][O / 128].
  int epi;
  float* ysc;
};

// Stores one row's 8 output values of a 128-column block after the output transform; the
// 16 lanes of a DPP row hold the block (epi 1 or 2 of GemmPlane).  fp16 form: the block is
// divided by 2^sh, sh = floor(log2 max|v|) - 14 (exact: a power of two), so its largest
// magnitude lies in [2^14, 2^15) and every value is rounded to fp16 once, with the full
// fp16 precision and no overflow; a block holding inf or NaN is stored unscaled.
__device__ __forceinline__ void StoreBlockRow(const GemmPlane& pl, size_t row, int c0, int O, const float v[8]) {
  if (pl.epi == 1) {
    StoreF8(pl.y + row * pl.ldy + c0, v);
    return;
  }
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(v[i]));
  m = fmaxf(m, Dpp<kDppQuadSwap1>(m));
  m = fmaxf(m, Dpp<kDppQuadSwap2>(m));
  m = fmaxf(m, Dpp<kDppRowHalfMirror>(m));
  m = fmaxf(m, Dpp<kDppRowMirror>(m));
  int sh = 0;
  if (m > 0.f && m <= 3.4e38f) sh = min(max((int)((__float_as_uint(m) >> 23) & 0xff) - 127 - 14, -100), 100);
  const float inv = ldexpf(1.f, -sh);
  uint32_t h[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) h[k] = __builtin_bit_cast(uint32_t, __floats2half2_rn(v[2 * k] * inv, v[2 * k + 1] * inv));
  __half* d = reinterpret_cast<__half*>(pl.y) + row * pl.ldy + c0;
  *reinterpret_cast<uint4*>(d) = make_uint4(h[0], h[1], h[2], h[3]);
  if ((threadIdx.x & 15) == 0) pl.ysc[row * (O / 128) + c0 / 128] = ldexpf(1.f, sh);
}

// Counters of the decode stage launch, one per 128-byte line (the waiting workgroups' polls
// of one entry do not share a line with another entry's arrivals).
constexpr int kStageCtrStride = 32;

struct GemmArgs {
  GemmPlane plane[2];
  const int4* entries;   // {matrix, row0, nrows, unused}; nullptr: dense rows (below)
  const int* n_entries;  // device-side count (nullptr: use n_entries_host)
  int n_entries_host;
  int entry_base;        // blockIdx.y + entry_base indexes entries
  int A;    // k-tiles (I / 16)
  int ncp;  // column pairs (O / 32)
  int S;    // K segments across workgroups
  // Dense rows (entries == nullptr): entry e is rows [e chunk, min(M, (e + 1) chunk)) of
  // the single matrix `mat` (no device-side tables).
  MatPtr mat;
  int rows, chunk;
  // Activation gather (nullable): compact row p < xmap_n reads activation row xmap[p]
  // (rows at or above xmap_n read row p).  Decode GEMM only.
  const int* xmap;
  int xmap_n;
  // Gate/up GEMMs with the mid fused in (Exl3GemmPrefillKernel<..., MID = true>, and the
  // tall GEMM with tall_seq_mid): the down projection's packed input scales [E + 1][O]
  // and its input rows xd [rows][O] fp16 (MFMA row order), row p at xd + p * O.  The
  // decode down GEMM's prologue mid (MIDX) reads mid_suh too.
  const __half* mid_suh;
  __half* mid_xd;
  // Decode down GEMM with the mid in its prologue (Exl3GemmKernel<..., MIDX = true>): the
  // gate/up raw sums [rows][I] fp32 (compact row order) and the packed gate / up output
  // scales [E + 1][I]; the down input scales are mid_suh.  The workgroup transforms its
  // entry's rows into LDS and never reads plane.x.
  const float* mid_yg;
  const float* mid_yu;
  const __half* mid_svg;
  const __half* mid_svu;
  // Tall gate/up GEMM with the mid fused (grid z = 1): a workgroup runs plane 0 (gate),
  // parks its raw sums in plane 0's y, runs plane 1 (up) and computes the mid of its rows
  // into mid_xd from the parked gate sums and the up sums in registers.
  int tall_seq_mid;
  // Decode stage launch (Exl3DecodeStageKernel): per row entry a counter, zero at launch;
  // each gate/up workgroup adds 1 after its sums are stored (stage_arrivals of them), the
  // last one computes the entry's mid and adds 1 more; the entry's down workgroups wait for
  // stage_arrivals + 1.
  int* stage_ctr;  // entry e's counter at stage_ctr[e * kStageCtrStride]
  int stage_arrivals;
};

// The mid of one row's 128-column block on 16 lanes (lane j: columns c0 + 8j..8j+7): the
// gate and up output transforms of the raw sums gv, uv (fp32: WHT128 * norm * svh), then
// RoundH(RoundH(SiLU(g) * u) * suh_down), WHT128, * norm -> fp16 in MFMA row order at dst
// (the block's first half).  engine/layers/moe_rows.h:543-566.
// The values before the fp16 store (v times kHadNorm * WhtLaneSign() is the stored row).
__device__ __forceinline__ void MidValues(float gv[8], float uv[8], const __half* svg_p, const __half* svu_p,
                                          const __half* sud_p, float v[8]) {
  float svg[8], svu[8], sud[8];
  LoadH8(svg_p, svg);
  LoadH8(svu_p, svu);
  LoadH8(sud_p, sud);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    gv[i] = 0.f + gv[i];
    uv[i] = 0.f + uv[i];
  }
  Wht128x8Signed(gv);
  Wht128x8Signed(uv);
  const float sg = WhtLaneSign();
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float a = gv[i] * (sg * (kHadNorm * svg[i]));
    const float b = uv[i] * (sg * (kHadNorm * svu[i]));
    v[i] = RoundH(RoundH(SiLU(a) * b) * sud[i]);
  }
  Wht128x8Signed(v);
}
__device__ __forceinline__ void MidBlock(float gv[8], float uv[8], const __half* svg_p, const __half* svu_p,
                                         const __half* sud_p, __half* dst) {
  float v[8];
  MidValues(gv, uv, svg_p, svu_p, sud_p, v);
  StorePerm32x8(dst, v, kHadNorm * WhtLaneSign());
}

// Gate/up role of the decode stage launch, after the workgroup stored its raw sums (plain
// stores): every wave waits for its stores' acknowledgement, then one thread counts the
// workgroup in the entry's counter (agent scope).  The last of the entry's stage_arrivals
// workgroups computes the entry's mid (rows [row0, row0 + nrows), expert e), reading the
// gate / up sums with the L2 policy (all written on this XCD), writes the down input rows
// (mid_xd, MFMA row order), waits for their acknowledgement and counts once more.  The same
// arithmetic as MoeMidKernel (MidBlock), so the rows are bitwise equal.
__device__ __forceinline__ void StagePublishMid(const GemmArgs& g, int ei, int e, int row0, int nrows) {
  __shared__ int s_last;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0)
    s_last = __hip_atomic_fetch_add(g.stage_ctr + ei * kStageCtrStride, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
             g.stage_arrivals - 1;
  __syncthreads();
  if (!s_last) return;
  const int I = g.ncp * 32, nb = I / 128, j = threadIdx.x & 15;
  const __amdgpu_buffer_rsrc_t rg = MakeRsrc(g.plane[0].y, 0x7fffffffu), ru = MakeRsrc(g.plane[1].y, 0x7fffffffu);
  const __half* svg = g.mid_svg + (size_t)e * I;
  const __half* svu = g.mid_svu + (size_t)e * I;
  const __half* sud = g.mid_suh + (size_t)e * I;
  for (int it = (int)threadIdx.x >> 4; it < nrows * nb; it += 16) {  // uniform per 16 lanes
    const int r = it / nb, blk = it % nb, c0 = blk * 128 + 8 * j;
    const size_t p = (size_t)(row0 + r);
    const uint32_t og = (uint32_t)((p * g.plane[0].ldy + c0) * 4), ou = (uint32_t)((p * g.plane[1].ldy + c0) * 4);
    float gv[8], uv[8];
    const u32x4_t g0 = BufLoad128L2(rg, og, 0), g1 = BufLoad128L2(rg, og + 16, 0);
    const u32x4_t u0 = BufLoad128L2(ru, ou, 0), u1 = BufLoad128L2(ru, ou + 16, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      gv[i] = __uint_as_float(g0[i]);
      gv[4 + i] = __uint_as_float(g1[i]);
      uv[i] = __uint_as_float(u0[i]);
      uv[4 + i] = __uint_as_float(u1[i]);
    }
    MidBlock(gv, uv, svg + c0, svu + c0, sud + c0, g.mid_xd + p * I + blk * 128);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_fetch_add(g.stage_ctr + ei * kStageCtrStride, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wave-uniform load through the scalar cache (device tables written by earlier launches).
template <typename T>
__device__ __forceinline__ T ScalarLoad(const T* p) {
  static_assert(sizeof(T) % 4 == 0, "dword-sized objects only");
  typedef const __attribute__((address_space(4))) uint32_t* ConstDwords;
  const ConstDwords q = (ConstDwords)(p);
  struct W {
    uint32_t w[sizeof(T) / 4];
  } v;
#pragma unroll
  for (unsigned i = 0; i < sizeof(T) / 4; ++i) v.w[i] = q[i];
  return __builtin_bit_cast(T, v);
}

// Row entry ei: from the device table, or the dense split of rows.
__device__ __forceinline__ int4 EntryOf(const GemmArgs& g, int ei) {
  if (g.entries) return ScalarLoad(g.entries + ei);
  const int r0 = ei * g.chunk;
  return make_int4(0, r0, min(g.chunk, g.rows - r0), 0);
}
__device__ __forceinline__ MatPtr MatOf(const GemmArgs& g, const GemmPlane& pl, int id) {
  return g.entries ? ScalarLoad(pl.mats + id) : g.mat;
}

// One wave streams `steps` steps of one column pair (tiles from `tiles`, already offset
// to the wave's first step) against NRB 16-row blocks of MFMA-ordered activations
// (`x` at the first row, 32 k-columns per step starting at step 0) into acc.
// `x` is the activation base at the wave's first k column; xrow[rb] is the byte offset of
// the lane's row of block rb (at or beyond x_bytes: a row of zeros, no memory access).
// XL: the activations come from LDS instead (xl at the lane's row and k-group, 16-byte
// units, 4 per step); x, x_bytes and xrow are then unused, and fill() (which writes them,
// all waves of the workgroup together) runs after the first weight loads are issued, so
// their latency overlaps it.
struct NoFill {
  __device__ void operator()() const {}
};
// XL2: activation loads with the L2 policy (BufLoad128L2: rows published by other
// workgroups of the same XCD during the launch), and fill() (the wait for them) runs
// between the first weight loads and the first activation loads.
template <int K2, int CB, int NRB, int U, bool XL = false, typename Fill = NoFill, bool XL2 = false>
__device__ __forceinline__ void StreamColumnPair(const uint32_t* tiles, int steps, const __half* x, uint32_t x_bytes,
                                                 const uint32_t (&xrow)[NRB], uint32_t* slot, int lane,
                                                 float4_t (&acc)[NRB][2], const u32x4_t* xl = nullptr,
                                                 Fill&& fill = Fill{}) {
  constexpr int T = TileDwords(K2);    // dwords per tile
  constexpr int SD = 4 * T;            // dwords per step
  constexpr int DPL = (SD + 63) / 64;  // dwords each lane loads per step
  constexpr int ND = WindowDwords(K2);
  const __amdgpu_buffer_rsrc_t rw = MakeRsrc(tiles, (uint32_t)steps * SD * 4);
  const __amdgpu_buffer_rsrc_t rx = MakeRsrc(x, x_bytes);
  const LaneRun<K2> lr(lane);
  // LDS dword offsets of the lane's windows: run t of tile (k-tile j, column tile tau).
  uint32_t woff[2][ND];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int i = 0; i < ND; ++i) woff[j][i] = (uint32_t)StagePad<K2>((2 * j + lr.tile) * T + (lr.d0 + i) % T);
  const uint32_t loff = (uint32_t)lane * DPL * 4;
  uint32_t xoff[NRB];
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb) xoff[rb] = xrow[rb] + (uint32_t)(16 * (lane >> 4));

#pragma unroll
  for (int rb = 0; rb < NRB; ++rb) acc[rb][0] = acc[rb][1] = float4_t{0.f, 0.f, 0.f, 0.f};

  auto load_w = [&](int s) { return BufLoadN<DPL>(rw, loff, (uint32_t)s * SD * 4); };
  auto load_x = [&](int s, int rb) {
    if constexpr (XL)
      return xl[s * 4];
    else if constexpr (XL2)
      return BufLoad128L2(rx, xoff[rb], (uint32_t)s * 64);
    else
      return BufLoad128(rx, xoff[rb], (uint32_t)s * 64);
  };
  auto step = [&](const Dwords<DPL>& w, const u32x4_t (&xv)[NRB]) {
    // Stage the step in the wave's slot; LDS executes a wave's operations in order, so
    // the window reads below see these writes and the next step's writes follow them.
    StageWrite<K2, DPL>(slot, lane, w.v);
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
      const half8_t av = __builtin_bit_cast(half8_t, xv[rb]);
      acc[rb][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, b0, acc[rb][0], 0, 0, 0);
      acc[rb][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, b1, acc[rb][1], 0, 0, 0);
    }
  };

  // Register double buffering: the loads of the next U steps are in flight while the
  // current U steps are decoded.  Loads are issued unconditionally, also past the last
  // step: weight loads there fall outside the buffer resource (no memory access, zeros)
  // and their results are not used.  Conditional loads would make the compiler wait for
  // every outstanding load at each group (vmcnt(0)), since it cannot count them on every
  // path.
  Dwords<DPL> wa[U], wb[U];
  u32x4_t xa[U][NRB], xb[U][NRB];
  auto load_group = [&](Dwords<DPL> (&w)[U], u32x4_t (&xg)[U][NRB], int sb) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      w[u] = load_w(sb + u);
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb) xg[u][rb] = load_x(sb + u, rb);
    }
  };
  if constexpr (XL || XL2) {
#pragma unroll
    for (int u = 0; u < U; ++u) wa[u] = load_w(u);
    fill();
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb) xa[u][rb] = load_x(u, rb);
  } else {
    load_group(wa, xa, 0);
  }
  for (int s = 0; s < steps; s += 2 * U) {
    load_group(wb, xb, s + U);
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (s + u < steps) step(wa[u], xa[u]);
    load_group(wa, xa, s + 2 * U);
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (s + U + u < steps) step(wb[u], xb[u]);
  }
}

// One 16-row block per wave (decode) at up to 4 bpw asks for 8 waves per SIMD (64
// registers, no spills there): the decode is VALU-bound and the extra waves hide the
// LDS round trip of each step.
//
// MIDX (one row block, no K split): the down projection of the decode MoE layer with the
// mid computed in the prologue.  The workgroup transforms its entry's rows (at most 16)
// from the gate/up sums into LDS in MFMA row order (dynamic LDS: 16 rows of I + 8 halves;
// the pad keeps the 16 rows of a k-group in distinct banks), and the K loop reads them
// there; rows past the entry read its last row (their sums are discarded).  Each of the
// entry's column-block workgroups computes the mid again: a few hundred VALU per row
// block instead of a launch and the down input's round trip through memory.
//
// STAGE (one role of Exl3DecodeStageKernel, gate/up and down of a decode call in one
// launch): 1 = gate/up, publishing its sums through the entry's counter and, in the last
// workgroup of the entry, computing the mid; 2 = down, waiting for the entry's mid rows and
// reading them with the L2 policy.  (bx, by, bz) are the workgroup's coordinates in the
// grid of the GEMM's own launch.
template <int K2, int CB, int NRB, int KSW, int U, bool MIDX, int STAGE>
__device__ __forceinline__ void GemmBody(const GemmArgs& g, int bx, int by, int bz) {
  static_assert(!MIDX || (NRB == 1 && KSW == 1), "the prologue mid is for the decode down projection");
  constexpr int CPW = 4 / KSW;
  constexpr int T = TileDwords(K2);
  constexpr int DPL = (4 * T + 63) / 64;
  __shared__ uint32_t stage[4][StageDwords<K2, DPL>()];
  // Device tables: entries past the last real one have 0 rows (the grid never exceeds the
  // table), so a wave's first weight load waits on two dependent scalar loads (entry,
  // matrix pointers) and no entry count.
  const int ei = by + g.entry_base;
  const int4 ent = EntryOf(g, ei);
  if (g.entries ? ent.z <= 0 : ei >= g.n_entries_host) return;
  const GemmPlane& pl = g.plane[bz];
  const int ncpg = g.ncp / CPW;
  const int cpg = bx % ncpg, kseg = bx / ncpg;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int cp = cpg * CPW + wave / KSW, ks = wave % KSW;
  const int nsplit = g.S * KSW, split = kseg * KSW + ks;
  const int A2 = g.A / 2;
  const int s0 = A2 * split / nsplit, s1 = A2 * (split + 1) / nsplit;
  const int steps = s1 - s0, a0 = 2 * s0;
  const int row0 = ent.y, nrows = ent.z;
  const MatPtr m = MatOf(g, pl, ent.x);
  // Byte offset of each lane's activation row (rows past the entry: beyond the buffer).
  uint32_t xrow[NRB];
  const __half* xb;
  uint32_t xbytes;
  if (g.xmap) {
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
      const int r = rb * 16 + (lane & 15), p = row0 + r;
      const int src = p < g.xmap_n ? g.xmap[min(p, g.xmap_n - 1)] : p;
      xrow[rb] = r < nrows ? (uint32_t)src * pl.ldx * 2 : 0xF0000000u;
    }
    xb = pl.x + a0 * 16;
    xbytes = 0xE0000000u;
  } else {
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) xrow[rb] = (uint32_t)((rb * 16 + (lane & 15)) * pl.ldx * 2);
    xb = pl.x + (size_t)row0 * pl.ldx + a0 * 16;
    xbytes = (uint32_t)nrows * pl.ldx * 2;
  }
  float4_t acc[NRB][2];
  extern __shared__ u32x4_t xmid[];  // MIDX only (no dynamic LDS otherwise)
  if constexpr (MIDX) {
    const int I = g.A * 16, nb = I / 128, rs = I / 8 + 1;  // 16-byte units per LDS row
    auto fill = [&]() {
      const int e = ent.x, j = lane & 15;
      const __half* svg = g.mid_svg + (size_t)e * I;
      const __half* svu = g.mid_svu + (size_t)e * I;
      const __half* sud = g.mid_suh + (size_t)e * I;
      for (int it = (int)threadIdx.x >> 4; it < nrows * nb; it += 16) {  // uniform per 16 lanes
        const int r = it / nb, blk = it % nb, c0 = blk * 128 + 8 * j;
        const size_t p = (size_t)(row0 + r);
        float gv[8], uv[8], v[8];
        LoadF8(g.mid_yg + p * I + c0, gv);
        LoadF8(g.mid_yu + p * I + c0, uv);
        MidValues(gv, uv, svg + c0, svu + c0, sud + c0, v);
        int h[4];
        Perm32x8Chunk(v, kHadNorm * WhtLaneSign(), h);
        xmid[r * rs + blk * 16 + 4 * (j >> 2) + (j & 3)] =
            u32x4_t{(uint32_t)h[0], (uint32_t)h[1], (uint32_t)h[2], (uint32_t)h[3]};
      }
      __syncthreads();
    };
    const int rr = min(lane & 15, nrows - 1);
    StreamColumnPair<K2, CB, NRB, U, true>(m.tiles + ((size_t)cp * g.A + a0) * 2 * T, steps, xb, xbytes, xrow,
                                           stage[wave], lane, acc, xmid + rr * rs + 2 * a0 + (lane >> 4), fill);
  } else if constexpr (STAGE == 2) {
    // The entry's mid rows are ready once its counter reaches arrivals + 1.  Bounded: every
    // gate/up workgroup precedes every down workgroup in dispatch order and never waits, so
    // the count arrives; the bound only guarantees that every wave exits.
    // The wait runs after the first weight loads are issued, so their latency overlaps it.
    __shared__ int s_ready;
    auto wait = [&]() {
      if (threadIdx.x == 0) {
        int it = 0;
        while (__hip_atomic_load(g.stage_ctr + ei * kStageCtrStride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) <
                   g.stage_arrivals + 1 &&
               ++it < (1 << 20))
          __builtin_amdgcn_s_sleep(16);
        s_ready = it < (1 << 20);
      }
      __syncthreads();
    };
    StreamColumnPair<K2, CB, NRB, U, false, decltype(wait)&, true>(m.tiles + ((size_t)cp * g.A + a0) * 2 * T, steps,
                                                                    xb, xbytes, xrow, stage[wave], lane, acc, nullptr,
                                                                    wait);
    if (!s_ready) return;  // never taken when the dispatch order holds (the output rows stay unwritten)
  } else {
    StreamColumnPair<K2, CB, NRB, U>(m.tiles + ((size_t)cp * g.A + a0) * 2 * T, steps, xb, xbytes, xrow, stage[wave],
                                     lane, acc);
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
    if constexpr (STAGE == 1) {
      static_assert(CPW == 1 && NRB == 1, "one storing wave per gate/up workgroup");
      if (ks == 0) {
#pragma unroll
        for (int k = 0; k < KSW - 1; ++k) {
          acc[0][0] += red[c][k][0][lane];
          acc[0][1] += red[c][k][1][lane];
        }
        float* yr0 = pl.y + (size_t)kseg * pl.seg_stride;
        const int col = (2 * cp + ((lane & 15) >> 3)) * 16 + (lane & 7);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = 4 * (lane >> 4) + i;
          if (r < nrows) {
            float* yr = yr0 + (size_t)(row0 + r) * pl.ldy;
            yr[col] = acc[0][0][i];
            yr[col + 8] = acc[0][1][i];
          }
        }
      }
      StagePublishMid(g, ei, ent.x, row0, nrows);
      return;
    }
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
      // engine/exl3/exl3.h:69-82), fp32.  MIDX: in the mid rows' LDS, once every wave is
      // done with them (8.4 KB of the 16.6 KB; 8 workgroups per CU still fit).
      float(*ebuf)[132];
      if constexpr (MIDX) {
        __syncthreads();
        ebuf = reinterpret_cast<float(*)[132]>(xmid);
      } else {
        __shared__ float ebuf_s[16 * NRB][132];
        ebuf = ebuf_s;
      }
      // The output scales are loaded first: their latency overlaps the staging.
      const int j = threadIdx.x & 15, c0 = cpg * 128 + 8 * j;
      float sv[8];
      LoadH8(m.svh + c0, sv);
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
      for (int r = threadIdx.x >> 4; r < nrows; r += 16) {
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = 0.f + ebuf[r][8 * j + i];
        Wht128x8Signed(v);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] *= WhtLaneSign() * (kHadNorm * sv[i]);
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

template <int K2, int CB, int NRB, int KSW, int U, bool MIDX = false>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(NRB == 1 && K2 <= 8 ? 8 : 1)))
Exl3GemmKernel(GemmArgs g) {
  GemmBody<K2, CB, NRB, KSW, U, MIDX, 0>(g, (int)blockIdx.x, (int)blockIdx.y, (int)blockIdx.z);
}

// Several GEMMs of one rate, codebook and row-block count in one launch (a group of linears
// over the same rows, engine/exl3/exl3.h:328-389 runs them as one LinPolicyKernel): job j
// owns workgroups [start[j], start[j + 1]), laid out as its own launch's (gx[j], entries)
// grid, x fastest.  Each workgroup runs the same body as that launch, so the outputs are
// bitwise those of one launch per job.
constexpr int kMaxMultiJobs = 12;  // the table stays within the 4 KB of kernel arguments
struct GemmMulti {
  int n;
  int start[kMaxMultiJobs + 1];
  int gx[kMaxMultiJobs];
  GemmArgs g[kMaxMultiJobs];
};
template <int K2, int CB, int NRB, int KSW, int U>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(NRB == 1 && K2 <= 8 ? 8 : 1)))
Exl3GemmMultiKernel(GemmMulti gm) {
  const int L = (int)blockIdx.x;
  int j = 0;
  while (j + 1 < gm.n && L >= gm.start[j + 1]) ++j;  // uniform
  const int loc = L - gm.start[j];
  GemmBody<K2, CB, NRB, KSW, U, false, 0>(gm.g[j], loc % gm.gx[j], loc / gm.gx[j], 0);
}

// Decode calls: the gate/up GEMM, the mid and the down GEMM (output transform in its
// epilogue) in one launch, with no fence and no data leaving an XCD.  Workgroups go to the
// 8 XCDs round-robin by linear id; workgroup L serves row entry e with e % 8 = L % 8, so
// an entry's gate/up sums and mid rows are written and read in one XCD's L2 (plain stores,
// acknowledged before an agent-scope counter; reads with the L2 policy).  With n the
// device-side entry count rounded up to 8: ids [0, n_gu = 2 gu.ncp n): gate/up (per XCD,
// entry-major: 2 gu.ncp workgroups per entry, column pair then plane); the next dn.ncp / 4
// n ids: down (column-block workgroups per entry); the rest (the grid is sized for the
// table's nyp entries) exit at once, after every real workgroup in dispatch order, so the
// dispatcher's time on them falls in the launch's drain instead of between the gate/up and
// the down workgroups.  Every gate/up workgroup precedes every down workgroup in dispatch
// order, and only down workgroups wait, so every wait ends.  nyp: the entry table's
// length, a multiple of 8 (entries past the device-side count have 0 rows).  The counters
// are zeroed by the grouping launch before.  K2: the gate/up rate, K2D the down rate.
template <int K2, int K2D, int CB>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(K2 <= 8 && K2D <= 8 ? 8 : 1)))
Exl3DecodeStageKernel(GemmArgs gu, GemmArgs dn, int nyp) {
  const int L = (int)blockIdx.x, x = L & 7;
  const int n = (min(*gu.n_entries, nyp) + 7) & ~7;
  const int per_gu = 2 * gu.ncp, n_gu = per_gu * n, per_dn = dn.ncp / 4;
  if (L < n_gu) {
    const int k = L >> 3, e = 8 * (k / per_gu) + x, j = k % per_gu;
    GemmBody<K2, CB, 1, 4, 2, false, 1>(gu, j % gu.ncp, e, j / gu.ncp);
  } else if (L < n_gu + per_dn * n) {
    const int k = (L - n_gu) >> 3, e = 8 * (k / per_dn) + x, j = k % per_dn;
    GemmBody<K2D, CB, 1, 1, 2, false, 2>(dn, j, e, 0);
  }
}

}  // namespace cx

namespace cx {

// Workgroups go to the 8 XCDs round-robin by linear id.  This remap puts all gridDim.x *
// gridDim.z workgroups of row entry y on XCD y % 8, consecutively, so an entry's activation
// rows are fetched into one L2 and reused there.  gridDim.y must be a multiple of 8.
struct GridPos {
  int x, y, z;
};
__device__ __forceinline__ GridPos XcdEntryMajor() {
  const int X = gridDim.x, subs = X * gridDim.z;
  const int L = blockIdx.x + X * (blockIdx.y + gridDim.y * blockIdx.z);
  const int k = L >> 3, sub = k % subs;
  return {sub % X, 8 * (k / subs) + (L & 7), sub / X};
}

// Prefill GEMM (register-blocked): a workgroup = WPG waves owns WPG CPWV column pairs
// (32 WPG CPWV columns) x up to 16 NRBT rows of one expert, full K.  Each wave decodes
// its own CPWV column pairs (B fragments stay in registers, every tile decoded once per
// workgroup) and multiplies them with all the workgroup's row blocks; the activation
// tile of a step (16 NRBT rows x 32 inputs) is loaded once into LDS and shared by the
// waves, so more waves per workgroup read the activations fewer times.  One barrier per
// step double-buffers the activation tile.
//
// MID: gate and up in one workgroup (2 WPG waves: the first WPG on gate, the others on up,
// each plane with its own activation tiles), and the mid computed in the epilogue from
// both planes' sums (MidBlock), written as the down projection's input rows; the raw
// gate / up sums never leave the workgroup.  Needs 32 WPG CPWV = 128 (one block).
template <int K2, int CB, int NRBT, int CPWV, int WPG, bool MID = false>
__global__ void __launch_bounds__(64 * WPG * (MID ? 2 : 1)) Exl3GemmPrefillKernel(GemmArgs g) {
  static_assert(!MID || 32 * WPG * CPWV == 128, "the fused mid needs one 128-column block per workgroup");
  constexpr int NP = MID ? 2 : 1;       // planes per workgroup
  constexpr int T = TileDwords(K2);
  constexpr int SD = 4 * T;
  constexpr int DPL = (SD + 63) / 64;
  constexpr int ND = WindowDwords(K2);
  constexpr int R = 16 * NRBT;          // rows per workgroup
  // Staged activation rows of 32 halves, unpadded; 16-byte chunk c of row r sits at chunk
  // c ^ ((r >> 1) & 3), so the 16-byte fragment reads of 8 consecutive rows and the tile
  // writes (4 threads per row) each cover all 32 banks.  Measured bank-conflict cycles per
  // LDS instruction of the config-4 launches: 0.07 (gate/up) and 0.26 (down) against 0.99
  // and 1.13 with rows padded to 48 halves (the launch times did not change).
  constexpr int XS = 32;
  auto xcol = [](int r, int c) { return 8 * (c ^ ((r >> 1) & 3)); };
  constexpr int NT = 64 * WPG;             // threads per plane
  constexpr int XL = (R * 4 + NT - 1) / NT;  // 16-byte activation loads per thread per step
  // The epilogue stages 16-row slabs (8.4 KB), so the activation tiles set the LDS size and
  // more workgroups fit a CU.
  constexpr int ER = 16;
  constexpr int NXB = 4;  // activation tile buffers (written for s + 1, read by the MFMAs of s - 1)
  constexpr int XBYTES = NP * NXB * R * XS * 2, EBYTES = NP * ER * 132 * 4;
  __shared__ uint32_t stage[NP * WPG][CPWV][StageDwords<K2, DPL>()];
  // Activation tiles during the main loop; the epilogue's row staging afterwards.
  __shared__ __align__(16) char smem[XBYTES > EBYTES ? XBYTES : EBYTES];
  const int n_entries = g.n_entries ? *g.n_entries : g.n_entries_host;
  const GridPos gp = XcdEntryMajor();
  const int ei = gp.y + g.entry_base;
  if (ei >= n_entries) return;
  const int4 ent = EntryOf(g, ei);
  const int cpg = gp.x;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int plane = MID ? wave / WPG : 0, lw = MID ? wave % WPG : wave;  // plane, wave within it
  const int tp = (int)threadIdx.x - plane * NT;                            // thread within the plane
  const GemmPlane& pl = g.plane[MID ? plane : gp.z];
  __half(*xs)[R][XS] = reinterpret_cast<__half(*)[R][XS]>(smem + plane * (XBYTES / NP));
  const int steps = g.A / 2;
  const int row0 = ent.y, nrows = ent.z;
  const int nrb = (nrows + 15) / 16;
  const MatPtr m = MatOf(g, pl, ent.x);
  const LaneRun<K2> lr(lane);

  __amdgpu_buffer_rsrc_t rw[CPWV];
#pragma unroll
  for (int c = 0; c < CPWV; ++c) {
    const int cp = (cpg * WPG + lw) * CPWV + c;
    rw[c] = MakeRsrc(m.tiles + (size_t)cp * g.A * 2 * T, (uint32_t)steps * SD * 4);
  }
  uint32_t woff[2][ND];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int i = 0; i < ND; ++i) woff[j][i] = (uint32_t)StagePad<K2>((2 * j + lr.tile) * T + (lr.d0 + i) % T);
  const uint32_t loff = (uint32_t)lane * DPL * 4;

  // Activation tile loads: thread t moves rows t / 4 + 64 i, quarter t % 4 (16 bytes).
  const __amdgpu_buffer_rsrc_t rx = MakeRsrc(pl.x + (size_t)row0 * pl.ldx, (uint32_t)nrows * pl.ldx * 2);
  uint32_t xoff[XL];
#pragma unroll
  for (int i = 0; i < XL; ++i) {
    const int row = tp / 4 + (NT / 4) * i;
    xoff[i] = (uint32_t)((row * pl.ldx + 8 * (tp & 3)) * 2);
  }
  auto load_x = [&](u32x4_t (&xv)[XL], int s) {
#pragma unroll
    for (int i = 0; i < XL; ++i) xv[i] = BufLoad128(rx, xoff[i], (uint32_t)s * 64);
  };
  auto store_x = [&](const u32x4_t (&xv)[XL], int buf) {
#pragma unroll
    for (int i = 0; i < XL; ++i) {
      const int row = tp / 4 + (NT / 4) * i;
      if ((NT / 4) * (i + 1) <= R || row < R)  // statically true when the loads cover R rows exactly
        *reinterpret_cast<u32x4_t*>(&xs[buf][row][xcol(row, tp & 3)]) = xv[i];
    }
  };

  float4_t acc[NRBT][CPWV][2];
#pragma unroll
  for (int i = 0; i < NRBT; ++i)
#pragma unroll
    for (int c = 0; c < CPWV; ++c) acc[i][c][0] = acc[i][c][1] = float4_t{0.f, 0.f, 0.f, 0.f};

  constexpr int PFW = 4;  // weight steps in flight
  constexpr int PFX = 2;  // activation steps in flight
  Dwords<DPL> wq[PFW][CPWV];
  u32x4_t xq[PFX][XL];
  // Every load is unconditional, also past the last step (weight loads there fall outside
  // the buffer resource: no memory access; activation loads read rows' other columns):
  // with conditional loads the compiler cannot count the loads in flight and waits for
  // all of them (vmcnt(0)) at every use, which empties the prefetch queues.
#pragma unroll
  for (int k = 0; k < PFW; ++k)
#pragma unroll
    for (int c = 0; c < CPWV; ++c) wq[k][c] = BufLoadN<DPL>(rw[c], loff, (uint32_t)k * SD * 4);
#pragma unroll
  for (int k = 0; k < PFX; ++k) load_x(xq[k], k);
  store_x(xq[0], 0);
  load_x(xq[0], PFX);
  // The MFMAs issued at step 0 (for the step before the first) read tile buffer NXB - 1
  // with zero fragments: zero it so they add exact zeros.
  for (int i = tp; i < R * XS / 8; i += NT)
    reinterpret_cast<u32x4_t*>(&xs[NXB - 1][0][0])[i] = u32x4_t{0u, 0u, 0u, 0u};
  __syncthreads();

  uint32_t* slot[CPWV];
#pragma unroll
  for (int c = 0; c < CPWV; ++c) slot[c] = stage[wave][c];

  // The main loop is instantiated per count of live row blocks NA, so the accumulators
  // stay in fixed registers (a runtime guard per MFMA makes the compiler copy them).
  // Software pipeline: step s decodes its weights while the MFMAs of step s - 1 (its
  // decoded fragments kept in registers, its activation tile still in LDS) execute, so the
  // matrix core works under the decode's VALU stream instead of after it.
  auto main_loop = [&](auto nac) {
    constexpr int NA = decltype(nac)::value;
    half8_t bp[CPWV][2];  // fragments of the previous step (zero before the first)
#pragma unroll
    for (int c = 0; c < CPWV; ++c) bp[c][0] = bp[c][1] = half8_t{};
    // MFMAs of row blocks [i0, i1) of the previous step.
    auto mfma = [&](int buf, int i0, int i1) {
#pragma unroll
      for (int i = 0; i < NRBT; ++i) {
        if (i < NA && i >= i0 && i < i1) {
          const half8_t av =
              *reinterpret_cast<const half8_t*>(&xs[buf][i * 16 + (lane & 15)][xcol(lane & 15, lane >> 4)]);
#pragma unroll
          for (int c = 0; c < CPWV; ++c) {
            acc[i][c][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bp[c][0], acc[i][c][0], 0, 0, 0);
            acc[i][c][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bp[c][1], acc[i][c][1], 0, 0, 0);
          }
        }
      }
    };
    constexpr int HALF = (NA + 1) / 2;
    // Unrolled by lcm(PFW, PFX, NXB) = 4 (steps is a multiple of 4): every queue slot and
    // tile buffer is fixed and a step is one basic block, so the scheduler can interleave
    // the MFMAs of step s - 1 with the decode of step s.  Loads and tile stores past the
    // last step are unconditional: weight loads there fall outside the buffer resource (no
    // memory access), activation loads read rows' other columns, and the tile stored for
    // step `steps` is never read.
    constexpr int UN = 4;
    for (int s0 = 0; s0 < steps; s0 += UN) {
#pragma unroll
      for (int u = 0; u < UN; ++u) {
        const int s = s0 + u;
        const int qw = u % PFW, qx = (u + 1) % PFX;
        store_x(xq[qx], (u + 1) % NXB);
        load_x(xq[qx], s + 1 + PFX);
        half8_t b[CPWV][2];
#pragma unroll
        for (int c = 0; c < CPWV; ++c) {
          StageWrite<K2, DPL>(slot[c], lane, wq[qw][c].v);
          __builtin_amdgcn_wave_barrier();
          uint32_t v[2][3];
#pragma unroll
          for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int i = 0; i < ND; ++i) v[j][i] = slot[c][woff[j][i]];
            if constexpr (ND == 2) v[j][2] = 0u;
          }
          __builtin_amdgcn_wave_barrier();
          wq[qw][c] = BufLoadN<DPL>(rw[c], loff, (uint32_t)(s + PFW) * SD * 4);
          // The previous step's MFMAs go between the two runs' decode (scheduling
          // fences keep them there): the matrix core works while the VALU decodes.
          half4_t lo0, hi0, lo1, hi1;
          DecodeRun<K2, CB>(v[0][0], v[0][1], v[0][2], lr.shift, lo0, hi0);
          if (c == 0) {
            __builtin_amdgcn_sched_barrier(0);
            mfma((u + NXB - 1) % NXB, 0, HALF);
            __builtin_amdgcn_sched_barrier(0);
          }
          DecodeRun<K2, CB>(v[1][0], v[1][1], v[1][2], lr.shift, lo1, hi1);
          if (c == 0) {
            __builtin_amdgcn_sched_barrier(0);
            mfma((u + NXB - 1) % NXB, HALF, NA);
            __builtin_amdgcn_sched_barrier(0);
          }
          b[c][0] = half8_t{lo0[0], lo0[1], lo0[2], lo0[3], lo1[0], lo1[1], lo1[2], lo1[3]};
          b[c][1] = half8_t{hi0[0], hi0[1], hi0[2], hi0[3], hi1[0], hi1[1], hi1[2], hi1[3]};
        }
#pragma unroll
        for (int c = 0; c < CPWV; ++c) {
          bp[c][0] = b[c][0];
          bp[c][1] = b[c][1];
        }
        __syncthreads();
      }
    }
    mfma((steps - 1) % NXB, 0, NA);
    __syncthreads();  // the epilogue reuses the tile buffers
  };
  using std::integral_constant;
  // main_loop<NA> for NA = clamp(nrb, 1, NRBT): a chain of compile-time tests.
  [&]<int... Is>(std::integer_sequence<int, Is...>) {
    const int na = nrb < 1 ? 1 : nrb > NRBT ? NRBT : nrb;
    (void)((na == Is + 1 ? (main_loop(integral_constant<int, Is + 1>{}), true) : false) || ...);
  }(std::make_integer_sequence<int, NRBT>{});

  if constexpr (MID) {
    // Mid per 16-row slab: both planes' raw sums staged in LDS, then one row's block per
    // 16 lanes of the first 16 ER threads.
    float(*eb)[ER][132] = reinterpret_cast<float(*)[ER][132]>(smem);
    const MatPtr mg = MatOf(g, g.plane[0], ent.x), mu = MatOf(g, g.plane[1], ent.x);
    const int j = threadIdx.x & 15, c0 = cpg * 128 + 8 * j;
    const int O = g.ncp * 32;
    for (int r0 = 0; r0 < nrows; r0 += ER) {
#pragma unroll
      for (int i = 0; i < NRBT; ++i) {
        if (i * 16 < r0 || i * 16 >= r0 + ER) continue;
        const int cl = lw * 32 + ((lane & 15) >> 3) * 16 + (lane & 7);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = i * 16 - r0 + 4 * (lane >> 4) + e;
          eb[plane][r][cl] = acc[i][0][0][e];
          eb[plane][r][cl + 8] = acc[i][0][1][e];
        }
      }
      __syncthreads();
      const int rr = threadIdx.x >> 4;
      if (rr < ER && r0 + rr < nrows) {
        float gv[8], uv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          gv[e] = eb[0][rr][8 * j + e];
          uv[e] = eb[1][rr][8 * j + e];
        }
        const size_t p = (size_t)(row0 + r0 + rr);
        MidBlock(gv, uv, mg.svh + c0, mu.svh + c0, g.mid_suh + (size_t)ent.x * O + c0,
                 g.mid_xd + p * O + cpg * 128);
      }
      __syncthreads();
    }
    return;
  }
  if (pl.epi >= 1) {
    // Output transform per 128-column block: stage y_h rows in LDS, ER rows at a time
    // (reusing the activation tile area), WHT128 * norm * svh per row.
    float(*eb)[132] = reinterpret_cast<float(*)[132]>(smem);
    const int j = threadIdx.x & 15;
#pragma unroll
    for (int blk = 0; blk < WPG * CPWV / 4; ++blk) {
      // Column block blk of this workgroup holds column pairs 4 blk .. 4 blk + 3 of the
      // workgroup = waves (4 blk + q) / CPWV, their pair (4 blk + q) % CPWV.
      const int c0 = (cpg * WPG * CPWV / 4 + blk) * 128 + 8 * j;
      float sv[8];
      LoadH8(m.svh + c0, sv);
      for (int r0 = 0; r0 < nrows; r0 += ER) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int wpair = 4 * blk + q;  // column pair index within the workgroup
          if (wave == wpair / CPWV) {
            const int c = wpair % CPWV;
            const int cl = q * 32 + ((lane & 15) >> 3) * 16 + (lane & 7);
#pragma unroll
            for (int i = 0; i < NRBT; ++i) {
              if (i * 16 < r0 || i * 16 >= r0 + ER) continue;
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const int r = i * 16 - r0 + 4 * (lane >> 4) + e;
                eb[r][cl] = acc[i][c][0][e];
                eb[r][cl + 8] = acc[i][c][1][e];
              }
            }
          }
        }
        __syncthreads();
        for (int rr = threadIdx.x >> 4; rr < ER && r0 + rr < nrows; rr += NT / 16) {
          float v[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = 0.f + eb[rr][8 * j + e];
          Wht128x8Signed(v);
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] *= WhtLaneSign() * (kHadNorm * sv[e]);
          StoreBlockRow(pl, (size_t)(row0 + r0 + rr), c0, g.ncp * 32, v);
        }
        __syncthreads();
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < NRBT; ++i) {
    if (i >= nrb) break;
#pragma unroll
    for (int c = 0; c < CPWV; ++c) {
      const int cp = (cpg * WPG + wave) * CPWV + c;
      const int col = (2 * cp + ((lane & 15) >> 3)) * 16 + (lane & 7);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = i * 16 + 4 * (lane >> 4) + e;
        if (r < nrows) {
          float* yr = pl.y + (size_t)(row0 + r) * pl.ldy;
          yr[col] = acc[i][c][0][e];
          yr[col + 8] = acc[i][c][1][e];
        }
      }
    }
  }
}

}  // namespace cx

namespace cx {

// Tall prefill GEMM for long entries: a workgroup = 4 waves owns 128 columns (4 column
// pairs) x up to 16 NRBW row blocks of one entry, full K.  Wave w decodes column pair w
// per step and passes its B fragments to the other waves through LDS; wave w multiplies
// row blocks w, w + 4, ... by all 8 column tiles.  So every tile is decoded once per
// entry of up to 64 NRBW rows, and every activation fragment is loaded by exactly one
// wave, straight into registers (no activation staging, no sharing needed).
//
// tall_seq_mid (gate/up): the workgroup runs the gate plane, then the up plane over the same
// entry and columns, and computes the mid in the epilogue (grid z = 1).
//
// Step pipeline (B fragments in 4 LDS buffers, decode two steps ahead of the MFMAs):
//   [barrier at even s] | read B(s) | MFMAs of step s, decode of step s + 2 | write B(s + 2)
// One workgroup barrier per two steps: every B write and its reads, and every read and the
// next write of its buffer, have an even step's barrier between them.
template <int K2, int CB, int NRBW>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
Exl3GemmTallKernel(GemmArgs g) {
  constexpr int T = TileDwords(K2);
  constexpr int SD = 4 * T;
  constexpr int DPL = (SD + 63) / 64;
  constexpr int ND = WindowDwords(K2);
  constexpr int ER = 16;                       // epilogue slab rows (one row block)
  // Steps the decode runs ahead of the MFMAs (one workgroup barrier per DA steps).
  // Measured on config 5: 1 and 4 no better than 2 (4: gate/up -1.5%, down +1%).
  constexpr int DA = 2;
  constexpr int NBB = 2 * DA;        // B buffers
  constexpr int BBYTES = NBB * 4 * 2 * 64 * 16;  // [buffer][column pair][fragment][lane] x 16 B
  constexpr int EBYTES = 4 * ER * 132 * 4;     // one slab per wave
  __shared__ uint32_t stage[4][StageDwords<K2, DPL>()];
  __shared__ __align__(16) char smem[BBYTES > EBYTES ? BBYTES : EBYTES];
  u32x4_t* bs = reinterpret_cast<u32x4_t*>(smem);
  const int n_entries = g.n_entries ? *g.n_entries : g.n_entries_host;
  const GridPos gp = XcdEntryMajor();
  const int ei = gp.y + g.entry_base;
  if (ei >= n_entries) return;
  const int4 ent = EntryOf(g, ei);
  const bool seq = g.tall_seq_mid != 0;  // both planes in this workgroup, the mid fused
  const int cpg = gp.x;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int steps = g.A / 2;
  const int row0 = ent.y, nrows = ent.z;
  if (nrows <= 0) return;
  const int nrb = (nrows + 15) / 16;
  const LaneRun<K2> lr(lane);
  const int cp = cpg * 4 + wave;
  uint32_t woff[2][ND];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int i = 0; i < ND; ++i) woff[j][i] = (uint32_t)StagePad<K2>((2 * j + lr.tile) * T + (lr.d0 + i) % T);
  const uint32_t loff = (uint32_t)lane * DPL * 4;
  uint32_t* slot = stage[wave];

  // A step's weights go through the wave's LDS slot: staged (written) one step before its
  // decode, windows read back at the start of the decode's step.
  auto stage_w = [&](const Dwords<DPL>& w) { StageWrite<K2, DPL>(slot, lane, w.v); };
  auto read_windows = [&](uint32_t (&v)[2][3]) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int i = 0; i < ND; ++i) v[j][i] = slot[woff[j][i]];
      if constexpr (ND == 2) v[j][2] = 0u;
    }
  };
  auto decode = [&](const uint32_t (&v)[2][3], half8_t& b0, half8_t& b1) {
    half4_t lo0, hi0, lo1, hi1;
    DecodeRun<K2, CB>(v[0][0], v[0][1], v[0][2], lr.shift, lo0, hi0);
    DecodeRun<K2, CB>(v[1][0], v[1][1], v[1][2], lr.shift, lo1, hi1);
    b0 = half8_t{lo0[0], lo0[1], lo0[2], lo0[3], lo1[0], lo1[1], lo1[2], lo1[3]};
    b1 = half8_t{hi0[0], hi0[1], hi0[2], hi0[3], hi1[0], hi1[1], hi1[2], hi1[3]};
  };
  auto write_b = [&](int buf, const half8_t& b0, const half8_t& b1) {
    bs[((buf * 4 + wave) * 2 + 0) * 64 + lane] = __builtin_bit_cast(u32x4_t, b0);
    bs[((buf * 4 + wave) * 2 + 1) * 64 + lane] = __builtin_bit_cast(u32x4_t, b1);
  };

  auto main_loop = [&](auto nac) {
    constexpr int NA = decltype(nac)::value;  // row blocks per wave
    constexpr int PFW = 2;                    // weight steps in flight (beyond the staged one)
    constexpr int PFA = 2;                    // activation steps in flight
    for (int pz = seq ? 0 : gp.z;; ++pz) {  // one plane, or gate then up (seq)
      const GemmPlane& pl = g.plane[pz];
      const MatPtr m = MatOf(g, pl, ent.x);
      const __amdgpu_buffer_rsrc_t rw = MakeRsrc(m.tiles + (size_t)cp * g.A * 2 * T, (uint32_t)steps * SD * 4);
      // Activations: rows past the entry lie outside the buffer resource and read as zeros.
      const __amdgpu_buffer_rsrc_t rx = MakeRsrc(pl.x + (size_t)row0 * pl.ldx, (uint32_t)nrows * pl.ldx * 2);
      uint32_t xoff[NA];
#pragma unroll
      for (int i = 0; i < NA; ++i)
        xoff[i] = (uint32_t)(((wave + 4 * i) * 16 + (lane & 15)) * pl.ldx * 2 + 16 * (lane >> 4));
      float4_t acc[NA][4][2];
#pragma unroll
      for (int i = 0; i < NA; ++i)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[i][c][0] = acc[i][c][1] = float4_t{0.f, 0.f, 0.f, 0.f};
      Dwords<DPL> wq[PFW];  // slot j % PFW: step j's weights until they are staged
      u32x4_t aq[PFA][NA];
      // Loads are unconditional, also past the last step (outside the buffer resources: no
      // memory access, zeros), so the compiler can count the loads in flight.
#pragma unroll
      for (int k = 0; k < PFW; ++k) wq[k] = BufLoadN<DPL>(rw, loff, (uint32_t)k * SD * 4);
#pragma unroll
      for (int k = 0; k < PFA; ++k)
#pragma unroll
        for (int i = 0; i < NA; ++i) aq[k][i] = BufLoad128(rx, xoff[i], (uint32_t)k * 64);
      // Steps 0 .. DA - 1 decoded and published, step DA staged.
#pragma unroll
      for (int k = 0; k < DA; ++k) {
        stage_w(wq[k % PFW]);
        wq[k % PFW] = BufLoadN<DPL>(rw, loff, (uint32_t)(PFW + k) * SD * 4);
        __builtin_amdgcn_wave_barrier();
        uint32_t v[2][3];
        read_windows(v);
        __builtin_amdgcn_wave_barrier();
        half8_t b0, b1;
        decode(v, b0, b1);
        write_b(k, b0, b1);
      }
      stage_w(wq[DA % PFW]);
      wq[DA % PFW] = BufLoadN<DPL>(rw, loff, (uint32_t)(PFW + DA) * SD * 4);
      // Decode runs two steps ahead of the MFMAs into 4 B buffers (buffer s % 4), so a
      // workgroup barrier is needed at even steps only: B(s + 2), written in step s, is read
      // in step s + 2 with the even step's barrier in between, and buffer (s + 2) % 4 was last
      // read in step s - 2, also one barrier earlier.
      constexpr int UN = NBB > 4 ? NBB : 4;  // lcm(PFW, PFA, NBB): fixed queue slots and buffers per unrolled step
      constexpr int NM = NA * 8;  // MFMAs per step
      for (int s0 = 0; s0 < steps; s0 += UN) {
#pragma unroll
        for (int u = 0; u < UN; ++u) {
          const int s = s0 + u;
          if (u % DA == 0) __syncthreads();
          half8_t bf[4][2];
#pragma unroll
          for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int f = 0; f < 2; ++f) bf[c][f] = __builtin_bit_cast(half8_t, bs[(((u % NBB) * 4 + c) * 2 + f) * 64 + lane]);
          uint32_t v[2][3];
          read_windows(v);  // step s + DA, staged in the previous step
          __builtin_amdgcn_sched_barrier(0);
          // MFMAs of step s (column-tile major, so the first ones need only the first B
          // fragment) interleaved with the decode of step s + 2: the matrix core and the
          // VALU work side by side within the wave.
          half8_t n0, n1;
          decode(v, n0, n1);
#pragma unroll
          for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int f = 0; f < 2; ++f)
#pragma unroll
              for (int i = 0; i < NA; ++i)
                acc[i][c][f] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, aq[u % PFA][i]),
                                                                      bf[c][f], acc[i][c][f], 0, 0, 0);
#pragma unroll
          for (int i = 0; i < NA; ++i) {
            aq[u % PFA][i] = BufLoad128(rx, xoff[i], (uint32_t)(s + PFA) * 64);
          }
          __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
#pragma unroll
          for (int k = 0; k < NM - 2; ++k) {
            __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          }
          __builtin_amdgcn_sched_barrier(0);
          write_b((u + DA) % NBB, n0, n1);  // step s + DA (past the last step: never read)
          stage_w(wq[(u + DA + 1) % PFW]);  // step s + DA + 1
          wq[(u + DA + 1) % PFW] = BufLoadN<DPL>(rw, loff, (uint32_t)(s + DA + 1 + PFW) * SD * 4);
        }
      }
      __syncthreads();  // every wave is done with the B buffers: the epilogue reuses them

      if (seq && pz == 1) {
        // The mid of the wave's rows: up sums staged per row block in the wave's slab, gate
        // sums read back from plane 0's y, where this wave wrote them (the workgroup
        // barriers since then order the writes before these reads).
        float(*eb)[132] = reinterpret_cast<float(*)[132]>(smem + wave * ER * 132 * 4);
        const GemmPlane& p0 = g.plane[0];
        const MatPtr mg = MatOf(g, p0, ent.x);
        const int j = lane & 15, c0 = cpg * 128 + 8 * j, O = g.ncp * 32;
#pragma unroll
        for (int i = 0; i < NA; ++i) {
          const int rb = wave + 4 * i;
          if (rb >= nrb) break;  // wave-uniform
#pragma unroll
          for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int cl = c * 32 + ((lane & 15) >> 3) * 16 + (lane & 7);
              eb[4 * (lane >> 4) + e][cl] = acc[i][c][0][e];
              eb[4 * (lane >> 4) + e][cl + 8] = acc[i][c][1][e];
            }
          __builtin_amdgcn_wave_barrier();
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int rr = 4 * q + (lane >> 4), r = rb * 16 + rr;
            if (r < nrows) {  // uniform over the row's 16 lanes
              const size_t p = (size_t)(row0 + r);
              float gv[8], uv[8];
              LoadF8(p0.y + p * p0.ldy + c0, gv);
#pragma unroll
              for (int e = 0; e < 8; ++e) uv[e] = eb[rr][8 * j + e];
              MidBlock(gv, uv, mg.svh + c0, m.svh + c0, g.mid_suh + (size_t)ent.x * O + c0,
                       g.mid_xd + p * O + cpg * 128);
            }
          }
          __builtin_amdgcn_wave_barrier();
        }
        return;
      }
      if (pl.epi >= 1) {
        // Output transform per row: the wave holds all 128 columns of its row blocks.
        // Stage one row block (16 x 128 fp32) in the wave's slab, then WHT128 * norm * svh.
        float(*eb)[132] = reinterpret_cast<float(*)[132]>(smem + wave * ER * 132 * 4);
        const int j = lane & 15;
        const int c0 = cpg * 128 + 8 * j;
        float sv[8];
        LoadH8(m.svh + c0, sv);
#pragma unroll
        for (int i = 0; i < NA; ++i) {
          const int rb = wave + 4 * i;
          if (rb >= nrb) break;  // wave-uniform
#pragma unroll
          for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int cl = c * 32 + ((lane & 15) >> 3) * 16 + (lane & 7);
              eb[4 * (lane >> 4) + e][cl] = acc[i][c][0][e];
              eb[4 * (lane >> 4) + e][cl + 8] = acc[i][c][1][e];
            }
          __builtin_amdgcn_wave_barrier();
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int rr = 4 * q + (lane >> 4);
            float v[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = 0.f + eb[rr][8 * j + e];
            Wht128x8Signed(v);
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] *= WhtLaneSign() * (kHadNorm * sv[e]);
            const int r = rb * 16 + rr;
            if (r < nrows) StoreBlockRow(pl, (size_t)(row0 + r), c0, g.ncp * 32, v);
          }
          __builtin_amdgcn_wave_barrier();
        }
        return;
      }
      // Raw sums: each row block (16 x 128 fp32) staged in the wave's slab and written as
      // 16-byte pieces, 8 store instructions per lane instead of 32 single-float ones.
      float(*eb)[132] = reinterpret_cast<float(*)[132]>(smem + wave * ER * 132 * 4);
#pragma unroll
      for (int i = 0; i < NA; ++i) {
        const int rb = wave + 4 * i;
        if (rb >= nrb) break;  // wave-uniform
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int cl = c * 32 + ((lane & 15) >> 3) * 16 + (lane & 7);
            eb[4 * (lane >> 4) + e][cl] = acc[i][c][0][e];
            eb[4 * (lane >> 4) + e][cl + 8] = acc[i][c][1][e];
          }
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const int rr = 2 * k + (lane >> 5), c4 = 4 * (lane & 31);
          const int r = rb * 16 + rr;
          if (r < nrows)
            *reinterpret_cast<float4*>(pl.y + (size_t)(row0 + r) * pl.ldy + cpg * 128 + c4) =
                *reinterpret_cast<const float4*>(&eb[rr][c4]);
        }
        __builtin_amdgcn_wave_barrier();
      }
      if (!seq) return;
      __syncthreads();  // the slabs are the next plane's B buffers
    }
  };
  using std::integral_constant;
  [&]<int... Is>(std::integer_sequence<int, Is...>) {
    const int na = (nrb + 3) / 4;
    (void)((na <= Is + 1 ? (main_loop(integral_constant<int, Is + 1>{}), true) : false) || ...);
  }(std::make_integer_sequence<int, NRBW>{});
}

}  // namespace cx

