// EXL3 trellis decode for wave64 + MFMA on gfx950.
//
// Format (docs/EXL3_FORMAT.md §2-3 of the reference; ref/exl3_ref.py:40-86): a 16x16
// tile is a circular bitstream of 256 symbols, 8K dwords (K = bits per weight, or
// floor(K) / floor(K)+1 alternating for K = 1.5, 2.5, 3.5), read MSB first.  Decoder
// position i holds the 16-bit state ending at the end of symbol i; position i = 8t + j
// is element (2(t%4) + (j&1) + 8((j>>1)&1), t/4 + 8(j>>2)) of the tile.
//
// Lane mapping.  A wave processes a step of two k-tiles of a column pair (32 input rows,
// 32 output columns: 4 tiles) with two v_mfma_f32_16x16x32_f16.  MFMA lane L (column
// n = L % 16, k-group q = L / 16) decodes run t = 4 (n % 8) + q of column tile n / 8 in
// both k-tiles: the 8 consecutive positions 8t..8t+7.  Positions 8t..8t+3 are column
// n % 8 at rows {2q, 2q+1, 2q+8, 2q+9} and 8t+4..8t+7 the same rows of column n % 8 + 8;
// the first four of each k-tile form the first MFMA's B operand (8 halves), the second
// four the second's.  Activations are stored in the matching 32-row order (PermPos32 in
// common.hpp), so no decoded weight ever crosses lanes.
//
// A run needs the 16 - d bits before it (its first state's history): the lane reads
// the (at most 3) dwords that hold its window, at offsets fixed per lane.
#pragma once

#include "common.hpp"

namespace cx {

enum Codebook { kCb3Inst = 0, kCbMcg = 1, kCbMul1 = 2 };

// Symbol width of position i at rate K2 = 2 x bits per weight.
__host__ __device__ constexpr int SymWidth(int k2, int i) { return (k2 >> 1) + ((k2 & 1) ? (i & 1) : 0); }
__host__ __device__ constexpr int TileDwords(int k2) { return 4 * k2; }
// End of state j of a run, in bits from the start of the run's window.
__host__ __device__ constexpr int RunEnd(int k2, int j) {
  int e = 16;
  for (int i = 1; i <= j; ++i) e += SymWidth(k2, i);
  return e;
}
// First window bit of run t (may be negative: the ring wraps).
__host__ __device__ constexpr int RunStart(int k2, int t) { return 4 * t * k2 + (k2 >> 1) - 16; }
__host__ __device__ constexpr int FloorDiv32(int s) { return s >= 0 ? s / 32 : -((31 - s) / 32); }
// Window start as (first dword, bit offset 1..32 from that dword's MSB).  An offset of
// 1..32 keeps every funnel-shift amount 32 - shift in 0..31.
__host__ __device__ constexpr int RunShift(int k2, int t) { return RunStart(k2, t) - 32 * FloorDiv32(RunStart(k2, t) - 1); }
__host__ __device__ constexpr int RunDword0(int k2, int t) {
  const int T = TileDwords(k2);
  return ((FloorDiv32(RunStart(k2, t) - 1) % T) + T) % T;
}
__host__ __device__ constexpr int MaxSpan(int k2) {
  int m = 0;
  for (int t = 0; t < 32; ++t) m = m > RunShift(k2, t) + RunEnd(k2, 7) ? m : RunShift(k2, t) + RunEnd(k2, 7);
  return m;
}
// Dwords a lane loads per tile.
__host__ __device__ constexpr int WindowDwords(int k2) { return MaxSpan(k2) <= 64 ? 2 : 3; }
// The shift is the same for every lane when a run is a whole number of dwords.
__host__ __device__ constexpr bool UniformShift(int k2) { return (4 * k2) % 32 == 0; }

__device__ __forceinline__ uint32_t AlignBit(uint32_t hi, uint32_t lo, uint32_t s) {
  return __builtin_amdgcn_alignbit(hi, lo, s);
}

// 32-bit state * mult for the state in the low (HI = false) or high half of r: the state
// is isolated by one shift or mask (2-cycle ops on gfx950) and multiplied by one
// v_mul_lo_u32 (a 4-cycle op there, like the packed 16-bit multiply and v_mad_u32_u16 a
// two-instruction 16-bit split would need).
template <bool HI>
__device__ __forceinline__ uint32_t StateProduct(uint32_t r, uint32_t mult) {
  const uint32_t st = HI ? (r >> 16) : (r & 0xffffu);
  return st * mult;
}

// Per-state codebook term of the state in the low (HI = false) or high half of r.
// mul1: the 32-bit product p = s * 0x83DCD12D (its byte sum is taken per pair below).
// mcg / 3inst: the fp16 value bits in the low 16 bits (high bits not defined).
template <int CB, bool HI>
__device__ __forceinline__ uint32_t CodeTerm(uint32_t r) {
  if constexpr (CB == kCbMul1) {
    return StateProduct<HI>(r, 0x83DCD12Du);
  } else {
    uint32_t p = StateProduct<HI>(r, CB == kCbMcg ? 0xCBAC1FEDu : 89226354u);
    if constexpr (CB == kCb3Inst) p += 64248484u;
    p = (p & 0x8fff8fffu) ^ 0x3b603b60u;
    const half2_t h = __builtin_bit_cast(half2_t, p);
    const _Float16 s = h.x + h.y;  // one fp16 rounding (docs/EXL3_FORMAT.md:133-144)
    return (uint32_t)__builtin_bit_cast(unsigned short, s);
  }
}

// Two states' terms -> packed fp16 weights (lo = a, hi = b).
// mul1: 0x6400 + bytesum(p) is the fp16 encoding of 1024 + bytesum.  The byte sums of a
// and b land directly in the two halves: v_dot4_u32_u8 adds bytesum(a) to 0x64006400
// (at most 0x67fc, no carry into the high half), v_sad_hi_u8 against zero adds
// bytesum(b) << 16.  Then the affine map h * 0x1eee + 0xc931 as one fp16 FMA (one
// rounding, docs/EXL3_FORMAT.md:120-131) on the pair.
template <int CB>
__device__ __forceinline__ half2_t PairWeights(uint32_t a, uint32_t b) {
  if constexpr (CB == kCbMul1) {
    uint32_t r = __builtin_amdgcn_udot4(a, 0x01010101u, 0x64006400u, false);
    r = __builtin_amdgcn_sad_hi_u8(b, 0u, r);
    const half2_t inv = {__builtin_bit_cast(_Float16, (unsigned short)0x1eee),
                         __builtin_bit_cast(_Float16, (unsigned short)0x1eee)};
    const half2_t bias = {__builtin_bit_cast(_Float16, (unsigned short)0xc931),
                          __builtin_bit_cast(_Float16, (unsigned short)0xc931)};
    return __builtin_elementwise_fma(__builtin_bit_cast(half2_t, r), inv, bias);
  } else {
    return __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(b, a, 0x05040100u));
  }
}

// Per-lane constants of the run window.
template <int K2>
struct LaneRun {
  int t;      // run index 0..31 within the tile
  int tile;   // 0 or 1: which tile of the pair
  int shift;  // 1..32
  int d0;     // first window dword within the tile
  __device__ __forceinline__ explicit LaneRun(int lane) {
    const int n = lane & 15, q = lane >> 4;
    tile = n >> 3;
    t = 4 * (n & 7) + q;
    if constexpr (UniformShift(K2)) {
      shift = RunShift(K2, 0);
    } else {
      const int s = RunStart(K2, t);
      const int dw = FloorDiv32(s - 1);
      shift = s - 32 * dw;
    }
    d0 = RunDword0(K2, t);
  }
  // Byte offset of window dword i relative to the tile pair.
  __device__ __forceinline__ uint32_t ByteOffset(int i) const {
    constexpr int T = TileDwords(K2);
    return (uint32_t)(tile * T + (d0 + i) % T) * 4u;
  }
};

// Decode one lane's run from its window dwords into the two MFMA B operands:
// lo = positions 8t..8t+3, hi = 8t+4..8t+7 (fp16).
template <int K2, int CB>
__device__ __forceinline__ void DecodeRun(uint32_t w0, uint32_t w1, uint32_t w2, int shift, half4_t& lo, half4_t& hi) {
  if constexpr (UniformShift(K2) && RunEnd(K2, 4) - RunEnd(K2, 0) == 16 && RunShift(K2, 0) + RunEnd(K2, 7) <= 64) {
    // K = 4 with a lane-invariant window start: the register holding state j + 4 (low
    // half) and state j (high half) is window bits [e - 32, e), e = end of state j + 4,
    // i.e. one funnel shift of (w0, w1) by a compile-time amount.
    constexpr int S0 = RunShift(K2, 0);
    uint32_t c[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = S0 + RunEnd(K2, j + 4);  // bit position after the state, from w0's MSB
      const uint32_t r = e == 64 ? w1 : AlignBit(w0, w1, (uint32_t)(64 - e));
      c[j] = CodeTerm<CB, true>(r);
      c[j + 4] = CodeTerm<CB, false>(r);
    }
    const half2_t p0 = PairWeights<CB>(c[0], c[1]), p1 = PairWeights<CB>(c[2], c[3]);
    const half2_t p2 = PairWeights<CB>(c[4], c[5]), p3 = PairWeights<CB>(c[6], c[7]);
    lo = half4_t{p0.x, p0.y, p1.x, p1.y};
    hi = half4_t{p2.x, p2.y, p3.x, p3.y};
    return;
  }
  const uint32_t sh = UniformShift(K2) ? (uint32_t)(32 - RunShift(K2, 0)) : (uint32_t)(32 - shift);
  const uint32_t a0 = AlignBit(w0, w1, sh);
  const uint32_t a1 = AlignBit(w1, w2, sh);
  uint32_t a2 = 0;
  if constexpr (RunEnd(K2, 7) > 64) a2 = AlignBit(w2, 0u, sh);
  uint32_t c[8];
  if constexpr (RunEnd(K2, 4) - RunEnd(K2, 0) == 16 && RunEnd(K2, 7) <= 64) {
    // K = 4: the register holding state j + 4 carries state j in its high half.
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = RunEnd(K2, j + 4);
      const uint32_t r = e <= 32 ? (a0 >> (32 - e)) : AlignBit(a0, a1, 64 - e);
      c[j] = CodeTerm<CB, true>(r);
      c[j + 4] = CodeTerm<CB, false>(r);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int e = RunEnd(K2, j);
      uint32_t r;
      if (e <= 32) r = a0 >> (32 - e);
      else if (e <= 64) r = AlignBit(a0, a1, 64 - e);
      else r = AlignBit(a1, a2, 96 - e);
      c[j] = CodeTerm<CB, false>(r);
    }
  }
  const half2_t p0 = PairWeights<CB>(c[0], c[1]), p1 = PairWeights<CB>(c[2], c[3]);
  const half2_t p2 = PairWeights<CB>(c[4], c[5]), p3 = PairWeights<CB>(c[6], c[7]);
  lo = half4_t{p0.x, p0.y, p1.x, p1.y};
  hi = half4_t{p2.x, p2.y, p3.x, p3.y};
}

}  // namespace cx
