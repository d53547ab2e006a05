// Device helpers for the MI355X (gfx950, CDNA4, wave64) EXL3 MoE path.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

namespace cx {

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef unsigned short ushort2_t __attribute__((ext_vector_type(2)));

constexpr float kHadNorm = 0.088388347648f;  // 1/sqrt(128) as EXL3 stores it (binary32)

__device__ __forceinline__ float RoundH(float v) { return __half2float(__float2half(v)); }
__device__ __forceinline__ float H2F(__half h) { return __half2float(h); }
__device__ __forceinline__ float SiLU(float v) { return v / (1.f + __expf(-v)); }
__device__ __forceinline__ float Sigmoid(float v) { return 1.f / (1.f + __expf(-v)); }

// 128-point natural-order Sylvester butterfly over fp32 values, 32 lanes per block
// (a wave64 holds two blocks: lanes 0-31 and 32-63).  Lane j of a block holds elements
// 4j..4j+3.  Strides 1 and 2 are in-lane, strides 4..64 are lane xors 1..16, in
// increasing order, each output being lo + hi or lo - hi of the same two operands, so
// the result is the same fp32 value as any other evaluation of that butterfly network.
__device__ __forceinline__ void Wht128x4(float v[4]) {
  const int lane = threadIdx.x & 31;
  const float a0 = v[0] + v[1], a1 = v[0] - v[1], a2 = v[2] + v[3], a3 = v[2] - v[3];
  v[0] = a0 + a2;
  v[1] = a1 + a3;
  v[2] = a0 - a2;
  v[3] = a1 - a3;
#pragma unroll
  for (int m = 1; m < 32; m <<= 1) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float o = __shfl_xor(v[i], m, 64);
      v[i] = (lane & m) ? (o - v[i]) : (v[i] + o);
    }
  }
}

// ---- cross-lane moves inside 16-lane rows (DPP, plain VALU: no LDS traffic) ----------
template <int CTRL>
__device__ __forceinline__ float Dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
template <int CTRL>
__device__ __forceinline__ int DppI(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}
constexpr int kDppQuadSwap1 = 0xB1;     // quad_perm [1,0,3,2]: lane ^ 1
constexpr int kDppQuadSwap2 = 0x4E;     // quad_perm [2,3,0,1]: lane ^ 2
constexpr int kDppQuadReverse = 0x1B;   // quad_perm [3,2,1,0]: lane ^ 3
constexpr int kDppRowMirror = 0x140;    // lane 15 - i within 16
constexpr int kDppRowHalfMirror = 0x141;  // lane 7 - i within 8 (lane ^ 7)
// Value of lane ^ M (M = 1, 2, 4, 8) within each 16-lane row.
template <int M>
__device__ __forceinline__ float XorLane(float v) {
  if constexpr (M == 1) return Dpp<kDppQuadSwap1>(v);
  else if constexpr (M == 2) return Dpp<kDppQuadSwap2>(v);
  else if constexpr (M == 4) return Dpp<kDppQuadReverse>(Dpp<kDppRowHalfMirror>(v));  // (i ^ 7) ^ 3
  else return Dpp<kDppRowHalfMirror>(Dpp<kDppRowMirror>(v));                          // (i ^ 15) ^ 7
}

// 128-point natural-order Sylvester butterfly, 16 lanes per block (a wave64 holds four
// blocks, one per 16-lane row).  Lane j of a block holds elements 8j..8j+7.  Strides
// 1, 2, 4 are in-lane, strides 8..64 are lane xors 1..8 by DPP, in increasing order; each
// output is lo + hi or lo - hi of the same two fp32 operands, so the values are those of
// any evaluation of the same butterfly network.  All 64 lanes must be active.
__device__ __forceinline__ void Wht128x8(float v[8]) {
#pragma unroll
  for (int st = 1; st < 8; st <<= 1)
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (!(i & st)) {
        const float lo = v[i], hi = v[i + st];
        v[i] = lo + hi;
        v[i + st] = lo - hi;
      }
  const int j = threadIdx.x & 15;
  auto stage = [&](auto mc) {
    constexpr int M = decltype(mc)::value;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float o = XorLane<M>(v[i]);
      v[i] = (j & M) ? (o - v[i]) : (v[i] + o);
    }
  };
  stage(std::integral_constant<int, 1>{});
  stage(std::integral_constant<int, 2>{});
  stage(std::integral_constant<int, 4>{});
  stage(std::integral_constant<int, 8>{});
}

// Wave-uniform max / min by DPP row reductions and four lane reads.
__device__ __forceinline__ float WaveMaxF(float v) {
  v = fmaxf(v, Dpp<kDppQuadSwap1>(v));
  v = fmaxf(v, Dpp<kDppQuadSwap2>(v));
  v = fmaxf(v, Dpp<kDppRowHalfMirror>(v));
  v = fmaxf(v, Dpp<kDppRowMirror>(v));
  const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float d = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return fmaxf(fmaxf(a, b), fmaxf(c, d));
}
__device__ __forceinline__ int WaveMinI(int v) {
  v = min(v, DppI<kDppQuadSwap1>(v));
  v = min(v, DppI<kDppQuadSwap2>(v));
  v = min(v, DppI<kDppRowHalfMirror>(v));
  v = min(v, DppI<kDppRowMirror>(v));
  return min(min(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
             min(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}

// Position of input row r (0..15 of a 16-row block) in the MFMA-ordered activation
// layout.  Lane group q of a 16x16x16 MFMA feeds rows {2q, 2q+1, 2q+8, 2q+9} of a
// weight tile (the decoder's run layout), so activations are stored as
// [.., 4q + s, ..] with row(q, s) = 2q + (s & 1) + 8 (s >> 1).
__host__ __device__ constexpr int PermPos16(int r) { return 4 * ((r & 7) >> 1) + (r & 1) + 2 * (r >> 3); }
__host__ __device__ constexpr int PermRow16(int p) { return 2 * (p >> 2) + (p & 1) + 8 * ((p >> 1) & 1); }
// The same for a 16x16x32 MFMA over two k-tiles (32 input rows): lane group q holds
// slots 8q..8q+7 = rows {2q, 2q+1, 2q+8, 2q+9} of the first k-tile, then of the second.
__host__ __device__ constexpr int PermPos32(int r) { return 8 * ((r & 7) >> 1) + 4 * (r >> 4) + (r & 1) + 2 * ((r >> 3) & 1); }
__host__ __device__ constexpr int PermRow32(int p) {
  return 16 * ((p >> 2) & 1) + 2 * (p >> 3) + (p & 1) + 8 * ((p >> 1) & 1);
}

// Stores 8 fp16 values of elements 8j..8j+7 of a 128-block (j = lane & 15) in the
// 32-row MFMA order: element 8j + i goes to 32 (j >> 2) + PermPos32(8 (j & 3) + i), so
// the lanes t = j & 3 of a quad hold pairs (i, i + 1) that interleave: chunk k (8 halves)
// of the quad's 32 is [pair k of lane 0, of lane 1, of lane 2, of lane 3].  A 4 x 4
// transpose of the packed pairs across the quad (two DPP exchange rounds) gives every
// lane one whole chunk, stored with one 16-byte write.  d: the block's first half.
__device__ __forceinline__ void StorePerm32x8(__half* d, const float v[8], float scale) {
  const int j = threadIdx.x & 15, t = j & 3;
  int h[4];
#pragma unroll
  for (int k = 0; k < 4; ++k)
    h[k] = __builtin_bit_cast(int, __floats2half2_rn(v[2 * k] * scale, v[2 * k + 1] * scale));
  // Round 1 (lane ^ 1): lanes exchange the pairs whose index differs from them in bit 0.
  {
    const bool odd = t & 1;
    const int a = DppI<kDppQuadSwap1>(odd ? h[0] : h[1]);
    const int b = DppI<kDppQuadSwap1>(odd ? h[2] : h[3]);
    if (odd) {
      h[0] = a;
      h[2] = b;
    } else {
      h[1] = a;
      h[3] = b;
    }
  }
  // Round 2 (lane ^ 2): the same for bit 1.
  {
    const bool hi = t & 2;
    const int a = DppI<kDppQuadSwap2>(hi ? h[0] : h[2]);
    const int b = DppI<kDppQuadSwap2>(hi ? h[1] : h[3]);
    if (hi) {
      h[0] = a;
      h[1] = b;
    } else {
      h[2] = a;
      h[3] = b;
    }
  }
  // Now h[q] is pair t of lane q: chunk t of the quad.
  *reinterpret_cast<int4*>(d + 32 * (j >> 2) + 8 * t) = make_int4(h[0], h[1], h[2], h[3]);
}
__device__ __forceinline__ void LoadH8(const __half* p, float v[8]) {
  const uint4 u = *reinterpret_cast<const uint4*>(p);
  const __half2* h = reinterpret_cast<const __half2*>(&u);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float2 f = __half22float2(h[k]);
    v[2 * k] = f.x;
    v[2 * k + 1] = f.y;
  }
}
__device__ __forceinline__ void LoadF8(const float* p, float v[8]) {
  const float4 a = *reinterpret_cast<const float4*>(p), b = *reinterpret_cast<const float4*>(p + 4);
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}
__device__ __forceinline__ void StoreF8(float* p, const float v[8]) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  *reinterpret_cast<float4*>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
}

// Raw buffer resource over [base, base + bytes): loads past the end return zero.  Every
// resource here is wave-uniform; the explicit lane-0 reads keep it in SGPRs even when the
// compiler cannot prove the base uniform (a base loaded through a selected pointer would
// otherwise put a waterfall loop around every load).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t MakeRsrc(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32));
  const int n = __builtin_amdgcn_readfirstlane((int)bytes);
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(lo | (hi << 32)), (short)0, n, 0x00020000);
}
__device__ __forceinline__ uint32_t BufLoad32(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
}
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x3_t __attribute__((ext_vector_type(3)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x2_t BufLoad64(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0);
}
__device__ __forceinline__ u32x4_t BufLoad128(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
}
// N consecutive dwords (N = 1..4) from a buffer.
template <int N>
struct Dwords {
  uint32_t v[N];
};
template <int N>
__device__ __forceinline__ Dwords<N> BufLoadN(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  Dwords<N> d;
  if constexpr (N == 1) {
    d.v[0] = __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
  } else if constexpr (N == 2) {
    const u32x2_t t = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0);
    d.v[0] = t.x;
    d.v[1] = t.y;
  } else if constexpr (N == 3) {
    const u32x3_t t = __builtin_amdgcn_raw_buffer_load_b96(r, voff, soff, 0);
    d.v[0] = t.x;
    d.v[1] = t.y;
    d.v[2] = t.z;
  } else {
    const u32x4_t t = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
    d.v[0] = t.x;
    d.v[1] = t.y;
    d.v[2] = t.z;
    d.v[3] = t.w;
  }
  return d;
}

}  // namespace cx
