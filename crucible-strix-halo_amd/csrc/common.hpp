// Device helpers for the MI355X (gfx950, CDNA4, wave64) EXL3 MoE path.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdint>

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

// Raw buffer resource over [base, base + bytes): loads past the end return zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t MakeRsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
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
