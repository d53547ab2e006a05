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

// ---- cross-lane moves inside 16-lane rows (DPP, plain VALU: no LDS traffic) ----------
// Every pattern used here reads an in-range lane of the same row with all rows and banks
// enabled, so the moves need no `old` value (bound_ctrl set: nothing is read from it).
template <int CTRL>
__device__ __forceinline__ float Dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xf, 0xf, true));
}
template <int CTRL>
__device__ __forceinline__ int DppI(int v) {
  return __builtin_amdgcn_mov_dpp(v, CTRL, 0xf, 0xf, true);
}
constexpr int kDppQuadSwap1 = 0xB1;     // quad_perm [1,0,3,2]: lane ^ 1
constexpr int kDppQuadSwap2 = 0x4E;     // quad_perm [2,3,0,1]: lane ^ 2
constexpr int kDppQuadReverse = 0x1B;   // quad_perm [3,2,1,0]: lane ^ 3
constexpr int kDppRowMirror = 0x140;    // lane 15 - i within 16
constexpr int kDppRowHalfMirror = 0x141;  // lane 7 - i within 8 (lane ^ 7)
constexpr int kDppRowRor8 = 0x128;       // lane (i + 8) % 16 within 16 (lane ^ 8)
// Value of lane ^ M (M = 1, 2, 4, 8) within each 16-lane row.
template <int M>
__device__ __forceinline__ float XorLane(float v) {
  if constexpr (M == 1) return Dpp<kDppQuadSwap1>(v);
  else if constexpr (M == 2) return Dpp<kDppQuadSwap2>(v);
  else if constexpr (M == 4) return Dpp<kDppQuadReverse>(Dpp<kDppRowHalfMirror>(v));  // (i ^ 7) ^ 3
  else return Dpp<kDppRowRor8>(v);                                                  // (i + 8) % 16
}

// 128-point natural-order Sylvester butterfly, 16 lanes per block (a wave64 holds four
// blocks, one per 16-lane row).  Lane j of a block holds elements 8j..8j+7.  Strides
// 1, 2, 4 are in-lane, strides 8..64 are lane xors 1..8 by DPP, in increasing order; each
// output is lo + hi or lo - hi of the same two fp32 operands, so the values are those of
// any evaluation of the same butterfly network.  All 64 lanes must be active.
//
// The cross-lane stages run in a signed form: lane j keeps sigma_j * value with
// sigma_j = (-1)^popcount(j), so every stage is one fused multiply-add per value with the
// partner's value (the DPP move folds into it): v = fma(partner, (j & M) ? -1 : 1, v).
// The low lane gets sigma (lo + hi) and the high lane sigma (hi - lo) = -sigma (lo - hi),
// which is what flips its sign.  Negation is exact and round-to-nearest is symmetric, so
// every nonzero value equals the natural-order network's; an exactly-zero output may
// carry the other sign of zero.  Callers fold WhtLaneSign() into the scale they apply
// after the transform (a multiplication by +-1 is exact).
//
// Relabelled form (PHI): physical lane L of a 16-lane row holds the elements of lane
// index e = L ^ 3 when L & 4 (else e = L).  The partners e ^ 1, e ^ 2, e ^ 4, e ^ 8 then
// sit at physical lanes L ^ 1, L ^ 2, L ^ 7, L ^ 8, one DPP pattern each (the natural
// layout needs two DPP moves for e ^ 4); signs follow e.  The network and its operands
// are the same, so are the values.  The caller loads and stores by e
// (StorePerm32x8LdsBuf<true>).
__device__ __forceinline__ int PhiLane() {
  const int L = threadIdx.x & 15;
  return L ^ (3 * ((L >> 2) & 1));
}
template <bool PHI = false>
__device__ __forceinline__ float WhtLaneSign() {
  const int e = PHI ? PhiLane() : (threadIdx.x & 15);
  return (__builtin_popcount(e) & 1) ? -1.f : 1.f;
}

// In-lane butterfly stages of strides ST0, 2 ST0, ... < 8.
template <int ST0>
__device__ __forceinline__ void WhtInLane(float v[8]) {
#pragma unroll
  for (int st = ST0; st < 8; st <<= 1)
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (!(i & st)) {
        const float lo = v[i], hi = v[i + st];
        v[i] = lo + hi;
        v[i + st] = lo - hi;
      }
}

// Cross-lane stages (strides 8..64) in the signed form (PHI: the relabelled lanes).
template <bool PHI = false>
__device__ __forceinline__ void WhtCrossLaneSigned(float v[8]) {
  const int j = PHI ? PhiLane() : (threadIdx.x & 15);
  // v_fmac_f32_dpp d, a, s: d += dpp(a) * s.  The compiler does not fold a DPP move into a
  // multiply-add, so the stages are written out; each block starts with the two wait
  // states a DPP read of a just-written VGPR needs.
#define CX_WHT_FMAC8(DPP, A0, A1, A2, A3, A4, A5, A6, A7, ...)                                    \
  asm volatile("s_nop 1\n"                                                                         \
               "v_fmac_f32_dpp %0, " A0 ", %8 " DPP "\n"                                           \
               "v_fmac_f32_dpp %1, " A1 ", %8 " DPP "\n"                                           \
               "v_fmac_f32_dpp %2, " A2 ", %8 " DPP "\n"                                           \
               "v_fmac_f32_dpp %3, " A3 ", %8 " DPP "\n"                                           \
               "v_fmac_f32_dpp %4, " A4 ", %8 " DPP "\n"                                           \
               "v_fmac_f32_dpp %5, " A5 ", %8 " DPP "\n"                                           \
               "v_fmac_f32_dpp %6, " A6 ", %8 " DPP "\n"                                           \
               "v_fmac_f32_dpp %7, " A7 ", %8 " DPP                                                 \
               : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]), \
                 "+v"(v[7])                                                                        \
               : "v"(sg), ##__VA_ARGS__)
  // In place (a lane reads its partner's value before any lane writes): stages 1, 2, 8.
#define CX_WHT_STAGE_INPLACE(DPP) CX_WHT_FMAC8(DPP, "%0", "%1", "%2", "%3", "%4", "%5", "%6", "%7")
  {
    const float sg = (j & 1) ? -1.f : 1.f;
    CX_WHT_STAGE_INPLACE("quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf");
  }
  {
    const float sg = (j & 2) ? -1.f : 1.f;
    CX_WHT_STAGE_INPLACE("quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf");
  }
  if constexpr (PHI) {
    const float sg = (j & 4) ? -1.f : 1.f;  // element e ^ 4 is physical lane L ^ 7
    CX_WHT_STAGE_INPLACE("row_half_mirror row_mask:0xf bank_mask:0xf");
  } else {
    float a[8];  // lane ^ 4 = (lane ^ 7) ^ 3: the first move by the compiler, the second folded
#pragma unroll
    for (int i = 0; i < 8; ++i) a[i] = Dpp<kDppRowHalfMirror>(v[i]);
    const float sg = (j & 4) ? -1.f : 1.f;
    CX_WHT_FMAC8("quad_perm:[3,2,1,0] row_mask:0xf bank_mask:0xf", "%9", "%10", "%11", "%12", "%13", "%14", "%15",
                 "%16", "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5]), "v"(a[6]), "v"(a[7]));
  }
  {
    const float sg = (j & 8) ? -1.f : 1.f;
    CX_WHT_STAGE_INPLACE("row_ror:8 row_mask:0xf bank_mask:0xf");
  }
#undef CX_WHT_STAGE_INPLACE
#undef CX_WHT_FMAC8
}

__device__ __forceinline__ void Wht128x8Signed(float v[8]) {
  WhtInLane<1>(v);
  WhtCrossLaneSigned(v);
}

// The same transform of 8 fp16 inputs packed in pairs (h[k] = elements 2k, 2k + 1): the
// stride-1 stage is v_fma_mix_f32 lo * 1 + (+-hi), the fp32 sum of the two values with
// one rounding, i.e. the conversion to fp32 folded into the first butterfly.
template <bool PHI = false>
__device__ __forceinline__ void Wht128x8SignedH(const uint32_t h[4], float v[8]) {
#pragma unroll
  for (int k = 0; k < 4; ++k)
    asm("v_fma_mix_f32 %0, %2, 1.0, %2 op_sel:[0,0,1] op_sel_hi:[1,0,1]\n"
        "v_fma_mix_f32 %1, %2, 1.0, -%2 op_sel:[0,0,1] op_sel_hi:[1,0,1]"
        : "=&v"(v[2 * k]), "=v"(v[2 * k + 1])
        : "v"(h[k]));
  WhtInLane<2>(v);
  WhtCrossLaneSigned<PHI>(v);
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

// Input row of slot p (0..15) of one k-tile in the decoder's run layout: lane group q
// (lanes 16q..16q+15) decodes rows {2q, 2q+1, 2q+8, 2q+9} of a weight tile as slots
// 4q..4q+3, i.e. row(q, s) = 2q + (s & 1) + 8 (s >> 1) (the dequantizer's element order).
__host__ __device__ constexpr int PermRow16(int p) { return 2 * (p >> 2) + (p & 1) + 8 * ((p >> 1) & 1); }
// The v_mfma_f32_16x16x32_f16 order over two k-tiles (32 input rows): lane group q holds
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
// The quad transpose of StorePerm32x8: on return h[q] is pair t of lane q, i.e. chunk t
// (8 halves) of the quad's 32 in MFMA row order, for lane t = (lane & 15) & 3.
__device__ __forceinline__ void Perm32x8Chunk(const float v[8], float scale, int (&h)[4]);
__device__ __forceinline__ void StorePerm32x8(__half* d, const float v[8], float scale) {
  const int j = threadIdx.x & 15, t = j & 3;
  int h[4];
  Perm32x8Chunk(v, scale, h);
  *reinterpret_cast<int4*>(d + 32 * (j >> 2) + 8 * t) = make_int4(h[0], h[1], h[2], h[3]);
}
__device__ __forceinline__ void Perm32x8Chunk(const float v[8], float scale, int (&h)[4]) {
  const int t = threadIdx.x & 3;
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
}
__device__ __forceinline__ void H8ToF(const uint4& u, float v[8]) {
  const __half2* h = reinterpret_cast<const __half2*>(&u);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float2 f = __half22float2(h[k]);
    v[2 * k] = f.x;
    v[2 * k + 1] = f.y;
  }
}
__device__ __forceinline__ void LoadH8(const __half* p, float v[8]) {
  H8ToF(*reinterpret_cast<const uint4*>(p), v);
}
// 8 consecutive activations at element idx of x as packed fp16: fp16 sources as they
// are, fp32 sources rounded to nearest-even (RoundH of each value).  16- / 32-byte loads.
__device__ __forceinline__ uint4 LoadAsH8(const void* x, bool f32, size_t idx) {
  if (f32) {
    const float* p = static_cast<const float*>(x) + idx;
    const float4 a = *reinterpret_cast<const float4*>(p), b = *reinterpret_cast<const float4*>(p + 4);
    return make_uint4(__builtin_bit_cast(uint32_t, __floats2half2_rn(a.x, a.y)),
                      __builtin_bit_cast(uint32_t, __floats2half2_rn(a.z, a.w)),
                      __builtin_bit_cast(uint32_t, __floats2half2_rn(b.x, b.y)),
                      __builtin_bit_cast(uint32_t, __floats2half2_rn(b.z, b.w)));
  }
  return *reinterpret_cast<const uint4*>(static_cast<const __half*>(x) + idx);
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
// Loads with the device-scope (sc1) cache policy: they miss in the CU's L1 and read the
// XCD's L2, so they see what other workgroups on the same XCD stored with plain stores and
// published (stores acknowledged, then an agent-scope flag) during the same launch.  The L2
// of another XCD is not coherent with it: such data must stay on one XCD.
constexpr int kPolicyL2 = 16;  // sc1
__device__ __forceinline__ u32x4_t BufLoad128L2(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, kPolicyL2);
}
// The same store through a buffer resource: the block at byte offset voff + soff (voff may
// differ per lane group, soff is uniform), the lane's chunk at + (32 (j >> 2) + 8 t) * 2.
__device__ __forceinline__ void StorePerm32x8Buf(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                                 const float v[8], float scale) {
  const int j = threadIdx.x & 15, t = j & 3;
  int h[4];
  Perm32x8Chunk(v, scale, h);
  __builtin_amdgcn_raw_buffer_store_b128(u32x4_t{(uint32_t)h[0], (uint32_t)h[1], (uint32_t)h[2], (uint32_t)h[3]}, r,
                                         voff + (uint32_t)(32 * (j >> 2) + 8 * t) * 2, soff, 0);
}
// StorePerm32x8Buf with the quad transpose through LDS instead of DPP exchanges: lane
// (q, s) = (lane / 4, lane % 4) writes its pair k to dword 16 q + 4 (k ^ f(q)) + s of the
// wave's 256-dword area (f(q) = (q >> 1) & 3: each of the four writes covers all 32 banks
// per half wave), then reads its chunk t = s, 16 bytes at 16 q + 4 (t ^ f(q)) (8
// consecutive lanes cover all banks).  A wave's LDS operations run in order, so no
// barrier is needed; the area must be the calling wave's own.  PHI: the lanes hold the
// relabelled elements (PhiLane), written at their element slot s = e & 3.
template <bool PHI = false>
__device__ __forceinline__ void StorePerm32x8LdsBuf(uint32_t* area, __amdgpu_buffer_rsrc_t r, uint32_t voff,
                                                    uint32_t soff, const float v[8], float scale) {
  const int lane = threadIdx.x & 63, j = lane & 15, q = lane >> 2, t = lane & 3, f = (q >> 1) & 3;
  const int te = PHI ? (PhiLane() & 3) : t;  // the values' lane index within the quad
  uint32_t h[4];
#pragma unroll
  for (int k = 0; k < 4; ++k)
    h[k] = __builtin_bit_cast(uint32_t, __floats2half2_rn(v[2 * k] * scale, v[2 * k + 1] * scale));
#pragma unroll
  for (int k = 0; k < 4; ++k) area[16 * q + 4 * (k ^ f) + te] = h[k];
  const u32x4_t c = *reinterpret_cast<const u32x4_t*>(area + 16 * q + 4 * (t ^ f));
  __builtin_amdgcn_raw_buffer_store_b128(c, r, voff + (uint32_t)(32 * (j >> 2) + 8 * t) * 2, soff, 0);
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
