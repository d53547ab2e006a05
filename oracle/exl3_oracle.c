/*
 * CPU oracle for the EXL3 quantized MoE expert path.  TEST INFRASTRUCTURE ONLY:
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this
 * library, as the checker or as the timed CPU baseline.  The product path never
 * calls it.
 *
 * A plain-C restatement of the reference algorithm, each function citing the
 * reference file:line it follows (paths relative to the reference root):
 *   - trellis state extraction      ref/exl3_ref.py:40-65, docs/EXL3_FORMAT.md:76-112
 *   - codebooks mul1 / mcg / 3inst  ref/exl3_ref.py:68-86, docs/EXL3_FORMAT.md:114-144
 *   - tensor-core element order     ref/exl3_ref.py:29-37, docs/EXL3_FORMAT.md:62-74
 *   - reconstruct_inner             ref/exl3_ref.py:110-119
 *   - 128-point Hadamard transform  ref/exl3_ref.py:140-156, engine/gfx1151/common.h:62-77
 *   - matvec (fp16 / fp32 output)   ref/exl3_ref.py:159-178, engine/exl3/exl3.h:48-82
 *   - router top-k + weights        engine/layers/ops.h:683-713, docs/FLASHNEXT_FORWARD.md:236-250
 *   - stable expert-major dispatch  ref/prefill_ref.py:37-45, engine/layers/kernels/prefill_moe.h:9-100
 *   - MoE layer with engine rounding points
 *                                   ref/oracle.py:226-239, engine/layers/moe_rows.h:102-125,543-566,634-682
 *
 * Dot products accumulate in binary64 (each fp16*fp16 product is exact there) and
 * round once to binary32, which is at least as accurate as the reference's fp32 BLAS.
 * Every other rounding point (fp16 activations, fp32 transforms) follows the reference.
 *
 * Built with OpenMP: the same code is the timed CPU baseline.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define HAD_SCALE 0.088388347648f
#define MUL1 0x83DCD12Du
#define MCG 0xCBAC1FEDu

/* ---------------------------------------------------------------- fp16 ---- */

/* binary32 -> binary16, round to nearest even, with subnormals, inf and nan. */
uint16_t or_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t exp = (x >> 23) & 0xffu;
  uint32_t man = x & 0x7fffffu;
  if (exp == 0xffu) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u | (man >> 13) : 0u));
  int e = (int)exp - 127 + 15;
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    man |= 0x800000u;
    int shift = 14 - e; /* 24-bit mantissa to a subnormal with 10 bits */
    uint32_t half = man >> shift;
    uint32_t rem = man & ((1u << shift) - 1u);
    uint32_t mid = 1u << (shift - 1);
    if (rem > mid || (rem == mid && (half & 1u))) ++half;
    return (uint16_t)(sign | half);
  }
  uint32_t half = ((uint32_t)e << 10) | (man >> 13);
  uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) ++half; /* may carry into the exponent: correct */
  return (uint16_t)(sign | half);
}

float or_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t x;
  if (exp == 0) {
    if (man == 0) {
      x = sign;
    } else {
      int e = -1;
      do { ++e; man <<= 1; } while (!(man & 0x400u));
      x = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ffu) << 13);
    }
  } else if (exp == 31) {
    x = sign | 0x7f800000u | (man << 13);
  } else {
    x = sign | ((exp + 127 - 15) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &x, 4);
  return f;
}

static inline float round_h(float v) { return or_f16_to_f32(or_f32_to_f16(v)); }

/* ----------------------------------------------------- trellis decoding ---- */

/* Width of symbol i for the bitrate 2K = k2 (integer K: K; half-integer: floor(K)
 * plus one on odd positions).  ref/exl3_ref.py:57, docs/EXL3_FORMAT.md:70-72. */
static inline int sym_width(int k2, int i) { return (k2 >> 1) + ((k2 & 1) ? (i & 1) : 0); }

int or_valid_k2(int k2) { return (k2 >= 2 && k2 <= 16 && !(k2 & 1)) || k2 == 3 || k2 == 5 || k2 == 7; }

/* The 256 sliding 16-bit states of one tile in decoder order.  words: the tile's
 * 16K little-endian int16 storage words; u32[q] = w[2q] | w[2q+1] << 16 and the
 * stream is read MSB first within each u32.  State i is the 16 ring bits ending
 * at the end of symbol i, wrapping inside the tile.  ref/exl3_ref.py:40-65. */
void or_decode_states(const uint16_t* words, int k2, uint16_t* states) {
  const int ndw = 4 * k2; /* 8K dwords */
  const int bits = 128 * k2;
  uint32_t u32[64];
  for (int q = 0; q < ndw; ++q) u32[q] = (uint32_t)words[2 * q] | ((uint32_t)words[2 * q + 1] << 16);
  int end = bits; /* E_i + B keeps indices nonnegative */
  for (int i = 0; i < 256; ++i) {
    end += sym_width(k2, i);
    const int start = end - 16;
    const int first = start / 32, last = (end - 1) / 32;
    const int shift = (last + 1) * 32 - end;
    const uint64_t a = u32[first % ndw], b = u32[last % ndw];
    states[i] = (uint16_t)((((a << 32) | b) >> shift) & 0xffffu);
  }
}

/* Exact fp16 codebook value (bits) of one state.  cb: 0 = 3inst, 1 = mcg,
 * 2 = mul1.  ref/exl3_ref.py:68-86, docs/EXL3_FORMAT.md:114-144. */
uint16_t or_codebook(uint16_t state, int cb) {
  if (cb == 2) {
    const uint32_t p = (uint32_t)state * MUL1;
    const uint32_t b = (p & 255u) + ((p >> 8) & 255u) + ((p >> 16) & 255u) + (p >> 24);
    /* (1024 + b) * inv + bias is exact in binary64; one rounding to fp16. */
    const double h = 1024.0 + (double)b;
    const double inv = (double)or_f16_to_f32(0x1eee), bias = (double)or_f16_to_f32(0xc931);
    const double v = h * inv + bias;
    /* v has at most 22 significant bits, so binary64 -> binary32 is exact and the
     * binary32 -> binary16 conversion is the single rounding. */
    return or_f32_to_f16((float)v);
  }
  uint32_t p = cb == 1 ? (uint32_t)state * MCG : (uint32_t)state * 89226354u + 64248484u;
  p = (p & 0x8fff8fffu) ^ 0x3b603b60u;
  /* fp16 + fp16 is exact in binary32; one rounding to fp16. */
  return or_f32_to_f16(or_f16_to_f32((uint16_t)(p & 0xffffu)) + or_f16_to_f32((uint16_t)(p >> 16)));
}

/* Decoder position i -> row-major element of the 16x16 tile.  ref/exl3_ref.py:29-37. */
int or_tc_perm(int i) {
  const int t = i >> 3, j = i & 7;
  const int r = 2 * (t & 3) + (j & 1) + ((j & 2) ? 8 : 0);
  const int c = (t >> 2) + ((j & 4) ? 8 : 0);
  return r * 16 + c;
}

/* The 256 fp16 weights of one tile, row-major [16][16]. */
void or_decode_tile(const uint16_t* words, int k2, int cb, uint16_t* out256) {
  uint16_t st[256];
  or_decode_states(words, k2, st);
  for (int i = 0; i < 256; ++i) out256[or_tc_perm(i)] = or_codebook(st[i], cb);
}

/* reconstruct_inner: rotated-basis fp16 W_hat [I][O] from trellis
 * [I/16][O/16][16K] (checkpoint order).  ref/exl3_ref.py:110-119. */
void or_reconstruct_inner(const uint16_t* trellis, int in_f, int out_f, int k2, int cb, uint16_t* w) {
  const int A = in_f / 16, B = out_f / 16, T = 8 * k2;
#pragma omp parallel for schedule(static)
  for (int a = 0; a < A; ++a) {
    uint16_t tile[256];
    for (int b = 0; b < B; ++b) {
      or_decode_tile(trellis + ((size_t)a * B + b) * T, k2, cb, tile);
      for (int r = 0; r < 16; ++r)
        for (int c = 0; c < 16; ++c) w[(size_t)(a * 16 + r) * out_f + b * 16 + c] = tile[r * 16 + c];
    }
  }
}

/* ------------------------------------------------------------ Hadamard ---- */

/* Natural-order Sylvester butterfly over one 128-block, fp32, strides 1..64.
 * ref/exl3_ref.py:146-151, engine/gfx1151/common.h:62-77. */
void or_wht128(float* v) {
  for (int s = 1; s < 128; s <<= 1)
    for (int base = 0; base < 128; base += 2 * s)
      for (int i = base; i < base + s; ++i) {
        const float lo = v[i], hi = v[i + s];
        v[i] = lo + hi;
        v[i + s] = lo - hi;
      }
}

/* Input transform of one fp16 row: RoundH(RoundH(x) * suh), WHT, * norm, fp16.
 * ref/exl3_ref.py:140-152 (fp16 path), engine/exl3/exl3.h:60-64. */
void or_input_transform(const uint16_t* x, const uint16_t* suh, int n, uint16_t* xh) {
  float v[128];
  for (int b = 0; b < n; b += 128) {
    for (int i = 0; i < 128; ++i) v[i] = round_h(or_f16_to_f32(x[b + i]) * or_f16_to_f32(suh[b + i]));
    or_wht128(v);
    for (int i = 0; i < 128; ++i) xh[b + i] = or_f32_to_f16(v[i] * HAD_SCALE);
  }
}

/* Input transform of an fp32 row (the engine's src path): RoundH(RoundH(x) * suh). */
void or_input_transform_f32(const float* x, const uint16_t* suh, int n, uint16_t* xh) {
  float v[128];
  for (int b = 0; b < n; b += 128) {
    for (int i = 0; i < 128; ++i) v[i] = round_h(round_h(x[b + i]) * or_f16_to_f32(suh[b + i]));
    or_wht128(v);
    for (int i = 0; i < 128; ++i) xh[b + i] = or_f32_to_f16(v[i] * HAD_SCALE);
  }
}

/* Output transform, fp32 (engine LinOutBlock, engine/exl3/exl3.h:69-82):
 * WHT, then * (norm * svh). */
void or_output_transform_f32(const float* y_raw, const uint16_t* svh, int n, float* y) {
  float v[128];
  for (int b = 0; b < n; b += 128) {
    for (int i = 0; i < 128; ++i) v[i] = 0.f + y_raw[b + i];
    or_wht128(v);
    for (int i = 0; i < 128; ++i) y[b + i] = v[i] * (HAD_SCALE * or_f16_to_f32(svh[b + i]));
  }
}

/* Output transform, fp16 activations (ref/exl3_ref.py:153-156, 175):
 * y_h rounded to fp16, WHT in fp32, * norm -> fp16, * svh -> fp16. */
void or_output_transform_f16(const float* y_raw, const uint16_t* svh, int n, uint16_t* y) {
  float v[128];
  for (int b = 0; b < n; b += 128) {
    for (int i = 0; i < 128; ++i) v[i] = round_h(y_raw[b + i]);
    or_wht128(v);
    for (int i = 0; i < 128; ++i)
      y[b + i] = or_f32_to_f16(round_h(v[i] * HAD_SCALE) * or_f16_to_f32(svh[b + i]));
  }
}

/* Generic hadamard_kernel on fp32 or fp16 data (ref/exl3_ref.py:140-156).
 * is_f16: data is fp16 bits, else fp32.  pre/post: nullable fp16 scales. */
void or_hadamard(void* data, int is_f16, long rows, int n, const uint16_t* pre, const uint16_t* post) {
#pragma omp parallel for schedule(static)
  for (long r = 0; r < rows; ++r) {
    float v[128];
    for (int b = 0; b < n; b += 128) {
      for (int i = 0; i < 128; ++i) {
        float x = is_f16 ? or_f16_to_f32(((uint16_t*)data)[r * n + b + i]) : ((float*)data)[r * n + b + i];
        if (pre) {
          x = x * or_f16_to_f32(pre[b + i]);
          if (is_f16) x = round_h(x);
        }
        v[i] = x;
      }
      or_wht128(v);
      for (int i = 0; i < 128; ++i) {
        float y = v[i] * HAD_SCALE;
        if (is_f16) y = round_h(y);
        if (post) {
          y = y * or_f16_to_f32(post[b + i]);
          if (is_f16) y = round_h(y);
        }
        if (is_f16) ((uint16_t*)data)[r * n + b + i] = or_f32_to_f16(y);
        else ((float*)data)[r * n + b + i] = y;
      }
    }
  }
}

/* y_raw[o] = sum_k xh[k] * W[k][o], binary64 accumulation, one rounding. */
static void dot_rows(const uint16_t* xh, const uint16_t* w, int in_f, int out_f, float* y_raw, double* acc) {
  for (int o = 0; o < out_f; ++o) acc[o] = 0.0;
  for (int k = 0; k < in_f; ++k) {
    const double xv = (double)or_f16_to_f32(xh[k]);
    if (xv == 0.0) continue;
    const uint16_t* wr = w + (size_t)k * out_f;
    for (int o = 0; o < out_f; ++o) acc[o] += xv * (double)or_f16_to_f32(wr[o]);
  }
  for (int o = 0; o < out_f; ++o) y_raw[o] = (float)acc[o];
}

/* matvec over M rows with a decoded W_hat [I][O] (or_reconstruct_inner output).
 * out_f16 != 0: fp16 output per exl3_ref.matvec's default; else fp32 output with
 * the engine's output transform.  ref/exl3_ref.py:159-178, engine/exl3/exl3.h:48-82. */
void or_matvec(const uint16_t* x, long M, const uint16_t* w, const uint16_t* suh, const uint16_t* svh,
               int in_f, int out_f, int out_f16, void* y) {
#pragma omp parallel
  {
    uint16_t* xh = (uint16_t*)malloc(sizeof(uint16_t) * in_f);
    float* yr = (float*)malloc(sizeof(float) * out_f);
    double* acc = (double*)malloc(sizeof(double) * out_f);
#pragma omp for schedule(dynamic, 1)
    for (long m = 0; m < M; ++m) {
      or_input_transform(x + m * in_f, suh, in_f, xh);
      dot_rows(xh, w, in_f, out_f, yr, acc);
      if (out_f16) or_output_transform_f16(yr, svh, out_f, (uint16_t*)y + m * out_f);
      else or_output_transform_f32(yr, svh, out_f, (float*)y + m * out_f);
    }
    free(xh);
    free(yr);
    free(acc);
  }
}

/* -------------------------------------------------------------- routing ---- */

/* Top-k of E fp32 logits per row (logit descending, lower expert id on ties) and
 * the selection softmax w_k = exp(l_k - l_0) / sum_j exp(l_j - l_0) summed in rank
 * order; wts[k] = sigmoid(shared logit).  engine/layers/ops.h:683-713,
 * ref/oracle.py:227-230, docs/FLASHNEXT_FORWARD.md:238,250.
 * Non-finite logits: a NaN ranks and weighs as -inf (the reference's rank count leaves
 * NaN undefined: it flags it in a debug build, engine/layers/ops.h:691-693); +-inf rank as
 * themselves, so a +inf top logit gives NaN weights, as exp(inf - inf) does there. */
static double or_route_key(float v) { return v != v ? -INFINITY : (double)v; }
void or_route(const float* logits, long ld, long M, int E, int topk, const float* shared_logit,
              int32_t* sel, float* wts) {
#pragma omp parallel for schedule(static)
  for (long r = 0; r < M; ++r) {
    const float* lg = logits + r * ld;
    int32_t* s = sel + r * topk;
    for (int k = 0; k < topk; ++k) {
      int best = -1;
      for (int e = 0; e < E; ++e) {
        int taken = 0;
        for (int j = 0; j < k; ++j) taken |= s[j] == e;
        if (taken) continue;
        if (best < 0 || or_route_key(lg[e]) > or_route_key(lg[best])) best = e; /* strict: lower id wins ties */
      }
      s[k] = best;
    }
    const double top = or_route_key(lg[s[0]]);
    double sum = 0.0;
    for (int k = 0; k < topk; ++k) sum += exp(or_route_key(lg[s[k]]) - top);
    float* w = wts + r * (topk + 1);
    for (int k = 0; k < topk; ++k) w[k] = (float)(exp(or_route_key(lg[s[k]]) - top) / sum);
    const double sl = shared_logit ? shared_logit[r] : lg[E];
    w[topk] = (float)(1.0 / (1.0 + exp(-sl)));
  }
}

/* Stable expert-major dispatch: counts[E], exclusive offsets[E+1], pairs = stable
 * argsort of the flattened selection (row*topk + slot), row_ids = pairs / topk.
 * Returns -1 on an out-of-range expert id.  ref/prefill_ref.py:37-45. */
int or_dispatch(const int32_t* sel, long M, int E, int topk, int32_t* counts, int32_t* offsets,
                int32_t* pairs, int32_t* row_ids) {
  const long n = M * topk;
  for (long i = 0; i < n; ++i)
    if (sel[i] < 0 || sel[i] >= E) return -1;
  for (int e = 0; e < E; ++e) counts[e] = 0;
  for (long i = 0; i < n; ++i) ++counts[sel[i]];
  offsets[0] = 0;
  for (int e = 0; e < E; ++e) offsets[e + 1] = offsets[e] + counts[e];
  int32_t* cursor = (int32_t*)malloc(sizeof(int32_t) * (E > 0 ? E : 1));
  for (int e = 0; e < E; ++e) cursor[e] = offsets[e];
  for (long i = 0; i < n; ++i) {
    const int32_t p = cursor[sel[i]]++;
    pairs[p] = (int32_t)i;
    if (row_ids) row_ids[p] = (int32_t)(i / topk);
  }
  free(cursor);
  return 0;
}

/* ------------------------------------------------------------ MoE layer ---- */

/* One expert's decoded matrices.  w*: fp16 W_hat [I][O] (or_reconstruct_inner). */
typedef struct {
  const uint16_t *wg, *wu, *wd;       /* gate [H][Ie], up [H][Ie], down [Ie][H] */
  const uint16_t *sg, *su, *sd;       /* suh of gate, up, down */
  const uint16_t *vg, *vu, *vd;       /* svh of gate, up, down */
} or_expert;

/* The SwiGLU expert on one fp16 row, with the engine's rounding points:
 * gate/up input transforms (each matrix its own suh), fp32 GEMV, fp32 output
 * transform, mid RoundH(RoundH(SiLU(g) * u) * suh_down) -> WHT -> fp16, down GEMV,
 * fp32 output transform.  engine/layers/moe_rows.h:102-125, 543-566;
 * ref/oracle.py:232-233.  out: fp32 [H]. */
static void expert_row(const or_expert* ex, const uint16_t* x, int H, int Ie, float* out, uint16_t* xh,
                       float* g, float* u, float* t, double* acc) {
  or_input_transform(x, ex->sg, H, xh);
  dot_rows(xh, ex->wg, H, Ie, t, acc);
  or_output_transform_f32(t, ex->vg, Ie, g);
  or_input_transform(x, ex->su, H, xh);
  dot_rows(xh, ex->wu, H, Ie, t, acc);
  or_output_transform_f32(t, ex->vu, Ie, u);
  float v[128];
  for (int b = 0; b < Ie; b += 128) {
    for (int i = 0; i < 128; ++i) {
      const float gv = g[b + i];
      const float silu = (float)((double)gv / (1.0 + exp(-(double)gv)));
      v[i] = round_h(round_h(silu * u[b + i]) * or_f16_to_f32(ex->sd[b + i]));
    }
    or_wht128(v);
    for (int i = 0; i < 128; ++i) xh[b + i] = or_f32_to_f16(v[i] * HAD_SCALE);
  }
  dot_rows(xh, ex->wd, Ie, H, t, acc);
  or_output_transform_f32(t, ex->vd, H, out);
}

/* MoE layer: y[r] = sum_{k<topk} w_k * expert_{sel[r][k]}(x[r]) + w_topk * shared(x[r]),
 * fp32, accumulated in slot order with the shared expert last.
 * sel/wts: or_route output.  experts[E] plus shared.  ref/oracle.py:226-239,
 * engine/layers/moe_rows.h:634-682 (combine order). */
void or_moe_layer(const or_expert* experts, const or_expert* shared, const uint16_t* x, long M, int H, int Ie,
                  int topk, const int32_t* sel, const float* wts, float* y) {
#pragma omp parallel
  {
    uint16_t* xh = (uint16_t*)malloc(sizeof(uint16_t) * (H > Ie ? H : Ie));
    float* g = (float*)malloc(sizeof(float) * Ie);
    float* u = (float*)malloc(sizeof(float) * Ie);
    float* t = (float*)malloc(sizeof(float) * (H > Ie ? H : Ie));
    float* o = (float*)malloc(sizeof(float) * H);
    double* acc = (double*)malloc(sizeof(double) * (H > Ie ? H : Ie));
#pragma omp for schedule(dynamic, 1)
    for (long r = 0; r < M; ++r) {
      float* yr = y + r * H;
      for (int i = 0; i < H; ++i) yr[i] = 0.f;
      for (int k = 0; k <= topk; ++k) {
        const or_expert* ex = k < topk ? &experts[sel[r * topk + k]] : shared;
        expert_row(ex, x + r * H, H, Ie, o, xh, g, u, t, acc);
        const float w = wts[r * (topk + 1) + k];
        for (int i = 0; i < H; ++i) yr[i] += w * o[i];
      }
    }
    free(xh);
    free(g);
    free(u);
    free(t);
    free(o);
    free(acc);
  }
}

/* One expert on a batch of rows (the CPU baseline's unit of work). out: fp32 [M][H]. */
void or_expert_rows(const or_expert* ex, const uint16_t* x, long M, int H, int Ie, float* out) {
#pragma omp parallel
  {
    uint16_t* xh = (uint16_t*)malloc(sizeof(uint16_t) * (H > Ie ? H : Ie));
    float* g = (float*)malloc(sizeof(float) * Ie);
    float* u = (float*)malloc(sizeof(float) * Ie);
    float* t = (float*)malloc(sizeof(float) * (H > Ie ? H : Ie));
    double* acc = (double*)malloc(sizeof(double) * (H > Ie ? H : Ie));
#pragma omp for schedule(dynamic, 1)
    for (long r = 0; r < M; ++r) expert_row(ex, x + r * H, H, Ie, out + r * H, xh, g, u, t, acc);
    free(xh);
    free(g);
    free(u);
    free(t);
    free(acc);
  }
}

int or_num_threads(void) {
#ifdef _OPENMP
  extern int omp_get_max_threads(void);
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* Sets the OpenMP thread count of later calls (timing runs at 1 thread and at all). */
void or_set_num_threads(int n) {
#ifdef _OPENMP
  extern void omp_set_num_threads(int);
  omp_set_num_threads(n > 0 ? n : 1);
#else
  (void)n;
#endif
}
