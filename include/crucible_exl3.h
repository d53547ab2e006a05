/*
 * crucible_exl3.h — C-ABI of the MI355X (gfx950) EXL3 quantized MoE expert path.
 *
 * Drop-in boundary for Crucible's EXL3 linear op and MoE layer (the reference is the
 * engine's in-process C++: file:line citations are relative to the reference root).
 * All pointers are device pointers unless a parameter says "host".  Every compute call
 * is asynchronous on the given HIP stream, allocates nothing (workspace is caller
 * memory, sized by the matching *_workspace_size query and 256-byte aligned, as hipMalloc
 * and torch allocations are), never exits, and returns:
 *     0  success
 *    <0  invalid argument or shape (CX_E_*)
 *    >0  a hipError_t from a launch
 *
 * fp16 data is passed as uint16_t bit patterns (IEEE binary16).
 *
 * The exceptions are set-up calls: cx_moe_plan_create / _destroy allocate and free the
 * plan's device tables (synchronously), and the checkpoint reader does host I/O.  One
 * host thread drives a plan at a time (its trace ring is plan state), as one host
 * thread owns the reference engine (engine/serve/README.md:13-14).
 */
#ifndef CRUCIBLE_EXL3_H
#define CRUCIBLE_EXL3_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* cx_stream_t; /* a hipStream_t; NULL = the null stream */

enum {
  CX_OK = 0,
  CX_E_ARG = -1,       /* null pointer or bad enum */
  CX_E_SHAPE = -2,     /* dimension not a multiple of 128, rows out of range, ... */
  CX_E_BITRATE = -3,   /* bits per weight not in 1..8 or 1.5 / 2.5 / 3.5 */
  CX_E_WORKSPACE = -4, /* workspace too small */
  CX_E_EXPERT = -5,    /* expert id out of range */
  CX_E_UNSUPPORTED = -6,
  CX_E_FORMAT = -7     /* checkpoint file or tensor format error (cx_last_error has the reason) */
};

enum { CX_CB_3INST = 0, CX_CB_MCG = 1, CX_CB_MUL1 = 2 };   /* codebook, docs/EXL3_FORMAT.md §3 */
enum { CX_F16 = 0, CX_F32 = 1 };                            /* activation dtypes */
enum { CX_MOE_AUTO = 0, CX_MOE_DECODE = 1, CX_MOE_PREFILL = 2 };

/* One EXL3 linear [in_features x out_features] on the device, with its tiles already in
 * this library's layout (cx_exl3_repack).  Replaces the weight half of
 * `LinJob{tiles,suh,svh,...,I,O,K}` (engine/exl3/exl3.h:20-33) and `Lin`
 * (engine/model/flashnext/model.h:40-46). */
typedef struct cx_exl3_matrix {
  const uint32_t* tiles;   /* column-pair-major tiles, 8K dwords each */
  const uint16_t* suh;     /* fp16 [in_features] input sign/scale */
  const uint16_t* svh;     /* fp16 [out_features] output sign/scale */
  int32_t in_features;     /* multiple of 128 */
  int32_t out_features;    /* multiple of 128 */
  int32_t k2;              /* 2 x bits per weight: 2..16, or 3 / 5 / 7 for K = 1.5 / 2.5 / 3.5 */
  int32_t codebook;        /* CX_CB_* */
} cx_exl3_matrix;

/* Bytes of a matrix's packed tiles (I * O * K / 8). */
size_t cx_exl3_tile_bytes(int32_t in_features, int32_t out_features, int32_t k2);

/* Loader repack: checkpoint trellis [I/16][O/16][16K] int16 (docs/EXL3_FORMAT.md §1-2)
 * -> this library's column-pair-major tiles.  Replaces the loader's trellis repack to
 * "crucible order" (engine/model/flashnext/model.h:503-527).  src and dst must not overlap. */
int cx_exl3_repack(const int16_t* trellis, int32_t in_features, int32_t out_features, int32_t k2,
                   uint32_t* tiles, cx_stream_t stream);

/* Dequantize to the rotated-basis fp16 W_hat [I][O] (bit-exact decoded weights).  The
 * parity hook for ref/exl3_ref.py:110-119 `reconstruct_inner`. */
int cx_exl3_dequant(const cx_exl3_matrix* m, uint16_t* w_hat, cx_stream_t stream);

/* The input transform of a linear alone: per 128-block of each row, xh =
 * fp16(WHT128(RoundH(RoundH(x) * suh)) * norm), written in this library's MFMA row order
 * (natural element e of a 128-block at position 32 (e >> 5) + p(e & 31), p(r) =
 * 8 ((r & 7) >> 1) + 4 (r >> 4) + (r & 1) + 2 ((r >> 3) & 1)).  The parity hook for
 * LinInKernel / LinInLane (engine/exl3/exl3.h:48-65, 96-102) and hadamard_kernel with
 * pre_scale (ref/exl3_ref.py:140-156): it runs the kernel cx_exl3_linear uses.
 *   x   fp16 (CX_F16) or fp32 (CX_F32) [M][ldx], ldx >= in_features, ldx % 8 == 0
 *   xh  fp16 [M][in_features] */
int cx_exl3_input_transform(const cx_exl3_matrix* m, const void* x, int32_t x_dtype, int32_t ldx, int32_t M,
                            uint16_t* xh, cx_stream_t stream);

/* The output transform alone: y = WHT128(y_raw) * (norm * svh) in fp32 (CX_F32, the
 * engine's LinOutBlock, engine/exl3/exl3.h:69-82) or fp16(RoundH(WHT128(RoundH(y_raw)) *
 * norm) * svh) (CX_F16, ref/exl3_ref.py:153-156, 175), per 128-block.  The parity hook for
 * the output transform cx_exl3_linear runs.  y_raw fp32 [M][out_features]; y [M][out_features]. */
int cx_exl3_output_transform(const cx_exl3_matrix* m, const float* y_raw, int32_t M, void* y, int32_t y_dtype,
                             cx_stream_t stream);

/* y = EXL3 linear of M packed activation rows.  Replaces `Build` + `RunGroup`
 * (engine/engine.hip:1046, 1731) over one `LinJob` with R = M rows, i.e. LinInKernel
 * -> split-K GEMV -> LinOutKernel (engine/exl3/exl3.h:48-82, 330-389).
 *   x         x_dtype CX_F16 or CX_F32, [M][ldx], ldx >= in_features, ldx % 8 == 0; fp32 rows
 *             are rounded to fp16 inside the input transform (LinInLane's RoundH of the
 *             engine's fp32 `src`, engine/exl3/exl3.h:60-64), no separate conversion pass
 *   row_offsets  host, nullable: n_sessions + 1 exclusive prefix sums of the rows each
 *             session packed (ragged verify spans); checked, must end at M
 *   y_dtype   CX_F32: y_h kept fp32 through the output transform (engine LinOutBlock);
 *             CX_F16: y_h rounded to fp16 before it (ref/exl3_ref.py:175 default)
 *   workspace device scratch of cx_exl3_linear_workspace_size(m, M) bytes */
size_t cx_exl3_linear_workspace_size(const cx_exl3_matrix* m, int32_t M);
int cx_exl3_linear(const cx_exl3_matrix* m, const void* x, int32_t x_dtype, int32_t ldx, int32_t M,
                   const int32_t* row_offsets,
                   int32_t n_sessions, void* y, int32_t y_dtype, void* workspace, size_t workspace_bytes,
                   cx_stream_t stream);

/* Router: top-k of E fp32 logits per row (logit descending, lower id on ties), the
 * selection softmax w_k = exp(l_k - l_0) / sum_j exp(l_j - l_0), and w_topk =
 * sigmoid(shared logit).  Replaces MoeRouteKernel (engine/layers/ops.h:683-713) and
 * PrefillMoeRouteWaveKernel (engine/layers/prefill_moe.h:567-615).
 *   logits        fp32 [M][ld], ld >= E
 *   shared_logit  fp32 [M], nullable: then column E of logits (ld >= E + 1), the
 *                 engine's [M][E+1] router output layout
 *   sel int32 [M][topk], wts fp32 [M][topk + 1] */
int cx_moe_route(const float* logits, int32_t ld, int32_t M, int32_t E, int32_t topk, const float* shared_logit,
                 int32_t* sel, float* wts, cx_stream_t stream);

/* Stable expert-major grouping with on-device prefix sums (no host round trip).
 * counts [E], exclusive offsets [E+1], pairs [M*topk] (row * topk + slot, stable by
 * route index), row_ids [M*topk] (pairs / topk).  sel values must lie in [0, E): the
 * kernels check every id before using it, and a route with an id outside that range is
 * dropped (not counted, given no position), so offsets[E] < M * topk reports it and the
 * entries of pairs / row_ids from offsets[E] on are not written.  cx_moe_route never
 * produces such ids; the reference traps on them (engine/layers/moe_rows.h:31, 35).  Replaces the MoeDispatch kernels
 * (engine/layers/kernels/prefill_moe.h:9-100); oracle ref/prefill_ref.py:37-45. */
size_t cx_moe_group_workspace_size(int32_t M, int32_t E, int32_t topk);
int cx_moe_group(const int32_t* sel, int32_t M, int32_t E, int32_t topk, int32_t* counts, int32_t* offsets,
                 int32_t* pairs, int32_t* row_ids, void* workspace, size_t workspace_bytes, cx_stream_t stream);

/* A SwiGLU expert: gate [H][I], up [H][I], down [I][H].  Replaces `ExpertPtrs`
 * (engine/layers/ops.h:673-678). */
typedef struct cx_moe_expert {
  cx_exl3_matrix gate, up, down;
} cx_moe_expert;

/* A group of EXL3 linears applied to the same M rows, each with its own input and output
 * (e.g. the attention projections or the expert matrices of one decode step): one input-
 * transform launch for all jobs, one decode-GEMM launch per rate and codebook (up to 12
 * jobs each), one output-transform launch for all jobs.  Replaces Build + RunGroup over
 * LinJobs (engine/engine.hip:1046-1106, 1731-1746; engine/exl3/exl3.h:20-41, the group's
 * LinPolicyKernel launch engine/exl3/exl3.h:328-389).  fp32 inputs are rounded to fp16
 * before the input transform, as the reference's fp32 sources are.
 *   x   [M][ldx] of x_dtype (CX_F16 / CX_F32), y [M][ldy] of y_dtype; ldx, ldy multiples of 8
 *   at most 16 jobs; workspace per cx_exl3_group_workspace_size */
typedef struct cx_exl3_job {
  cx_exl3_matrix m;
  const void* x;
  int32_t x_dtype;
  int32_t ldx;
  void* y;
  int32_t y_dtype;
  int32_t ldy;
} cx_exl3_job;
size_t cx_exl3_group_workspace_size(const cx_exl3_job* jobs, int32_t n_jobs, int32_t M);
int cx_exl3_group(const cx_exl3_job* jobs, int32_t n_jobs, int32_t M, const int32_t* row_offsets, int32_t n_sessions,
                  void* workspace, size_t workspace_bytes, cx_stream_t stream);

/* Dense fp16-weight linear y[r][o] = W[o] . x[r] for r < M, o < O: the MoE router
 * (W = [E + 1][H], the shared-expert gate logit as output E).  Replaces LaunchDense
 * (engine/engine.hip:1824-1870) over DenseGemvKernel (engine/layers/ops.h:30-61) and the
 * prefill dense kernels.  Up to 8 rows of fp32 x: fp32 products and sums; otherwise x is
 * rounded to fp16 (as the reference packs it) and multiplied on MFMA with fp32 sums.
 *   W   fp16 [O][I] row-major, I a multiple of 32
 *   x   x_dtype CX_F32 / CX_F16, [M][ldx]   (fp32 rows 16-byte aligned: ldx % 4 == 0)
 *   y   fp32 [M][ldy] */
int cx_dense_linear(const uint16_t* W, int32_t O, int32_t I, const void* x, int32_t x_dtype, int32_t ldx, int32_t M,
                    float* y, int32_t ldy, cx_stream_t stream);

/* One MoE layer.  `experts` is a HOST array of E routed experts; the shared expert is
 * always on (slot topk).  Every routed expert must share the gate/up and the down
 * bitrate and codebook (the shared expert may differ).  Replaces `Moe`
 * (engine/model/flashnext/model.h:71-76). */
typedef struct cx_moe_layer {
  int32_t hidden;        /* H, multiple of 128 */
  int32_t intermediate;  /* I, multiple of 128 */
  int32_t n_experts;     /* E */
  int32_t topk;          /* k */
  const cx_moe_expert* experts; /* host [E] */
  cx_moe_expert shared;
} cx_moe_layer;

/* Prepared (device-resident) expert tables of a layer: built once, reused by every
 * call.  Replaces the d_experts upload (engine/model/flashnext/model.h:75).  The plan
 * keeps packed device copies of every expert's suh / svh vectors taken at creation
 * (2 H + 3 I halves per expert); the tiles are referenced, not copied.  Synchronous. */
typedef struct cx_moe_plan cx_moe_plan;
int cx_moe_plan_create(const cx_moe_layer* layer, cx_moe_plan** plan);
void cx_moe_plan_destroy(cx_moe_plan* plan);

/* y = MoE layer over M packed rows: route, group, gate/up, SiLU * up, down, and the
 * weighted combine (routed slots in selection order, shared expert last, fp32).
 * Replaces Engine::BlockMoe (engine/engine.hip:1327-1342, decode) and the MoE half of
 * Engine::PrefillBlock (engine/runtime/prefill_engine.inc:365-435, prefill).
 *   x             hidden states [M][ldx] of x_dtype: CX_F32 (the engine's fp32 residual-mixed
 *                 x_, engine/engine.hip:1332; each value is rounded to fp16 inside the input
 *                 transform as MoeRowsInSlotsKernel does, engine/layers/moe_rows.h:118-121)
 *                 or CX_F16; ldx >= H, ldx % 8 == 0
 *   logits        fp32 [M][ld] router logits (see cx_moe_route for shared_logit)
 *   row_offsets   host, nullable: session prefix sums, checked, must end at M
 *   y             fp32 [M][H]
 *   sel, wts      nullable outputs: int32 [M][topk] and fp32 [M][topk + 1]
 *   mode          CX_MOE_DECODE / PREFILL / AUTO (by M) */
size_t cx_moe_layer_workspace_size(const cx_moe_plan* plan, int32_t M, int32_t mode);
int cx_moe_layer_forward(const cx_moe_plan* plan, const void* x, int32_t x_dtype, int32_t ldx, const float* logits,
                         int32_t ld,
                 const float* shared_logit, int32_t M, const int32_t* row_offsets, int32_t n_sessions, float* y,
                 int32_t* sel, float* wts, int32_t mode, void* workspace, size_t workspace_bytes, cx_stream_t stream);

/* The layer without a workspace argument, for callers that cannot allocate (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  No
 * counterpart in the reference.  The workspace is a static device array of
 * CX_STATIC_SCRATCH_BYTES inside the library (one per GPU, held until the process ends;
 * its address is looked up when the first plan is created on that GPU); the call
 * allocates nothing.  Returns CX_E_WORKSPACE when cx_moe_layer_workspace_size(plan, M,
 * mode) exceeds CX_STATIC_SCRATCH_BYTES (at H = 2048, I = 512, top-10: decode calls up to
 * M = 64 rows fit).  Every call on one GPU shares the array: calls that overlap in time on
 * one GPU (other streams, other host threads) race and must be serialised by the caller.
 * Nothing in the array needs to start at zero.  Arguments as for cx_moe_layer_forward. */
#define CX_STATIC_SCRATCH_BYTES (24 << 20)
int cx_moe_layer_forward_static(const cx_moe_plan* plan, const void* x, int32_t x_dtype, int32_t ldx,
                                const float* logits, int32_t ld, const float* shared_logit, int32_t M,
                                const int32_t* row_offsets, int32_t n_sessions, float* y, int32_t* sel, float* wts,
                                int32_t mode, cx_stream_t stream);

/* The same layer with the reference's residual write-back in place of storing y:
 * H[r][s][c] += post[r][s] * y[r][c] for the n_streams hyper-connection streams of row r
 * (H row r at H + r * ldh, stream s at + s * H-width; ldh >= n_streams * hidden), fp32.
 * H is read and written in 16-byte pieces: H must be 16-byte aligned and ldh % 4 == 0.
 * Replaces the combine's write-back in MoeRowsCombineKernel (engine/layers/moe_rows.h:
 * 672-681) and PrefillMoeCombineKernel (engine/layers/prefill_moe.h:670-679).
 *   post          fp32 [M][n_streams] */
int cx_moe_layer_forward_hc(const cx_moe_plan* plan, const void* x, int32_t x_dtype, int32_t ldx,
                            const float* logits, int32_t ld,
                            const float* shared_logit, int32_t M, const int32_t* row_offsets, int32_t n_sessions,
                            const float* post, int32_t n_streams, float* H, int64_t ldh, int32_t* sel, float* wts,
                            int32_t mode, void* workspace, size_t workspace_bytes, cx_stream_t stream);

/* Stage tracing (the reference's per-stage hipEvent marks, engine/engine.hip:2086-2095,
 * stages named at engine/engine.hip:1349-1363).  With n_events > 0 every
 * cx_moe_layer_forward records CX_MOE_TRACE_MARKS events on its stream, into the caller's
 * hipEvent_t array used as a ring: mark 0 before the router, then one after each stage:
 * route, group, input transform, gate/up GEMM, mid, down GEMM, combine.  The plan keeps a
 * copy of the handles; n_events = 0 turns tracing off. */
#define CX_MOE_TRACE_MARKS 8
int cx_moe_plan_set_trace(cx_moe_plan* plan, void* const* events, int32_t n_events);

/* ---- checkpoints (host) and the EXL3 linear loader -------------------------------------
 * A checkpoint is one .safetensors file or a directory with model.safetensors.index.json
 * and its shards; every shard is memory-mapped read-only until cx_checkpoint_close.
 * Headers are parsed and every tensor is checked when the checkpoint opens (dtype known,
 * shape x dtype == data_offsets span inside the payload, unique names, shard names plain
 * file names).  Replaces st::Checkpoint (engine/exl3/safetensors.h) for the expert
 * weights.  Errors return CX_E_FORMAT with the file, tensor and reason in cx_last_error. */
enum {
  CX_DT_BOOL = 0, CX_DT_U8 = 1, CX_DT_I8 = 2, CX_DT_I16 = 3, CX_DT_U16 = 4, CX_DT_F16 = 5, CX_DT_BF16 = 6,
  CX_DT_I32 = 7, CX_DT_U32 = 8, CX_DT_F32 = 9, CX_DT_I64 = 10, CX_DT_U64 = 11, CX_DT_F64 = 12
};
#define CX_MAX_RANK 8
typedef struct cx_checkpoint cx_checkpoint;
int cx_checkpoint_open(const char* path, cx_checkpoint** ck);
void cx_checkpoint_close(cx_checkpoint* ck);
/* Tensor names in sorted order: i in [0, cx_checkpoint_count). */
int32_t cx_checkpoint_count(const cx_checkpoint* ck);
const char* cx_checkpoint_name(const cx_checkpoint* ck, int32_t i);
/* dtype (CX_DT_*), rank, shape (CX_MAX_RANK entries), host pointer to the mapped bytes;
 * any output may be NULL. */
int cx_checkpoint_tensor(const cx_checkpoint* ck, const char* name, int32_t* dtype, int32_t* rank, int64_t* shape,
                         const void** data, uint64_t* bytes);
/* Validates the EXL3 linear `prefix` (docs/EXL3_FORMAT.md §2: prefix.trellis I16
 * [I/16][O/16][16 K], prefix.suh F16 [I], prefix.svh F16 [O], marker prefix.mul1 =
 * 0x83DCD12D or prefix.mcg = 0xCBAC1FED as I32 scalars, neither = 3inst; I, O multiples of
 * 128) and returns its geometry.  The loader check of engine/model/flashnext/model.h:503-512. */
int cx_exl3_linear_info(const cx_checkpoint* ck, const char* prefix, int32_t* in_features, int32_t* out_features,
                        int32_t* k2, int32_t* codebook);
/* Uploads the linear into caller-owned device buffers (tiles: cx_exl3_tile_bytes; suh,
 * svh: I and O halves; staging: at least the trellis bytes, I O K / 8) and repacks it on
 * the device; *m describes the result.  Returns after the uploads finished.  Replaces the
 * repack-on-load of engine/model/flashnext/model.h:513-527. */
int cx_exl3_load_linear(const cx_checkpoint* ck, const char* prefix, cx_exl3_matrix* m, uint32_t* tiles,
                        uint16_t* suh, uint16_t* svh, void* staging, size_t staging_bytes, cx_stream_t stream);
/* The reason for the calling thread's last CX_E_FORMAT (or other checkpoint) error. */
const char* cx_last_error(void);

/* Library version string. */
const char* cx_version(void);

#ifdef __cplusplus
}
#endif
#endif /* CRUCIBLE_EXL3_H */
