// EXL3 MoE layer on MI355X: router top-k, stable expert-major grouping built on the
// device (prefix sums and GEMM work lists, no host round trip), per-expert input
// transforms, grouped gate/up decode-GEMM, mid (SiLU * up + down input transform),
// grouped down decode-GEMM, and the weighted combine with the shared expert.
//
// Row space of one call with M rows and top-k routing: P = M k + M "compact rows".
// Rows [0, M k) are the routed (row, slot) pairs in stable expert-major order (pairs[]),
// rows [M k, M k + M) are the shared expert's rows 0..M-1.  Every expert's rows are
// contiguous, so an expert GEMM reads one contiguous block of activation rows.
#include <cstdlib>
#include <mutex>
#include <new>

#include "internal.hpp"

namespace cx {

constexpr int kMaxExperts = 1024;
constexpr int kMaxTopK = 32;
constexpr int kSmallRoutes = 2048;  // single-workgroup grouping up to this many routes

// ---- router ---------------------------------------------------------------------------

// True when (va, ia) ranks before (vb, ib): logit descending, lower expert id on ties.
__device__ __forceinline__ bool RanksBefore(float va, int ia, float vb, int ib) {
  return va > vb || (va == vb && ia < ib);
}

// Sorts a lane's V candidates into rank order (Batcher's odd-even merge sort, V a power
// of two; the compare-exchanges of one stage are independent).
template <int V>
__device__ __forceinline__ void SortLane(float (&v)[V], int (&id)[V]) {
#pragma unroll
  for (int p = 1; p < V; p <<= 1)
#pragma unroll
    for (int k = p; k >= 1; k >>= 1)
#pragma unroll
      for (int j = k % p; j + k < V; j += 2 * k)
#pragma unroll
        for (int i = 0; i < k; ++i) {
          const int a = i + j, b = i + j + k;
          if (b < V && a / (2 * p) == b / (2 * p)) {
            const bool sw = RanksBefore(v[b], id[b], v[a], id[a]);
            const float va = v[a];
            const int ia = id[a];
            v[a] = sw ? v[b] : va;
            id[a] = sw ? id[b] : ia;
            v[b] = sw ? va : v[b];
            id[b] = sw ? ia : id[b];
          }
        }
}

// Routes one row with one wave: top-k of E logits by (logit descending, id ascending),
// then the selection softmax exp(l_k - l_0) / sum_j exp(l_j - l_0) summed in rank order,
// and sigmoid of the shared logit.  engine/layers/ops.h:683-713.  Lane l holds logits
// l, l + 64, ... (E <= 64 V), sorted per lane once; each of the k rounds takes the wave
// maximum of the lane heads, and the winning lane (the only one holding the max, or the
// lowest id among equal maxima) pops its head.  NaN logits rank as -inf.
// Writes sel_row[0..k), wts_row[0..k] (unless sel_row is null) and, if s_row is given,
// s_row[0..k) (LDS copy).
template <int V>
__device__ __forceinline__ void RouteRowWave(const float* __restrict__ lg, int E, int topk, float shared,
                                             int* __restrict__ sel_row, float* __restrict__ wts_row, int* s_row) {
  const int lane = threadIdx.x & 63;
  float v[V];
  int id[V];
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int e = i * 64 + lane;
    const float x = e < E ? lg[e] : -INFINITY;
    v[i] = x == x ? x : -INFINITY;
    id[i] = e;
  }
  SortLane<V>(v, id);
  float mine = 0.f, top = 0.f;
  int myid = 0;
  for (int k = 0; k < topk; ++k) {
    const float mx = WaveMaxF(v[0]);
    const unsigned long long tie = __ballot(v[0] == mx);
    int win;
    if (__popcll(tie) == 1)
      win = __builtin_amdgcn_readlane(id[0], __ffsll((long long)tie) - 1);
    else
      win = WaveMinI(v[0] == mx ? id[0] : 0x7fffffff);
    if (id[0] == win) {  // ids are unique across the wave: the winning lane only
#pragma unroll
      for (int i = 0; i + 1 < V; ++i) {
        v[i] = v[i + 1];
        id[i] = id[i + 1];
      }
      v[V - 1] = -INFINITY;
      id[V - 1] = 0x7fffffff;
    }
    if (lane == k) {
      mine = mx;
      myid = win;
    }
    if (k == 0) top = mx;
  }
  const float ex = lane < topk ? __expf(mine - top) : 0.f;
  float sum = 0.f;
  for (int k = 0; k < topk; ++k) sum += __shfl(ex, k, 64);
  if (lane < topk) {
    if (sel_row) {
      sel_row[lane] = myid;
      wts_row[lane] = ex / sum;
    }
    if (s_row) s_row[lane] = myid;
  }
  if (lane == 0 && wts_row) wts_row[topk] = Sigmoid(shared);
}

// One wave per row; blockDim.x / 64 rows per workgroup.
template <int V>
__global__ void __launch_bounds__(256) RouteKernel(const float* __restrict__ logits, int ld, int M, int E, int topk,
                                                   const float* __restrict__ shared_logit, int* __restrict__ sel,
                                                   float* __restrict__ wts) {
  const int row = blockIdx.x * (int)(blockDim.x >> 6) + (int)(threadIdx.x >> 6);
  if (row >= M) return;  // whole waves leave together
  const float* lg = logits + (size_t)row * ld;
  RouteRowWave<V>(lg, E, topk, shared_logit ? shared_logit[row] : lg[E], sel + (size_t)row * topk,
                  wts + (size_t)row * (topk + 1), nullptr);
}

struct ExpertTables {
  const MatPtr* gate;  // [E + 1], index E = shared expert
  const MatPtr* up;
  const MatPtr* down;
  // Packed copies of the scale vectors, expert-major ([E + 1][H] or [E + 1][I]): the
  // transforms address them from the expert index alone, one dependent load fewer than
  // through the pointer tables.
  const __half* gate_suh;
  const __half* up_suh;
  const __half* gate_svh;
  const __half* up_svh;
  const __half* down_suh;
};

// ---- grouping --------------------------------------------------------------------------

struct GroupOut {
  int* counts;     // [E]
  int* offsets;    // [E + 1]
  int* pairs;      // [n]  route index (row * topk + slot) in expert-major stable order
  int* row_ids;    // [n]  pairs / topk
  int* inv;        // [n]  position of route i in pairs (nullable)
  int* expert;     // [n]  expert of compact row p (nullable)
  int4* entries;   // GEMM row entries (nullable): shared chunks first, then per-expert chunks
  int* n_entries;  // total entries
  int chunk;       // rows per entry
  int M, topk, E;
  int max_entries;  // entries [n_entries, max_entries) are written empty (rows = 0)
  int* zero;        // the decode stage launch's nzero counters, zero[i * kStageCtrStride], which the
  int nzero;        // grouping sets to 0 (nullable)
};

// Empty entries after the last real one, so a GEMM launched over max_entries rows of the
// table needs no entry count (an entry with 0 rows ends its workgroup).
__device__ void FillEmptyEntries(const GroupOut& o, int n_real) {
  for (int i = n_real + (int)threadIdx.x; i < o.max_entries; i += blockDim.x) o.entries[i] = make_int4(0, 0, 0, 0);
}

// Shared-expert entries [0, ceil(M / chunk)), then expert e's ceil(count / chunk) chunks,
// in expert order.  nch_base[e]: exclusive prefix of per-expert chunk counts.
__device__ void WriteEntries(const GroupOut& o, int e, int nch_base, int count, int offset) {
  const int nsh = (o.M + o.chunk - 1) / o.chunk;
  for (int c = 0; c * o.chunk < count; ++c)
    o.entries[nsh + nch_base + c] = make_int4(e, offset + c * o.chunk, min(o.chunk, count - c * o.chunk), 0);
}
__device__ void WriteSharedEntries(const GroupOut& o, int t, int nt) {
  const int nsh = (o.M + o.chunk - 1) / o.chunk;
  const int base = o.M * o.topk;
  for (int c = t; c < nsh; c += nt) o.entries[c] = make_int4(o.E, base + c * o.chunk, min(o.chunk, o.M - c * o.chunk), 0);
}

// Exclusive block scan of one int per thread (blockDim.x == 1024); returns the prefix,
// *total gets the sum.
__device__ int BlockExclusiveScan(int v, int* scratch, int* total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(x, d, 64);
    if (lane >= d) x += y;
  }
  if (lane == 63) scratch[w] = x;
  __syncthreads();
  if (threadIdx.x < 64) {
    const int nw = blockDim.x >> 6;
    int s = threadIdx.x < nw ? scratch[threadIdx.x] : 0;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int y = __shfl_up(s, d, 64);
      if ((int)threadIdx.x >= d) s += y;
    }
    if (threadIdx.x < nw) scratch[64 + threadIdx.x] = s;
  }
  __syncthreads();
  const int before = (w ? scratch[64 + w - 1] : 0) + x - v;
  *total = scratch[64 + (blockDim.x >> 6) - 1];
  __syncthreads();
  return before;
}

// Stable append of one route per thread (route index i in thread order; e < 0: none):
// its position is cursor[e] + (routes of expert e in earlier waves) + (earlier lanes of
// this wave with expert e).  Lanes of one expert are found by ballots over the id bits;
// the waves take their cursor ranges in wave order, so positions follow route order.
// Returns the position (or -1).  All threads of the block must call it.
// nw: waves that may hold valid routes (the others have e < 0); uniform over the block.
__device__ int StableAppend(int e, int* cursor, int nw) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const bool valid = e >= 0;
  unsigned long long peers = __ballot(valid);
#pragma unroll
  for (int b = 0; b < 10; ++b) {
    const bool bit = (e >> b) & 1;
    const unsigned long long bb = __ballot(bit);
    peers &= bit ? bb : ~bb;
  }
  const int rank = __popcll(peers & ((1ull << lane) - 1ull));
  const int leader = valid ? __ffsll((long long)peers) - 1 : lane;
  int base = 0;
  for (int ww = 0; ww < nw; ++ww) {
    if (w == ww && valid && rank == 0) base = atomicAdd(&cursor[e], __popcll(peers));
    __syncthreads();
  }
  base = __shfl(base, leader, 64);
  return valid ? base + rank : -1;
}

// An expert id in [0, E), or -1 for an id outside it (such a route is dropped).
__device__ __forceinline__ int ValidExpert(int e, int E) { return (unsigned)e < (unsigned)E ? e : -1; }

__device__ void WritePair(const GroupOut& o, int p, int i, int e) {
  o.pairs[p] = i;
  o.row_ids[p] = i / o.topk;
  if (o.inv) o.inv[i] = p;
  if (o.expert) o.expert[p] = e;
}

// Whole grouping in one 1024-thread workgroup (up to kSmallRoutes routes); sel may be
// in global memory or in LDS.  ref/prefill_ref.py:37-45.
__device__ void GroupSmallBody(const int* sel, const GroupOut& o, int* s_cur, int* s_scan) {
  const int n = o.M * o.topk;
  for (int i = threadIdx.x; i < o.nzero; i += blockDim.x) o.zero[i * kStageCtrStride] = 0;
  for (int e = threadIdx.x; e < o.E; e += blockDim.x) s_cur[e] = 0;
  __syncthreads();
  for (int i = threadIdx.x; i < n; i += blockDim.x) {  // counts only; ids outside [0, E) are dropped
    const int e = sel[i];
    if ((unsigned)e < (unsigned)o.E) atomicAdd(&s_cur[e], 1);
  }
  __syncthreads();
  const int e = threadIdx.x;
  const int cnt = e < o.E ? s_cur[e] : 0;
  const int nch = o.entries ? (cnt + o.chunk - 1) / o.chunk : 0;
  // Route and chunk counts scanned together (both < 2^16 here).
  int packed = 0;
  const int pre = BlockExclusiveScan(cnt | (nch << 16), s_scan, &packed);
  const int off = pre & 0xffff, chb = pre >> 16;
  const int total = packed & 0xffff, ctotal = packed >> 16;
  if (e < o.E) {
    o.counts[e] = cnt;
    o.offsets[e] = off;
    s_cur[e] = off;
    if (o.entries) WriteEntries(o, e, chb, cnt, off);
  }
  if (e == 0) o.offsets[o.E] = total;
  if (o.entries) {
    WriteSharedEntries(o, threadIdx.x, blockDim.x);
    if (threadIdx.x == 0) *o.n_entries = (o.M + o.chunk - 1) / o.chunk + ctotal;
    FillEmptyEntries(o, (o.M + o.chunk - 1) / o.chunk + ctotal);
  }
  __syncthreads();
  for (int base = 0; base < n; base += blockDim.x) {
    const int i = base + threadIdx.x;
    const int e = i < n ? ValidExpert(sel[i], o.E) : -1;
    const int p = StableAppend(e, s_cur, min((int)blockDim.x, n - base + 63) >> 6);
    if (p >= 0) WritePair(o, p, i, e);
  }
}

__global__ void __launch_bounds__(1024) GroupSmallKernel(const int* __restrict__ sel, GroupOut o) {
  __shared__ int s_cur[kMaxExperts];
  __shared__ int s_scan[128];
  GroupSmallBody(sel, o, s_cur, s_scan);
}

// The gate and up input transforms of one lane's 8 elements of a 128-block (signed
// form, before the norm): x, suh_gate, suh_up as 8 packed fp16 each.  RoundH(x * suh) is
// the fp16 product (an fp16 x fp16 product is exact in fp32, so one fp16 rounding).
template <bool PHI = false>
__device__ __forceinline__ void InputPairTransform(const uint4& x, const uint4& sg, const uint4& su, float a[8],
                                                   float v[8]) {
  const uint32_t hx[4] = {x.x, x.y, x.z, x.w};
  const uint32_t hg[4] = {sg.x, sg.y, sg.z, sg.w};
  const uint32_t hu[4] = {su.x, su.y, su.z, su.w};
  uint32_t pa[4], pv[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    pa[k] = __builtin_bit_cast(uint32_t, __hmul2(__builtin_bit_cast(__half2, hx[k]), __builtin_bit_cast(__half2, hg[k])));
    pv[k] = __builtin_bit_cast(uint32_t, __hmul2(__builtin_bit_cast(__half2, hx[k]), __builtin_bit_cast(__half2, hu[k])));
  }
  Wht128x8SignedH<PHI>(pa, a);
  Wht128x8SignedH<PHI>(pv, v);
}

// Decode: grouping and the gate/up input transforms in one launch, after routing.
// Workgroup 0 groups all rows (GroupSmallBody); the other workgroups, a few per row, write
// the gate and up input transforms (engine/exl3/exl3.h:48-65: RoundH(x * suh) -> WHT128 ->
// * norm, fp16 in MFMA row order) of row r's k routed slots and of the shared expert, in
// route order: row r * k + slot, shared expert row M k + r.  The transforms need only the
// row's own selection, so the workgroups are independent; the gate/up GEMM gathers its
// compact rows through pairs[].
__global__ void __launch_bounds__(1024) GroupInputKernel(const int* __restrict__ sel, const void* __restrict__ x,
                                                         int xf32, long long ldx, ExpertTables tb, int H,
                                                         __half* __restrict__ xg,
                                                         __half* __restrict__ xu, GroupOut o) {
  __shared__ int s_e[kMaxTopK + 1];
  __shared__ int s_cur[kMaxExperts];
  __shared__ int s_scan[128];
  if (blockIdx.x == 0) {
    GroupSmallBody(sel, o, s_cur, s_scan);
    return;
  }
  const int topk = o.topk, M = o.M, nb = H / 128, j = threadIdx.x & 15;
  const int items = (topk + 1) * nb, per = blockDim.x >> 4;  // (slot, 128-block) items of a row
  const int wpr = (items + per - 1) / per;                    // workgroups per row
  const int row = (blockIdx.x - 1) / wpr, part = (blockIdx.x - 1) % wpr;
  if ((int)threadIdx.x <= topk) s_e[threadIdx.x] = (int)threadIdx.x < topk ? sel[(size_t)row * topk + threadIdx.x] : o.E;
  __syncthreads();
  const size_t xr = (size_t)row * ldx;
  for (int it = part * per + (threadIdx.x >> 4); it < min(items, (part + 1) * per); it += per) {
    const int slot = it / nb, blk = it % nb;
    const int e = s_e[slot];
    const size_t q = slot < topk ? (size_t)row * topk + slot : (size_t)M * topk + row;
    const int c0 = blk * 128 + 8 * j;
    float a[8], v[8];
    InputPairTransform(LoadAsH8(x, xf32, xr + c0),
                       *reinterpret_cast<const uint4*>(tb.gate_suh + (size_t)e * H + c0),
                       *reinterpret_cast<const uint4*>(tb.up_suh + (size_t)e * H + c0), a, v);
    StorePerm32x8(xg + q * H + blk * 128, a, kHadNorm * WhtLaneSign());
    StorePerm32x8(xu + q * H + blk * 128, v, kHadNorm * WhtLaneSign());
  }
}

// Routing, grouping and the input transforms of a decode call in one launch.  Workgroup 0
// routes every row (16 waves, rows r, r + 16, ...), writes sel and wts, keeps the
// selections in LDS and groups from there; every other workgroup routes its own row with
// its first wave (the same deterministic result, kept in LDS only) and writes that row's
// gate/up input transforms in route order, as GroupInputKernel does.
template <int V>
__global__ void __launch_bounds__(1024) RouteGroupInputKernel(const float* __restrict__ logits, int ld,
                                                              const float* __restrict__ shared_logit,
                                                              int* __restrict__ sel, float* __restrict__ wts,
                                                              const void* __restrict__ x, int xf32, long long ldx,
                                                              ExpertTables tb, int H, __half* __restrict__ xg,
                                                              __half* __restrict__ xu, GroupOut o) {
  __shared__ int s_sel[kSmallRoutes];
  __shared__ int s_cur[kMaxExperts];
  __shared__ int s_scan[128];
  const int topk = o.topk, M = o.M, E = o.E;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (blockIdx.x == 0) {
    for (int r = wave; r < M; r += 16) {
      const float* lg = logits + (size_t)r * ld;
      RouteRowWave<V>(lg, E, topk, shared_logit ? shared_logit[r] : lg[E], sel + (size_t)r * topk,
                      wts + (size_t)r * (topk + 1), s_sel + r * topk);
    }
    __syncthreads();
    GroupSmallBody(s_sel, o, s_cur, s_scan);
    return;
  }
  const int nb = H / 128, j = threadIdx.x & 15;
  const int items = (topk + 1) * nb, per = blockDim.x >> 4;
  const int wpr = (items + per - 1) / per;
  const int row = (blockIdx.x - 1) / wpr, part = (blockIdx.x - 1) % wpr;
  int* s_e = s_sel;
  if (wave == 0) {
    const float* lg = logits + (size_t)row * ld;
    RouteRowWave<V>(lg, E, topk, shared_logit ? shared_logit[row] : lg[E], nullptr, nullptr, s_e);
    if (lane == 0) s_e[topk] = E;
  }
  (void)lane;
  __syncthreads();
  const size_t xr = (size_t)row * ldx;
  for (int it = part * per + (threadIdx.x >> 4); it < min(items, (part + 1) * per); it += per) {
    const int slot = it / nb, blk = it % nb;
    const int e = s_e[slot];
    const size_t q = slot < topk ? (size_t)row * topk + slot : (size_t)M * topk + row;
    const int c0 = blk * 128 + 8 * j;
    float a[8], v[8];
    InputPairTransform(LoadAsH8(x, xf32, xr + c0),
                       *reinterpret_cast<const uint4*>(tb.gate_suh + (size_t)e * H + c0),
                       *reinterpret_cast<const uint4*>(tb.up_suh + (size_t)e * H + c0), a, v);
    StorePerm32x8(xg + q * H + blk * 128, a, kHadNorm * WhtLaneSign());
    StorePerm32x8(xu + q * H + blk * 128, v, kHadNorm * WhtLaneSign());
  }
}

// Multi-workgroup grouping for long prefill chunks: per-tile histograms, one scan, and
// a stable in-tile scatter.  Tiles hold 1024 routes.
constexpr int kTile = 1024;

__global__ void __launch_bounds__(1024) GroupCountKernel(const int* __restrict__ sel, int n, int E, int ntiles,
                                                         int* __restrict__ tile_counts) {
  __shared__ int h[kMaxExperts];
  for (int e = threadIdx.x; e < E; e += blockDim.x) h[e] = 0;
  __syncthreads();
  const int i = blockIdx.x * kTile + threadIdx.x;
  if (i < n) {  // counts only; never decides order
    const int e = ValidExpert(sel[i], E);
    if (e >= 0) atomicAdd(&h[e], 1);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += blockDim.x) tile_counts[(size_t)e * ntiles + blockIdx.x] = h[e];
}

// Scan and scatter in one launch, one workgroup per tile: every workgroup reads all tile
// histograms (ntiles x E counts, a few tens of KB from L2) and scans them itself in
// (expert, tile) order for its own tile bases, so no separate scan launch has to finish
// first, then does a stable in-tile scatter.  One extra workgroup (index ntiles) writes
// counts, offsets and the GEMM entries meanwhile.
__global__ void __launch_bounds__(1024) GroupScatterKernel(const int* __restrict__ sel,
                                                           const int* __restrict__ tile_counts, int ntiles,
                                                           GroupOut o) {
  __shared__ int s_scan[128];
  __shared__ int s_cur[kMaxExperts];
  const int e = threadIdx.x, tile = blockIdx.x;
  int cnt = 0, before = 0;
  if (e < o.E) {
    // Independent loads issued 8 at a time (a dependent chain would wait ntiles times).
    const int* tc = tile_counts + (size_t)e * ntiles;
    int t = 0;
    for (; t + 8 <= ntiles; t += 8) {
      int v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = tc[t + i];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        before += t + i < tile ? v[i] : 0;
        cnt += v[i];
      }
    }
    for (; t < ntiles; ++t) {
      const int v = tc[t];
      before += t < tile ? v : 0;
      cnt += v;
    }
  }
  int total = 0;
  const int off = BlockExclusiveScan(cnt, s_scan, &total);
  if (e < o.E) s_cur[e] = off + before;
  if (tile == ntiles) {  // the extra workgroup: counts, offsets, entries
    int ctotal = 0;
    const int nch = o.entries ? (cnt + o.chunk - 1) / o.chunk : 0;
    const int chb = BlockExclusiveScan(nch, s_scan, &ctotal);
    if (e < o.E) {
      o.counts[e] = cnt;
      o.offsets[e] = off;
      if (o.entries) WriteEntries(o, e, chb, cnt, off);
    }
    if (e == 0) o.offsets[o.E] = total;
    if (o.entries) {
      WriteSharedEntries(o, threadIdx.x, blockDim.x);
      if (threadIdx.x == 0) *o.n_entries = (o.M + o.chunk - 1) / o.chunk + ctotal;
      FillEmptyEntries(o, (o.M + o.chunk - 1) / o.chunk + ctotal);
    }
    return;
  }
  __syncthreads();
  const int n = o.M * o.topk;
  const int i = tile * kTile + threadIdx.x;
  const int se = i < n ? ValidExpert(sel[i], o.E) : -1;
  const int p = StableAppend(se, s_cur, min((int)blockDim.x, n - tile * kTile + 63) >> 6);
  if (p >= 0) WritePair(o, p, i, se);
}

// ---- activation transforms of the experts ----------------------------------------------

// Gate and up input transforms of every compact row (each matrix has its own suh):
// RoundH(x * suh) -> WHT128 -> * norm -> fp16 in MFMA row order.  S waves per compact
// row: its route and expert are looked up once per wave, then lane group g (16 lanes) of
// part t transforms the 128-blocks 4 t + g, 4 (t + S) + g, ... of both inputs (S = 1 for
// long calls; short calls split rows for parallelism).  Compact-row order keeps the
// writes sequential; walking routes in row order instead (reads shared, writes scattered
// in 4 KB pieces) measured 8% slower.  engine/layers/moe_rows.h:102-125.
template <bool XF32>
__global__ void __launch_bounds__(256) MoeInputKernel(const void* __restrict__ x, long long ldx,
                                                      const int* __restrict__ rexp,
                                                      const int* __restrict__ rows, ExpertTables tb, int M, int topk,
                                                      int E, int H, int S, __half* __restrict__ xg,
                                                      __half* __restrict__ xu) {
  __shared__ __align__(16) uint32_t tarea[4][256];  // per-wave transpose areas
  const int P = M * topk + M;
  const int w = blockIdx.x * 4 + (int)(threadIdx.x >> 6);
  const int p = w / S, part = w % S;
  if (p >= P) return;  // whole waves
  int row, e;
  if (p < M * topk) {  // row and expert of the compact row, written by the grouping
    row = __builtin_amdgcn_readfirstlane(rows[p]);
    e = __builtin_amdgcn_readfirstlane(rexp[p]);
  } else {
    row = p - M * topk;
    e = E;
  }
  const __half* sg = tb.gate_suh + (size_t)e * H;
  const __half* su = tb.up_suh + (size_t)e * H;
  // Lanes hold relabelled elements (PhiLane): the stride-32 butterfly is one DPP pattern.
  const int g = (threadIdx.x >> 4) & 3, j = PhiLane();
  const int nb = H / 128, st = 4 * S;
  // Every row touched here is addressed through a buffer resource on its (wave-uniform)
  // start: the lanes' offsets are 32-bit and each block's offset is the uniform soffset,
  // no 64-bit address arithmetic per load and store.
  constexpr int esz = XF32 ? 4 : 2;
  const __amdgpu_buffer_rsrc_t rxr =
      MakeRsrc(static_cast<const char*>(x) + (size_t)row * ldx * esz, (uint32_t)(H * esz));
  const __amdgpu_buffer_rsrc_t rsg = MakeRsrc(sg, (uint32_t)H * 2), rsu = MakeRsrc(su, (uint32_t)H * 2);
  const __amdgpu_buffer_rsrc_t rdg = MakeRsrc(xg + (size_t)p * H, (uint32_t)H * 2);
  const __amdgpu_buffer_rsrc_t rdu = MakeRsrc(xu + (size_t)p * H, (uint32_t)H * 2);
  // Up to 4 blocks per lane group at a time: all their loads are issued before the first
  // transform, so a wave keeps 12 16-byte loads in flight instead of 3.
  for (int b0 = 4 * part + g; b0 < nb; b0 += 4 * st) {
    const uint32_t e0 = (uint32_t)(b0 * 128 + 8 * j);  // the lane's first element, block b0
    uint4 rx[4], rg[4], ru[4];
    // Loads are unconditional: past the row's end they fall outside the buffer resource (no
    // memory access, zeros) and are not used.
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const uint32_t so = (uint32_t)(it * st * 128);  // block it's element offset (uniform)
        if constexpr (XF32) {
          const u32x4_t lo = BufLoad128(rxr, e0 * 4, so * 4), hi = BufLoad128(rxr, e0 * 4 + 16, so * 4);
          rx[it] = make_uint4(__builtin_bit_cast(uint32_t, __floats2half2_rn(__uint_as_float(lo[0]), __uint_as_float(lo[1]))),
                              __builtin_bit_cast(uint32_t, __floats2half2_rn(__uint_as_float(lo[2]), __uint_as_float(lo[3]))),
                              __builtin_bit_cast(uint32_t, __floats2half2_rn(__uint_as_float(hi[0]), __uint_as_float(hi[1]))),
                              __builtin_bit_cast(uint32_t, __floats2half2_rn(__uint_as_float(hi[2]), __uint_as_float(hi[3]))));
        } else {
          const u32x4_t u = BufLoad128(rxr, e0 * 2, so * 2);
          rx[it] = make_uint4(u[0], u[1], u[2], u[3]);
        }
        const u32x4_t a = BufLoad128(rsg, e0 * 2, so * 2), b = BufLoad128(rsu, e0 * 2, so * 2);
        rg[it] = make_uint4(a[0], a[1], a[2], a[3]);
        ru[it] = make_uint4(b[0], b[1], b[2], b[3]);
      }
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int blk = b0 + it * st;
      if (blk >= nb) break;  // uniform over the 16-lane group
      float a[8], v[8];
      InputPairTransform<true>(rx[it], rg[it], ru[it], a, v);
      const uint32_t so = (uint32_t)(it * st * 128) * 2;
      uint32_t* ta = tarea[threadIdx.x >> 6];
      StorePerm32x8LdsBuf<true>(ta, rdg, (uint32_t)(b0 * 128) * 2, so, a, kHadNorm * WhtLaneSign<true>());
      StorePerm32x8LdsBuf<true>(ta, rdu, (uint32_t)(b0 * 128) * 2, so, v, kHadNorm * WhtLaneSign<true>());
    }
  }
}

// Mid: gate and up output transforms (fp32), RoundH(RoundH(SiLU(g) * u) * suh_down),
// WHT128, * norm -> fp16 down input in MFMA row order.  engine/layers/moe_rows.h:543-566.
// One wave per compact row (lookups once); lane group g transforms 128-blocks g, g + 4, ...
__global__ void __launch_bounds__(256) MoeMidKernel(const float* __restrict__ yg, const float* __restrict__ yu,
                                                    const int* __restrict__ rexp,
                                                    ExpertTables tb, int M, int topk, int E, int I,
                                                    __half* __restrict__ xd) {
  const int P = M * topk + M;
  const int p = blockIdx.x * 4 + (int)(threadIdx.x >> 6);
  if (p >= P) return;  // whole waves
  const int e = p < M * topk ? __builtin_amdgcn_readfirstlane(rexp[p]) : E;
  const __half* svg_p = tb.gate_svh + (size_t)e * I;
  const __half* svu_p = tb.up_svh + (size_t)e * I;
  const __half* sud_p = tb.down_suh + (size_t)e * I;
  const int g = (threadIdx.x >> 4) & 3, j = threadIdx.x & 15;
  for (int blk = g; blk < I / 128; blk += 4) {
    const int c0 = blk * 128 + 8 * j;
    float gv[8], uv[8];
    LoadF8(yg + (size_t)p * I + c0, gv);
    LoadF8(yu + (size_t)p * I + c0, uv);
    MidBlock(gv, uv, svg_p + c0, svu_p + c0, sud_p + c0, xd + (size_t)p * I + blk * 128);
  }
}

// Residual write-back of the combine (hyper-connection streams): H row r, stream s at
// H + r * ldh + s * hidden gets H += post[r][s] * y[r].
struct HcArgs {
  const float* post;  // [M][n_streams]
  float* H;
  long long ldh;
  int n_streams;
};

// One combine weight step: acc + w * d with one rounding.
__device__ __forceinline__ float CombineStep(float acc, float w, float d) { return __builtin_fmaf(w, d, acc); }
// topk below this: every slot's row and weight are loaded at once (unrolled).
constexpr int kCombineSlots = 16;

// Combine: per row, slots 0..topk-1 in selection order then the shared expert:
// y += w_k * d_k, fp32, where d_k = WHT(y_h) * (norm * svh) came out of the down GEMM's
// epilogue: fp32 rows (decode), or fp16 rows with a power-of-two scale per 128-column
// block (F16, prefill: the reference's prefill keeps d_k in fp16 too,
// engine/layers/prefill_moe.h:648).  engine/layers/moe_rows.h:634-682.  HC: accumulate
// into the residual streams instead of storing y (engine/layers/moe_rows.h:672-681).
template <bool HC, bool F16>
__global__ void __launch_bounds__(256) MoeCombineKernel(const void* __restrict__ pd, const float* __restrict__ psc,
                                                        const float* __restrict__ wts, const int* __restrict__ inv,
                                                        int M, int topk, int H, float* __restrict__ y, HcArgs hc) {
  // Columns per thread: 8 for fp16 rows (one 16-byte load per slot), 4 for fp32 rows.
  constexpr int CW = F16 ? 8 : 4;
  const int nq = H / CW;
  const int item = blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= M * nq) return;
  const int r = item / nq, c0 = (item % nq) * CW;
  auto slot_row = [&](int k) { return k < topk ? inv[r * topk + k] : M * topk + r; };
  struct Cols {
    float v[CW];
  };
  auto load = [&](int p) {
    Cols d;
    if constexpr (F16) {
      const uint4 u = *reinterpret_cast<const uint4*>(static_cast<const __half*>(pd) + (size_t)p * H + c0);
      const float sc = psc[(size_t)p * (H / 128) + c0 / 128];
      const uint32_t h[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float2 f = __half22float2(__builtin_bit_cast(__half2, h[k]));
        d.v[2 * k] = f.x * sc;
        d.v[2 * k + 1] = f.y * sc;
      }
    } else {
      const float4 f = *reinterpret_cast<const float4*>(static_cast<const float*>(pd) + (size_t)p * H + c0);
      d.v[0] = f.x;
      d.v[1] = f.y;
      d.v[2] = f.z;
      d.v[3] = f.w;
    }
    return d;
  };
  float acc[CW];
#pragma unroll
  for (int i = 0; i < CW; ++i) acc[i] = 0.f;
  auto add = [&](float w, const Cols& d) {
#pragma unroll
    for (int i = 0; i < CW; ++i) acc[i] = CombineStep(acc[i], w, d.v[i]);
  };
  if (topk < kCombineSlots) {
    // All slot rows, then all their loads, issued before the first use (the rows and
    // weights of slots past topk repeat the last slot and are not added): one memory
    // latency per stage instead of one per slot.
    int p[kCombineSlots];
    float w[kCombineSlots];
    Cols d[kCombineSlots];
#pragma unroll
    for (int k = 0; k < kCombineSlots; ++k) {
      p[k] = slot_row(min(k, topk));
      w[k] = wts[(size_t)r * (topk + 1) + min(k, topk)];
    }
#pragma unroll
    for (int k = 0; k < kCombineSlots; ++k) d[k] = load(p[k]);
#pragma unroll
    for (int k = 0; k < kCombineSlots; ++k)
      if (k <= topk) add(w[k], d[k]);
  } else {
    for (int k = 0; k <= topk; ++k) add(wts[(size_t)r * (topk + 1) + k], load(slot_row(k)));
  }
#pragma unroll
  for (int h4 = 0; h4 < CW / 4; ++h4) {
    const float4 a = make_float4(acc[4 * h4], acc[4 * h4 + 1], acc[4 * h4 + 2], acc[4 * h4 + 3]);
    const int c = c0 + 4 * h4;
    if constexpr (HC) {
      for (int st = 0; st < hc.n_streams; ++st) {
        const float g = hc.post[(size_t)r * hc.n_streams + st];
        float4* h = reinterpret_cast<float4*>(hc.H + (size_t)r * hc.ldh + (size_t)st * H + c);
        float4 v = *h;
        v.x = CombineStep(v.x, g, a.x);
        v.y = CombineStep(v.y, g, a.y);
        v.z = CombineStep(v.z, g, a.z);
        v.w = CombineStep(v.w, g, a.w);
        *h = v;
      }
    } else {
      *reinterpret_cast<float4*>(y + (size_t)r * H + c) = a;
    }
  }
}

// Environment switches (the defaults are the measured best), read when a plan is created
// and kept in it, so each plan runs one fixed configuration:
//   CX_PREFILL_NRB (4 | 8) and CX_PREFILL_WPG (4 | 8 | 16): a register-blocked prefill
//     workgroup of wpg waves covers 16 nrb rows x 32 wpg columns;
//   CX_PREFILL_GEMM: 0 register-blocked, 1 tall, -1 by the rows per expert;
//   CX_PREFILL_MID: the mid fused into the register-blocked gate/up GEMM (needs nrb = 4);
//   CX_TALL_SEQMID: tall prefill with gate, up and the mid in one workgroup, one plane after
//     the other (0: separate plane workgroups and a mid launch);
//   CX_DOWN_MID: -1 the decode mid in the down GEMM's prologue at M (topk + 1) <= 128, 0 / 1
//     never / always (I <= 1024);
//   CX_FUSED_ROUTE: -1 routing inside the grouping launch at M <= 16, 0 / 1 never / for every
//     small call;
//   CX_STAGE: decode calls with gate/up, mid and down in one launch (0: separate launches).
struct Switches {
  int nrb, wpg;
  int kernel;
  int mid;
  int tall_mid;
  int down_mid;
  int fused_route;
  int stage;
};
inline Switches ReadSwitches() {
  auto env = [](const char* k, int d) {
    const char* e = std::getenv(k);
    return e ? std::atoi(e) : d;
  };
  const int nrb = env("CX_PREFILL_NRB", 4) == 8 ? 8 : 4;
  const int w = env("CX_PREFILL_WPG", 4);
  return Switches{nrb, w == 16 && nrb == 4 ? 16 : w == 4 ? 4 : 8, env("CX_PREFILL_GEMM", -1), env("CX_PREFILL_MID", 1),
                  env("CX_TALL_SEQMID", 1), env("CX_DOWN_MID", -1), env("CX_FUSED_ROUTE", -1), env("CX_STAGE", 1)};
}

}  // namespace cx

// ---- plan ----------------------------------------------------------------------------------

struct cx_moe_plan {
  int H, I, E, topk;
  int k2_gu, cb_gu, k2_d, cb_d;      // routed experts
  int k2_sgu, cb_sgu, k2_sd, cb_sd;  // shared expert
  cx::MatPtr* d_tables;              // device: gate[E+1], up[E+1], down[E+1]
  __half* d_scales;                  // device: packed scale copies (ExpertTables)
  cx::ExpertTables tb;
  hipEvent_t* trace;                 // caller's events (nullable), recorded between stages
  int n_trace, trace_cursor;
  void* scratch;                     // this device's address of the library's static scratch (nullable)
  bool xcd_rr;                       // workgroups go to the XCDs round-robin (XcdRoundRobin)
  cx::Switches sw;                   // environment switches, read when the plan is created
};

namespace cx {

struct MoeSizes {
  int M, P, n, nsh, chunk, nrb, wpg, max_entries, ntiles;
  bool small, prefill, tall, mid, down_mid, tall_mid, stage;
  size_t off_sel, off_wts, off_counts, off_offsets, off_pairs, off_rows, off_inv, off_rexp, off_ent, off_nent, off_tiles;
  size_t off_xg, off_xu, off_yg, off_yu, off_xd, off_yd, off_ysc, off_ctr, total;
  int nyp;  // entry table length of the decode stage launch (max_entries rounded up to 8)
};

bool FrontEndFits(int M, int E, int topk);

MoeSizes PlanMoe(const cx_moe_plan* pl, int M, int mode) {
  MoeSizes s{};
  s.M = M;
  s.n = M * pl->topk;
  s.P = s.n + M;
  const bool decode = mode == CX_MOE_DECODE || (mode == CX_MOE_AUTO && M <= 64);
  s.prefill = !decode;
  const Switches& ps = pl->sw;
  s.nrb = decode ? 1 : ps.nrb;
  s.wpg = decode ? 4 : ps.wpg;
  // The tall GEMM when experts average at least 96 rows (one decode then serves up to 192
  // rows); below that most entries fit the register-blocked GEMM's 64 rows.
  const int kern = ps.kernel >= 0 ? ps.kernel : (long)M * pl->topk >= 96L * pl->E ? 1 : 0;
  s.tall = !decode && kern == 1;
  if (s.tall) s.nrb = 4 * kTallRowBlocksPerWave;
  // Register-blocked prefill: gate and up in one workgroup with the mid fused into the
  // epilogue (64-row entries, 4 waves per plane).
  s.mid = !decode && !s.tall && s.nrb == 4 && ps.mid;
  s.tall_mid = s.tall && ps.tall_mid;
  // Decode: the mid in the down GEMM's prologue (16 rows of I halves in LDS per workgroup)
  // while at most 128 entries can exist (M (topk + 1) <= 128): the down launch is then at
  // most one generation of workgroups (16 per entry, 8 per CU), and the mid launch it
  // saves is pure latency.  Measured on config 3: -2 to -2.5 us per layer at 1-8 rows, no
  // change at 12-32, +2 to +4 us at 40 (every workgroup recomputes its entry's mid).
  // Switch CX_DOWN_MID = 0 / 1 forces it off / on (decode, I <= 1024).
  s.down_mid = decode && pl->I <= 1024 &&
               (ps.down_mid < 0 ? (long)M * (pl->topk + 1) <= 128 : ps.down_mid != 0);
  // Decode calls through the grouping launch with one codebook and the stage launch's rates,
  // above the prologue mid's range: gate/up, the mid and down in one launch
  // (Exl3DecodeStageKernel).  Measured on config 3 (median per layer call, 200 calls):
  // 12 rows 74.8 -> 66.3 us, 16 rows 87.6 -> 80.4, 24 rows 111.7 -> 102.7, 32 rows
  // 128.8 -> 124, 64 rows 188.7 -> 181; at 1-8 rows, against the down GEMM with the
  // prologue mid, no change (29.4 / 58.5 us) or a little slower (R = 1 in bench: 31.6
  // against 30.8 us).
  // The down rate may exceed the gate/up rate by one or two steps for mul1 layers (the
  // launch's instantiations); the shared expert at the routed experts' rates.
  const bool stage_rates = pl->k2_d == pl->k2_gu || (pl->cb_d == kCbMul1 && (pl->k2_d == pl->k2_gu + 2 || pl->k2_d == pl->k2_gu + 4));
  s.stage = decode && ps.stage != 0 && pl->xcd_rr && FrontEndFits(M, pl->E, pl->topk) && !s.down_mid && stage_rates &&
            pl->k2_gu == pl->k2_sgu && pl->k2_d == pl->k2_sd && pl->cb_gu == pl->cb_d && pl->cb_gu == pl->cb_sgu &&
            pl->cb_gu == pl->cb_sd && pl->I % 128 == 0;
  // Decode: one 16-row block per entry; prefill: every row of an entry shares each decoded tile.
  s.chunk = 16 * s.nrb;
  s.nsh = (M + s.chunk - 1) / s.chunk;
  s.max_entries = s.nsh + std::min(pl->E, s.n) + s.n / s.chunk;
  s.nyp = (s.max_entries + 7) / 8 * 8;
  if (s.stage) s.max_entries = s.nyp;  // the stage launch's XCD mapping reads whole groups of 8
  s.small = s.n <= kSmallRoutes;
  s.ntiles = (s.n + kTile - 1) / kTile;
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o += AlignUp(bytes, 256);
    return at;
  };
  s.off_sel = take((size_t)s.n * 4);
  s.off_wts = take((size_t)M * (pl->topk + 1) * 4);
  s.off_counts = take((size_t)pl->E * 4);
  s.off_offsets = take((size_t)(pl->E + 1) * 4);
  s.off_pairs = take((size_t)s.n * 4);
  s.off_rows = take((size_t)s.n * 4);
  s.off_inv = take((size_t)s.n * 4);
  s.off_rexp = take((size_t)s.n * 4);
  s.off_ent = take((size_t)s.max_entries * 16);
  s.off_nent = take(4);
  s.off_tiles = take((size_t)pl->E * s.ntiles * 4);
  s.off_xg = take((size_t)s.P * pl->H * 2);
  s.off_xu = take((size_t)s.P * pl->H * 2);
  s.off_yg = take((size_t)s.P * pl->I * 4);
  s.off_yu = take((size_t)s.P * pl->I * 4);
  s.off_xd = take((size_t)s.P * pl->I * 2);
  s.off_yd = take((size_t)s.P * pl->H * (s.prefill ? 2 : 4));
  s.off_ysc = take(s.prefill ? (size_t)s.P * (pl->H / 128) * 4 : 0);
  s.off_ctr = take(s.stage ? (size_t)s.nyp * kStageCtrStride * 4 : 0);
  s.total = o;
  return s;
}

// ---- the allocation-free variant's scratch --------------------------------------------
// One static device array per GPU, used as the workspace of cx_moe_layer_forward_static.
// Host code never uses the array's name as an address (on the host it is a stand-in):
// its device address is looked up once per device, with that device current, when the
// first plan is created there, and kept in g_scratch[device] and in every plan.
static __device__ __align__(256) unsigned char scratch[CX_STATIC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices];

// Device address of `scratch` on the current device (nullptr with *err set on failure).
void* StaticScratch(hipError_t* err) {
  int dev = 0;
  *err = hipGetDevice(&dev);
  if (*err != hipSuccess) return nullptr;
  if (dev < 0 || dev >= kMaxDevices) {
    *err = hipErrorInvalidDevice;
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    *err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (*err != hipSuccess) return nullptr;
    g_scratch[dev] = p;
  }
  return g_scratch[dev];
}

// The decode stage launch (Exl3DecodeStageKernel) keeps each row entry on one XCD by
// relying on workgroups going to the XCDs round-robin by linear id (ids equal modulo 8 on
// one XCD; also true of partition modes with 4, 2 or 1 XCDs).  Checked once per device: a
// probe launch records the XCC id of each of 256 workgroups.
__global__ void __launch_bounds__(64) XccProbeKernel(int* out) {
  if (threadIdx.x == 0) {
    uint32_t v;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
    out[blockIdx.x] = (int)(v & 0xf);
  }
}
int g_xcd_rr[kMaxDevices];  // 0 not probed yet, 1 round-robin, -1 not (or the probe failed)

bool XcdRoundRobin() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return false;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_xcd_rr[dev] == 0) {
    constexpr int kN = 256;
    int* d = nullptr;
    int h[kN];
    bool ok = hipMalloc(&d, kN * sizeof(int)) == hipSuccess;
    if (ok) {
      hipLaunchKernelGGL(XccProbeKernel, dim3(kN), dim3(64), 0, nullptr, d);
      ok = hipGetLastError() == hipSuccess && hipMemcpy(h, d, sizeof h, hipMemcpyDeviceToHost) == hipSuccess;
    }
    if (d) (void)hipFree(d);
    for (int i = 8; ok && i < kN; ++i) ok = h[i] == h[i % 8];
    (void)hipGetLastError();
    g_xcd_rr[dev] = ok ? 1 : -1;
  }
  return g_xcd_rr[dev] > 0;
}

void LaunchRoute(const float* logits, int ld, int M, int E, int topk, const float* shared_logit, int* sel, float* wts,
                 hipStream_t s) {
  // A row's k rounds are a chain of scalar work (lane reads, ballot counts, branches), and
  // the CU's scalar unit is shared by its waves: small calls put one routing wave on each
  // CU.
  const int wpb = M <= 256 ? 1 : 4;  // waves (rows) per workgroup
  const dim3 grid((unsigned)((M + wpb - 1) / wpb)), block((unsigned)(64 * wpb));
  if (E <= 512)
    hipLaunchKernelGGL(RouteKernel<8>, grid, block, 0, s, logits, ld, M, E, topk, shared_logit, sel, wts);
  else
    hipLaunchKernelGGL(RouteKernel<16>, grid, block, 0, s, logits, ld, M, E, topk, shared_logit, sel, wts);
}

// Grouping fused with the input transforms (route-order rows) for small decode calls.
bool FrontEndFits(int M, int E, int topk) { return M <= 64 && M * topk <= kSmallRoutes && E <= kMaxExperts; }

int LaunchGroup(const int* sel, GroupOut& o, int* tile_counts, int ntiles, hipStream_t s) {
  const int n = o.M * o.topk;
  if (n <= kSmallRoutes) {
    hipLaunchKernelGGL(GroupSmallKernel, dim3(1), dim3(1024), 0, s, sel, o);
  } else {
    hipLaunchKernelGGL(GroupCountKernel, dim3(ntiles), dim3(1024), 0, s, sel, n, o.E, ntiles, tile_counts);
    hipLaunchKernelGGL(GroupScatterKernel, dim3(ntiles + 1), dim3(1024), 0, s, sel, tile_counts, ntiles, o);
  }
  return LaunchStatus();
}

// Expert GEMM over the device-built entries: shared-expert entries [0, nsh) and routed
// entries [nsh, n_entries).  Routed and shared matrices with different rates go in
// separate launches.
GemmArgs ExpertGemmArgs(const cx_moe_plan* pl, const MoeSizes& sz, bool gate_up, const __half* xa, const __half* xb,
                        float* ya, float* yb, float* ysc, __half* xd, const int4* ent, const int* xmap,
                        const float* mid_yg, const float* mid_yu) {
  GemmArgs g{};
  if (mid_yg) {
    g.mid_yg = mid_yg;
    g.mid_yu = mid_yu;
    g.mid_svg = pl->tb.gate_svh;
    g.mid_svu = pl->tb.up_svh;
  }
  g.mid_suh = pl->tb.down_suh;
  g.mid_xd = xd;
  g.xmap = xmap;
  g.xmap_n = sz.n;
  const int in = gate_up ? pl->H : pl->I, out = gate_up ? pl->I : pl->H;
  g.A = in / 16;
  g.ncp = out / 32;
  g.S = 1;
  g.entries = ent;
  if (gate_up) {
    g.plane[0] = GemmPlane{pl->tb.gate, xa, ya, in, out, 0, 0, nullptr};
    g.plane[1] = GemmPlane{pl->tb.up, xb, yb, in, out, 0, 0, nullptr};
  } else {
    // The down projection's output transform runs in the GEMM epilogue (a workgroup
    // holds one whole 128-column block), so the combine is a plain weighted sum.
    // Prefill stores it as fp16 rows with a scale per 128-column block (half the bytes).
    g.plane[0] = sz.prefill ? GemmPlane{pl->tb.down, xa, ya, in, out, 0, 2, ysc}
                            : GemmPlane{pl->tb.down, xa, ya, in, out, 0, 1, nullptr};
    g.plane[1] = g.plane[0];
  }
  g.tall_seq_mid = gate_up && sz.tall_mid;
  return g;
}

bool LaunchExpertGemm(const cx_moe_plan* pl, const MoeSizes& sz, bool gate_up, const __half* xa, const __half* xb,
                      float* ya, float* yb, float* ysc, __half* xd, const int4* ent, const int* nent, const int* xmap,
                      const float* mid_yg, const float* mid_yu, hipStream_t s) {
  GemmArgs g = ExpertGemmArgs(pl, sz, gate_up, xa, xb, ya, yb, ysc, xd, ent, xmap, mid_yg, mid_yu);
  const int ksw = gate_up ? 4 : 1;
  const int planes = gate_up && !sz.tall_mid ? 2 : 1;
  const int k2r = gate_up ? pl->k2_gu : pl->k2_d, cbr = gate_up ? pl->cb_gu : pl->cb_d;
  const int k2s = gate_up ? pl->k2_sgu : pl->k2_sd, cbs = gate_up ? pl->cb_sgu : pl->cb_sd;
  const int wpg = g.ncp % sz.wpg == 0 ? sz.wpg : 4;
  const bool mid = gate_up && sz.mid;  // both planes in one workgroup, the mid fused
  const int cpg = sz.tall ? g.ncp / 4 : mid ? g.ncp / 4 : sz.prefill ? g.ncp / wpg : g.ncp / (4 / ksw);
  auto launch = [&](int k2, int cb, int ny) {
    if (sz.tall) return LaunchGemmTall(k2, cb, dim3(cpg, (ny + 7) / 8 * 8, planes), g, s);
    if (sz.prefill)  // entry-major XCD placement needs the entry count padded to 8
      return LaunchGemmPrefill(k2, cb, sz.nrb, mid ? 4 : wpg, mid, dim3(cpg, (ny + 7) / 8 * 8, mid ? 1 : planes), g,
                               s);
    return LaunchGemm(k2, cb, sz.nrb, ksw, 4, dim3(cpg, ny, planes), g, s);
  };
  if (k2r == k2s && cbr == cbs) {
    g.n_entries = nent;
    g.entry_base = 0;
    return launch(k2r, cbr, sz.max_entries);
  }
  g.n_entries = nullptr;
  g.n_entries_host = sz.nsh;
  g.entry_base = 0;
  if (!launch(k2s, cbs, sz.nsh)) return false;
  g.n_entries = nent;
  g.entry_base = sz.nsh;
  return launch(k2r, cbr, sz.max_entries - sz.nsh);
}

int CheckExpertShapes(const cx_moe_expert& ex, int H, int I) {
  int rc;
  if ((rc = CheckMatrix(&ex.gate)) || (rc = CheckMatrix(&ex.up)) || (rc = CheckMatrix(&ex.down))) return rc;
  if (ex.gate.in_features != H || ex.gate.out_features != I || ex.up.in_features != H || ex.up.out_features != I ||
      ex.down.in_features != I || ex.down.out_features != H)
    return CX_E_SHAPE;
  if (ex.gate.k2 != ex.up.k2 || ex.gate.codebook != ex.up.codebook) return CX_E_UNSUPPORTED;
  return CX_OK;
}

}  // namespace cx

using namespace cx;

extern "C" {

int cx_moe_route(const float* logits, int32_t ld, int32_t M, int32_t E, int32_t topk, const float* shared_logit,
                 int32_t* sel, float* wts, cx_stream_t stream) {
  if (!logits || !sel || !wts) return CX_E_ARG;
  if (M <= 0 || E <= 0 || E > kMaxExperts || topk <= 0 || topk > kMaxTopK || topk > E || topk > 64) return CX_E_SHAPE;
  if (ld < E || (!shared_logit && ld < E + 1)) return CX_E_SHAPE;
  LaunchRoute(logits, ld, M, E, topk, shared_logit, sel, wts, (hipStream_t)stream);
  return LaunchStatus();
}

size_t cx_moe_group_workspace_size(int32_t M, int32_t E, int32_t topk) {
  if (M <= 0 || E <= 0 || topk <= 0) return 0;
  const int n = M * topk;
  return AlignUp((size_t)E * ((n + kTile - 1) / kTile) * 4, 256);
}

int cx_moe_group(const int32_t* sel, int32_t M, int32_t E, int32_t topk, int32_t* counts, int32_t* offsets,
                 int32_t* pairs, int32_t* row_ids, void* workspace, size_t workspace_bytes, cx_stream_t stream) {
  if (!sel || !counts || !offsets || !pairs || !row_ids) return CX_E_ARG;
  if (M <= 0 || E <= 0 || E > kMaxExperts || topk <= 0 || topk > E) return CX_E_SHAPE;
  if (workspace && !WorkspaceAligned(workspace)) return CX_E_SHAPE;
  const int n = M * topk;
  const int ntiles = (n + kTile - 1) / kTile;
  if (n > kSmallRoutes && (!workspace || workspace_bytes < cx_moe_group_workspace_size(M, E, topk)))
    return CX_E_WORKSPACE;
  GroupOut o{counts, offsets, pairs, row_ids, nullptr, nullptr, nullptr, nullptr, 16, M, topk, E};
  return LaunchGroup(sel, o, static_cast<int*>(workspace), ntiles, (hipStream_t)stream);
}

int cx_moe_plan_create(const cx_moe_layer* layer, cx_moe_plan** out) {
  if (!layer || !out || !layer->experts) return CX_E_ARG;
  *out = nullptr;
  const int H = layer->hidden, I = layer->intermediate, E = layer->n_experts;
  if (H <= 0 || I <= 0 || H % 128 || I % 128) return CX_E_SHAPE;
  if (E <= 0 || E > kMaxExperts || layer->topk <= 0 || layer->topk > E || layer->topk > kMaxTopK) return CX_E_SHAPE;
  int rc;
  for (int e = 0; e < E; ++e) {
    if ((rc = CheckExpertShapes(layer->experts[e], H, I))) return rc;
    const cx_moe_expert& a = layer->experts[e];
    const cx_moe_expert& b = layer->experts[0];
    if (a.gate.k2 != b.gate.k2 || a.gate.codebook != b.gate.codebook || a.down.k2 != b.down.k2 ||
        a.down.codebook != b.down.codebook)
      return CX_E_UNSUPPORTED;
  }
  if ((rc = CheckExpertShapes(layer->shared, H, I))) return rc;
  cx_moe_plan* pl = new (std::nothrow) cx_moe_plan{};
  if (!pl) return CX_E_ARG;
  pl->H = H;
  pl->I = I;
  pl->E = E;
  pl->topk = layer->topk;
  pl->k2_gu = layer->experts[0].gate.k2;
  pl->cb_gu = layer->experts[0].gate.codebook;
  pl->k2_d = layer->experts[0].down.k2;
  pl->cb_d = layer->experts[0].down.codebook;
  pl->k2_sgu = layer->shared.gate.k2;
  pl->cb_sgu = layer->shared.gate.codebook;
  pl->k2_sd = layer->shared.down.k2;
  pl->cb_sd = layer->shared.down.codebook;
  const size_t n = (size_t)(E + 1);
  MatPtr* host = static_cast<MatPtr*>(std::malloc(sizeof(MatPtr) * 3 * n));
  if (!host) {
    delete pl;
    return CX_E_ARG;
  }
  auto mp = [](const cx_exl3_matrix& m) {
    return MatPtr{m.tiles, reinterpret_cast<const __half*>(m.suh), reinterpret_cast<const __half*>(m.svh)};
  };
  for (int e = 0; e <= E; ++e) {
    const cx_moe_expert& ex = e < E ? layer->experts[e] : layer->shared;
    host[e] = mp(ex.gate);
    host[n + e] = mp(ex.up);
    host[2 * n + e] = mp(ex.down);
  }
  hipError_t err = hipMalloc(&pl->d_tables, sizeof(MatPtr) * 3 * n);
  if (err == hipSuccess) err = hipMemcpy(pl->d_tables, host, sizeof(MatPtr) * 3 * n, hipMemcpyHostToDevice);
  std::free(host);
  if (err != hipSuccess) {
    if (pl->d_tables) (void)hipFree(pl->d_tables);
    delete pl;
    return (int)err;
  }
  // Packed scale copies: gate suh, up suh [E+1][H]; gate svh, up svh, down suh [E+1][I].
  const size_t nsc = n * (2 * (size_t)H + 3 * (size_t)I);
  err = hipMalloc(&pl->d_scales, nsc * sizeof(__half));
  __half* g_suh = pl->d_scales;
  __half* u_suh = g_suh + n * H;
  __half* g_svh = u_suh + n * H;
  __half* u_svh = g_svh + n * I;
  __half* d_suh = u_svh + n * I;
  for (int e = 0; e <= E && err == hipSuccess; ++e) {
    const cx_moe_expert& ex = e < E ? layer->experts[e] : layer->shared;
    const struct {
      __half* dst;
      const void* src;
      int len;
    } cp[5] = {{g_suh + (size_t)e * H, ex.gate.suh, H},
               {u_suh + (size_t)e * H, ex.up.suh, H},
               {g_svh + (size_t)e * I, ex.gate.svh, I},
               {u_svh + (size_t)e * I, ex.up.svh, I},
               {d_suh + (size_t)e * I, ex.down.suh, I}};
    for (const auto& c : cp)
      if (err == hipSuccess) err = hipMemcpyAsync(c.dst, c.src, (size_t)c.len * sizeof(__half), hipMemcpyDefault, nullptr);
  }
  if (err == hipSuccess) err = hipStreamSynchronize(nullptr);
  if (err != hipSuccess) {
    if (pl->d_scales) (void)hipFree(pl->d_scales);
    (void)hipFree(pl->d_tables);
    delete pl;
    return (int)err;
  }
  pl->tb = ExpertTables{pl->d_tables, pl->d_tables + n, pl->d_tables + 2 * n, g_suh, u_suh, g_svh, u_svh, d_suh};
  // The static scratch serves only cx_moe_layer_forward_static: a failed lookup leaves it
  // null (that entry point then returns CX_E_ARG) and does not fail the plan.
  pl->xcd_rr = XcdRoundRobin();
  pl->scratch = StaticScratch(&err);
  if (err != hipSuccess) {
    pl->scratch = nullptr;
    (void)hipGetLastError();
  }
  pl->sw = ReadSwitches();
  *out = pl;
  return CX_OK;
}

void cx_moe_plan_destroy(cx_moe_plan* plan) {
  if (!plan) return;
  if (plan->d_tables) (void)hipFree(plan->d_tables);
  if (plan->d_scales) (void)hipFree(plan->d_scales);
  std::free(plan->trace);
  delete plan;
}

size_t cx_moe_layer_workspace_size(const cx_moe_plan* plan, int32_t M, int32_t mode) {
  if (!plan || M <= 0) return 0;
  return PlanMoe(plan, M, mode).total;
}

}  // extern "C"

namespace cx {

int MoeForward(const cx_moe_plan* pl, const void* x, int32_t x_dtype, int32_t ldx, const float* logits, int32_t ld,
               const float* shared_logit,
               int32_t M, const int32_t* row_offsets, int32_t n_sessions, float* y, const HcArgs* hc, int32_t* sel_out,
               float* wts_out, int32_t mode, void* workspace, size_t workspace_bytes, cx_stream_t stream) {
  if (!pl || !x || !logits || (!y && !hc) || !workspace) return CX_E_ARG;
  if (mode < CX_MOE_AUTO || mode > CX_MOE_PREFILL) return CX_E_ARG;
  if (x_dtype != CX_F16 && x_dtype != CX_F32) return CX_E_ARG;
  if (M <= 0) return CX_E_SHAPE;
  if (!WorkspaceAligned(workspace) || reinterpret_cast<uintptr_t>(y) % 16) return CX_E_SHAPE;  // y: float4 rows
  // Rows are read in 16- / 32-byte pieces.
  if (ldx < pl->H || ldx % 8 || reinterpret_cast<uintptr_t>(x) % 16) return CX_E_SHAPE;
  if (ld < pl->E || (!shared_logit && ld < pl->E + 1)) return CX_E_SHAPE;
  int rc;
  if ((rc = RowOffsetsCheck(row_offsets, n_sessions, M))) return rc;
  const MoeSizes sz = PlanMoe(pl, M, mode);
  if (workspace_bytes < sz.total) return CX_E_WORKSPACE;
  hipStream_t s = (hipStream_t)stream;
  char* ws = static_cast<char*>(workspace);
  int* sel = sel_out ? sel_out : reinterpret_cast<int*>(ws + sz.off_sel);
  float* wts = wts_out ? wts_out : reinterpret_cast<float*>(ws + sz.off_wts);
  int* counts = reinterpret_cast<int*>(ws + sz.off_counts);
  int* offsets = reinterpret_cast<int*>(ws + sz.off_offsets);
  int* pairs = reinterpret_cast<int*>(ws + sz.off_pairs);
  int* rows = reinterpret_cast<int*>(ws + sz.off_rows);
  int* inv = reinterpret_cast<int*>(ws + sz.off_inv);
  int* rexp = reinterpret_cast<int*>(ws + sz.off_rexp);
  int4* ent = reinterpret_cast<int4*>(ws + sz.off_ent);
  int* nent = reinterpret_cast<int*>(ws + sz.off_nent);
  int* tiles = reinterpret_cast<int*>(ws + sz.off_tiles);
  __half* xg = reinterpret_cast<__half*>(ws + sz.off_xg);
  __half* xu = reinterpret_cast<__half*>(ws + sz.off_xu);
  float* yg = reinterpret_cast<float*>(ws + sz.off_yg);
  float* yu = reinterpret_cast<float*>(ws + sz.off_yu);
  __half* xd = reinterpret_cast<__half*>(ws + sz.off_xd);
  float* yd = reinterpret_cast<float*>(ws + sz.off_yd);
  float* ysc = reinterpret_cast<float*>(ws + sz.off_ysc);

  cx_moe_plan* mp = const_cast<cx_moe_plan*>(pl);
  auto mark = [&]() {
    if (mp->trace && mp->n_trace > 0) {
      (void)hipEventRecord(mp->trace[mp->trace_cursor], s);
      mp->trace_cursor = (mp->trace_cursor + 1) % mp->n_trace;
    }
  };
  mark();
  int* ctr = reinterpret_cast<int*>(ws + sz.off_ctr);
  GroupOut o{counts, offsets, pairs, rows, inv, rexp, ent, nent, sz.chunk, M, pl->topk, pl->E, sz.max_entries,
             sz.stage ? ctr : nullptr, sz.stage ? sz.nyp : 0};
  const bool front = !sz.prefill && FrontEndFits(M, pl->E, pl->topk);
  // Routing fused into the grouping launch when workgroup 0 routes every row in one round
  // of its 16 waves (M <= 16; CX_FUSED_ROUTE = 0 / 1 forces it off / on for any small call).
  const bool fused_route = pl->sw.fused_route < 0 ? M <= 16 : pl->sw.fused_route != 0;
  if (front && fused_route) {
    // Routing, grouping and input transforms in one launch; the trace records it as the
    // route stage (group and input stages empty).
    const int wpr = ((pl->topk + 1) * (pl->H / 128) + 63) / 64;
    if (pl->E <= 512)
      hipLaunchKernelGGL(RouteGroupInputKernel<8>, dim3(1 + M * wpr), dim3(1024), 0, s, logits, ld, shared_logit, sel,
                         wts, x, (int)(x_dtype == CX_F32), (long long)ldx, pl->tb, pl->H, xg, xu, o);
    else
      hipLaunchKernelGGL(RouteGroupInputKernel<16>, dim3(1 + M * wpr), dim3(1024), 0, s, logits, ld, shared_logit, sel,
                         wts, x, (int)(x_dtype == CX_F32), (long long)ldx, pl->tb, pl->H, xg, xu, o);
    mark();
    mark();
  } else {
    LaunchRoute(logits, ld, M, pl->E, pl->topk, shared_logit, sel, wts, s);
    mark();
  }
  if (front && fused_route) {
  } else if (front) {
    // Grouping and input transforms in one launch; the trace records it as the group
    // stage (input stage empty).
    const int wpr = ((pl->topk + 1) * (pl->H / 128) + 63) / 64;
    hipLaunchKernelGGL(GroupInputKernel, dim3(1 + M * wpr), dim3(1024), 0, s, sel, x, (int)(x_dtype == CX_F32),
                       (long long)ldx, pl->tb, pl->H, xg, xu, o);
    mark();
  } else {
    if ((rc = LaunchGroup(sel, o, tiles, sz.ntiles, s))) return rc;
    mark();
    // Split rows over more waves when there are few of them (decode).
    const int S = sz.P >= 4096 ? 1 : std::max(1, std::min(4, pl->H / 512));
    const dim3 grid((unsigned)(((long)sz.P * S + 3) / 4));
    if (x_dtype == CX_F32)
      hipLaunchKernelGGL(MoeInputKernel<true>, grid, dim3(256), 0, s, x, (long long)ldx, rexp, rows, pl->tb, M, pl->topk,
                         pl->E, pl->H, S, xg, xu);
    else
      hipLaunchKernelGGL(MoeInputKernel<false>, grid, dim3(256), 0, s, x, (long long)ldx, rexp, rows, pl->tb, M,
                         pl->topk, pl->E, pl->H, S, xg, xu);
  }
  mark();
  if (sz.stage) {
    // Gate/up, mid and down in one launch (the counters were zeroed by the grouping launch);
    // the trace records it as the gate/up stage (mid and down stages empty).
    GemmArgs gu = ExpertGemmArgs(pl, sz, true, xg, xu, yg, yu, nullptr, xd, ent, pairs, nullptr, nullptr);
    GemmArgs dn = ExpertGemmArgs(pl, sz, false, xd, nullptr, yd, nullptr, nullptr, nullptr, ent, nullptr, nullptr,
                                 nullptr);
    gu.mid_svg = pl->tb.gate_svh;
    gu.mid_svu = pl->tb.up_svh;
    gu.n_entries = dn.n_entries = nent;
    gu.stage_ctr = dn.stage_ctr = ctr;
    gu.stage_arrivals = dn.stage_arrivals = 2 * gu.ncp;
    if (!LaunchDecodeStage(pl->k2_gu, pl->k2_d, pl->cb_gu, gu, dn, sz.nyp, s)) return CX_E_UNSUPPORTED;
    mark();
    mark();
  } else {
    if (!LaunchExpertGemm(pl, sz, true, xg, xu, yg, yu, nullptr, xd, ent, nent, front ? pairs : nullptr, nullptr,
                          nullptr, s))
      return CX_E_UNSUPPORTED;
    mark();
    if (!sz.mid && !sz.down_mid && !sz.tall_mid)  // else a GEMM computes the down projection's input rows itself
      hipLaunchKernelGGL(MoeMidKernel, dim3((unsigned)((sz.P + 3) / 4)), dim3(256), 0, s, yg, yu, rexp,
                         pl->tb, M, pl->topk, pl->E, pl->I, xd);
    mark();
    if (!LaunchExpertGemm(pl, sz, false, xd, nullptr, yd, nullptr, ysc, nullptr, ent, nent, nullptr,
                          sz.down_mid ? yg : nullptr, sz.down_mid ? yu : nullptr, s))
      return CX_E_UNSUPPORTED;
  }
  mark();
  {
    const long items = (long)M * (pl->H / (sz.prefill ? 8 : 4));  // columns per thread: MoeCombineKernel's CW
    const dim3 grid((unsigned)((items + 255) / 256));
    const HcArgs h = hc ? *hc : HcArgs{};
    if (hc && sz.prefill)
      hipLaunchKernelGGL((MoeCombineKernel<true, true>), grid, dim3(256), 0, s, yd, ysc, wts, inv, M, pl->topk, pl->H,
                         nullptr, h);
    else if (hc)
      hipLaunchKernelGGL((MoeCombineKernel<true, false>), grid, dim3(256), 0, s, yd, ysc, wts, inv, M, pl->topk, pl->H,
                         nullptr, h);
    else if (sz.prefill)
      hipLaunchKernelGGL((MoeCombineKernel<false, true>), grid, dim3(256), 0, s, yd, ysc, wts, inv, M, pl->topk, pl->H,
                         y, h);
    else
      hipLaunchKernelGGL((MoeCombineKernel<false, false>), grid, dim3(256), 0, s, yd, ysc, wts, inv, M, pl->topk, pl->H,
                         y, h);
  }
  mark();
  return LaunchStatus();
}

}  // namespace cx

extern "C" {

int cx_moe_layer_forward(const cx_moe_plan* pl, const void* x, int32_t x_dtype, int32_t ldx, const float* logits,
                         int32_t ld, const float* shared_logit, int32_t M, const int32_t* row_offsets,
                         int32_t n_sessions, float* y, int32_t* sel, float* wts, int32_t mode, void* workspace,
                         size_t workspace_bytes, cx_stream_t stream) {
  if (!y) return CX_E_ARG;
  return MoeForward(pl, x, x_dtype, ldx, logits, ld, shared_logit, M, row_offsets, n_sessions, y, nullptr, sel, wts, mode, workspace,
                    workspace_bytes, stream);
}

int cx_moe_layer_forward_hc(const cx_moe_plan* pl, const void* x, int32_t x_dtype, int32_t ldx,
                            const float* logits, int32_t ld, const float* shared_logit, int32_t M, const int32_t* row_offsets, int32_t n_sessions,
                            const float* post, int32_t n_streams, float* H, int64_t ldh, int32_t* sel, float* wts,
                            int32_t mode, void* workspace, size_t workspace_bytes, cx_stream_t stream) {
  if (!pl || !post || !H) return CX_E_ARG;
  if (n_streams < 1 || n_streams > 64 || ldh < (int64_t)n_streams * pl->H) return CX_E_SHAPE;
  // The combine reads and writes H in 16-byte pieces.
  if (ldh % 4 || reinterpret_cast<uintptr_t>(H) % 16) return CX_E_SHAPE;
  const HcArgs hc{post, H, (long long)ldh, n_streams};
  return MoeForward(pl, x, x_dtype, ldx, logits, ld, shared_logit, M, row_offsets, n_sessions, nullptr, &hc, sel, wts, mode,
                    workspace, workspace_bytes, stream);
}

int cx_moe_layer_forward_static(const cx_moe_plan* pl, const void* x, int32_t x_dtype, int32_t ldx,
                                const float* logits, int32_t ld, const float* shared_logit, int32_t M,
                                const int32_t* row_offsets, int32_t n_sessions, float* y, int32_t* sel, float* wts,
                                int32_t mode, cx_stream_t stream) {
  if (!pl || !y) return CX_E_ARG;
  if (!pl->scratch) return CX_E_ARG;
  if (M <= 0) return CX_E_SHAPE;
  // The whole workspace lives in the static array; nothing is allocated here.
  if (PlanMoe(pl, M, mode).total > (size_t)CX_STATIC_SCRATCH_BYTES) return CX_E_WORKSPACE;
  return MoeForward(pl, x, x_dtype, ldx, logits, ld, shared_logit, M, row_offsets, n_sessions, y, nullptr, sel, wts,
                    mode, pl->scratch, (size_t)CX_STATIC_SCRATCH_BYTES, stream);
}

int cx_moe_plan_set_trace(cx_moe_plan* plan, void* const* events, int32_t n_events) {
  if (!plan || n_events < 0 || (n_events > 0 && !events)) return CX_E_ARG;
  std::free(plan->trace);
  plan->trace = nullptr;
  plan->n_trace = 0;
  plan->trace_cursor = 0;
  if (n_events == 0) return CX_OK;
  plan->trace = static_cast<hipEvent_t*>(std::malloc(sizeof(hipEvent_t) * n_events));
  if (!plan->trace) return CX_E_ARG;
  for (int i = 0; i < n_events; ++i) plan->trace[i] = static_cast<hipEvent_t>(events[i]);
  plan->n_trace = n_events;
  return CX_OK;
}

}  // extern "C"
