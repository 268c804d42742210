// HBM-streaming skinny matmul (M <= 4 rows of activations): the
// decode-shaped linear (M = 1 GEMV) and the W8A16 linear with int8 weights
// dequantized in-kernel, for B = W [K,N] row-major (the split-K kernel
// below) and for W [N,K] (the row-dot kernel, further down).
//
// In the reference such a dispatch is still an HMX matmul: M is padded to the
// 32-row HMX tile (CG/Transforms/HexagonConvertMatmulToHmx.cpp:51-70) and the
// VTCM plan keeps K whole (CG/Strategy/Planning/VTCMPlanning.cpp:156-260).
// With M = 1 the work is reading W once, so on MI355X it is a bandwidth
// kernel, not an MFMA kernel:
//  * each lane streams one 16-byte column segment of W (8 f16 or 16 int8
//    weights) down a run of rows, 16 loads in flight, and accumulates in
//    f32; x is read once per lane and broadcast, nothing is staged first;
//  * a wave covers 64 segments of one row, or (half-wave form) 32 segments
//    of two rows, each 32-lane half streaming its own run: half the columns
//    per workgroup, so fewer K splits and a smaller final sum per column
//    block;
//  * K is split over a 2-D grid (column block x K split) sized to about one
//    workgroup per CU; each workgroup sums its waves' runs through LDS and
//    writes an f32 partial;
//  * the last workgroup to finish a column block (device-scope arrival
//    counter) sums the partials, applies the per-column scale (W8A16), adds
//    the DPS init if asked, rounds once and re-arms the counter, so the
//    whole matmul is one launch.
#include <type_traits>

#include "device_common.h"
#include "kernels_internal.h"

namespace ihp {

namespace {

constexpr int kThreads = kGemvThreads;  // 8 waves
constexpr int kWaves = kThreads / 64;
constexpr int kBatch = 8;        // 16-byte loads per batch; two batches in flight
constexpr int kSumBatch = 32;    // partial loads in flight in the final sum
constexpr int kMaxRowsPerWave = 64;

template <typename WT>
struct WTraits;
template <>
struct WTraits<f16> {
  static constexpr int kCols = 8;  // weights per 16-byte load
  static __device__ __forceinline__ void widen(i32x4 v, float *w) {
    f16x8 h = __builtin_bit_cast(f16x8, v);
#pragma unroll
    for (int c = 0; c < 8; ++c)
      w[c] = (float)h[c];
  }
};
template <>
struct WTraits<int8_t> {
  static constexpr int kCols = 16;
  static __device__ __forceinline__ void widen(i32x4 v, float *w) {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const int x = v[d];
#pragma unroll
      for (int b = 0; b < 4; ++b)
        w[d * 4 + b] = (float)(int)(int8_t)(x >> (8 * b));
    }
  }
};

__device__ __forceinline__ void store_y(float *p, float v, int acc) {
  *p = acc ? *p + v : v;
}
__device__ __forceinline__ void store_y(f16 *p, float v, int acc) {
  *p = (f16)(acc ? (float)*p + v : v);
}

}  // namespace

// Grid: (column blocks, K splits). A workgroup owns (64 / H) * kCols columns
// (H = 1: 512 f16 / 1024 int8, one 16-byte segment per lane of a row; H = 2:
// half that, one segment per lane of a 32-lane half) and k_chunk rows, which
// its 8 waves split into contiguous runs of rows_per_wave, and each wave's H
// lane groups into runs of rows_per_wave / H. Each lane streams its column
// segment down its group's rows, two batches of kBatch loads in flight, and
// accumulates in f32; x[r][k] is uniform across a lane group and broadcast
// with readlane.
template <typename WT, int MR, typename OutT, int H>
__global__ __launch_bounds__(kThreads, 1) void gemv_splitk_kernel(
    const f16 *__restrict__ X, const WT *__restrict__ W,
    const f16 *__restrict__ scale, OutT *__restrict__ Y, int N, int K,
    int64_t ldx, int64_t ldw, int64_t ldy, int k_chunk, int rows_per_wave,
    int accumulate, float *__restrict__ partials,
    unsigned *__restrict__ counters, int64_t sx, int64_t sw, int64_t sy,
    Epi epi, int64_t s_mul) {
  typedef WTraits<WT> Tr;
  static_assert(H == 1 || H == 2, "one or two lane groups per wave");
  constexpr int CPT = Tr::kCols;
  constexpr int LPR = 64 / H;  // lanes per row
  constexpr int BNC = LPR * CPT;
  __shared__ float red[kWaves * H][MR][BNC];
  __shared__ unsigned last_flag;

  // Batch z: this workgroup's x, W, y, partials and counters.
  {
    const int64_t z = blockIdx.z;
    X += z * sx;
    W += z * sw;
    Y += z * sy;
    epi.mul += z * s_mul;  // s_mul is 0 without a multiplier
    partials += z * (int64_t)gridDim.y * MR * N;
    counters += z * gridDim.x * kCounterStride;
  }
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int half = H == 2 ? lane / LPR : 0;  // this lane's group
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int split = blockIdx.y, splits = gridDim.y;
  const int64_t n_base = (int64_t)blockIdx.x * BNC;
  const int64_t n0 = n_base + (lane % LPR) * CPT;
  const bool col_ok = n0 < N;  // N is a multiple of CPT
  const int64_t kc0 = (int64_t)split * k_chunk;
  const int64_t kc1 = kc0 + k_chunk < K ? kc0 + k_chunk : K;
  const int64_t kw0 = kc0 + (int64_t)wave * rows_per_wave;
  const int64_t kw1 = kw0 + rows_per_wave < kc1 ? kw0 + rows_per_wave : kc1;
  // The wave's run of nrows rows: group 0 owns the first cnt0 and group 1
  // the other cnt1 (<= cnt0). Both stream cnt0 steps, group 1 over the cnt0
  // rows that end the run, whose first cnt0 - cnt1 (group 0's) it re-reads
  // and skips: every step is a row of the run for both groups, and the step
  // count is wave-uniform.
  const int hr = rows_per_wave / H;
  const int nrows = kw1 > kw0 ? (int)(kw1 - kw0) : 0;
  const int cnt0 = nrows < hr ? nrows : hr;
  const int skip1 = H == 1 ? 0 : 2 * cnt0 - nrows;  // cnt0 - cnt1
  const int64_t hk0 = half ? kw1 - cnt0 : kw0;

  float acc[MR][CPT];
#pragma unroll
  for (int r = 0; r < MR; ++r)
#pragma unroll
    for (int c = 0; c < CPT; ++c)
      acc[r][c] = 0.0f;

  // x[r][k] for this lane group's steps (at most 64), loaded before any
  // weight so that the in-order return of vector loads lets the weights stay
  // in flight while it is read. Lane s holds step s of each group as f16
  // bits, group 1's in the upper half; a step's value is broadcast with
  // readlane and each group shifts its half down.
  int xl[MR];
  const unsigned short *xbits = (const unsigned short *)X;
#pragma unroll
  for (int r = 0; r < MR; ++r) {
    int v = lane < cnt0 ? (int)xbits[r * ldx + kw0 + lane] : 0;
    if constexpr (H == 2)
      if (lane < cnt0)
        v |= (int)xbits[r * ldx + kw1 - cnt0 + lane] << 16;
    xl[r] = v;
  }
  const int x_shift = 16 * half;
  auto x_at = [&](int r, int idx) {
    const int bits = __builtin_amdgcn_readlane(xl[r], idx);
    return (float)__builtin_bit_cast(
        f16, (unsigned short)(H == 2 ? bits >> x_shift : bits));
  };

  // Lanes past N read column 0 instead (never stored), so every load of a
  // batch is unpredicated and only the wave-uniform step bound branches.
  const int64_t ldw_b = ldw * (int64_t)sizeof(WT);
  const char *wrow = (const char *)(W + (col_ok ? n0 : 0)) + hk0 * ldw_b;
  // Steps past the run re-read its last step (their products are skipped),
  // so a batch is 8 unconditional loads the wait counter can track exactly.
  auto load_batch = [&](int sb, i32x4 *v) {
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int st = sb + u < cnt0 ? sb + u : cnt0 - 1;
      v[u] = __builtin_nontemporal_load(
          (const i32x4 *)(wrow + (int64_t)st * ldw_b));
    }
  };
  auto consume = [&](int sb, const i32x4 *v) {
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int st = sb + u;
      // Wave-uniform except in the half-wave form's ragged runs, whose
      // first steps group 1 skips.
      if (st < cnt0 && (H == 1 || st >= skip1 || half == 0)) {
        float w[CPT];
        Tr::widen(v[u], w);
#pragma unroll
        for (int r = 0; r < MR; ++r) {
          const float xv = x_at(r, st);
#pragma unroll
          for (int c = 0; c < CPT; ++c)
            acc[r][c] += xv * w[c];
        }
      }
    }
  };
  // Two register batches in turn, the loop unrolled by two, so that no
  // batch is copied (a copy would wait for its loads) and every consume
  // follows a known sequence of loads: the next batch stays in flight while
  // the current one is consumed.
  if (cnt0 > 0) {
    i32x4 va[kBatch], vb[kBatch];
    int sb = 0;
    load_batch(sb, va);
    while (true) {
      if (sb + kBatch >= cnt0) {
        consume(sb, va);
        break;
      }
      load_batch(sb + kBatch, vb);
      consume(sb, va);
      sb += kBatch;
      if (sb + kBatch >= cnt0) {
        consume(sb, vb);
        break;
      }
      load_batch(sb + kBatch, va);
      consume(sb, vb);
      sb += kBatch;
    }
  }

  // Sum the waves' (and groups') row runs through LDS, in row order.
#pragma unroll
  for (int r = 0; r < MR; ++r)
#pragma unroll
    for (int c = 0; c < CPT; ++c)
      red[wave * H + half][r][(lane % LPR) * CPT + c] = acc[r][c];
  __syncthreads();

  // Output of one element: scale, fused epilogue (chosen once per
  // workgroup, outside the loops: testing the epilogue fields per element
  // slows the plain store), one rounding.
  auto finish = [&](auto with_epi, float s, int r, int64_t n) {
    float v = s * (scale ? (float)scale[n] : 1.0f);
    if constexpr (decltype(with_epi)::value)
      v = epi_apply(v, r, n, epi);
    store_y(Y + r * ldy + n, v, accumulate);
  };
  const bool plain = epi_plain(epi);
  const bool direct = splits == 1;
  auto first = [&](auto with_epi) {
    for (int i = tid; i < MR * BNC; i += kThreads) {
      const int r = i / BNC, col = i % BNC;
      const int64_t n = n_base + col;
      if (n >= N)
        continue;
      float s = red[0][r][col];
#pragma unroll
      for (int w = 1; w < kWaves * H; ++w)
        s += red[w][r][col];
      if (direct) {
        finish(with_epi, s, r, n);
      } else {
        // Device-scope store: written through past this XCD's L2, so a
        // workgroup on another XCD reads it with a device-scope load.
        store_device(&partials[((int64_t)split * MR + r) * N + n], s);
      }
    }
  };
  if (plain)
    first(std::false_type());
  else
    first(std::true_type());
  if (direct)
    return;

  // Every partial store of this workgroup is acknowledged before its arrival
  // is counted: vmcnt(0) per thread, then the barrier. Only the partials and
  // the counter are shared between workgroups, and both are accessed at
  // device scope, so no L2 write-back / invalidate fence is needed.
  wait_vmcnt<0>();
  __syncthreads();
  if (tid == 0) {
    const unsigned prev = __hip_atomic_fetch_add(
        &counters[blockIdx.x * kCounterStride], 1u, __ATOMIC_RELAXED,
        __HIP_MEMORY_SCOPE_AGENT);
    last_flag = prev == (unsigned)(splits - 1);
  }
  __syncthreads();
  if (!last_flag)
    return;
  auto last = [&](auto with_epi) {
    for (int i = tid; i < MR * BNC; i += kThreads) {
      const int r = i / BNC, col = i % BNC;
      const int64_t n = n_base + col;
      if (n >= N)
        continue;
      const float s = partial_sum<float, kSumBatch>(
          &partials[(int64_t)r * N + n], (int64_t)MR * N, splits);
      finish(with_epi, s, r, n);
    }
  };
  if (plain)
    last(std::false_type());
  else
    last(std::true_type());
  if (tid == 0)  // re-arm for the next call on this workspace
    __hip_atomic_store(&counters[blockIdx.x * kCounterStride], 0u,
                       __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// Row-dot form for W [N,K] (K contiguous: the B_TRANSPOSED layout, a torch
// Linear's weight): y[r][n] = sum_k x[r][k] W[n][k]. Workgroup g owns the
// output columns [g P, g P + P) (P = ceil(N / grid)); its waves take them
// from an LDS counter, one (f16 weights) or two (int8) at a time. A wave
// streams those columns' rows of W in 16-byte segments (lane l: segments
// l, l + 64, ...; kBatch loads a row in flight) against x, staged whole in
// LDS once per workgroup, and sums each row wave-wide; lane 0 then scales
// (W8A16), applies the epilogue and stores y[r][n] for each r. K is never
// split: nothing is published and the launch takes no workspace.
template <typename WT, int MR, typename OutT>
__global__ __launch_bounds__(kThreads) void gemv_rowdot_kernel(
    const f16 *__restrict__ X, const WT *__restrict__ W,
    const f16 *__restrict__ scale, OutT *__restrict__ Y, int N, int K,
    int64_t ldx, int64_t ldw, int64_t ldy, int accumulate, int64_t sx,
    int64_t sw, int64_t sy, Epi epi, int64_t s_mul) {
  extern __shared__ __attribute__((aligned(16))) f16 xs[];  // [MR][K]
  __shared__ unsigned next_col;
  constexpr int EPS = 16 / (int)sizeof(WT);  // weights per 16-byte segment
  {
    const int64_t z = blockIdx.z;
    X += z * sx;
    W += z * sw;
    Y += z * sy;
    epi.mul += z * s_mul;
  }
  const int tid = threadIdx.x, lane = tid & 63;
  // x rows into LDS, 16 bytes a step (K is a multiple of 8 and each x row
  // 16-byte aligned, both checked by the planner).
  const int xc = K / 8;
  for (int i = tid; i < MR * xc; i += kThreads) {
    const int r = i / xc, c = i - r * xc;
    *(i32x4 *)(xs + (int64_t)r * K + 8 * c) =
        *(const i32x4 *)(X + r * ldx + 8 * c);
  }
  const int per = (N + (int)gridDim.x - 1) / (int)gridDim.x;
  const int n_begin = (int)blockIdx.x * per;
  const int n_end = min(N, n_begin + per);
  if (tid == 0)
    next_col = (unsigned)n_begin;
  __syncthreads();
  const int segs = K / EPS;  // 16-byte segments of a row of W
  // Vector elements are copied out before __builtin_bit_cast: a bit cast of
  // a vector element expression reads element 0 whatever the index (hipcc
  // 7.2).
  auto dot = [](float a, int w, int x) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w),
                                  __builtin_bit_cast(f16x2, x), a, false);
  };
  // A wave takes COLS columns at a time: their rows' loads are in flight
  // together and each x value read from LDS serves all of them. An odd last
  // column re-reads its own row as the second (its sums are not stored).
  // Two for int8 weights (C5 M=1 N=11008: 11.9 against 13.9 us for one);
  // f16 rows, twice the bytes, measured 2-7 % slower with two.
  constexpr int COLS = sizeof(WT) == 1 ? 2 : 1;
  while (true) {
    int n = 0;
    if (lane == 0)
      n = (int)atomicAdd(&next_col, (unsigned)COLS);
    n = __builtin_amdgcn_readfirstlane(n);
    if (n >= n_end)
      break;
    const bool two = COLS == 2 && n + 1 < n_end;
    const WT *wrow[COLS];
    wrow[0] = W + (int64_t)n * ldw;
    if constexpr (COLS == 2)
      wrow[1] = two ? wrow[0] + ldw : wrow[0];
    float acc[COLS][MR];
#pragma unroll
    for (int c = 0; c < COLS; ++c)
#pragma unroll
      for (int r = 0; r < MR; ++r)
        acc[c][r] = 0.0f;
    for (int s0 = 0; s0 < segs; s0 += 64 * kBatch) {
      i32x4 v[COLS][kBatch];
#pragma unroll
      for (int b = 0; b < kBatch; ++b) {
        const int s = s0 + 64 * b + lane;
        if (s < segs) {
#pragma unroll
          for (int c = 0; c < COLS; ++c)
            v[c][b] = __builtin_nontemporal_load(
                (const i32x4 *)(wrow[c] + (int64_t)s * EPS));
        }
      }
#pragma unroll
      for (int b = 0; b < kBatch; ++b) {
        const int s = s0 + 64 * b + lane;
        if (s >= segs)
          continue;
        const int k0 = s * EPS;
        if constexpr (sizeof(WT) == 2) {
#pragma unroll
          for (int r = 0; r < MR; ++r) {
            const i32x4 xv = *(const i32x4 *)(xs + (int64_t)r * K + k0);
#pragma unroll
            for (int d = 0; d < 4; ++d) {
              const int xd = xv[d];
#pragma unroll
              for (int c = 0; c < COLS; ++c) {
                const int wd = v[c][b][d];
                acc[c][r] = dot(acc[c][r], wd, xd);
              }
            }
          }
        } else {
          // 16 int8 weights as 16 exact f16 values, in k order
          i32x4 w0[COLS], w1[COLS];
#pragma unroll
          for (int c = 0; c < COLS; ++c) {
            w0[c] = i8x8_to_f16x8(i32x2{v[c][b][0], v[c][b][1]});
            w1[c] = i8x8_to_f16x8(i32x2{v[c][b][2], v[c][b][3]});
          }
#pragma unroll
          for (int r = 0; r < MR; ++r) {
            const i32x4 x0 = *(const i32x4 *)(xs + (int64_t)r * K + k0);
            const i32x4 x1 = *(const i32x4 *)(xs + (int64_t)r * K + k0 + 8);
#pragma unroll
            for (int d = 0; d < 4; ++d) {
              const int xa = x0[d], xb = x1[d];
#pragma unroll
              for (int c = 0; c < COLS; ++c) {
                const int wa = w0[c][d], wb = w1[c][d];
                acc[c][r] = dot(acc[c][r], wa, xa);
                acc[c][r] = dot(acc[c][r], wb, xb);
              }
            }
          }
        }
      }
    }
#pragma unroll
    for (int c = 0; c < COLS; ++c)
#pragma unroll
      for (int r = 0; r < MR; ++r) {
        float t = acc[c][r];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1)
          t += __shfl_xor(t, off);
        acc[c][r] = t;
      }
    if (lane == 0) {
#pragma unroll
      for (int c = 0; c < COLS; ++c) {
        if (c == 1 && !two)
          break;
        const int col = n + c;
#pragma unroll
        for (int r = 0; r < MR; ++r) {
          float t = acc[c][r];
          if constexpr (sizeof(WT) == 1)
            t *= (float)scale[col];
          store_y(Y + r * ldy + col, epi_apply(t, r, col, epi), accumulate);
        }
      }
    }
  }
}

// The plan with h lane groups per wave.
static GemvPlan gemv_plan_h(int64_t n, int64_t k, int cpt, int64_t batch,
                            int h) {
  GemvPlan p;
  p.halves = h;
  p.cols_per_wg = 64 / h * cpt;
  const int64_t col_blocks = (n + p.cols_per_wg - 1) / p.cols_per_wg;
  // About one workgroup per CU (256): measured over 128..1024 workgroups on
  // the C3 / C5 shapes, fewer and longer K runs shorten the split-K tail (the
  // partial publish, arrival count and final sum are three memory round
  // trips) but leave CUs idle, more add tail latency. Split K so that
  // col_blocks x splits is about that, each lane group's run of rows a
  // multiple of the load batch.
  const int64_t per_batch = (kGemvTargetWgs + batch - 1) / batch;
  int64_t want = (per_batch + col_blocks / 2) / col_blocks;
  if (want < 1)
    want = 1;
  const int64_t unit = (int64_t)h * kBatch;
  int64_t rpw = (k + want * kWaves - 1) / (want * kWaves);
  rpw = (rpw + unit - 1) / unit * unit;
  if (rpw < unit)
    rpw = unit;
  if (rpw > (int64_t)h * kMaxRowsPerWave)  // x of a run: one value per lane
    rpw = (int64_t)h * kMaxRowsPerWave;
  p.rows_per_wave = (int)rpw;
  p.k_chunk = (int)(rpw * kWaves);
  p.splits = k > 0 ? (int)((k + p.k_chunk - 1) / p.k_chunk) : 1;
  p.col_blocks = col_blocks;
  return p;
}

GemvPlan gemv_plan(int64_t m, int64_t n, int64_t k, int w_bytes,
                   int64_t batch) {
  (void)m;
  const int cpt = w_bytes == 2 ? 8 : 16;
  const GemvPlan one = gemv_plan_h(n, k, cpt, batch, 1);
  const GemvPlan two = gemv_plan_h(n, k, cpt, batch, 2);
  // The last workgroup of a column block reads splits x columns partials
  // alone: the half-wave form halves the columns and about halves the
  // splits. Taken when it shrinks that read and keeps the grid within 1/16
  // of the full-wave one (and its column blocks within the workspace's
  // arrival counters, which the full-wave form's eligibility checked).
  const int64_t wgs1 = one.col_blocks * one.splits;
  const int64_t wgs2 = two.col_blocks * two.splits;
  const int64_t read1 = (int64_t)one.splits * one.cols_per_wg;
  const int64_t read2 =
      two.splits > 1 ? (int64_t)two.splits * two.cols_per_wg : 0;
  const bool counters_fit =
      two.splits == 1 || two.col_blocks * batch <= kMaxWorkspaceCounters;
  if (one.splits > 1 && read2 < read1 && wgs2 <= wgs1 + wgs1 / 16 &&
      counters_fit)
    return two;
  return one;
}

// Workspace layout: [the fixed counter region, one counter per column block]
// [f32 partials (splits x rows x N)]. Each call leaves the counters it used at
// zero again.
static size_t counter_bytes(int64_t col_blocks) {
  (void)col_blocks;
  return kWorkspaceCounterBytes;
}

size_t gemv_workspace_bytes(int64_t m, int64_t n, int64_t k, int w_bytes,
                            int64_t batch) {
  GemvPlan p = gemv_plan(m, n, k, w_bytes, batch);
  if (p.splits <= 1)
    return 0;
  return counter_bytes(p.col_blocks) +
         (size_t)batch * p.splits * kGemvMaxRows * (size_t)n * 4;
}

template <typename WT, int MR, typename OutT>
static hipError_t launch_gemv_t(const MatmulArgs &a, const void *scale,
                                void *workspace, const GemvPlan &p) {
  unsigned *counters = (unsigned *)workspace;
  float *partials =
      workspace ? (float *)((char *)workspace + counter_bytes(p.col_blocks))
                : nullptr;
  dim3 grid((unsigned)p.col_blocks, (unsigned)p.splits, (unsigned)a.batch);
  auto run = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, grid, dim3(kThreads), 0,
                       (hipStream_t)a.stream, (const f16 *)a.a,
                       (const WT *)a.b, (const f16 *)scale, (OutT *)a.c,
                       (int)a.n, (int)a.k, a.lda, a.ldb, a.ldc, p.k_chunk,
                       p.rows_per_wave, a.accumulate, partials, counters,
                       a.sa, a.sb, a.sc, make_epi(a), epi_batch_stride(a));
    return hipGetLastError();
  };
  return p.halves == 2 ? run(gemv_splitk_kernel<WT, MR, OutT, 2>)
                       : run(gemv_splitk_kernel<WT, MR, OutT, 1>);
}

template <typename WT, typename OutT>
static hipError_t launch_gemv_rows(const MatmulArgs &a, const void *scale,
                                   void *ws, const GemvPlan &p) {
  switch (a.m) {
    case 1:
      return launch_gemv_t<WT, 1, OutT>(a, scale, ws, p);
    case 2:
      return launch_gemv_t<WT, 2, OutT>(a, scale, ws, p);
    case 3:
      return launch_gemv_t<WT, 3, OutT>(a, scale, ws, p);
    case 4:
      return launch_gemv_t<WT, 4, OutT>(a, scale, ws, p);
  }
  return hipErrorInvalidValue;
}

template <typename WT, int MR, typename OutT>
static hipError_t launch_rowdot_t(const MatmulArgs &a, const void *scale) {
  const dim3 grid((unsigned)rowdot_workgroups(a.n), 1, (unsigned)a.batch);
  const size_t x_bytes = (size_t)MR * (size_t)a.k * sizeof(f16);
  hipLaunchKernelGGL((gemv_rowdot_kernel<WT, MR, OutT>), grid, dim3(kThreads),
                     x_bytes, (hipStream_t)a.stream, (const f16 *)a.a,
                     (const WT *)a.b, (const f16 *)scale, (OutT *)a.c,
                     (int)a.n, (int)a.k, a.lda, a.ldb, a.ldc, a.accumulate,
                     a.sa, a.sb, a.sc, make_epi(a), epi_batch_stride(a));
  return hipGetLastError();
}

template <typename WT, typename OutT>
static hipError_t launch_rowdot(const MatmulArgs &a, const void *scale) {
  switch (a.m) {
    case 1:
      return launch_rowdot_t<WT, 1, OutT>(a, scale);
    case 2:
      return launch_rowdot_t<WT, 2, OutT>(a, scale);
    case 3:
      return launch_rowdot_t<WT, 3, OutT>(a, scale);
    case 4:
      return launch_rowdot_t<WT, 4, OutT>(a, scale);
  }
  if constexpr (sizeof(WT) == 1) {  // W8A16 launches of up to 8 rows
    switch (a.m) {
      case 5:
        return launch_rowdot_t<WT, 5, OutT>(a, scale);
      case 6:
        return launch_rowdot_t<WT, 6, OutT>(a, scale);
      case 7:
        return launch_rowdot_t<WT, 7, OutT>(a, scale);
      case 8:
        return launch_rowdot_t<WT, 8, OutT>(a, scale);
    }
  }
  return hipErrorInvalidValue;
}

hipError_t launch_gemv(const MatmulArgs &a, int w_bytes, const void *scale,
                       int out_f32, void *workspace) {
  if (a.b_transposed) {
    const int64_t rows =
        w_bytes == 1 ? rowdot_w8a16_rows(a.m, a.k) : a.m;
    if (rows < 1 || rows * a.k * (int64_t)sizeof(f16) > kRowdotMaxXBytes ||
        a.k % 16 != 0 ||
        a.m > (w_bytes == 1 ? kRowdotMaxRowsW8A16 : kGemvMaxRows))
      return hipErrorInvalidValue;
    if (w_bytes == 2)
      return out_f32 ? launch_rowdot<f16, float>(a, nullptr)
                     : launch_rowdot<f16, f16>(a, nullptr);
    // W8A16: blocks of `rows` rows of x (and of y and the multiplier), one
    // launch each
    for (int64_t r0 = 0; r0 < a.m; r0 += rows) {
      MatmulArgs b = a;
      b.m = a.m - r0 < rows ? a.m - r0 : rows;
      b.a = (const f16 *)a.a + r0 * a.lda;
      b.c = (f16 *)a.c + r0 * a.ldc;
      if (a.mul)
        b.mul = (const f16 *)a.mul + r0 * a.ld_mul;
      const hipError_t e = launch_rowdot<int8_t, f16>(b, scale);
      if (e != hipSuccess)
        return e;
    }
    return hipSuccess;
  }
  const GemvPlan p = gemv_plan(a.m, a.n, a.k, w_bytes, a.batch);
  if (w_bytes == 2)
    return out_f32 ? launch_gemv_rows<f16, float>(a, nullptr, workspace, p)
                   : launch_gemv_rows<f16, f16>(a, nullptr, workspace, p);
  return launch_gemv_rows<int8_t, f16>(a, scale, workspace, p);
}

}  // namespace ihp

namespace ihp {

// Every GEMV kernel: rows 1..4 for f16 weights (f16 / f32 out) and W8A16,
// in the full-wave and the half-wave (_h2) form for W [K,N], and the
// row-dot form for W [N,K].
const KernelEntry *gemv_kernels(int *count) {
  const uint32_t f16x = kExportMatmulF16 | kExportBatchMatmulF16;
  static const KernelEntry all[] = {
      {"gemv_f16_r1", (const void *)&gemv_splitk_kernel<f16, 1, f16, 1>, kThreads, f16x},
      {"gemv_f16_r2", (const void *)&gemv_splitk_kernel<f16, 2, f16, 1>, kThreads, f16x},
      {"gemv_f16_r3", (const void *)&gemv_splitk_kernel<f16, 3, f16, 1>, kThreads, f16x},
      {"gemv_f16_r4", (const void *)&gemv_splitk_kernel<f16, 4, f16, 1>, kThreads, f16x},
      {"gemv_f16f32_r1", (const void *)&gemv_splitk_kernel<f16, 1, float, 1>, kThreads, f16x},
      {"gemv_f16f32_r2", (const void *)&gemv_splitk_kernel<f16, 2, float, 1>, kThreads, f16x},
      {"gemv_f16f32_r3", (const void *)&gemv_splitk_kernel<f16, 3, float, 1>, kThreads, f16x},
      {"gemv_f16f32_r4", (const void *)&gemv_splitk_kernel<f16, 4, float, 1>, kThreads, f16x},
      {"gemv_w8a16_r1", (const void *)&gemv_splitk_kernel<int8_t, 1, f16, 1>, kThreads, kExportW8A16},
      {"gemv_w8a16_r2", (const void *)&gemv_splitk_kernel<int8_t, 2, f16, 1>, kThreads, kExportW8A16},
      {"gemv_w8a16_r3", (const void *)&gemv_splitk_kernel<int8_t, 3, f16, 1>, kThreads, kExportW8A16},
      {"gemv_w8a16_r4", (const void *)&gemv_splitk_kernel<int8_t, 4, f16, 1>, kThreads, kExportW8A16},
      {"gemv_f16_r1_h2", (const void *)&gemv_splitk_kernel<f16, 1, f16, 2>, kThreads, f16x},
      {"gemv_f16_r2_h2", (const void *)&gemv_splitk_kernel<f16, 2, f16, 2>, kThreads, f16x},
      {"gemv_f16_r3_h2", (const void *)&gemv_splitk_kernel<f16, 3, f16, 2>, kThreads, f16x},
      {"gemv_f16_r4_h2", (const void *)&gemv_splitk_kernel<f16, 4, f16, 2>, kThreads, f16x},
      {"gemv_f16f32_r1_h2", (const void *)&gemv_splitk_kernel<f16, 1, float, 2>, kThreads, f16x},
      {"gemv_f16f32_r2_h2", (const void *)&gemv_splitk_kernel<f16, 2, float, 2>, kThreads, f16x},
      {"gemv_f16f32_r3_h2", (const void *)&gemv_splitk_kernel<f16, 3, float, 2>, kThreads, f16x},
      {"gemv_f16f32_r4_h2", (const void *)&gemv_splitk_kernel<f16, 4, float, 2>, kThreads, f16x},
      {"gemv_w8a16_r1_h2", (const void *)&gemv_splitk_kernel<int8_t, 1, f16, 2>, kThreads, kExportW8A16},
      {"gemv_w8a16_r2_h2", (const void *)&gemv_splitk_kernel<int8_t, 2, f16, 2>, kThreads, kExportW8A16},
      {"gemv_w8a16_r3_h2", (const void *)&gemv_splitk_kernel<int8_t, 3, f16, 2>, kThreads, kExportW8A16},
      {"gemv_w8a16_r4_h2", (const void *)&gemv_splitk_kernel<int8_t, 4, f16, 2>, kThreads, kExportW8A16},
      {"gemv_rowdot_f16_r1", (const void *)&gemv_rowdot_kernel<f16, 1, f16>, kThreads, f16x},
      {"gemv_rowdot_f16_r2", (const void *)&gemv_rowdot_kernel<f16, 2, f16>, kThreads, f16x},
      {"gemv_rowdot_f16_r3", (const void *)&gemv_rowdot_kernel<f16, 3, f16>, kThreads, f16x},
      {"gemv_rowdot_f16_r4", (const void *)&gemv_rowdot_kernel<f16, 4, f16>, kThreads, f16x},
      {"gemv_rowdot_f16f32_r1", (const void *)&gemv_rowdot_kernel<f16, 1, float>, kThreads, f16x},
      {"gemv_rowdot_f16f32_r2", (const void *)&gemv_rowdot_kernel<f16, 2, float>, kThreads, f16x},
      {"gemv_rowdot_f16f32_r3", (const void *)&gemv_rowdot_kernel<f16, 3, float>, kThreads, f16x},
      {"gemv_rowdot_f16f32_r4", (const void *)&gemv_rowdot_kernel<f16, 4, float>, kThreads, f16x},
      {"gemv_rowdot_w8a16_r1", (const void *)&gemv_rowdot_kernel<int8_t, 1, f16>, kThreads, kExportW8A16},
      {"gemv_rowdot_w8a16_r2", (const void *)&gemv_rowdot_kernel<int8_t, 2, f16>, kThreads, kExportW8A16},
      {"gemv_rowdot_w8a16_r3", (const void *)&gemv_rowdot_kernel<int8_t, 3, f16>, kThreads, kExportW8A16},
      {"gemv_rowdot_w8a16_r4", (const void *)&gemv_rowdot_kernel<int8_t, 4, f16>, kThreads, kExportW8A16},
      {"gemv_rowdot_w8a16_r5", (const void *)&gemv_rowdot_kernel<int8_t, 5, f16>, kThreads, kExportW8A16},
      {"gemv_rowdot_w8a16_r6", (const void *)&gemv_rowdot_kernel<int8_t, 6, f16>, kThreads, kExportW8A16},
      {"gemv_rowdot_w8a16_r7", (const void *)&gemv_rowdot_kernel<int8_t, 7, f16>, kThreads, kExportW8A16},
      {"gemv_rowdot_w8a16_r8", (const void *)&gemv_rowdot_kernel<int8_t, 8, f16>, kThreads, kExportW8A16},
  };
  *count = (int)(sizeof(all) / sizeof(all[0]));
  return all;
}

}  // namespace ihp
