// HBM-streaming skinny matmul (M <= 4 rows of activations) for B = W [K,N]
// row-major: the decode-shaped linear (M = 1 GEMV) and the W8A16 linear with
// int8 weights dequantized in-kernel.
//
// In the reference such a dispatch is still an HMX matmul: M is padded to the
// 32-row HMX tile (CG/Transforms/HexagonConvertMatmulToHmx.cpp:51-70) and the
// VTCM plan keeps K whole (CG/Strategy/Planning/VTCMPlanning.cpp:156-260).
// With M = 1 the work is reading W once, so on MI355X it is a bandwidth
// kernel, not an MFMA kernel:
//  * each lane streams one 16-byte column segment of W (8 f16 or 16 int8
//    weights) down a run of rows, 16 loads in flight, and accumulates in
//    f32; x is read through the scalar cache, nothing is staged first;
//  * K is split over a 2-D grid (column block x K split) sized to about one
//    workgroup per CU; each workgroup sums its 8 waves through LDS and writes
//    an f32 partial;
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

// Grid: (column blocks, K splits). A workgroup owns 64 * kCols columns
// (512 f16 / 1024 int8: one 16-byte segment per lane of a row) and k_chunk
// rows, which its 8 waves split into contiguous runs of rows_per_wave. Each
// lane streams its column segment down its wave's rows, two batches of
// kBatch loads in flight, and accumulates in f32; x[r][k] is wave-uniform and
// comes through the scalar cache.
template <typename WT, int MR, typename OutT>
__global__ __launch_bounds__(kThreads, 1) void gemv_splitk_kernel(
    const f16 *__restrict__ X, const WT *__restrict__ W,
    const f16 *__restrict__ scale, OutT *__restrict__ Y, int N, int K,
    int64_t ldx, int64_t ldw, int64_t ldy, int k_chunk, int rows_per_wave,
    int accumulate, float *__restrict__ partials,
    unsigned *__restrict__ counters, int64_t sx, int64_t sw, int64_t sy,
    Epi epi, int64_t s_mul) {
  typedef WTraits<WT> Tr;
  constexpr int CPT = Tr::kCols;
  constexpr int BNC = 64 * CPT;
  __shared__ float red[kWaves][MR][BNC];
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
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int split = blockIdx.y, splits = gridDim.y;
  const int64_t n_base = (int64_t)blockIdx.x * BNC;
  const int64_t n0 = n_base + lane * CPT;
  const bool col_ok = n0 < N;  // N is a multiple of CPT
  const int64_t kc0 = (int64_t)split * k_chunk;
  const int64_t kc1 = kc0 + k_chunk < K ? kc0 + k_chunk : K;
  const int64_t kw0 = kc0 + (int64_t)wave * rows_per_wave;
  const int64_t kw1 = kw0 + rows_per_wave < kc1 ? kw0 + rows_per_wave : kc1;

  float acc[MR][CPT];
#pragma unroll
  for (int r = 0; r < MR; ++r)
#pragma unroll
    for (int c = 0; c < CPT; ++c)
      acc[r][c] = 0.0f;

  // x[r][kw0 + lane] for this wave's rows (at most 64), loaded before any
  // weight so that the in-order return of vector loads lets the weights stay
  // in flight while it is read; row u of the run is then lane u's value,
  // broadcast with readlane.
  int xl[MR];  // raw f16 bits, widened when broadcast
  const unsigned short *xbits = (const unsigned short *)X;
#pragma unroll
  for (int r = 0; r < MR; ++r)
    xl[r] = kw0 + lane < kw1 ? (int)xbits[r * ldx + kw0 + lane] : 0;

  // Lanes past N read column 0 instead (never stored), so every load of a
  // batch is unpredicated and only the wave-uniform row bound branches.
  const char *wcol = (const char *)(W + (col_ok ? n0 : 0));
  const int64_t ldw_b = ldw * (int64_t)sizeof(WT);
  // Rows past the run re-read its last row (their products are skipped), so
  // a batch is 8 unconditional loads the wait counter can track exactly.
  auto load_batch = [&](int64_t kb, i32x4 *v) {
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int64_t k = kb + u < kw1 ? kb + u : kw1 - 1;
      v[u] = __builtin_nontemporal_load((const i32x4 *)(wcol + k * ldw_b));
    }
  };
  auto consume = [&](int64_t kb, const i32x4 *v) {
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int64_t k = kb + u;
      if (k < kw1) {  // wave-uniform
        float w[CPT];
        Tr::widen(v[u], w);
        const int idx = (int)(k - kw0);
#pragma unroll
        for (int r = 0; r < MR; ++r) {
          const float xv = (float)__builtin_bit_cast(
              f16, (unsigned short)__builtin_amdgcn_readlane(xl[r], idx));
#pragma unroll
          for (int c = 0; c < CPT; ++c)
            acc[r][c] += xv * w[c];
        }
      }
    }
  };
  if (kw0 < kw1) {
    i32x4 cur[kBatch], nxt[kBatch];
    int64_t kb = kw0;
    load_batch(kb, cur);
    while (true) {
      const bool more = kb + kBatch < kw1;
      if (more)
        load_batch(kb + kBatch, nxt);
      consume(kb, cur);
      if (!more)
        break;
      kb += kBatch;
#pragma unroll
      for (int u = 0; u < kBatch; ++u)
        cur[u] = nxt[u];
    }
  }

  // Sum the 8 waves' row runs through LDS, in wave order.
#pragma unroll
  for (int r = 0; r < MR; ++r)
#pragma unroll
    for (int c = 0; c < CPT; ++c)
      red[wave][r][lane * CPT + c] = acc[r][c];
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
      for (int w = 1; w < kWaves; ++w)
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

GemvPlan gemv_plan(int64_t m, int64_t n, int64_t k, int w_bytes,
                   int64_t batch) {
  (void)m;
  const int cpt = w_bytes == 2 ? 8 : 16;
  GemvPlan p;
  p.cols_per_wg = 64 * cpt;
  const int64_t col_blocks = (n + p.cols_per_wg - 1) / p.cols_per_wg;
  // About one workgroup per CU (256): measured over 128..1024 workgroups on
  // the C3 / C5 shapes, fewer and longer K runs shorten the split-K tail (the
  // partial publish, arrival count and final sum are three memory round
  // trips) but leave CUs idle, more add tail latency. Split K so that
  // col_blocks x splits is about that, each wave's run of rows a multiple of
  // the load batch.
  const int64_t per_batch = (kGemvTargetWgs + batch - 1) / batch;
  int64_t want = (per_batch + col_blocks / 2) / col_blocks;
  if (want < 1)
    want = 1;
  int64_t rpw = (k + want * kWaves - 1) / (want * kWaves);
  rpw = (rpw + kBatch - 1) / kBatch * kBatch;
  if (rpw < kBatch)
    rpw = kBatch;
  if (rpw > kMaxRowsPerWave)  // x of a run is one value per lane
    rpw = kMaxRowsPerWave;
  p.rows_per_wave = (int)rpw;
  p.k_chunk = (int)(rpw * kWaves);
  p.splits = k > 0 ? (int)((k + p.k_chunk - 1) / p.k_chunk) : 1;
  p.col_blocks = col_blocks;
  return p;
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
  hipLaunchKernelGGL((gemv_splitk_kernel<WT, MR, OutT>), grid, dim3(kThreads),
                     0, (hipStream_t)a.stream, (const f16 *)a.a,
                     (const WT *)a.b, (const f16 *)scale, (OutT *)a.c,
                     (int)a.n, (int)a.k, a.lda, a.ldb, a.ldc, p.k_chunk,
                     p.rows_per_wave, a.accumulate, partials, counters, a.sa,
                     a.sb, a.sc, make_epi(a), epi_batch_stride(a));
  return hipGetLastError();
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

hipError_t launch_gemv(const MatmulArgs &a, int w_bytes, const void *scale,
                       int out_f32, void *workspace) {
  const GemvPlan p = gemv_plan(a.m, a.n, a.k, w_bytes, a.batch);
  if (w_bytes == 2)
    return out_f32 ? launch_gemv_rows<f16, float>(a, nullptr, workspace, p)
                   : launch_gemv_rows<f16, f16>(a, nullptr, workspace, p);
  return launch_gemv_rows<int8_t, f16>(a, scale, workspace, p);
}

}  // namespace ihp

namespace ihp {

// Every GEMV kernel: rows 1..4 for f16 weights (f16 / f32 out) and W8A16.
const KernelEntry *gemv_kernels(int *count) {
  const uint32_t f16x = kExportMatmulF16 | kExportBatchMatmulF16;
  static const KernelEntry all[] = {
      {"gemv_f16_r1", (const void *)&gemv_splitk_kernel<f16, 1, f16>, kThreads, f16x},
      {"gemv_f16_r2", (const void *)&gemv_splitk_kernel<f16, 2, f16>, kThreads, f16x},
      {"gemv_f16_r3", (const void *)&gemv_splitk_kernel<f16, 3, f16>, kThreads, f16x},
      {"gemv_f16_r4", (const void *)&gemv_splitk_kernel<f16, 4, f16>, kThreads, f16x},
      {"gemv_f16f32_r1", (const void *)&gemv_splitk_kernel<f16, 1, float>, kThreads, f16x},
      {"gemv_f16f32_r2", (const void *)&gemv_splitk_kernel<f16, 2, float>, kThreads, f16x},
      {"gemv_f16f32_r3", (const void *)&gemv_splitk_kernel<f16, 3, float>, kThreads, f16x},
      {"gemv_f16f32_r4", (const void *)&gemv_splitk_kernel<f16, 4, float>, kThreads, f16x},
      {"gemv_w8a16_r1", (const void *)&gemv_splitk_kernel<int8_t, 1, f16>, kThreads, kExportW8A16},
      {"gemv_w8a16_r2", (const void *)&gemv_splitk_kernel<int8_t, 2, f16>, kThreads, kExportW8A16},
      {"gemv_w8a16_r3", (const void *)&gemv_splitk_kernel<int8_t, 3, f16>, kThreads, kExportW8A16},
      {"gemv_w8a16_r4", (const void *)&gemv_splitk_kernel<int8_t, 4, f16>, kThreads, kExportW8A16},
  };
  *count = (int)(sizeof(all) / sizeof(all[0]));
  return all;
}

}  // namespace ihp
