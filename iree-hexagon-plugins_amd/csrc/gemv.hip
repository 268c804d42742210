// HBM-streaming skinny matmul (M <= 4 rows of activations) for B = W [K,N]
// row-major: the decode-shaped linear (M = 1 GEMV) and the W8A16 linear with
// int8 weights dequantized in-kernel.
//
// In the reference such a dispatch is still an HMX matmul: M is padded to the
// 32-row HMX tile (CG/Transforms/HexagonConvertMatmulToHmx.cpp:51-70) and the
// VTCM plan keeps K whole (CG/Strategy/Planning/VTCMPlanning.cpp:156-260).
// With M = 1 the work is reading W once, so on MI355X it is a bandwidth
// kernel, not an MFMA kernel:
//  * each thread streams 16-byte row segments of W (8 f16 or 16 int8
//    weights), several loads in flight, and accumulates in f32;
//  * K is split over a 2-D grid (column block x K split) so the whole chip
//    streams at once; each workgroup reduces its 8 K-lanes through LDS and
//    writes an f32 partial;
//  * the last workgroup to finish a column block (device-scope arrival
//    counter) sums the partials, applies the per-column scale (W8A16), adds
//    the DPS init if asked, rounds once and re-arms the counter, so the
//    whole matmul is one launch.
#include "device_common.h"
#include "kernels_internal.h"

namespace ihp {

namespace {

constexpr int kThreads = 256;
constexpr int kTN = 32;                 // threads across columns
constexpr int kTK = kThreads / kTN;     // K lanes per workgroup
constexpr int kUnroll = 8;              // 16-byte loads in flight per thread
constexpr int kKChunkAlign = kTK * kUnroll;
constexpr int kMaxKChunk = 1024;        // rows of W per workgroup (x in LDS)

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

template <typename WT, int MR, typename OutT>
__global__ __launch_bounds__(kThreads) void gemv_splitk_kernel(
    const f16 *__restrict__ X, const WT *__restrict__ W,
    const f16 *__restrict__ scale, OutT *__restrict__ Y, int N, int K,
    int64_t ldx, int64_t ldw, int64_t ldy, int k_chunk, int accumulate,
    float *__restrict__ partials, unsigned *__restrict__ counters) {
  typedef WTraits<WT> Tr;
  constexpr int CPT = Tr::kCols;
  constexpr int BNC = kTN * CPT;
  __shared__ float xs[MR * kMaxKChunk];
  __shared__ float red[4][MR][BNC];
  __shared__ unsigned last_flag;

  const int tid = threadIdx.x;
  const int tn = tid % kTN, tk = tid / kTN;
  const int wave = tid >> 6;
  const int split = blockIdx.y, splits = gridDim.y;
  const int64_t k0 = (int64_t)split * k_chunk;
  const int64_t k1 = k0 + k_chunk < K ? k0 + k_chunk : K;
  const int64_t n_base = (int64_t)blockIdx.x * BNC;
  const int64_t n0 = n_base + tn * CPT;
  const bool col_ok = n0 < N;  // N is a multiple of CPT

  // Stage this split's slice of x (MR rows) into LDS as f32.
  for (int64_t i = tid; i < (int64_t)MR * (k1 - k0); i += kThreads) {
    const int r = (int)(i / (k1 - k0));
    const int64_t kk = i - r * (k1 - k0);
    xs[r * kMaxKChunk + kk] = (float)X[r * ldx + k0 + kk];
  }
  __syncthreads();

  float acc[MR][CPT];
#pragma unroll
  for (int r = 0; r < MR; ++r)
#pragma unroll
    for (int c = 0; c < CPT; ++c)
      acc[r][c] = 0.0f;

  const char *wrow = (const char *)(W + n0);
  const int64_t ldw_b = ldw * (int64_t)sizeof(WT);
  // Full groups of kUnroll rows: every load in range, no per-load branch.
  int64_t kb = k0 + tk;
  if (col_ok) {
    for (; kb + (int64_t)(kUnroll - 1) * kTK < k1; kb += kTK * kUnroll) {
      i32x4 v[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u)
        v[u] = __builtin_nontemporal_load(
            (const i32x4 *)(wrow + (kb + (int64_t)u * kTK) * ldw_b));
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int64_t k = kb + (int64_t)u * kTK;
        float w[CPT];
        Tr::widen(v[u], w);
#pragma unroll
        for (int r = 0; r < MR; ++r) {
          const float xv = xs[r * kMaxKChunk + (k - k0)];
#pragma unroll
          for (int c = 0; c < CPT; ++c)
            acc[r][c] += xv * w[c];
        }
      }
    }
  }
  // Tail (K not a multiple of the group).
  for (; kb < k1; kb += kTK * kUnroll) {
    i32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t k = kb + (int64_t)u * kTK;
      v[u] = (col_ok && k < k1)
                 ? __builtin_nontemporal_load((const i32x4 *)(wrow + k * ldw_b))
                 : i32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t k = kb + (int64_t)u * kTK;
      if (k < k1) {
        float w[CPT];
        Tr::widen(v[u], w);
#pragma unroll
        for (int r = 0; r < MR; ++r) {
          const float xv = xs[r * kMaxKChunk + (k - k0)];
#pragma unroll
          for (int c = 0; c < CPT; ++c)
            acc[r][c] += xv * w[c];
        }
      }
    }
  }

  // Reduce the two K lanes of each wave, then the four waves through LDS.
#pragma unroll
  for (int r = 0; r < MR; ++r)
#pragma unroll
    for (int c = 0; c < CPT; ++c)
      acc[r][c] += __shfl_xor(acc[r][c], 32);
  if ((tid & 63) < 32) {
#pragma unroll
    for (int r = 0; r < MR; ++r)
#pragma unroll
      for (int c = 0; c < CPT; ++c)
        red[wave][r][tn * CPT + c] = acc[r][c];
  }
  __syncthreads();

  const bool direct = splits == 1;
  for (int i = tid; i < MR * BNC; i += kThreads) {
    const int r = i / BNC, col = i % BNC;
    const float s = red[0][r][col] + red[1][r][col] + red[2][r][col] +
                    red[3][r][col];
    const int64_t n = n_base + col;
    if (n >= N)
      continue;
    if (direct) {
      const float sc = scale ? (float)scale[n] : 1.0f;
      store_y(Y + r * ldy + n, s * sc, accumulate);
    } else {
      // Device-scope store: written through past this XCD's L2, so a
      // workgroup on another XCD reads it with a device-scope load.
      store_device(&partials[((int64_t)split * MR + r) * N + n], s);
    }
  }
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
        &counters[blockIdx.x], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last_flag = prev == (unsigned)(splits - 1);
  }
  __syncthreads();
  if (!last_flag)
    return;
  for (int i = tid; i < MR * BNC; i += kThreads) {
    const int r = i / BNC, col = i % BNC;
    const int64_t n = n_base + col;
    if (n >= N)
      continue;
    const float s = partial_sum(&partials[(int64_t)r * N + n],
                                (int64_t)MR * N, splits);
    const float sc = scale ? (float)scale[n] : 1.0f;
    store_y(Y + r * ldy + n, s * sc, accumulate);
  }
  if (tid == 0)  // re-arm for the next call on this workspace
    __hip_atomic_store(&counters[blockIdx.x], 0u, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

static int round_up(int64_t v, int64_t a) { return (int)((v + a - 1) / a * a); }

GemvPlan gemv_plan(int64_t m, int64_t n, int64_t k, int w_bytes) {
  (void)m;
  const int cpt = w_bytes == 2 ? 8 : 16;
  GemvPlan p;
  p.cols_per_wg = kTN * cpt;
  const int64_t col_blocks = (n + p.cols_per_wg - 1) / p.cols_per_wg;
  // Aim for about three workgroups per CU over 256 CUs.
  int64_t want = (768 + col_blocks - 1) / col_blocks;
  if (want < 1)
    want = 1;
  int chunk = round_up((k + want - 1) / want, kKChunkAlign);
  if (chunk > kMaxKChunk)
    chunk = kMaxKChunk;
  if (chunk < kKChunkAlign)
    chunk = kKChunkAlign;
  p.k_chunk = chunk;
  p.splits = k > 0 ? (int)((k + chunk - 1) / chunk) : 1;
  p.col_blocks = col_blocks;
  return p;
}

// Workspace layout: [arrival counters, one per column block][f32 partials
// (splits x rows x N)]. The counters sit at offset 0 for every shape, so one
// zero-filled workspace serves any sequence of calls; each call leaves the
// counters it used at zero again.
static size_t counter_bytes(int64_t col_blocks) {
  return (size_t)((col_blocks * 4 + 255) / 256 * 256);
}

size_t gemv_workspace_bytes(int64_t m, int64_t n, int64_t k, int w_bytes) {
  GemvPlan p = gemv_plan(m, n, k, w_bytes);
  if (p.splits <= 1)
    return 0;
  return counter_bytes(p.col_blocks) +
         (size_t)p.splits * kGemvMaxRows * (size_t)n * 4;
}

template <typename WT, int MR, typename OutT>
static hipError_t launch_gemv_t(const MatmulArgs &a, const void *scale,
                                void *workspace, const GemvPlan &p) {
  unsigned *counters = (unsigned *)workspace;
  float *partials =
      workspace ? (float *)((char *)workspace + counter_bytes(p.col_blocks))
                : nullptr;
  dim3 grid((unsigned)p.col_blocks, (unsigned)p.splits);
  hipLaunchKernelGGL((gemv_splitk_kernel<WT, MR, OutT>), grid, dim3(kThreads),
                     0, (hipStream_t)a.stream, (const f16 *)a.a,
                     (const WT *)a.b, (const f16 *)scale, (OutT *)a.c,
                     (int)a.n, (int)a.k, a.lda, a.ldb, a.ldc, p.k_chunk,
                     a.accumulate, partials, counters);
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
  const GemvPlan p = gemv_plan(a.m, a.n, a.k, w_bytes);
  if (w_bytes == 2)
    return out_f32 ? launch_gemv_rows<f16, float>(a, nullptr, workspace, p)
                   : launch_gemv_rows<f16, f16>(a, nullptr, workspace, p);
  return launch_gemv_rows<int8_t, f16>(a, scale, workspace, p);
}

}  // namespace ihp
