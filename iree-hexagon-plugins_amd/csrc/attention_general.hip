// General attention forward: any head dims (Q/K and V/O may differ, up to
// 256), an optional additive mask, f16 or f32 output, strided operands and
// grouped KV heads.
//
// The reference lowers iree_linalg_ext.attention whatever its head dims,
// mask or output type, through online attention
// (CG/Pipelines/LoweringPipelines.cpp:561-595; the online_attention of the
// pipeline test test/codegen/pipelines/hexagon_lower_executable_target.mlir:
// 195-233 has a QK head dim of 4, a V head dim of 5, scale 0.5 and an f32
// accumulator). The
// MFMA kernel (attention.hip) takes the common shapes; this one takes the
// rest, with the same semantics:
//  * a workgroup owns 64 query rows of one (batch, head) (under the causal
//    mask two such blocks, x and the mirror one, for an even load); four
//    lanes share a row, each holding a quarter of its Q slice (f16 pairs)
//    and of its O accumulator (f32) in registers;
//  * 32-key blocks of K and V are staged in LDS (bounds-checked element
//    loads, zero past the sequence and head dims); a row's score is its four
//    lanes' partial dot products summed across the quad;
//  * scores are scaled, the mask added, causal and out-of-range keys set to
//    -inf, then an online softmax in f32 rescales the accumulator block by
//    block; a row that sees no key (fully masked) writes 0, as the
//    all-masked-row guard of the decomposed softmax does
//    (examples/attention_layer/attention_layer.mlir:80-102).
#include <type_traits>

#include "device_common.h"
#include "kernels_internal.h"

namespace ihp {

namespace {

constexpr int kGenThreads = 256;
constexpr int kGenRows = kGenThreads / 4;  // query rows per workgroup
constexpr int kGenKeys = 32;               // keys per LDS block

__device__ __forceinline__ float quad_sum(float x) {
  x += __shfl_xor(x, 1, 64);
  x += __shfl_xor(x, 2, 64);
  return x;
}

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ void store_o(f16 *p, float v) { *p = (f16)v; }
__device__ __forceinline__ void store_o(float *p, float v) { *p = v; }

}  // namespace

// MAXD: the head-dim bucket (a power of two >= both head dims); each of a
// row's four lanes holds MAXD / 4 elements of Q (as f16 pairs) and of the O
// accumulator (f32). Scores are v_dot2_f32_f16 sums of those pairs (f16
// products are exact in f32); PV multiplies the f16 V values into f32 (the
// widening folds into v_fma_mix).
template <int MAXD, typename OutT>
__global__ __launch_bounds__(kGenThreads) void attention_general_kernel(
    const f16 *__restrict__ Q, const f16 *__restrict__ K,
    const f16 *__restrict__ V, OutT *__restrict__ O,
    const f16 *__restrict__ Mask, AttentionGeneralLayout L) {
  constexpr int QC = MAXD / 4;
  constexpr int QP = QC / 2;    // f16 pairs a lane holds
  constexpr int PAD = 8;        // keeps the four quarters of a row off one bank
  constexpr int RS = MAXD + PAD;  // LDS row stride (elements; 16-byte rows)
  constexpr int CPR = MAXD / 8;   // 16-byte chunks of a row
  static_assert(QC % 2 == 0 && (RS * 2) % 16 == 0, "layout");
  __shared__ __attribute__((aligned(16))) f16 ks[kGenKeys][RS];
  __shared__ __attribute__((aligned(16))) f16 vs[kGenKeys][RS];
  __shared__ f16 ms[kGenRows][kGenKeys + 2];  // this block's mask values

  const int t = threadIdx.x;
  const int r = t >> 2, qd = t & 3;
  const int64_t b = blockIdx.z, h = blockIdx.y, hk = h / L.group;
  const f16 *kp = K + b * L.k[0] + hk * L.k[1];
  const f16 *vp = V + b * L.v[0] + hk * L.v[1];
  const f16 *mbase = Mask ? Mask + b * L.mask[0] + h * L.mask[1] : nullptr;
  const int d0 = qd * QC;
  // Under the causal mask row block x costs x + 1 key blocks: a workgroup
  // takes blocks x and nb - 1 - x (one when they coincide), so every
  // workgroup carries about the same keys; otherwise one block each.
  const int nb = (L.seq_q + kGenRows - 1) / kGenRows;
  const int x = blockIdx.x;
  const int n_items = L.causal && nb - 1 - x != x ? 2 : 1;
  for (int item = 0; item < n_items; ++item) {
    const int row0 = (item == 0 ? x : nb - 1 - x) * kGenRows;
    const int i = row0 + r;
    const bool row_ok = i < L.seq_q;
    const int ic = row_ok ? i : L.seq_q - 1;
    const f16 *qp = Q + b * L.q[0] + h * L.q[1] + (int64_t)ic * L.q[2];

    f16x2 q2[QP];
    float acc[QC];
#pragma unroll
    for (int c = 0; c < QP; ++c) {
      const int d = d0 + 2 * c;
      q2[c] = f16x2{d < L.dqk ? qp[d] : (f16)0,
                    d + 1 < L.dqk ? qp[d + 1] : (f16)0};
    }
#pragma unroll
    for (int c = 0; c < QC; ++c)
      acc[c] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;

    // 16-byte fills when every K (V) row starts 16-byte aligned and its head
    // dim is a multiple of 8 (decided on the host, uniform); element fills
    // with bounds checks otherwise. Both write zeros past the sequence and
    // the head dim.
    auto fill = [&](f16 (*dst)[RS], const f16 *src, int64_t pitch, int dim,
                    int vec, int kb0) {
      if (vec) {
        for (int e = t; e < kGenKeys * CPR; e += kGenThreads) {
          const int j = e / CPR, c8 = (e % CPR) * 8;
          const int key = kb0 + j;
          i32x4 v = i32x4{0, 0, 0, 0};
          if (key < L.seq_kv && c8 < dim)
            v = *(const i32x4 *)(src + (int64_t)key * pitch + c8);
          *(i32x4 *)&dst[j][c8] = v;
        }
      } else {
        for (int e = t; e < kGenKeys * MAXD; e += kGenThreads) {
          const int j = e / MAXD, d = e % MAXD;
          const int key = kb0 + j;
          dst[j][d] = key < L.seq_kv && d < dim
                          ? src[(int64_t)key * pitch + d]
                          : (f16)0;
        }
      }
    };

    // Keys this workgroup's rows may see.
    const int last_row = min(row0 + kGenRows, L.seq_q) - 1;
    const int kv_end = L.causal ? min(L.seq_kv, last_row + 1) : L.seq_kv;
    for (int kb0 = 0; kb0 < kv_end; kb0 += kGenKeys) {
      __syncthreads();  // the previous block's K, V and mask are no longer read
      fill(ks, kp, L.k[2], L.dqk, L.vec_k, kb0);
      fill(vs, vp, L.v[2], L.dv, L.vec_v, kb0);
      if (mbase) {
        for (int e = t; e < kGenRows * kGenKeys; e += kGenThreads) {
          const int rr = e / kGenKeys, j = e % kGenKeys;
          const int row = row0 + rr, key = kb0 + j;
          ms[rr][j] = row < L.seq_q && key < L.seq_kv
                          ? mbase[(int64_t)row * L.mask[2] +
                                  (int64_t)key * L.mask[3]]
                          : (f16)0;
        }
      }
      __syncthreads();
      float s[kGenKeys];
      float blk_max = -INFINITY;
#pragma unroll
      for (int j = 0; j < kGenKeys; ++j) {
        float part = 0.0f;
#pragma unroll
        for (int c = 0; c < QP; ++c)
          part = __builtin_amdgcn_fdot2(
              q2[c], *(const f16x2 *)&ks[j][d0 + 2 * c], part, false);
        const float dot = quad_sum(part);
        const int key = kb0 + j;
        const bool valid = key < L.seq_kv && (!L.causal || key <= ic);
        float v = dot * L.scale;
        if (mbase)
          v += (float)ms[r][j];
        s[j] = valid ? v : -INFINITY;
        blk_max = fmaxf(blk_max, s[j]);
      }
      const float m_new = fmaxf(m_run, blk_max);
      if (m_new == -INFINITY)
        continue;  // every key so far masked: nothing to accumulate
      const float alpha = m_run == -INFINITY ? 0.0f : __expf(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int c = 0; c < QC; ++c)
        acc[c] *= alpha;
#pragma unroll
      for (int j = 0; j < kGenKeys; ++j) {
        const float p = s[j] == -INFINITY ? 0.0f : __expf(s[j] - m_new);
        l_run += p;
#pragma unroll
        for (int c = 0; c < QC; ++c)
          acc[c] = __builtin_fmaf((float)vs[j][d0 + c], p, acc[c]);
      }
      m_run = m_new;
    }
    if (row_ok) {
      const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
      OutT *op = O + b * L.o[0] + h * L.o[1] + (int64_t)i * L.o[2];
#pragma unroll
      for (int c = 0; c < QC; ++c)
        if (d0 + c < L.dv)
          store_o(op + d0 + c, acc[c] * inv);
    }
  }
}

namespace {

template <typename OutT>
hipError_t launch_general_t(const void *q, const void *k, const void *v,
                            void *o, const void *mask, int64_t batch,
                            const AttentionGeneralLayout &l, void *stream) {
  const int d = l.dqk > l.dv ? l.dqk : l.dv;
  const int nb = (l.seq_q + kGenRows - 1) / kGenRows;
  dim3 grid((unsigned)(l.causal ? (nb + 1) / 2 : nb), (unsigned)l.heads,
            (unsigned)batch);
  const f16 *qp = (const f16 *)q, *kp = (const f16 *)k, *vp = (const f16 *)v,
            *mp = (const f16 *)mask;
  OutT *op = (OutT *)o;
  auto run = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, grid, dim3(kGenThreads), 0,
                       (hipStream_t)stream, qp, kp, vp, op, mp, l);
    return hipGetLastError();
  };
  if (d <= 16)
    return run(attention_general_kernel<16, OutT>);
  if (d <= 32)
    return run(attention_general_kernel<32, OutT>);
  if (d <= 64)
    return run(attention_general_kernel<64, OutT>);
  if (d <= 128)
    return run(attention_general_kernel<128, OutT>);
  if (d <= 256)
    return run(attention_general_kernel<256, OutT>);
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_attention_general(const void *q, const void *k,
                                    const void *v, void *o, const void *mask,
                                    int64_t batch,
                                    const AttentionGeneralLayout &layout,
                                    int out_f32, void *stream) {
  return out_f32 ? launch_general_t<float>(q, k, v, o, mask, batch, layout,
                                           stream)
                 : launch_general_t<f16>(q, k, v, o, mask, batch, layout,
                                         stream);
}

const KernelEntry *attention_general_kernels(int *count) {
  static const KernelEntry all[] = {
      {"attention_general_d16", (const void *)&attention_general_kernel<16, f16>, kGenThreads, kExportAttention},
      {"attention_general_d32", (const void *)&attention_general_kernel<32, f16>, kGenThreads, kExportAttention},
      {"attention_general_d64", (const void *)&attention_general_kernel<64, f16>, kGenThreads, kExportAttention},
      {"attention_general_d128", (const void *)&attention_general_kernel<128, f16>, kGenThreads, kExportAttention},
      {"attention_general_d256", (const void *)&attention_general_kernel<256, f16>, kGenThreads, kExportAttention},
      {"attention_general_d16_f32", (const void *)&attention_general_kernel<16, float>, kGenThreads, kExportAttention},
      {"attention_general_d32_f32", (const void *)&attention_general_kernel<32, float>, kGenThreads, kExportAttention},
      {"attention_general_d64_f32", (const void *)&attention_general_kernel<64, float>, kGenThreads, kExportAttention},
      {"attention_general_d128_f32", (const void *)&attention_general_kernel<128, float>, kGenThreads, kExportAttention},
      {"attention_general_d256_f32", (const void *)&attention_general_kernel<256, float>, kGenThreads, kExportAttention},
  };
  *count = (int)(sizeof(all) / sizeof(all[0]));
  return all;
}

}  // namespace ihp
