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
//  * a workgroup owns 64 query rows of one (batch, head); four lanes share a
//    row, each holding a quarter of its Q slice and of its O accumulator in
//    registers;
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

__device__ __forceinline__ void store_o(f16 *p, float v) { *p = (f16)v; }
__device__ __forceinline__ void store_o(float *p, float v) { *p = v; }

}  // namespace

// MAXD: the head-dim bucket (a power of two >= both head dims); each of a
// row's four lanes holds MAXD / 4 elements of Q and of the O accumulator.
template <int MAXD, typename OutT>
__global__ __launch_bounds__(kGenThreads) void attention_general_kernel(
    const f16 *__restrict__ Q, const f16 *__restrict__ K,
    const f16 *__restrict__ V, OutT *__restrict__ O,
    const f16 *__restrict__ Mask, AttentionGeneralLayout L) {
  constexpr int QC = MAXD / 4;
  constexpr int PAD = 8;  // keeps the four quarters of a row off one bank
  __shared__ f16 ks[kGenKeys][MAXD + PAD];
  __shared__ f16 vs[kGenKeys][MAXD + PAD];

  const int t = threadIdx.x;
  const int r = t >> 2, qd = t & 3;
  const int64_t b = blockIdx.z, h = blockIdx.y, hk = h / L.group;
  const int row0 = blockIdx.x * kGenRows;
  const int i = row0 + r;
  const bool row_ok = i < L.seq_q;
  const int ic = row_ok ? i : L.seq_q - 1;
  const f16 *qp = Q + b * L.q[0] + h * L.q[1] + (int64_t)ic * L.q[2];
  const f16 *kp = K + b * L.k[0] + hk * L.k[1];
  const f16 *vp = V + b * L.v[0] + hk * L.v[1];
  const f16 *mp = Mask ? Mask + b * L.mask[0] + h * L.mask[1] +
                             (int64_t)ic * L.mask[2]
                       : nullptr;
  const int d0 = qd * QC;

  float q[QC], acc[QC];
#pragma unroll
  for (int c = 0; c < QC; ++c) {
    q[c] = d0 + c < L.dqk ? (float)qp[d0 + c] : 0.0f;
    acc[c] = 0.0f;
  }
  float m_run = -INFINITY, l_run = 0.0f;

  // Keys this workgroup's rows may see.
  const int last_row = min(row0 + kGenRows, L.seq_q) - 1;
  const int kv_end = L.causal ? min(L.seq_kv, last_row + 1) : L.seq_kv;
  for (int kb0 = 0; kb0 < kv_end; kb0 += kGenKeys) {
    __syncthreads();  // the previous block's K and V are no longer read
    for (int e = t; e < kGenKeys * MAXD; e += kGenThreads) {
      const int j = e / MAXD, d = e % MAXD;
      const int key = kb0 + j;
      const bool in = key < L.seq_kv;
      ks[j][d] = in && d < L.dqk ? kp[(int64_t)key * L.k[2] + d] : (f16)0;
      vs[j][d] = in && d < L.dv ? vp[(int64_t)key * L.v[2] + d] : (f16)0;
    }
    __syncthreads();
    float s[kGenKeys];
    float blk_max = -INFINITY;
#pragma unroll
    for (int j = 0; j < kGenKeys; ++j) {
      float part = 0.0f;
#pragma unroll
      for (int c = 0; c < QC; ++c)
        part += q[c] * (float)ks[j][d0 + c];
      const float dot = quad_sum(part);
      const int key = kb0 + j;
      const bool valid = key < L.seq_kv && (!L.causal || key <= ic);
      float v = dot * L.scale;
      if (mp && valid)
        v += (float)mp[(int64_t)key * L.mask[3]];
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
        acc[c] += p * (float)vs[j][d0 + c];
    }
    m_run = m_new;
  }
  if (!row_ok)
    return;
  const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
  OutT *op = O + b * L.o[0] + h * L.o[1] + (int64_t)i * L.o[2];
#pragma unroll
  for (int c = 0; c < QC; ++c)
    if (d0 + c < L.dv)
      store_o(op + d0 + c, acc[c] * inv);
}

namespace {

template <typename OutT>
hipError_t launch_general_t(const void *q, const void *k, const void *v,
                            void *o, const void *mask, int64_t batch,
                            const AttentionGeneralLayout &l, void *stream) {
  const int d = l.dqk > l.dv ? l.dqk : l.dv;
  dim3 grid((unsigned)((l.seq_q + kGenRows - 1) / kGenRows),
            (unsigned)l.heads, (unsigned)batch);
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
