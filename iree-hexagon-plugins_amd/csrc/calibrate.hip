// Calibration kernels for bench.py: the ceilings the dispatch kernels are
// read against on the box that runs them. Built into a library of its own
// (lib/libiree_mi355x_calibrate.so), loaded only by the benchmark; nothing in
// the dispatch path calls it.
//
//  * stream_read: a pure HBM read of one buffer (16-byte non-temporal loads,
//    eight in flight per lane), the most a kernel that only streams its
//    operand once can reach. The GEMV streams the same bytes plus x and y.
//  * mfma_loop: MFMAs on operands held in registers, no memory traffic in
//    the loop, four independent accumulator chains per wave and two waves
//    per SIMD, so the issue rate is the MFMA pipe's at whatever clock the
//    operand data lets the chip hold. Random operands toggle more bits than
//    constant ones; that difference is the power ceiling the GEMMs meet.
//    The 32x32 and 16x16 shapes are both measured: they draw different
//    power per product.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "device_common.h"

namespace ihp {
namespace {

__global__ __launch_bounds__(512) void stream_read_kernel(
    const i32x4 *__restrict__ p, int64_t n16, uint32_t *__restrict__ sink) {
  constexpr int kUnroll = 8;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint32_t acc = 0;
  for (; i + (kUnroll - 1) * stride < n16; i += kUnroll * stride) {
    i32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      v[u] = __builtin_nontemporal_load(p + i + u * stride);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      acc ^= (uint32_t)(v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3]);
  }
  for (; i < n16; i += stride) {
    const i32x4 v = __builtin_nontemporal_load(p + i);
    acc ^= (uint32_t)(v[0] ^ v[1] ^ v[2] ^ v[3]);
  }
  // One store per workgroup keeps the loads live; it is 4 bytes against
  // the megabytes read.
  acc = __builtin_amdgcn_readfirstlane(acc);
  if (threadIdx.x == 0)
    sink[blockIdx.x] = acc;
}

// `iters` rounds of 4 independent MFMAs per wave on operands loaded once
// from `src` (64 lanes x 4 operands x 16 bytes per wave); MF is the 32x32
// or the 16x16 MFMA family (the same operand bytes per lane, half the
// products per instruction for 16x16).
template <typename MF>
__global__ __launch_bounds__(512) void mfma_loop_kernel(
    const i32x4 *__restrict__ src, int iters, int32_t *__restrict__ sink) {
  typedef typename MF::Acc Acc;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const i32x4 *w = src + ((int64_t)(blockIdx.x * 8 + wave) % 64) * 256;
  i32x4 a0 = w[lane], a1 = w[64 + lane], b0 = w[128 + lane],
        b1 = w[192 + lane];
  Acc c0 = {}, c1 = {}, c2 = {}, c3 = {};
  for (int it = 0; it < iters; ++it) {
    c0 = MF::mma(a0, b0, c0);
    c1 = MF::mma(a1, b0, c1);
    c2 = MF::mma(a0, b1, c2);
    c3 = MF::mma(a1, b1, c3);
  }
  // The bits of every result, folded, keep the chains live. Elements are
  // copied to scalars first: hipcc folded a bit cast taken directly of a
  // vector element to zero and dropped the whole loop.
  uint32_t s = 0;
#pragma unroll
  for (int r = 0; r < (int)(sizeof(Acc) / 4); ++r) {
    const typename MF::AccScalar e0 = c0[r], e1 = c1[r], e2 = c2[r],
                                 e3 = c3[r];
    s ^= __builtin_bit_cast(uint32_t, e0) ^ __builtin_bit_cast(uint32_t, e1) ^
         __builtin_bit_cast(uint32_t, e2) ^ __builtin_bit_cast(uint32_t, e3);
  }
  sink[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = (int32_t)s;
}

}  // namespace
}  // namespace ihp

using namespace ihp;

extern "C" {

// Pure read of `bytes` (a multiple of 16) from `src`; `sink` holds one u32
// per workgroup (`workgroups` of 512 threads).
int iree_mi355x_calibrate_stream_read(const void *src, int64_t bytes,
                                      void *sink, int workgroups,
                                      void *stream) {
  if (!src || !sink || bytes <= 0 || bytes % 16 || workgroups <= 0)
    return 1;
  hipLaunchKernelGGL(stream_read_kernel, dim3(workgroups), dim3(512), 0,
                     (hipStream_t)stream, (const i32x4 *)src, bytes / 16,
                     (uint32_t *)sink);
  return hipGetLastError() == hipSuccess ? 0 : 4;
}

// MFMA loop: `workgroups` x 8 waves, `iters` rounds of 4 MFMAs each;
// kind 0: v_mfma_i32_32x32x32_i8, 1: v_mfma_f32_32x32x16_f16,
// 2: v_mfma_i32_16x16x64_i8, 3: v_mfma_f32_16x16x32_f16. `src` holds
// 64 x 256 x 16 bytes of operands, `sink` workgroups x 512 x 4 bytes.
int iree_mi355x_calibrate_mfma_loop(int kind, const void *src, int iters,
                                    void *sink, int workgroups,
                                    void *stream) {
  if (!src || !sink || iters <= 0 || workgroups <= 0 || kind < 0 || kind > 3)
    return 1;
  const dim3 grid(workgroups), block(512);
  const hipStream_t s = (hipStream_t)stream;
  const i32x4 *in = (const i32x4 *)src;
  int32_t *out = (int32_t *)sink;
  switch (kind) {
    case 0:
      hipLaunchKernelGGL(mfma_loop_kernel<Mfma32<int8_t>>, grid, block, 0, s,
                         in, iters, out);
      break;
    case 1:
      hipLaunchKernelGGL(mfma_loop_kernel<Mfma32<f16>>, grid, block, 0, s, in,
                         iters, out);
      break;
    case 2:
      hipLaunchKernelGGL(mfma_loop_kernel<Mfma16<int8_t>>, grid, block, 0, s,
                         in, iters, out);
      break;
    default:
      hipLaunchKernelGGL(mfma_loop_kernel<Mfma16<f16>>, grid, block, 0, s, in,
                         iters, out);
  }
  return hipGetLastError() == hipSuccess ? 0 : 4;
}

}  // extern "C"
