// Fused causal attention forward (f16 in/out, f32 scores and softmax).
//
// The reference has no fused attention kernel: SDPA is imported in its math
// form and lowered as batch_matmul + softmax generics
// (examples/attention_layer/attention_layer.mlir:48-105), or, for
// iree_linalg_ext.attention, decomposed into an online-softmax loop over KV
// tiles (CG/Pipelines/LoweringPipelines.cpp:561-595). This kernel is that
// online-softmax loop on MFMA:
//  * a workgroup owns a 128-row query block of one (batch, head); each of its
//    4 waves owns 32 query rows held in registers for the whole loop;
//  * per 64-key block: S^T = K Q^T on v_mfma_f32_32x32x16_f16, laid out so a
//    lane holds all scores of one query row (the row max and row sum need one
//    cross-lane exchange, lane ^ 32);
//  * online softmax in f32 (exp2 with the scale folded in), running max and
//    sum per row, output rescaled in registers;
//  * O^T += V^T P^T on MFMA with P taken straight from the score registers
//    (rounded to f16) and V^T staged in LDS;
//  * causal blocks above the diagonal are skipped, the diagonal blocks are
//    masked, and query blocks are scheduled heaviest first.
#include "device_common.h"
#include "kernels_internal.h"

namespace ihp {

namespace {
constexpr int kBQ = 128;   // query rows per workgroup
constexpr int kBKV = 64;   // keys per block
constexpr int kVtPad = 4;  // halves of padding per V^T row (bank spread)
}  // namespace

template <int D>
__global__ __launch_bounds__(256, 2) void attention_fwd_kernel(
    const f16 *__restrict__ Q, const f16 *__restrict__ K,
    const f16 *__restrict__ V, f16 *__restrict__ O, int heads, int seq_q,
    int seq_kv, float scale_log2, int causal) {
  constexpr int DS = D / 16;         // 16-wide d steps of S^T = K Q^T
  constexpr int DT = D / 32;         // 32-row d tiles of O^T
  constexpr int KROW = D * 2;        // bytes per staged K row
  constexpr int KCH = KROW / 16;     // 16-byte chunks per K row
  constexpr int VT_ROW = kBKV + kVtPad;  // halves per V^T row
  __shared__ __attribute__((aligned(16))) char Ks[kBKV * KROW];
  __shared__ __attribute__((aligned(16))) f16 Vt[D * VT_ROW];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int q_blocks = (seq_q + kBQ - 1) / kBQ;
  // Heaviest (last) query blocks first under a causal mask.
  const int qb = q_blocks - 1 - (int)(blockIdx.x / (unsigned)(gridDim.x / q_blocks));
  const int plane = (int)(blockIdx.x % (unsigned)(gridDim.x / q_blocks));
  const int64_t q_off = (int64_t)plane * seq_q * D;
  const int64_t kv_off = (int64_t)plane * seq_kv * D;
  const int q0 = qb * kBQ + wave * 32;  // this wave's first query row
  const int my_q = q0 + l32;

  // Q fragments (B operand of S^T = K Q^T): lane holds query my_q, d chunk
  // 16*s + 8*g .. +7 for every step s.
  i32x4 qf[DS];
#pragma unroll
  for (int s = 0; s < DS; ++s) {
    if (my_q < seq_q)
      qf[s] = *(const i32x4 *)(Q + q_off + (int64_t)my_q * D + 16 * s + 8 * g);
    else
      qf[s] = i32x4{0, 0, 0, 0};
  }

  f32x16 o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r)
      o[t][r] = 0.0f;
  float m_run = -INFINITY, l_run = 0.0f;

  int kv_end = seq_kv;
  if (causal) {
    const int last_q = qb * kBQ + kBQ - 1;
    kv_end = last_q + 1 < seq_kv ? last_q + 1 : seq_kv;
  }
  const int n_blocks = (kv_end + kBKV - 1) / kBKV;

  for (int kb = 0; kb < n_blocks; ++kb) {
    const int kv0 = kb * kBKV;
    __syncthreads();  // previous block's K / V^T reads are done
    // Stage K [64][D] (16-byte chunks XOR-swizzled by row) and V^T [D][64].
    for (int it = tid; it < kBKV * KCH; it += 256) {
      const int key = it / KCH, c = it % KCH;
      i32x4 kv = i32x4{0, 0, 0, 0}, vv = i32x4{0, 0, 0, 0};
      if (kv0 + key < seq_kv) {
        kv = *(const i32x4 *)(K + kv_off + (int64_t)(kv0 + key) * D + 8 * c);
        vv = *(const i32x4 *)(V + kv_off + (int64_t)(kv0 + key) * D + 8 * c);
      }
      *(i32x4 *)(Ks + key * KROW + ((c ^ (key & 7)) * 16)) = kv;
      f16x8 vh = __builtin_bit_cast(f16x8, vv);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        Vt[(8 * c + e) * VT_ROW + key] = vh[e];
    }
    __syncthreads();

    // S^T tiles: keys 32t..32t+31 x this wave's 32 queries.
    f32x16 st[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int r = 0; r < 16; ++r)
        st[t][r] = 0.0f;
      const int key = 32 * t + l32;
#pragma unroll
      for (int s = 0; s < DS; ++s) {
        const int c = 2 * s + g;
        i32x4 kf = *(const i32x4 *)(Ks + key * KROW + ((c ^ (key & 7)) * 16));
        st[t] = Mfma32<f16>::mma(kf, qf[s], st[t]);
      }
    }

    // Mask (causal diagonal, sequence tail), then the online softmax update.
    const bool need_mask = (causal && kv0 + kBKV - 1 > q0) || kv0 + kBKV > seq_kv;
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float s = st[t][r] * scale_log2;
        if (need_mask) {
          const int key = kv0 + 32 * t + 8 * (r >> 2) + 4 * g + (r & 3);
          if (key >= seq_kv || (causal && key > my_q))
            s = -INFINITY;
        }
        st[t][r] = s;
        mx = fmaxf(mx, s);
      }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    // A row with every key masked so far keeps m = -inf; exp2 of a finite
    // offset from it must not produce nan.
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    const float alpha = exp2f(m_run - m_use);
    float psum = 0.0f;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = exp2f(st[t][r] - m_use);
        st[t][r] = p;
        psum += p;
      }
    psum += __shfl_xor(psum, 32);
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        o[t][r] *= alpha;

    // O^T[d][q] += V^T[d][key] P^T[key][q], 16 keys per MFMA.
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        f16x8 pf;
#pragma unroll
        for (int e = 0; e < 8; ++e)
          pf[e] = (f16)st[t][8 * h + e];
        const i32x4 pb = __builtin_bit_cast(i32x4, pf);
        const int kbase = 32 * t + 16 * h + 4 * g;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const f16 *vrow = Vt + (32 * dt + l32) * VT_ROW + kbase;
          const i32x2 lo = *(const i32x2 *)(vrow);
          const i32x2 hi = *(const i32x2 *)(vrow + 8);
          const i32x4 vf = i32x4{lo[0], lo[1], hi[0], hi[1]};
          o[dt] = Mfma32<f16>::mma(vf, pb, o[dt]);
        }
      }
    }
  }

  if (my_q >= seq_q)
    return;
  const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
  f16 *orow = O + q_off + (int64_t)my_q * D;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) {
      f16x4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        v[e] = (f16)(o[dt][4 * rq + e] * inv);
      *(f16x4 *)(orow + 32 * dt + 8 * rq + 4 * g) = v;
    }
  }
}

hipError_t launch_attention(const void *q, const void *k, const void *v,
                            void *o, int64_t batch, int64_t heads,
                            int64_t seq_q, int64_t seq_kv, int64_t head_dim,
                            float scale, int causal, void *stream) {
  const int64_t q_blocks = (seq_q + kBQ - 1) / kBQ;
  const int64_t planes = batch * heads;
  dim3 grid((unsigned)(q_blocks * planes));
  const float scale_log2 = scale * 1.4426950408889634f;  // log2(e)
  if (head_dim == 128)
    hipLaunchKernelGGL((attention_fwd_kernel<128>), grid, dim3(256), 0,
                       (hipStream_t)stream, (const f16 *)q, (const f16 *)k,
                       (const f16 *)v, (f16 *)o, (int)heads, (int)seq_q,
                       (int)seq_kv, scale_log2, causal);
  else if (head_dim == 64)
    hipLaunchKernelGGL((attention_fwd_kernel<64>), grid, dim3(256), 0,
                       (hipStream_t)stream, (const f16 *)q, (const f16 *)k,
                       (const f16 *)v, (f16 *)o, (int)heads, (int)seq_q,
                       (int)seq_kv, scale_log2, causal);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace ihp
