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
//    (rounded to f16) and V^T read transposed from key-major LDS
//    (ds_read_b64_tr_b16);
//  * K and V blocks stream HBM -> LDS (global_load_lds) one block ahead of
//    the block being computed;
//  * causal blocks above the diagonal are skipped, the diagonal blocks are
//    masked, and heavy query blocks are interleaved with light ones.
#include <type_traits>

#include "device_common.h"
#include "kernels_internal.h"

namespace ihp {

namespace {
constexpr int kBQ = 128;   // query rows per workgroup
constexpr int kBKV = 64;   // keys per block
constexpr int kThreads = 256;

template <int N, int I = 0, typename F>
__device__ __forceinline__ void static_for(F &&f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>());
    static_for<N, I + 1>(f);
  }
}

// Transposed 8-byte LDS read (ds_read_b64_tr_b16): within each 16-lane
// block, lane i receives element i%4 of the 8-byte loads of lanes
// 4r + i/4, r = 0..3.
__device__ __forceinline__ i32x2 lds_read_tr16(const IHP_LDS char *p) {
  i32x2 v;
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(v)
               : "v"((unsigned)(uintptr_t)p));
  return v;
}
__device__ __forceinline__ void tie2(i32x2 &v) { asm volatile("" : "+v"(v)); }

// ds_read_b64_tr_b16 with an immediate byte offset; the caller waits with
// lgkm_wait<N>() and ties the result before use.
template <int OFF>
__device__ __forceinline__ i32x2 lds_read_tr16_at(const IHP_LDS char *p) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset range");
  i32x2 v;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2"
               : "=v"(v)
               : "v"((unsigned)(uintptr_t)p), "i"(OFF));
  return v;
}

// x[l % 32] op x[l % 32 + 32] in every lane l (the two lane halves hold
// different keys of the same query row). v_permlane32_swap_b32 exchanges
// lanes 32..63 of its first operand with lanes 0..31 of its second: with
// both set to x, one then holds x[0..31] twice and the other x[32..63]
// twice. Issued as asm with both operands tied: the compiler's builtin for
// it maps both results to one register. s_nop 1 covers the VALU-write ->
// permlane-read wait states the compiler inserts before it.
__device__ __forceinline__ void half_swap(float x, float &lo, float &hi) {
  lo = x;
  hi = x;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1"
               : "+v"(lo), "+v"(hi));
}
__device__ __forceinline__ float pair_max(float x) {
  float a, b;
  half_swap(x, a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float pair_sum(float x) {
  float a, b;
  half_swap(x, a, b);
  return a + b;
}
}  // namespace

// K and V blocks are copied HBM -> LDS with global_load_lds into a two-slot
// ring (block kb+1 streams in while block kb is computed). Both are stored
// key-major as in HBM, 16-byte chunks XOR-swizzled on the copy side:
//  * K rows are read by ds_read_b128, 16 lanes = 16 consecutive keys at one
//    chunk: chunk ^ (key & 15) for 256-byte rows (D = 128),
//    chunk ^ ((key >> 1) & 7) for 128-byte rows (D = 64);
//  * V is read transposed (V^T operand) by ds_read_b64_tr_b16, 32 lanes =
//    4 consecutive keys x 32 d: chunk ^ 4 * (key & 3) (D = 128),
//    chunk ^ 4 * ((key >> 1) & 1) (D = 64).
template <int D>
__device__ __forceinline__ int k_swizzle(int key) {
  return D == 128 ? (key & 15) : ((key >> 1) & 7);
}
template <int D>
__device__ __forceinline__ int v_swizzle(int key) {
  return D == 128 ? 4 * (key & 3) : 4 * ((key >> 1) & 1);
}

template <int D>
__global__ __launch_bounds__(kThreads, 2) void attention_fwd_kernel(
    const f16 *__restrict__ Q, const f16 *__restrict__ K,
    const f16 *__restrict__ V, f16 *__restrict__ O, int heads, int seq_q,
    int seq_kv, float scale_log2, int causal) {
  constexpr int DS = D / 16;       // 16-wide d steps of S^T = K Q^T
  constexpr int DT = D / 32;       // 32-row d tiles of O^T
  constexpr int ROW = D * 2;       // bytes per staged K / V row
  constexpr int CH = ROW / 16;     // 16-byte chunks per row
  constexpr int BLK = kBKV * ROW;  // bytes of one staged K (or V) block
  constexpr int ROWS_PER_INSN = 64 / CH;             // rows per wave copy
  constexpr int PASSES = kBKV / (4 * ROWS_PER_INSN);  // per wave, per tensor
  static_assert(PASSES * 4 * ROWS_PER_INSN == kBKV, "copy shape");
  __shared__ __attribute__((aligned(1024))) char smem[2 * 2 * BLK];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, l32 = lane & 31;
  const int q_blocks = (seq_q + kBQ - 1) / kBQ;
  // Heaviest (last) query blocks first under a causal mask.
  // Under a causal mask query block qb costs qb + 1 units. The first half
  // of the grid takes the heavy blocks (heaviest first), the second half the
  // light ones (lightest first), so the two workgroups that share a CU sum to
  // about the same work.
  const int planes = (int)(gridDim.x / (unsigned)q_blocks);
  const int idx = (int)(blockIdx.x / (unsigned)planes);
  const int half = (q_blocks + 1) / 2;
  const int qb = idx < half ? q_blocks - 1 - idx : idx - half;
  const int plane = (int)(blockIdx.x % (unsigned)planes);
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

  int kv_end = seq_kv;
  if (causal) {
    const int last_q = qb * kBQ + kBQ - 1;
    kv_end = last_q + 1 < seq_kv ? last_q + 1 : seq_kv;
  }
  const int n_blocks = (kv_end + kBKV - 1) / kBKV;

  // Copy side: a wave instruction moves ROWS_PER_INSN rows of CH chunks;
  // lane -> (row, physical chunk), fetching the logical chunk that belongs
  // there. Keys past seq_kv are clamped to the last key (masked later).
  const int c_row = lane / CH, c_phys = lane % CH;
  IHP_LDS char *lds = (IHP_LDS char *)smem;
  auto copy_block = [&](int kb, int slot) {
    const int kv0 = kb * kBKV;
    IHP_LDS char *kd = lds + slot * 2 * BLK;
    IHP_LDS char *vd = kd + BLK;
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      const int row = (p * 4 + wave) * ROWS_PER_INSN + c_row;
      int key = kv0 + row;
      key = key < seq_kv ? key : seq_kv - 1;
      const f16 *kr = K + kv_off + (int64_t)key * D;
      const f16 *vr = V + kv_off + (int64_t)key * D;
      global_to_lds_16(kr + 8 * (c_phys ^ k_swizzle<D>(row)),
                       kd + (p * 4 + wave) * ROWS_PER_INSN * ROW);
      global_to_lds_16(vr + 8 * (c_phys ^ v_swizzle<D>(row)),
                       vd + (p * 4 + wave) * ROWS_PER_INSN * ROW);
    }
  };

  // V^T read side: for key step (t, h) lane group g needs keys
  // kstart = 32t + 16h + 4g .. +3 and kstart + 8 .. +11 (the order the S^T
  // registers hold them in). Load lane j = lane % 16 of block b = lane / 16
  // reads row kstart + j/4, d = 32 dt + 16 (b % 2) + 4 (j % 4) .. +3.
  // The swizzle of rows kstart + j/4 (+ 8) depends only on j/4, so each d
  // tile's read address is one per-lane offset; key step (t, h) and the +8
  // row half are immediate offsets.
  const int vj = lane & 15, vb = lane >> 4;
  const int v_row_in = vj >> 2;
  int v_off[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    const int b0 = 64 * dt + 2 * (16 * (vb & 1) + 4 * (vj & 3));
    v_off[dt] = (4 * g + v_row_in) * ROW +
                (((b0 >> 4) ^ v_swizzle<D>(v_row_in)) << 4) + (b0 & 15);
  }

  f32x16 o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r)
      o[t][r] = 0.0f;
  float m_run = -INFINITY, l_run = 0.0f;

  if (n_blocks > 0)
    copy_block(0, 0);
  for (int kb = 0; kb < n_blocks; ++kb) {
    const int kv0 = kb * kBKV;
    const int slot = kb & 1;
    // Block kb has landed for every wave, and every wave is done with block
    // kb-1, whose slot now receives block kb+1 while kb is computed.
    wait_vmcnt<0>();
    block_barrier();
    if (kb + 1 < n_blocks)
      copy_block(kb + 1, slot ^ 1);
    const IHP_LDS char *ks = lds + slot * 2 * BLK;
    const IHP_LDS char *vs = ks + BLK;

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
        const i32x4 kf =
            *(const IHP_LDS i32x4 *)(ks + key * ROW + ((c ^ k_swizzle<D>(key)) * 16));
        st[t] = Mfma32<f16>::mma(kf, qf[s], st[t]);
      }
    }

    // Mask (causal diagonal, sequence tail), then the online softmax update
    // in the log2 domain: p = 2^(s * scale_log2 - m). Off the diagonal the
    // row max is taken on the raw scores (scale_log2 > 0 keeps the order) and
    // the scale is fused into the exponent's FMA.
    const bool need_mask =
        (causal && kv0 + kBKV - 1 > q0) || kv0 + kBKV > seq_kv;
    float mx;
    float sc = scale_log2;  // multiplier applied inside the exponent
    if (need_mask || scale_log2 <= 0.0f) {
      mx = -INFINITY;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float s = st[t][r] * scale_log2;
          const int key = kv0 + 32 * t + 8 * (r >> 2) + 4 * g + (r & 3);
          if (key >= seq_kv || (causal && key > my_q))
            s = -INFINITY;
          st[t][r] = s;
          mx = fmaxf(mx, s);
        }
      }
      sc = 1.0f;
    } else {
      mx = -INFINITY;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          mx = fmaxf(mx, st[t][r]);
      mx *= scale_log2;
    }
    mx = pair_max(mx);
    const float m_new = fmaxf(m_run, mx);
    // A row with every key masked so far keeps m = -inf; exp2 of a finite
    // offset from it must not produce nan.
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    float psum = 0.0f;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(st[t][r], sc, -m_use));
        st[t][r] = p;
        psum += p;
      }
    psum = pair_sum(psum);
    l_run = l_run * alpha + psum;
    m_run = m_new;
    // rescale the running output only when some row's max moved
    if (!__all(alpha == 1.0f)) {
#pragma unroll
      for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          o[t][r] *= alpha;
    }

    // O^T[d][q] += V^T[d][key] P^T[key][q], 16 keys per MFMA; the V^T
    // reads of key step i+1 are in flight during the MFMAs of step i.
    i32x2 vr[2][DT][2];
    auto read_v = [&](auto step, i32x2 (&dst)[DT][2]) {
      constexpr int ST = decltype(step)::value;  // (t, h) = (ST / 2, ST % 2)
      constexpr int KOFF = 16 * ST * ROW;
      static_for<DT>([&](auto dt) {
        constexpr int DTI = decltype(dt)::value;
        dst[DTI][0] = lds_read_tr16_at<KOFF>(vs + v_off[DTI]);
        dst[DTI][1] = lds_read_tr16_at<KOFF + 8 * ROW>(vs + v_off[DTI]);
      });
    };
    read_v(std::integral_constant<int, 0>(), vr[0]);
    static_for<4>([&](auto step) {
      constexpr int ST = decltype(step)::value;
      constexpr int CUR = ST & 1;
      if constexpr (ST + 1 < 4) {
        read_v(std::integral_constant<int, ST + 1>(), vr[CUR ^ 1]);
        lgkm_wait<2 * DT>();
      } else {
        lgkm_wait<0>();
      }
      f16x8 pf;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        pf[e] = (f16)st[ST >> 1][8 * (ST & 1) + e];
      const i32x4 pb = __builtin_bit_cast(i32x4, pf);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        tie2(vr[CUR][dt][0]);
        tie2(vr[CUR][dt][1]);
        const i32x4 vf = i32x4{vr[CUR][dt][0][0], vr[CUR][dt][0][1],
                               vr[CUR][dt][1][0], vr[CUR][dt][1][1]};
        o[dt] = Mfma32<f16>::mma(vf, pb, o[dt]);
      }
    });
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
    hipLaunchKernelGGL((attention_fwd_kernel<128>), grid, dim3(kThreads), 0,
                       (hipStream_t)stream, (const f16 *)q, (const f16 *)k,
                       (const f16 *)v, (f16 *)o, (int)heads, (int)seq_q,
                       (int)seq_kv, scale_log2, causal);
  else if (head_dim == 64)
    hipLaunchKernelGGL((attention_fwd_kernel<64>), grid, dim3(kThreads), 0,
                       (hipStream_t)stream, (const f16 *)q, (const f16 *)k,
                       (const f16 *)v, (f16 *)o, (int)heads, (int)seq_q,
                       (int)seq_kv, scale_log2, causal);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace ihp

namespace ihp {

const KernelEntry *attention_kernels(int *count) {
  static const KernelEntry all[] = {
      {"attention_fwd_d128", (const void *)&attention_fwd_kernel<128>, kThreads, kExportAttention},
      {"attention_fwd_d64", (const void *)&attention_fwd_kernel<64>, kThreads, kExportAttention},
  };
  *count = (int)(sizeof(all) / sizeof(all[0]));
  return all;
}

}  // namespace ihp
