// General attention forward on the matrix cores: any head dims (Q/K and V/O
// may differ, up to 256), an optional additive mask, f16 or f32 output,
// strided operands and grouped KV heads.
//
// The reference lowers iree_linalg_ext.attention whatever its head dims,
// mask or output type, through online attention
// (CG/Pipelines/LoweringPipelines.cpp:561-595; the online_attention of the
// pipeline test test/codegen/pipelines/hexagon_lower_executable_target.mlir:
// 195-233 has a QK head dim of 4, a V head dim of 5, scale 0.5 and an f32
// accumulator). The fused kernel (attention.hip) takes the common shapes at
// full speed; this one takes the rest, with the same semantics:
//  * a workgroup of 4 waves owns 64 query rows of one (batch, head), 16 per
//    wave (under the causal mask two such blocks, x and the mirror one, for
//    an even load); a wave keeps its Q rows as 16x16x32 MFMA fragments
//    (zero past the head dim) and its O rows as f32 accumulators;
//  * 64-key blocks of K (row-major) and V (transposed, so that a lane reads
//    8 consecutive keys of one V column) are staged in LDS, zero past the
//    sequence and the head dims; 16-byte fills where rows allow them;
//  * S = Q K^T on v_mfma_f32_16x16x32_f16; scores are scaled, the mask
//    added, causal and out-of-range keys set to -inf; an online softmax in
//    f32 (row max and sum over a lane's 16-lane group) rescales O block by
//    block; the probabilities, rounded to f16, go through the wave's own LDS
//    tile into the A operand of O += P V;
//  * a row that sees no key (fully masked) writes 0, as the all-masked-row
//    guard of the decomposed softmax does
//    (examples/attention_layer/attention_layer.mlir:80-102).
#include <type_traits>

#include "device_common.h"
#include "kernels_internal.h"

namespace ihp {

namespace {

constexpr int kGenThreads = 256;           // 4 waves
constexpr int kGenRows = 64;               // query rows per workgroup
constexpr int kGenKeys = 64;               // keys per LDS block
constexpr int kGenPad = 8;                 // f16 padding per LDS row

// Max / sum over the 16 lanes of a lane's group (lanes sharing lane / 16,
// one DPP row): the lanes that hold one query row's scores. Four DPP moves,
// no LDS round trip: swap neighbours, swap pairs (each lane then holds its
// quad's result), then combine with the mirrored lane of the half row and
// of the row, which lie in the other quads.
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF,
                                      0xF, false));
}
constexpr int kDppSwap1 = 0xB1;        // quad_perm [1, 0, 3, 2]
constexpr int kDppSwap2 = 0x4E;        // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141;  // row_half_mirror
constexpr int kDppMirror = 0x140;      // row_mirror
__device__ __forceinline__ float group16_max(float x) {
  x = fmaxf(x, dpp<kDppSwap1>(x));
  x = fmaxf(x, dpp<kDppSwap2>(x));
  x = fmaxf(x, dpp<kDppHalfMirror>(x));
  return fmaxf(x, dpp<kDppMirror>(x));
}
__device__ __forceinline__ float group16_sum(float x) {
  x += dpp<kDppSwap1>(x);
  x += dpp<kDppSwap2>(x);
  x += dpp<kDppHalfMirror>(x);
  return x + dpp<kDppMirror>(x);
}

__device__ __forceinline__ void store_o(f16 *p, float v) { *p = (f16)v; }
__device__ __forceinline__ void store_o(float *p, float v) { *p = v; }

}  // namespace

// DP: the head-dim bucket (32, 64, 128 or 256, at least both head dims).
// MFMA operand layout (v_mfma_f32_16x16x32_f16): lane l supplies row l % 16
// and the 8 consecutive k of chunk l / 16; the result holds column l % 16 in
// lane l, row 4 (l / 16) + r in register r. S uses Q as the row operand and
// K as the column operand (k = head dim); O uses P (k = keys) and V^T.
// Per bucket: the 256 bucket runs one wave per SIMD whatever it does, so it
// prefetches the next K / V block into registers and reads each group of V
// fragments before the previous group's MFMAs; the smaller buckets keep
// registers for 2-4 workgroups per CU and read each fragment group just
// before its MFMAs. Measured at 2048 x 2048 (causal and not, 16-32 heads):
// against prefetching in every bucket, the small buckets ran 22-34 % faster
// on long non-causal rows and 30 % faster causal; the 256 bucket gains 6 %
// from its prefetch.
template <int DP>
struct GenTraits {
  static constexpr bool kPrefetch = DP >= 256;
  static constexpr bool kVLookahead = DP >= 256;
  static constexpr int kWgPerCu = DP <= 64 ? 4 : DP <= 128 ? 2 : 1;
};

template <int DP, typename OutT>
__global__ __launch_bounds__(kGenThreads, GenTraits<DP>::kWgPerCu) void
attention_general_kernel(
    const f16 *__restrict__ Q, const f16 *__restrict__ K,
    const f16 *__restrict__ V, OutT *__restrict__ O,
    const f16 *__restrict__ Mask, AttentionGeneralLayout L) {
  constexpr int QS = DP / 32;            // 32-wide head-dim steps of S
  constexpr int DB = DP / 16;            // 16-wide column blocks of O
  constexpr int KR = DP + kGenPad;       // K row in LDS (halves)
  constexpr int VR = kGenKeys + kGenPad; // V^T row (halves)
  constexpr int PR = kGenKeys + kGenPad; // P row (halves)
  constexpr int C8 = DP / 8;             // 16-byte chunks of a head-dim row
  static_assert(DP % 32 == 0, "head-dim bucket");
  __shared__ __attribute__((aligned(16))) f16 ks[kGenKeys * KR];
  __shared__ __attribute__((aligned(16))) f16 vt[DP * VR];
  __shared__ __attribute__((aligned(16))) f16 ps[kGenThreads / 64][16 * PR];
  __shared__ f16 ms[kGenRows][kGenKeys + 2];  // this block's mask values

  constexpr bool PF = GenTraits<DP>::kPrefetch;
  constexpr bool VLA = GenTraits<DP>::kVLookahead;
  constexpr int NK = kGenKeys * C8 / kGenThreads;  // 16-byte chunks a thread
                                                   // stages per K / V block
  static_assert(NK >= 1 && NK * kGenThreads == kGenKeys * C8, "staging");
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int lr = lane & 15, lg = lane >> 4;
  const int nb = (L.seq_q + kGenRows - 1) / kGenRows;
  const int gx = L.causal ? (nb + 1) / 2 : nb;  // workgroups per (batch, head)
  // A 1-D grid is renumbered so that the workgroups of one head run on one
  // XCD (dispatch is round-robin over the 8 XCDs): they read the same K and
  // V, which then stay in that XCD's L2. A grid too large for 1-D is 3-D,
  // (x, head, batch), in dispatch order.
  int x;
  int64_t b, h;
  if (gridDim.y == 1 && gridDim.z == 1) {
    const int64_t wg = blockIdx.x, nwg = gridDim.x;
    const int64_t logical = nwg % 8 == 0 ? (wg % 8) * (nwg / 8) + wg / 8 : wg;
    x = (int)(logical % gx);
    const int64_t hz = logical / gx;
    h = hz % L.heads;
    b = hz / L.heads;
  } else {
    x = blockIdx.x;
    h = blockIdx.y;
    b = blockIdx.z;
  }
  const int64_t hk = h / L.group;
  const f16 *kp = K + b * L.k[0] + hk * L.k[1];
  const f16 *vp = V + b * L.v[0] + hk * L.v[1];
  const f16 *mbase = Mask ? Mask + b * L.mask[0] + h * L.mask[1] : nullptr;
  f16 *pw = ps[wave];
  // Under the causal mask row block x costs x + 1 key blocks: a workgroup
  // takes blocks x and nb - 1 - x (one when they coincide), so every
  // workgroup carries about the same keys; otherwise one block each.
  const int n_items = L.causal && nb - 1 - x != x ? 2 : 1;
  for (int item = 0; item < n_items; ++item) {
    const int row0 = (item == 0 ? x : nb - 1 - x) * kGenRows;
    const int wrow0 = row0 + 16 * wave;  // this wave's first query row

    // Q fragments: row wrow0 + lr, head dims 32 s + 8 lg .. + 7.
    i32x4 qf[QS];
    {
      const int qi = wrow0 + lr;
      const bool q_ok = qi < L.seq_q;
      const f16 *qp = Q + b * L.q[0] + h * L.q[1] +
                      (int64_t)(q_ok ? qi : 0) * L.q[2];
#pragma unroll
      for (int st = 0; st < QS; ++st) {
        f16x8 v;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int d = 32 * st + 8 * lg + e;
          v[e] = q_ok && d < L.dqk ? qp[d] : (f16)0;
        }
        qf[st] = __builtin_bit_cast(i32x4, v);
      }
    }
    f32x4 o[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db)
      o[db] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // Rows 4 lg + r of the wave: running max (shared by the row's 16 lanes)
    // and this lane's share of the row sum.
    float m_run[4], l_run[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      m_run[r] = -INFINITY;
      l_run[r] = 0.0f;
    }

    // Keys this workgroup's rows may see.
    const int last_row = min(row0 + kGenRows, L.seq_q) - 1;
    const int kv_end = L.causal ? min(L.seq_kv, last_row + 1) : L.seq_kv;
    // K and V blocks with 16-byte rows go through registers: with PF the
    // next block is loaded while this one is computed and written to LDS
    // after the barrier. Element-wise K / V (rows not 16-byte aligned) and
    // mask values are staged straight from memory. Zeros past the sequence
    // and head dims.
    i32x4 pk[NK], pv[NK];
    auto prefetch = [&](int kb0) {
      if (L.vec_k) {
#pragma unroll
        for (int i = 0; i < NK; ++i) {
          const int e = t + i * kGenThreads;
          const int j = e / C8, c8 = (e % C8) * 8, key = kb0 + j;
          pk[i] = key < L.seq_kv && c8 < L.dqk
                      ? *(const i32x4 *)(kp + (int64_t)key * L.k[2] + c8)
                      : i32x4{0, 0, 0, 0};
        }
      }
      if (L.vec_v) {
#pragma unroll
        for (int i = 0; i < NK; ++i) {
          const int e = t + i * kGenThreads;
          const int j = e % kGenKeys, c8 = (e / kGenKeys) * 8, key = kb0 + j;
          pv[i] = key < L.seq_kv && c8 < L.dv
                      ? *(const i32x4 *)(vp + (int64_t)key * L.v[2] + c8)
                      : i32x4{0, 0, 0, 0};
        }
      }
    };
    auto stage = [&](int kb0) {
      if constexpr (!PF)
        prefetch(kb0);
      if (L.vec_k) {
#pragma unroll
        for (int i = 0; i < NK; ++i) {
          const int e = t + i * kGenThreads;
          *(i32x4 *)&ks[(e / C8) * KR + (e % C8) * 8] = pk[i];
        }
      } else {
        for (int e = t; e < kGenKeys * DP; e += kGenThreads) {
          const int j = e / DP, d = e % DP, key = kb0 + j;
          ks[j * KR + d] = key < L.seq_kv && d < L.dqk
                               ? kp[(int64_t)key * L.k[2] + d]
                               : (f16)0;
        }
      }
      if (L.vec_v) {
#pragma unroll
        for (int i = 0; i < NK; ++i) {
          const int e = t + i * kGenThreads;
          const int j = e % kGenKeys, c8 = (e / kGenKeys) * 8;
          const f16x8 hv = __builtin_bit_cast(f16x8, pv[i]);
#pragma unroll
          for (int u = 0; u < 8; ++u)
            vt[(c8 + u) * VR + j] = hv[u];
        }
      } else {
        for (int e = t; e < kGenKeys * DP; e += kGenThreads) {
          const int j = e % kGenKeys, d = e / kGenKeys, key = kb0 + j;
          vt[d * VR + j] = key < L.seq_kv && d < L.dv
                               ? vp[(int64_t)key * L.v[2] + d]
                               : (f16)0;
        }
      }
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
    };
    if (PF && kv_end > 0)
      prefetch(0);
    for (int kb0 = 0; kb0 < kv_end; kb0 += kGenKeys) {
      __syncthreads();  // the previous block's K, V, mask and P are read
      stage(kb0);
      __syncthreads();
      if (PF && kb0 + kGenKeys < kv_end)
        prefetch(kb0 + kGenKeys);

      // S for the block's four 16-key groups, each group's K fragments read
      // together before its MFMAs.
      f32x4 s[4];
      i32x4 kf[QS];
      auto read_k = [&](int kg, i32x4 *dst) {
        const f16 *krow = &ks[(16 * kg + lr) * KR + 8 * lg];
#pragma unroll
        for (int st = 0; st < QS; ++st)
          dst[st] = *(const i32x4 *)(krow + 32 * st);
      };
#pragma unroll
      for (int kg = 0; kg < 4; ++kg) {
        read_k(kg, kf);
        s[kg] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int st = 0; st < QS; ++st)
          s[kg] = Mfma16<f16>::mma(qf[st], kf[st], s[kg]);
      }
      // Scale, mask and bounds; this block's row max.
      float mx[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int qrow = wrow0 + 4 * lg + r;
        mx[r] = -INFINITY;
#pragma unroll
        for (int kg = 0; kg < 4; ++kg) {
          const int key = kb0 + 16 * kg + lr;
          const bool valid = key < L.seq_kv && (!L.causal || key <= qrow);
          float v = s[kg][r] * L.scale;
          if (mbase)
            v += (float)ms[16 * wave + 4 * lg + r][16 * kg + lr];
          s[kg][r] = valid ? v : -INFINITY;
          mx[r] = fmaxf(mx[r], s[kg][r]);
        }
        mx[r] = group16_max(mx[r]);
      }
      // Online softmax: rescale, probabilities (rounded to f16 once, the
      // values PV multiplies and the row sum adds) into the wave's P tile.
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float m_new = fmaxf(m_run[r], mx[r]);
        const float alpha =
            m_run[r] == -INFINITY ? 0.0f : __expf(m_run[r] - m_new);
        l_run[r] *= alpha;
#pragma unroll
        for (int db = 0; db < DB; ++db)
          o[db][r] *= alpha;
        m_run[r] = m_new;
#pragma unroll
        for (int kg = 0; kg < 4; ++kg) {
          const float sv = s[kg][r];
          const f16 p = (f16)(sv == -INFINITY ? 0.0f : __expf(sv - m_new));
          l_run[r] += (float)p;
          pw[(4 * lg + r) * PR + 16 * kg + lr] = p;
        }
      }
      // O += P V, 32 keys a step, V^T fragments read in groups of VG (with
      // VLA ahead of the previous group's MFMAs); the wave reads only its
      // own P tile, so its in-order LDS accesses need no barrier.
      constexpr int VG = DB < 4 ? DB : 4;
      constexpr int NG = 2 * DB / VG;  // groups over both key steps
      i32x4 pf[2], vf[2][VG];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
        pf[kt] = *(const i32x4 *)&pw[lr * PR + 32 * kt + 8 * lg];
      auto read_v = [&](int gi, i32x4 *dst) {
        const int kt = gi / (DB / VG), db0 = (gi % (DB / VG)) * VG;
#pragma unroll
        for (int u = 0; u < VG; ++u)
          dst[u] = *(const i32x4 *)&vt[(16 * (db0 + u) + lr) * VR + 32 * kt +
                                       8 * lg];
      };
      if (VLA)
        read_v(0, vf[0]);
#pragma unroll
      for (int gi = 0; gi < NG; ++gi) {
        if (!VLA)
          read_v(gi, vf[gi & 1]);
        else if (gi + 1 < NG)
          read_v(gi + 1, vf[(gi + 1) & 1]);
        const int kt = gi / (DB / VG), db0 = (gi % (DB / VG)) * VG;
#pragma unroll
        for (int u = 0; u < VG; ++u)
          o[db0 + u] = Mfma16<f16>::mma(pf[kt], vf[gi & 1][u], o[db0 + u]);
      }
    }
    // O / l for the wave's rows; columns past the V head dim are padding.
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float l = group16_sum(l_run[r]);
      const float inv = l > 0.0f ? 1.0f / l : 0.0f;
      const int qrow = wrow0 + 4 * lg + r;
      if (qrow < L.seq_q) {
        OutT *op = O + b * L.o[0] + h * L.o[1] + (int64_t)qrow * L.o[2];
#pragma unroll
        for (int db = 0; db < DB; ++db)
          if (16 * db + lr < L.dv)
            store_o(op + 16 * db + lr, o[db][r] * inv);
      }
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
  const int64_t gx = l.causal ? (nb + 1) / 2 : nb;
  const int64_t flat = gx * l.heads * batch;
  // 1-D (renumbered by XCD in the kernel) when it fits, else 3-D.
  const dim3 grid = flat <= 0x7fffffff
                        ? dim3((unsigned)flat, 1, 1)
                        : dim3((unsigned)gx, (unsigned)l.heads,
                               (unsigned)batch);
  const f16 *qp = (const f16 *)q, *kp = (const f16 *)k, *vp = (const f16 *)v,
            *mp = (const f16 *)mask;
  OutT *op = (OutT *)o;
  auto run = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, grid, dim3(kGenThreads), 0,
                       (hipStream_t)stream, qp, kp, vp, op, mp, l);
    return hipGetLastError();
  };
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
      {"attention_general_d32", (const void *)&attention_general_kernel<32, f16>, kGenThreads, kExportAttention},
      {"attention_general_d64", (const void *)&attention_general_kernel<64, f16>, kGenThreads, kExportAttention},
      {"attention_general_d128", (const void *)&attention_general_kernel<128, f16>, kGenThreads, kExportAttention},
      {"attention_general_d256", (const void *)&attention_general_kernel<256, f16>, kGenThreads, kExportAttention},
      {"attention_general_d32_f32", (const void *)&attention_general_kernel<32, float>, kGenThreads, kExportAttention},
      {"attention_general_d64_f32", (const void *)&attention_general_kernel<64, float>, kGenThreads, kExportAttention},
      {"attention_general_d128_f32", (const void *)&attention_general_kernel<128, float>, kGenThreads, kExportAttention},
      {"attention_general_d256_f32", (const void *)&attention_general_kernel<256, float>, kGenThreads, kExportAttention},
  };
  *count = (int)(sizeof(all) / sizeof(all[0]));
  return all;
}

}  // namespace ihp
