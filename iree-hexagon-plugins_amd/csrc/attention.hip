// Fused causal attention forward (f16 in/out, f32 scores and softmax).
//
// The reference has no fused attention kernel: SDPA is imported in its math
// form and lowered as batch_matmul + softmax generics
// (examples/attention_layer/attention_layer.mlir:48-105), or, for
// iree_linalg_ext.attention, decomposed into an online-softmax loop over KV
// tiles (CG/Pipelines/LoweringPipelines.cpp:561-595). This kernel is that
// online-softmax loop on MFMA:
//  * a workgroup owns a 128-row query block of one (batch, head) and fills a
//    CU: two groups of 4 waves take alternate 64-key blocks, each wave
//    owning 32 query rows held in registers for the whole loop, and merge
//    their partial (O, max, sum) through LDS at the end;
//  * per 64-key block: S^T = K Q^T on v_mfma_f32_32x32x16_f16, laid out so a
//    lane holds all scores of one query row (the row max and row sum need one
//    cross-lane exchange, lane ^ 32);
//  * online softmax in f32 (exp2 with the scale folded in), running max and
//    sum per row, output rescaled in registers;
//  * O^T += V^T P^T on MFMA with P taken straight from the score registers
//    (rounded to f16) and V^T read transposed from key-major LDS
//    (ds_read_b64_tr_b16);
//  * K and V blocks stream HBM -> LDS (global_load_lds) into per-group
//    rings;
//  * each wave alternates an M phase (PV of one block and S^T of the next:
//    MFMA and LDS reads only) and a V phase (that block's softmax: VALU),
//    one phase per workgroup barrier; group 1 runs one phase behind group 0,
//    and wave w (group 0) shares its SIMD with wave w + 4 (group 1), so one
//    wave of each SIMD feeds the matrix core while the other works on the
//    VALU;
//  * causal blocks above the diagonal are skipped, the diagonal blocks are
//    masked, and the grid runs the heaviest query blocks first.
#include <type_traits>

#include "device_common.h"
#include "kernels_internal.h"

namespace ihp {

namespace {
constexpr int kBQ = 128;   // query rows per workgroup
constexpr int kBKV = 64;   // keys per block
constexpr int kGroups = 2;  // wave groups, each taking every other key block
constexpr int kThreads = 256 * kGroups;
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
// Lazy running max: tolerated growth of a row's max (log2 units) before the
// reference max moves and the output is rescaled.
constexpr float kLazyMax = 8.0f;
// K fragment reads in flight ahead of the S^T MFMA that takes them.
constexpr int kKReadAhead = 3;

template <int N, int I = 0, typename F>
__device__ __forceinline__ void static_for(F &&f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>());
    static_for<N, I + 1>(f);
  }
}

__device__ __forceinline__ void tie2(i32x2 &v) { asm volatile("" : "+v"(v)); }

// Transposed 8-byte LDS read (ds_read_b64_tr_b16) with an immediate byte
// offset: within each 16-lane block, lane i receives element i%4 of the
// 8-byte loads of lanes 4r + i/4, r = 0..3. The caller waits with
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

// K and V blocks are copied HBM -> LDS with global_load_lds into two-slot
// rings (a block streams in while the one before is computed). Both are stored
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

// CONTIG: every operand is contiguous [B, H, S, D] with one KV head per
// query head (the layout's strides are then not read): rows are one
// compile-time row size apart and a plane's base is its index times its
// size, so the copies add no scalar arithmetic.
// MASK: an additive f16 mask M (strided instances only), read through the
// layout's (batch, head, row) strides with keys contiguous, scaled by log2(e)
// and added to the log2-domain scores of every block.
// DV: the head dim when it is a multiple of 16 below D (the LDS layout's):
// copies skip the chunks past it (those LDS bytes are never read as K or Q:
// S^T takes DV / 16 d steps), PV runs over all D / 32 tiles of O^T and the
// rows past DV it produces from the unwritten V chunks are not stored.
// OF32: O is f32 (strided instances only), stored from the merged
// registers, 16 bytes (4 d of one row) per lane and register quarter.
template <int D, bool CONTIG, bool MASK = false, int DV = D, bool OF32 = false>
__global__ __launch_bounds__(kThreads, 1) void attention_fwd_kernel(
    const f16 *__restrict__ Q, const f16 *__restrict__ K,
    const f16 *__restrict__ V, void *__restrict__ O, const f16 *__restrict__ M,
    AttentionLayout L, float scale_log2, int causal) {
  typedef typename std::conditional<OF32, float, f16>::type OutT;
  static_assert(!(CONTIG && (MASK || OF32)),
                "masks and f32 outputs take the strided instance");
  static_assert(DV % 16 == 0 && DV > 0 && DV <= D && (DV == D || !CONTIG),
                "head dim");
  const int heads = L.heads, seq_q = L.seq_q, seq_kv = L.seq_kv;
  constexpr int DS = D / 16;       // 16-wide d steps of S^T = K Q^T
  constexpr int DT = D / 32;       // 32-row d tiles of O^T
  constexpr int DSV = DV / 16;     // d steps of S^T over the head dim
  constexpr int CHV = DV / 8;      // 16-byte chunks of a row within it
  constexpr int ROW = D * 2;       // bytes per staged K / V row
  constexpr int CH = ROW / 16;     // 16-byte chunks per row
  constexpr int BLK = kBKV * ROW;  // bytes of one staged K (or V) block
  constexpr int ROWS_PER_INSN = 64 / CH;             // rows per wave copy
  constexpr int PASSES = kBKV / (4 * ROWS_PER_INSN);  // per wave, per tensor
  static_assert(PASSES * 4 * ROWS_PER_INSN == kBKV, "copy shape");
  // Per wave group: K ring (slots 0, 1) then V ring (slots 0, 1). After both
  // groups' rings: the (max, sum) pairs of the merge, one per (group, wave,
  // lane).
  // Slot 1 of the rings also stages, between key loops, the query block's
  // rows (Q in the V slots, rows 0-63 in group 0's, 64-127 in group 1's),
  // the merge's O hand-over, and the block's output rows (the K slots).
  constexpr int RING = 4 * BLK;
  constexpr int XML = kGroups * 4 * 64 * 8;
  __shared__ __attribute__((aligned(1024))) char smem[kGroups * RING + XML];
  // The merge hands half of a wave's O each way (DT / 2 tiles of 16 floats
  // per lane); both halves of a wave pair fill one ring slot.
  static_assert(DT * 4 * 64 * 16 == BLK, "a wave's O fills one ring slot");
  static_assert(DT % 2 == 0, "O tiles split between the groups");

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Group grp (waves 4 grp .. 4 grp + 3) takes key blocks grp, grp + 2, ...
  // of the same 128 query rows; wave wq of each group owns rows 32 wq ..
  const int grp = wave >> 2, wq = wave & 3;
  const int g = lane >> 5, l32 = lane & 31;
  const int q_blocks = (seq_q + kBQ - 1) / kBQ;
  // A workgroup fills a CU (its LDS) and takes query blocks
  // q_blocks - 1 - pair and pair of one plane, in that order (one block when
  // they coincide). Under a causal mask block qb costs qb + 1 units, so every
  // pair costs q_blocks + 1. Consecutive workgroups take consecutive planes:
  // with a multiple of 8 planes a plane's pairs share an XCD (and its L2).
  const int pairs = (q_blocks + 1) >> 1;
  const int planes = (int)(gridDim.x / (unsigned)pairs);
  const int pair = (int)(blockIdx.x / (unsigned)planes);
  const int plane = (int)(blockIdx.x % (unsigned)planes);
  const int n_items = q_blocks - 1 - pair == pair ? 1 : 2;
  // The plane's (batch, query head) and the KV head it reads; its rows of
  // Q, K, V and O start at these bases, one row pitch (bytes) apart.
  const char *Qp, *Kp, *Vp;
  OutT *Op;
  const f16 *Mp = nullptr;
  uint32_t q_pitch, k_pitch, v_pitch;
  int64_t o_row;
  if constexpr (CONTIG) {
    Qp = (const char *)(Q + (int64_t)plane * seq_q * D);
    Kp = (const char *)(K + (int64_t)plane * seq_kv * D);
    Vp = (const char *)(V + (int64_t)plane * seq_kv * D);
    Op = (OutT *)O + (int64_t)plane * seq_q * D;
    q_pitch = k_pitch = v_pitch = ROW;
    o_row = D;
  } else {
    const int pb = plane / heads, ph = plane - pb * heads, pk = ph / L.group;
    Qp = (const char *)(Q + pb * L.q[0] + ph * L.q[1]);
    Kp = (const char *)(K + pb * L.k[0] + pk * L.k[1]);
    Vp = (const char *)(V + pb * L.v[0] + pk * L.v[1]);
    Op = (OutT *)O + pb * L.o[0] + ph * L.o[1];
    if constexpr (MASK)
      Mp = M + pb * L.m[0] + ph * L.m[1];
    q_pitch = (uint32_t)(2 * L.q[2]);
    k_pitch = (uint32_t)(2 * L.k[2]);
    v_pitch = (uint32_t)(2 * L.v[2]);
    o_row = L.o[2];
  }

  // Per query block: this wave's first row, this group's key blocks (local
  // block i is key block 2 i + grp) and the barrier slots of the block's
  // phase schedule. A group with n blocks runs 2 n + 1 phases (M, V, M, ...,
  // M) and group 1 starts one slot after group 0, so the schedule takes
  // 2 n0 + 1 slots, one more when group 1 has as many blocks as group 0.
  int q0 = 0, n_mine = 0, n_slots = 0;
  auto setup = [&](int item) {
    const int qb = item == 0 ? q_blocks - 1 - pair : pair;
    q0 = qb * kBQ + wq * 32;
    const int kv_end = causal ? min(qb * kBQ + kBQ, seq_kv) : seq_kv;
    const int n_blocks = (kv_end + kBKV - 1) / kBKV;
    n_mine = (n_blocks - grp + 1) >> 1;
    const int n0 = (n_blocks + 1) >> 1, n1 = n_blocks >> 1;
    n_slots = 2 * n0 + 1 + (n1 == n0 ? 1 : 0);
  };

  // Q fragments (B operand of S^T = K Q^T): lane holds query q0 + l32, d chunk
  // 16*s + 8*g .. +7 for every step s.
  i32x4 qf[DS];
  // Row r (0..127) of a query block staged in LDS: rows 0-63 in group 0's
  // slot `slot`, 64-127 in group 1's, chunks swizzled as K rows are.
  auto staged_row = [&](int r, int slot) {
    return (IHP_LDS char *)smem + (r >> 6) * RING + slot * BLK + (r & 63) * ROW;
  };

  // Copy side: a wave instruction moves ROWS_PER_INSN rows of CH chunks;
  // lane -> (row, physical chunk), fetching the logical chunk that belongs
  // there. Keys past seq_kv are clamped to the last key (masked later). A
  // block copy is PASSES instructions per wave.
  const int c_row = lane / CH, c_phys = lane % CH;
  IHP_LDS char *lds = (IHP_LDS char *)smem + grp * RING;
  auto copy_block = [&](const char *src, uint32_t pitch, int kb,
                        IHP_LDS char *dst, auto is_v) {
    const int kv0 = kb * kBKV;
    // Opaque copies: the per-pass addresses are recomputed at each copy
    // instead of being hoisted into live registers.
    int lane_row = c_row, lane_chunk = c_phys;
    asm volatile("" : "+v"(lane_row), "+v"(lane_chunk));
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      const int row = (p * 4 + wq) * ROWS_PER_INSN + lane_row;
      int key = kv0 + row;
      key = key < seq_kv ? key : seq_kv - 1;
      const int sw = decltype(is_v)::value ? v_swizzle<D>(row)
                                           : k_swizzle<D>(row);
      // Uniform head base + 32-bit lane offset: one VGPR per address.
      const uint32_t off = (uint32_t)key * pitch + 16u * (lane_chunk ^ sw);
      if (DV == D || (lane_chunk ^ sw) < CHV)
        global_to_lds_16(src + off, dst + (p * 4 + wq) * ROWS_PER_INSN * ROW);
    }
  };
  // Full key blocks take the saddr copy form: the lane's byte offset inside
  // a block (its row and swizzled chunk) is the same for every block and
  // pass (the swizzles repeat every 16 rows, a pass moves 4 * ROWS_PER_INSN
  // rows), so it is computed once, and each copy adds only wave-uniform
  // terms in SGPRs (the block's and the pass's rows): no vector instruction
  // per copy. A tail block (keys past seq_kv, clamped per lane) takes
  // copy_block.
  const int f_row = wq * ROWS_PER_INSN + c_row;
  const uint32_t k_voff =
      (uint32_t)f_row * k_pitch + 16u * (c_phys ^ k_swizzle<D>(f_row));
  const uint32_t v_voff =
      (uint32_t)f_row * v_pitch + 16u * (c_phys ^ v_swizzle<D>(f_row));
  // The lane's logical chunk is the same in every pass: whether it lies
  // within the head dim.
  const bool k_in = DV == D || (c_phys ^ k_swizzle<D>(f_row)) < CHV;
  const bool v_in = DV == D || (c_phys ^ v_swizzle<D>(f_row)) < CHV;
  auto copy_full = [&](const char *src, uint32_t pitch, int kb,
                       IHP_LDS char *dst, uint32_t voff, bool in) {
    if (DV < D && !in)
      return;
    const char *base = src + (int64_t)kb * kBKV * pitch;
#pragma unroll
    for (int p = 0; p < PASSES; ++p)
      global_to_lds_16s(base + (int64_t)p * 4 * ROWS_PER_INSN * pitch, voff,
                        dst + (p * 4 + wq) * ROWS_PER_INSN * ROW);
  };
  auto copy_k = [&](int i) {
    const int kb = 2 * i + grp;
    if ((kb + 1) * kBKV <= seq_kv)
      copy_full(Kp, k_pitch, kb, lds + (i & 1) * BLK, k_voff, k_in);
    else
      copy_block(Kp, k_pitch, kb, lds + (i & 1) * BLK, std::false_type());
  };
  // The query block's rows into the V slots 1 (all 8 waves, PASSES
  // instructions each); rows past seq_q are clamped to the last row (their
  // outputs are not stored).
  auto copy_q = [&]() {
    int lane_row = c_row, lane_chunk = c_phys;
    asm volatile("" : "+v"(lane_row), "+v"(lane_chunk));
    const int qrow0 = q0 - wq * 32;  // the block's first row
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      const int r0 = (p * 8 + wave) * ROWS_PER_INSN;
      const int r = r0 + lane_row;
      const int row = min(qrow0 + r, seq_q - 1);
      const int chunk = lane_chunk ^ k_swizzle<D>(r);
      const uint32_t off = (uint32_t)row * q_pitch + 16u * chunk;
      if (DV == D || chunk < CHV)
        global_to_lds_16(Qp + off, staged_row(r0, 3));
    }
  };
  auto copy_v = [&](int i) {
    const int kb = 2 * i + grp;
    if ((kb + 1) * kBKV <= seq_kv)
      copy_full(Vp, v_pitch, kb, lds + (2 + (i & 1)) * BLK, v_voff, v_in);
    else
      copy_block(Vp, v_pitch, kb, lds + (2 + (i & 1)) * BLK, std::true_type());
  };
  // A query block's first key blocks (slots 0); K(1) goes out separately,
  // last, and the block's first barrier does not wait for it.
  auto copy_first = [&]() {
    if (n_mine > 0) {
      copy_k(0);
      copy_v(0);
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
  // K read base of this lane in ring slot 0 (absolute LDS address). The
  // group's ring is 64 KiB aligned and a d step's swizzle flips address
  // bits 5-7 only, so each step's address is this base XOR 32 s.
  uint32_t ka;
  {
    const int kl = lane & 31, kg = lane >> 5;
    const int k_sw = k_swizzle<D>(kl);
    ka = (uint32_t)(uintptr_t)lds +
         (uint32_t)(kl * ROW + 16 * (kg ^ (k_sw & 1)) + 32 * (k_sw >> 1));
  }

  // K read side: step s reads chunk c = 2s + g of key l32 (+32 for the
  // second key tile, which has the same swizzle). With w = k_swizzle(key),
  // c ^ w = 2 (s ^ w/2) + (g ^ w%2), so every step's address is one base
  // XOR 32 s (the key * ROW part has no bits below ROW).
  // S^T tiles of local block i: keys 32t..32t+31 x this wave's 32 queries.
  // Read r = 2 s + t feeds MFMA r; reads run KW ahead of their MFMA in KW + 1
  // rotating registers (read r + KW lands in the registers MFMA r - 1 took),
  // so an MFMA waits for a read issued KW MFMAs earlier instead of for the
  // LDS latency of one issued just before it.
  auto scores = [&](int i, f32x16 (&st)[2]) {
    const uint32_t kbase = ka + (uint32_t)((i & 1) * BLK);
    constexpr int NR = 2 * DSV, KW = kKReadAhead, NB = KW + 1;
    i32x4 kb[NB];
    auto issue = [&](auto r_c) {
      constexpr int R = decltype(r_c)::value;
      kb[R % NB] = lds_read_16_async<32 * (R % 2) * ROW>(
          (const IHP_LDS char *)(uintptr_t)(kbase ^ (32u * (R / 2))));
    };
    static_for<KW>(issue);
    static_for<NR>([&](auto r_c) {
      constexpr int R = decltype(r_c)::value;
      constexpr int S = R / 2, T = R % 2;
      // Reads issued so far: min(NR, R + KW); read R is done when at most
      // the ones after it are outstanding.
      constexpr int AHEAD = (R + KW < NR ? R + KW : NR) - R - 1;
      lgkm_wait<AHEAD>();
      lgkm_tie(kb[R % NB]);
      // The first step accumulates onto an inline zero.
      st[T] = Mfma32<f16>::mma(kb[R % NB], qf[S], S == 0 ? f32x16{} : st[T]);
      if constexpr (R + KW < NR)
        issue(std::integral_constant<int, R + KW>());
    });
  };
  // Max of a lane's 32 scores as 4 independent chains of 8 (the V phase
  // runs alone on its wave: a single 32-long chain would be latency-bound),
  // each seeded with -inf.
  auto row_max = [](const f32x16 (&st)[2]) {
    float m[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      m[c] = -INFINITY;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        m[c] = fmaxf(m[c], st[c >> 1][8 * (c & 1) + e]);
    }
    return fmaxf(fmaxf(m[0], m[1]), fmaxf(m[2], m[3]));
  };

  // Half H of this wave's merged O^T tiles (d tiles H DT/2 .. H DT/2 +
  // DT/2 - 1), normalised to f16, into the staged output rows (the K slots
  // 1): 4 d of row 32 wq + l32 per register quarter, 16-byte chunk 4 dt + rq
  // swizzled as K rows are, half g.
  auto stage_o = [&](const f32x16 (&acc)[DT], float inv, auto half_c) {
    constexpr int H = decltype(half_c)::value;
    const int r = wq * 32 + l32;
    IHP_LDS char *dst = staged_row(r, 1);
    const int sw = k_swizzle<D>(r);
#pragma unroll
    for (int dt = H * DT / 2; dt < (H + 1) * DT / 2; ++dt)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        f16x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          v[e] = (f16)(acc[dt][4 * rq + e] * inv);
        *(IHP_LDS f16x4 *)(dst + 16 * ((4 * dt + rq) ^ sw) + 8 * g) = v;
      }
  };
  // The staged rows to HBM, 16 bytes per lane (all 8 waves, PASSES
  // instructions each), written through past this XCD's L2 (the kernel never
  // reads O, and no dirty lines are left for the write-back at its end:
  // 0.5-1 % at the C4 shape); rows past seq_q are not written.
  auto store_rows = [&](int qrow0) {
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      const int r = (p * 8 + wave) * ROWS_PER_INSN + c_row;
      const i32x4 v = *(const IHP_LDS i32x4 *)(
          staged_row(r, 1) + 16 * (c_phys ^ k_swizzle<D>(r)));
      if (qrow0 + r < seq_q && (DV == D || c_phys < CHV))
        store_through16((f16 *)Op + (int64_t)(qrow0 + r) * o_row + 8 * c_phys,
                        v);
    }
  };

  f32x16 o[DT];
  // l_run is this lane's share of the row sum (the keys its lane half
  // holds) until the key loop ends; both halves share m_run, so they are
  // rescaled alike, and one pair_sum then gives the row's sum.
  float m_run = -INFINITY, l_run = 0.0f;
  // S^T of the block being scored (M phase) and turned into probabilities
  // (V phase); P of the block awaiting its PV, as f16 pairs: word w of
  // fragment st holds keys 16 st + 2 w, + 1.
  f32x16 st[2];
  i32x4 pw[4];

  // O^T[d][q] += V^T[d][key] P^T[key][q] for local block i, 16 keys per
  // MFMA. V^T fragments of key step ST in buffer ST % 2: the reads of step
  // ST + 1 are issued before the MFMAs of step ST, which wait only for their
  // own 2 DT reads. The row sum of P (the f16 values PV multiplies, added
  // with v_dot2 against (1, 1)) is taken here, between the MFMAs, by the
  // wave whose SIMD partner is then on the VALU softmax: it depends on P
  // only, and l_run needs it only at the end of the key loop.
  auto pv = [&](int i) {
    float psum[4];
    const IHP_LDS char *vs = lds + (2 + (i & 1)) * BLK;
    i32x2 vr[2][DT][2];
    auto read_v = [&](auto step_c) {
      constexpr int ST = decltype(step_c)::value;
      constexpr int KOFF = 16 * ST * ROW;
      static_for<DT>([&](auto dt) {
        constexpr int DTI = decltype(dt)::value;
        vr[ST % 2][DTI][0] = lds_read_tr16_at<KOFF>(vs + v_off[DTI]);
        vr[ST % 2][DTI][1] = lds_read_tr16_at<KOFF + 8 * ROW>(vs + v_off[DTI]);
      });
    };
    read_v(std::integral_constant<int, 0>());
    static_for<4>([&](auto step_c) {
      constexpr int ST = decltype(step_c)::value;
      if constexpr (ST < 3)
        read_v(std::integral_constant<int, ST + 1>());
      lgkm_wait<ST < 3 ? 2 * DT : 0>();
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        tie2(vr[ST % 2][dt][0]);
        tie2(vr[ST % 2][dt][1]);
        const i32x4 vf = i32x4{vr[ST % 2][dt][0][0], vr[ST % 2][dt][0][1],
                               vr[ST % 2][dt][1][0], vr[ST % 2][dt][1][1]};
        o[dt] = Mfma32<f16>::mma(vf, pw[ST], o[dt]);
      }
      psum[ST] = 0.0f;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        // Copied out first: __builtin_bit_cast of a vector element
        // expression reads element 0 whatever the index (hipcc 7.2).
        const int word = pw[ST][w];
        psum[ST] = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, word),
                                          f16x2{1, 1}, psum[ST], false);
      }
    });
    l_run += (psum[0] + psum[1]) + (psum[2] + psum[3]);
  };

  // The mask values of block k this lane's scores need (MASK): element
  // (t, r) of S^T is key kv0 + 4 g + 32 t + 8 (r / 4) + r % 4 of row
  // q0 + l32, so register quarter (t, r / 4) is one 8-byte load of 4
  // consecutive keys. Groups past seq_kv (a multiple of 4) load key 0
  // instead (those scores are masked anyway); rows past seq_q the last row.
  // Issued by the M phase that computes S^T(k); the V phase after it waits
  // for them before its copies.
  i32x2 mk[2][4];
  auto load_mask = [&](int k) {
    const int kv0 = (2 * k + grp) * kBKV;
    const f16 *mrow = Mp + (int64_t)min(q0 + l32, seq_q - 1) * L.m[2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int key = kv0 + 4 * g + 32 * t + 8 * rq;
        mk[t][rq] = *(const i32x2 *)(mrow + (key + 3 < seq_kv ? key : 0));
      }
  };

  // M phase: PV of block k - 1 (when DO_PV), then S^T of block k (when
  // DO_S); MFMA and LDS reads only, at raised wave priority so its MFMAs
  // issue ahead of the other group's VALU work on the same SIMD.
  float alpha = 1.0f;     // output rescale pending from the V phase
  bool rescale = false;   // wave-uniform
  auto m_phase = [&](int k, auto do_pv, auto do_s) {
    if constexpr (MASK && decltype(do_s)::value)
      load_mask(k);
    __builtin_amdgcn_s_setprio(1);
    if constexpr (decltype(do_pv)::value) {
      if (rescale) {
#pragma unroll
        for (int t = 0; t < DT; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            o[t][r] *= alpha;
        rescale = false;
      }
      pv(k - 1);
    }
    if constexpr (decltype(do_s)::value)
      scores(k, st);
    __builtin_amdgcn_s_setprio(0);
  };

  // Block k's softmax. Off the diagonal the row max is taken on the raw
  // scores (scale_log2 > 0 keeps the order) and the scale goes into the
  // exponent's FMA; masked blocks (causal diagonal, sequence tail) are
  // masked and scaled in place first. Two instances (MASKED true / false)
  // so that neither path merges S^T values with the other.
  auto softmax = [&](int k, auto masked_c) {
    constexpr bool MASKED = decltype(masked_c)::value;
    float mx, sc;
    if constexpr (MASKED) {
      // Element (t, r) holds key kv0 + 4 g + c, c = 32 t + 8 (r / 4) + r % 4;
      // keys at or past min(seq_kv, q0 + l32 + 1) (causal) are masked, i.e.
      // c >= thr: one compare against a constant and one select each.
      const int kv0 = (2 * k + grp) * kBKV;
      const int row = q0 + l32;
      const int lim = causal ? min(seq_kv, row + 1) : seq_kv;
      const int thr = lim - kv0 - 4 * g;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int c = 32 * t + 8 * (r >> 2) + (r & 3);
          float v = st[t][r] * scale_log2;
          if constexpr (MASK) {
            const i32x2 w = mk[t][r >> 2];
            const f16x4 h = __builtin_bit_cast(f16x4, w);
            v = __builtin_fmaf((float)h[r & 3], 1.4426950408889634f, v);
          }
          st[t][r] = c >= thr ? -INFINITY : v;
        }
      mx = row_max(st);
      sc = 1.0f;
    } else {
      mx = row_max(st) * scale_log2;
      sc = scale_log2;
    }
    mx = pair_max(mx);
    alpha = 1.0f;
    if (!__all(mx <= m_run + kLazyMax)) {
      const float m_new = fmaxf(m_run, mx);
      // A row with every key masked so far keeps m = -inf; exp2 of a
      // finite offset from it must not produce nan.
      alpha =
          __builtin_amdgcn_exp2f(m_run - (m_new == -INFINITY ? 0.0f : m_new));
      m_run = m_new;
      // O is rescaled by the next M phase, before PV(k) adds to it.
      rescale = true;
    }
    const float m_use = m_run == -INFINITY ? 0.0f : m_run;
    // Probabilities rounded to f16 pairs. Their row sum is added by the
    // next PV (which multiplies exactly these values); the sum so far is
    // rescaled here, before it.
#pragma unroll
    for (int f = 0; f < 4; ++f)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float p0 = __builtin_amdgcn_exp2f(
            __builtin_fmaf(st[f >> 1][8 * (f & 1) + 2 * w], sc, -m_use));
        const float p1 = __builtin_amdgcn_exp2f(
            __builtin_fmaf(st[f >> 1][8 * (f & 1) + 2 * w + 1], sc, -m_use));
        const f16x2 h = __builtin_convertvector(f32x2{p0, p1}, f16x2);
        pw[f][w] = __builtin_bit_cast(int, h);
      }
    l_run *= alpha;
  };

  // V phase k (k = 0 .. n_mine - 1): the copies of K(k + 2) into the K slot
  // S(k) was read from and of V(k + 1) into the V slot PV(k - 1) was read
  // from (both read in the M phase before, which every wave of the group
  // has finished), then block k's softmax. The reference max m_run moves
  // only when some row's block max exceeds it by more than kLazyMax (log2
  // units), so probabilities stay at most 2^kLazyMax (exact in f16) and most
  // blocks skip the output rescale (done by the M phase after, whose PV
  // adds the first terms relative to the new reference). Ends by waiting
  // for this wave's copies of K(k + 1) and V(k), which the next M phase
  // reads (the ones issued here may stay in flight).
  auto v_phase = [&](int k) {
    const bool next_k = k + 2 < n_mine, next_v = k + 1 < n_mine;
    if constexpr (MASK) {
      // Block k's mask values, and the copies issued before them, have
      // landed before this phase's copies go out.
      wait_vmcnt<0>();
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int rq = 0; rq < 4; ++rq)
          tie2(mk[t][rq]);
    }
    if (next_k)
      copy_k(k + 2);
    if (next_v)
      copy_v(k + 1);
    const int kv0 = (2 * k + grp) * kBKV;
    if (MASK || (causal && kv0 + kBKV - 1 > q0) || kv0 + kBKV > seq_kv ||
        scale_log2 <= 0.0f)
      softmax(k, std::true_type());
    else
      softmax(k, std::false_type());
    if (next_k)
      wait_vmcnt<2 * PASSES>();
    else if (next_v)
      wait_vmcnt<PASSES>();
    else
      wait_vmcnt<0>();
  };

  setup(0);
  copy_q();
  copy_first();
  if (n_mine > 1)
    copy_k(1);
  for (int item = 0;;) {
    // Q, K(0) of this block (and the previous block's output stores) have
    // completed in every wave; so has V(0), issued before Q. K(1), when
    // issued, is each wave's newest memory operation and may stay in flight.
    if (n_mine > 1)
      wait_vmcnt<PASSES>();
    else
      wait_vmcnt<0>();
    block_barrier();
    {
      // This wave's 32 query rows, read like K rows (conflict-free). They
      // have landed before the barrier below: group 0 overwrites its V slot
      // 1 with V(1) in the slot after it, while group 1 may not yet have
      // used its copy.
      const IHP_LDS char *qs = staged_row(wq * 32, 3);
      int ln = lane;
      asm volatile("" : "+v"(ln));
      const int kl = ln & 31, kg = ln >> 5;
      const int k_sw = k_swizzle<D>(kl);
      const int qaddr = kl * ROW + 16 * (kg ^ (k_sw & 1)) + 32 * (k_sw >> 1);
#pragma unroll
      for (int s = 0; s < DSV; ++s)
        qf[s] = *(const IHP_LDS i32x4 *)(qs + (qaddr ^ (32 * s)));
      wait_lgkmcnt0();
    }
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        o[t][r] = 0.0f;
    m_run = -INFINITY;
    l_run = 0.0f;

    // Phase schedule: M(0), V(0), M(1), ..., V(n - 1), M(n), one phase per
    // barrier slot (M(k): PV(k - 1) and S(k); M(0) has no PV, M(n) no S).
    // Group 1 starts one slot after group 0, so the two waves sharing a
    // SIMD (w and w + 4) are always in opposite phases: one issues MFMAs
    // while the other works on the VALU. Every wave passes n_slots
    // barriers: the schedule's 2 n_mine + 1 (+ 1 for group 1), then padding.
    {
      int pad = n_slots;
      if (n_mine > 0) {
        if (grp == 1)
          block_barrier();
        m_phase(0, std::false_type(), std::true_type());
        block_barrier();
        for (int k = 0; k + 1 < n_mine; ++k) {
          v_phase(k);
          block_barrier();
          m_phase(k + 1, std::true_type(), std::true_type());
          block_barrier();
        }
        v_phase(n_mine - 1);
        block_barrier();
        m_phase(n_mine, std::true_type(), std::false_type());
        block_barrier();
        pad -= grp + 2 * n_mine + 1;
      }
      for (; pad > 0; --pad)
        block_barrier();
    }
    // After the last slot's barrier every wave has finished its phases:
    // every ring slot is free. The two lane halves' shares of each row
    // sum are added.
    l_run = pair_sum(l_run);
    const int qrow0 = q0 - wq * 32;  // this block's first row
    const bool more = item + 1 < n_items;
    // The next block's first key blocks stream into slots 0 during the
    // merge, which uses slots 1.
    if (more) {
      setup(item + 1);
      copy_first();
    }

    // Merge: each group hands the other the half of its O tiles the other
    // keeps (group 1 its d tiles 0 .. DT/2 - 1, group 0 the rest) and its
    // (m, l); both then merge their kept half with the same weights, in the
    // same arithmetic order (group 0's term first), and stage it. Wave wq's
    // halves go through ring slot 1 (K, then V) of group wq / 2: float4 k
    // of tile dt at (dt 4 + k) 64 + lane; (m, l) after the rings at
    // (grp 4 + wq) 64 + lane.
    IHP_LDS f32x4 *xo = (IHP_LDS f32x4 *)(smem + (wq >> 1) * RING +
                                          (1 + 2 * (wq & 1)) * BLK);
    IHP_LDS f32x2 *xml = (IHP_LDS f32x2 *)(smem + kGroups * RING);
    auto hand = [&](auto half_c) {
      constexpr int H = decltype(half_c)::value;
#pragma unroll
      for (int dt = H * DT / 2; dt < (H + 1) * DT / 2; ++dt)
#pragma unroll
        for (int k = 0; k < 4; ++k)
          xo[(dt * 4 + k) * 64 + lane] =
              f32x4{o[dt][4 * k], o[dt][4 * k + 1], o[dt][4 * k + 2],
                    o[dt][4 * k + 3]};
    };
    if (grp == 1)
      hand(std::integral_constant<int, 0>());
    else
      hand(std::integral_constant<int, 1>());
    xml[(grp * 4 + wq) * 64 + lane] = f32x2{m_run, l_run};
    wait_lgkmcnt0();
    block_barrier();
    {
      const f32x2 ml = xml[((grp ^ 1) * 4 + wq) * 64 + lane];
      const float m0 = grp == 0 ? m_run : ml[0];
      const float m1 = grp == 0 ? ml[0] : m_run;
      const float l0 = grp == 0 ? l_run : ml[1];
      const float l1 = grp == 0 ? ml[1] : l_run;
      const float m = fmaxf(m0, m1);
      const float m_use = m == -INFINITY ? 0.0f : m;
      const float a0 = __builtin_amdgcn_exp2f(m0 - m_use);
      const float a1 = __builtin_amdgcn_exp2f(m1 - m_use);
      l_run = l0 * a0 + l1 * a1;
      auto merge = [&](auto half_c) {
        constexpr int H = decltype(half_c)::value;
#pragma unroll
        for (int dt = H * DT / 2; dt < (H + 1) * DT / 2; ++dt)
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const f32x4 x = xo[(dt * 4 + k) * 64 + lane];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float own = o[dt][4 * k + e];
              o[dt][4 * k + e] = H == 0 ? own * a0 + x[e] * a1
                                        : x[e] * a0 + own * a1;
            }
          }
      };
      if (grp == 0)
        merge(std::integral_constant<int, 0>());
      else
        merge(std::integral_constant<int, 1>());
    }
    // The slots 1 are free again: the next block's rows stream into the V
    // slots, this block's output rows are staged in the K slots.
    block_barrier();
    if (more)
      copy_q();
    {
      const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
      if constexpr (OF32) {
        // This group's half of the d tiles of this wave's row l32 of the
        // block (q0 already names the next block's rows), straight to O:
        // register quarter rq of tile dt is d = 32 dt + 8 rq + 4 g .. + 3.
        const int row = qrow0 + wq * 32 + l32;
        if (row < seq_q) {
          float *dst = (float *)Op + (int64_t)row * o_row + 4 * g;
          auto put = [&](auto half_c) {
            constexpr int H = decltype(half_c)::value;
#pragma unroll
            for (int dt = H * DT / 2; dt < (H + 1) * DT / 2; ++dt)
#pragma unroll
              for (int rq = 0; rq < 4; ++rq)
                if (DV == D || 32 * dt + 8 * rq < DV)
                  *(f32x4 *)(dst + 32 * dt + 8 * rq) =
                      f32x4{o[dt][4 * rq] * inv, o[dt][4 * rq + 1] * inv,
                            o[dt][4 * rq + 2] * inv, o[dt][4 * rq + 3] * inv};
          };
          if (grp == 0)
            put(std::integral_constant<int, 0>());
          else
            put(std::integral_constant<int, 1>());
        }
      } else if (grp == 0) {
        stage_o(o, inv, std::integral_constant<int, 0>());
      } else {
        stage_o(o, inv, std::integral_constant<int, 1>());
      }
    }
    wait_lgkmcnt0();
    block_barrier();
    if constexpr (!OF32)
      store_rows(qrow0);
    if (!more)
      return;
    // The staged rows have been read: K(1) of the next block may land.
    wait_lgkmcnt0();
    block_barrier();
    if (n_mine > 1)
      copy_k(1);
    ++item;
  }
}

hipError_t launch_attention(const void *q, const void *k, const void *v,
                            void *o, int64_t batch,
                            const AttentionLayout &layout, int64_t head_dim,
                            float scale, int causal, void *stream,
                            const void *mask, int out_f32) {
  const int64_t q_blocks = (layout.seq_q + kBQ - 1) / kBQ;
  const int64_t planes = batch * layout.heads;
  // One workgroup per pair of query blocks (q_blocks - 1 - k, k).
  dim3 grid((unsigned)((q_blocks + 1) / 2 * planes));
  const float scale_log2 = scale * 1.4426950408889634f;  // log2(e)
  const int64_t d = head_dim, sq = layout.seq_q, skv = layout.seq_kv,
                h = layout.heads;
  const bool contig =
      !mask && !out_f32 && layout.group == 1 && layout.q[2] == d && layout.o[2] == d &&
      layout.k[2] == d && layout.v[2] == d && layout.q[1] == sq * d &&
      layout.o[1] == sq * d && layout.k[1] == skv * d &&
      layout.v[1] == skv * d && layout.q[0] == h * sq * d &&
      layout.o[0] == h * sq * d && layout.k[0] == h * skv * d &&
      layout.v[0] == h * skv * d;
  const void *kernel;
  // The strided instances: (mask, f32 output) of head dim DVV in layout DD.
#define IHP_ATT_PICK(DVV, DD)                                                  \
  kernel = mask ? (out_f32 ? (const void *)&attention_fwd_kernel<DD, false, true, DVV, true>   \
                           : (const void *)&attention_fwd_kernel<DD, false, true, DVV>)        \
                : (out_f32 ? (const void *)&attention_fwd_kernel<DD, false, false, DVV, true>  \
                           : (const void *)&attention_fwd_kernel<DD, false, false, DVV>);      \
  break;
  switch (head_dim) {
    case 128:
      if (contig) {
        kernel = (const void *)&attention_fwd_kernel<128, true>;
        break;
      }
      IHP_ATT_PICK(128, 128)
    case 64:
      if (contig) {
        kernel = (const void *)&attention_fwd_kernel<64, true>;
        break;
      }
      IHP_ATT_PICK(64, 64)
    case 16: IHP_ATT_PICK(16, 64)
    case 32: IHP_ATT_PICK(32, 64)
    case 48: IHP_ATT_PICK(48, 64)
    case 80: IHP_ATT_PICK(80, 128)
    case 96: IHP_ATT_PICK(96, 128)
    case 112: IHP_ATT_PICK(112, 128)
    default:
      return hipErrorInvalidValue;
  }
#undef IHP_ATT_PICK
  const f16 *qp = (const f16 *)q, *kp = (const f16 *)k, *vp = (const f16 *)v;
  const f16 *mp = (const f16 *)mask;
  void *op = o;
  AttentionLayout l = layout;
  void *args[] = {&qp, &kp, &vp, &op, &mp, &l, (void *)&scale_log2, &causal};
  return hipLaunchKernel(kernel, grid, dim3(kThreads), args, 0,
                         (hipStream_t)stream);
}

}  // namespace ihp

namespace ihp {

const KernelEntry *attention_kernels(int *count) {
  static const KernelEntry all[] = {
      {"attention_fwd_d128", (const void *)&attention_fwd_kernel<128, true>, kThreads, kExportAttention},
      {"attention_fwd_d64", (const void *)&attention_fwd_kernel<64, true>, kThreads, kExportAttention},
      {"attention_fwd_d128_strided", (const void *)&attention_fwd_kernel<128, false>, kThreads, kExportAttention},
      {"attention_fwd_d64_strided", (const void *)&attention_fwd_kernel<64, false>, kThreads, kExportAttention},
      {"attention_fwd_d128_mask", (const void *)&attention_fwd_kernel<128, false, true>, kThreads, kExportAttention},
      {"attention_fwd_d64_mask", (const void *)&attention_fwd_kernel<64, false, true>, kThreads, kExportAttention},
      {"attention_fwd_d16", (const void *)&attention_fwd_kernel<64, false, false, 16>, kThreads, kExportAttention},
      {"attention_fwd_d32", (const void *)&attention_fwd_kernel<64, false, false, 32>, kThreads, kExportAttention},
      {"attention_fwd_d48", (const void *)&attention_fwd_kernel<64, false, false, 48>, kThreads, kExportAttention},
      {"attention_fwd_d80", (const void *)&attention_fwd_kernel<128, false, false, 80>, kThreads, kExportAttention},
      {"attention_fwd_d96", (const void *)&attention_fwd_kernel<128, false, false, 96>, kThreads, kExportAttention},
      {"attention_fwd_d112", (const void *)&attention_fwd_kernel<128, false, false, 112>, kThreads, kExportAttention},
      {"attention_fwd_d16_mask", (const void *)&attention_fwd_kernel<64, false, true, 16>, kThreads, kExportAttention},
      {"attention_fwd_d32_mask", (const void *)&attention_fwd_kernel<64, false, true, 32>, kThreads, kExportAttention},
      {"attention_fwd_d48_mask", (const void *)&attention_fwd_kernel<64, false, true, 48>, kThreads, kExportAttention},
      {"attention_fwd_d80_mask", (const void *)&attention_fwd_kernel<128, false, true, 80>, kThreads, kExportAttention},
      {"attention_fwd_d96_mask", (const void *)&attention_fwd_kernel<128, false, true, 96>, kThreads, kExportAttention},
      {"attention_fwd_d112_mask", (const void *)&attention_fwd_kernel<128, false, true, 112>, kThreads, kExportAttention},
#define IHP_ATT_F32(NAME, DD, DVV)                                                                               \
      {"attention_fwd_" NAME "_f32", (const void *)&attention_fwd_kernel<DD, false, false, DVV, true>, kThreads, kExportAttention}, \
      {"attention_fwd_" NAME "_mask_f32", (const void *)&attention_fwd_kernel<DD, false, true, DVV, true>, kThreads, kExportAttention},
      IHP_ATT_F32("d16", 64, 16) IHP_ATT_F32("d32", 64, 32) IHP_ATT_F32("d48", 64, 48)
      IHP_ATT_F32("d64", 64, 64) IHP_ATT_F32("d80", 128, 80) IHP_ATT_F32("d96", 128, 96)
      IHP_ATT_F32("d112", 128, 112) IHP_ATT_F32("d128", 128, 128)
#undef IHP_ATT_F32
  };
  *count = (int)(sizeof(all) / sizeof(all[0]));
  return all;
}

}  // namespace ihp
