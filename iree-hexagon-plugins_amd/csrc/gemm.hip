// gfx950 matmul kernels for the linalg.matmul / quantized_matmul dispatch.
//
// The reference stages VTCM tiles of A and B with double-buffered DMA
// (CG/Transforms/HexagonPipelineVTCMTransfers.cpp:388-524), packs them into
// 32x32 HMX tiles (UK/hmx.c:123-143,246-275) and issues one 32x32x32 HMX MMA
// per K step into an accumulator that is read back once per output tile
// (CG/Transforms/HexagonExpandHmxMatmul.cpp:286-331). Here:
//  * the VTCM tile becomes a BM x BN workgroup macro-tile whose A and B K-slabs
//    are copied straight from HBM into LDS (global_load_lds_dwordx4, no VGPR
//    round trip) through a STAGES-deep ring of LDS buffers;
//  * the HMX pack becomes an XOR swizzle of 16-byte chunks applied on the
//    global side of that copy, so MFMA operand reads from LDS are
//    bank-conflict free and no separate pack pass exists;
//  * the HMX MMA becomes v_mfma_{f32_32x32x16_f16, i32_32x32x32_i8} on
//    per-wave 32x32 fragments with f32/i32 accumulators held in registers for
//    the whole K loop (the reference reads its accumulator out as f16,
//    HexagonConvertMatmulToHmx.cpp:592-596; this keeps full precision);
//  * the unpack (add into the DPS init, UK/hmx.c:328-357) is the epilogue.
#include <type_traits>
#include <vector>

#include "device_common.h"
#include "kernels_internal.h"

namespace ihp {

// Compile-time loop: f(std::integral_constant<int, I>()) for I in [0, N).
template <int N, int I = 0, typename F>
__device__ __forceinline__ void static_for(F &&f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>());
    static_for<N, I + 1>(f);
  }
}

// ----------------------------------------------------------------------------
// Fast path: A [M,K] K-contiguous, every extent a multiple of the macro-tile,
// 16-byte aligned rows. Three B forms (BMODE):
//   kBTN   B [N,K] of the A type (K-contiguous, "column-major B")
//   kBNN16 B [K,N] f16 (N-contiguous, row-major weights)
//   kBW8   B [K,N] int8 with a per-column f16 scale (W8A16), dequantized to
//          f16 in registers after the LDS read, scale applied in the epilogue
//   kBNN8  B [K,N] int8 with int8 A (row-major int8 weights: the default map
//          of linalg.matmul and quantized_matmul), int32 accumulation
// ----------------------------------------------------------------------------

template <int CH>
__device__ __forceinline__ int chunk_swizzle(int row) {
  // 16-byte chunk permutation of a staged K-contiguous row of CH chunks.
  // gfx950 LDS has 64 four-byte banks (a 256-byte bank line) and serves a
  // ds_read_b128 16 lanes at a time; the 16 lanes of a fragment read 16
  // consecutive rows at one logical chunk. Rows sharing a bank line keep
  // their offset within it, and the chunk index is XORed with the bank-line
  // number, so the 16 reads hit 16 distinct 16-byte bank groups.
  return (row / (16 / CH)) % CH;
}

// Chunk swizzle of a staged N-contiguous B row (row = k). A transposed LDS
// read (ds_read_b64_tr_b16 / _b8) makes each 16-lane block read 4 (f16) or 8
// (int8) consecutive k rows at one 32- or 16-byte column window; XORing the
// chunk index with a multiple of the row index spreads the rows of two
// neighbouring blocks over all 64 banks. For the 32x32 MFMA those two
// blocks read the same rows at neighbouring windows; for the 16x16 MFMA they
// read one window at rows 8 apart, so row bit 3 also flips a chunk bit
// (the swizzle then repeats every 16 rows). int8 operands of the int8
// MFMA take 16 k rows per 16-lane block (two 8-row transposed reads); in the
// 16x16 form the two blocks served together read rows 16 apart, so row bit
// 4 flips the chunk's low bit (period 32 rows).
template <int BMODE, int MS = 32>
__device__ __forceinline__ int nn_swizzle(int k) {
  if constexpr (BMODE == kBNN8)
    return 2 * (k & 7) ^ (MS == 16 ? (k >> 4) & 1 : 0);
  const int hi = MS == 16 ? (k >> 3) & 1 : 0;
  return BMODE == kBNN16 ? 4 * (k & 3) ^ 2 * hi : 2 * (k & 7) ^ hi;
}
// Rows after which nn_swizzle repeats.
template <int BMODE, int MS>
constexpr int nn_swizzle_period() {
  return BMODE == kBNN8 ? (MS == 16 ? 32 : 8)
                        : (MS == 16 ? 16 : (BMODE == kBNN16 ? 4 : 8));
}

template <int OFF>
__device__ __forceinline__ i32x2 lds_read_tr16_async(const IHP_LDS char *p) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset range");
  i32x2 v;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2"
               : "=v"(v)
               : "v"((unsigned)(uintptr_t)p), "i"(OFF));
  return v;
}

template <int OFF>
__device__ __forceinline__ i32x2 lds_read_tr8_async(const IHP_LDS char *p) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset range");
  i32x2 v;
  asm volatile("ds_read_b64_tr_b8 %0, %1 offset:%2"
               : "=v"(v)
               : "v"((unsigned)(uintptr_t)p), "i"(OFF));
  return v;
}

__device__ __forceinline__ void lgkm_tie2(i32x2 &v) {
  asm volatile("" : "+v"(v));
}

// AT: A is stored [K,M] (M-contiguous, the (d2, d0) indexing map of a
// transposed LHS). Its K rows are staged like row-major f16 B and read with
// the same transposed LDS reads: the A and B operands of the 32x32x16 MFMA
// share one lane layout (lane % 32 = row / column, 8 * (lane / 32) = k run).
//
// SPLIT: the K extent is split over gridDim.y (k_split elements each); every
// workgroup publishes an f32 (i32) partial tile and the last one to arrive at
// a tile sums the partials in split order and writes C. With sk_steps > 0
// (stream-K) the workgroups instead take equal runs of the (tile, K stage)
// pairs, so tile counts that leave CUs idle still fill the chip; a tile
// split over several runs is reduced the same way. M need not be a
// multiple of BM: A rows past M are clamped to row M-1 on the copy side (rows
// of C depend only on their own row of A) and never stored.
//
// MS: the MFMA shape, 32 (v_mfma_*_32x32x{16,32}) or 16
// (v_mfma_*_16x16x{32,64}). Both read the same operand bytes per wave tile;
// on random operands the 16x16 instructions sustain 11-15 % more products
// per second on this chip (the calibration loop: int8 4075 against 3559
// TOPS, f16 1950 against 1754 TFLOP/s), the power per product being lower.
// For row-major B and transposed A the 16x16 operand (16 columns x 8 k per
// 16-lane block) comes from the same transposed reads, each block taking
// k rows 8 b .. 8 b + 7 of the 32-row K step.
template <typename T, typename OutT, int BM, int BN, int BKB, int WM, int WN,
          int STAGES, int BMODE, bool SPLIT, bool AT, int MS = 32>
__global__ __launch_bounds__(64 * WM *WN, 1) void gemm_lds_kernel(
    const T *__restrict__ A, const void *__restrict__ Bv, OutT *__restrict__ C,
    const f16 *__restrict__ scale, int M, int N, int K, int64_t lda,
    int64_t ldb, int64_t ldc, int store_mode, int k_split, int sk_steps,
    typename Mfma32<T>::AccScalar *__restrict__ partials,
    unsigned *__restrict__ counters, int64_t sa, int64_t sb, int64_t sc,
    Epi epi, int64_t s_mul) {
  static_assert(MS == 32 || MS == 16, "MFMA shape");
  typedef typename std::conditional<MS == 32, Mfma32<T>, Mfma16<T>>::type MF;
  typedef typename MF::Acc Acc;
  // Accumulator registers per fragment, K bytes per MFMA step and the
  // 16-byte chunks one step reads per row.
  constexpr int AR = MS == 32 ? 16 : 4;
  constexpr int KSB = MS == 32 ? 32 : 64;
  constexpr int KCH = KSB / 16;
  constexpr bool kNN = BMODE != kBTN;
  constexpr int TBB = BMODE == kBW8 ? 1 : (int)sizeof(T);  // B element bytes
  constexpr int NT = 64 * WM * WN;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int FM = WTM / MS, FN = WTN / MS;
  constexpr int KE = BKB / (int)sizeof(T);  // K elements per stage
  constexpr int CH = BKB / 16;              // chunks per staged A (TN B) row
  constexpr int ROWS_PER_WAVE = 64 / CH;
  constexpr int ROWS_PER_PASS = NT / CH;
  // A staging: K-contiguous rows are M (BKB bytes each); AT rows are K
  // (BM * 2 bytes each).
  constexpr int AROW = AT ? BM * 2 : BKB;
  constexpr int ACH = AROW / 16;
  constexpr int A_ROWS = AT ? KE : BM;
  constexpr int A_RPW = AT ? 64 / ACH : ROWS_PER_WAVE;  // rows per wave copy
  constexpr int A_RPP = AT ? NT / ACH : ROWS_PER_PASS;  // rows per pass
  constexpr int A_PASSES = A_ROWS / A_RPP;
  // B staging: TN rows are N (BKB bytes each); NN rows are K (BN*TBB bytes).
  constexpr int BROW = kNN ? BN * TBB : BKB;
  constexpr int BCH = BROW / 16;
  constexpr int B_ROWS = kNN ? KE : BN;
  constexpr int B_RPW = 64 / BCH;    // B rows per wave copy instruction
  constexpr int B_RPP = NT / BCH;    // B rows per block-wide pass
  constexpr int B_PASSES = B_ROWS / B_RPP;
  constexpr int LOADS_PER_STAGE = A_PASSES + B_PASSES;
  constexpr int A_BYTES = BM * BKB;
  constexpr int STAGE_BYTES = A_BYTES + B_ROWS * BROW;
  constexpr int KSTEPS = BKB / KSB;
  // LDS reads per K step: FM A fragments, FN B fragments (two transposed
  // reads each for f16 and int8 NN).
  constexpr bool kTwoReadB = BMODE == kBNN16 || BMODE == kBNN8;
  constexpr int B_READS = kTwoReadB ? 2 * FN : FN;
  constexpr int A_READS = AT ? 2 * FM : FM;
  constexpr int RD = A_READS + B_READS;
  static_assert(A_ROWS % A_RPP == 0 && B_ROWS % B_RPP == 0, "tile");
  static_assert(!AT || (sizeof(T) == 2 && !SPLIT && ACH >= 16 &&
                        A_RPP % 8 == 0 && A_RPW <= 8),
                "transposed A: f16, exact M tiling, BM >= 128");
  static_assert(B_RPP * BCH == NT && B_RPW * BCH == 64, "B copy shape");
  static_assert(FM >= 1 && FN >= 1 && (CH == 4 || CH == 8), "tile");
  static_assert(KSTEPS % 2 == 0, "fragment double buffer parity");
  // The A swizzle repeats every 16 rows; block-wide copy passes start on
  // that period, so a lane's swizzle depends only on its row in the pass.
  static_assert(ROWS_PER_PASS % 16 == 0 && (16 / CH) * CH == 16, "swz");
  static_assert(!kNN || (BCH >= 16 && B_RPP % 8 == 0 && B_RPW <= 8), "nn");
  // Copy passes start on the row swizzle's period (16 rows for 16x16, 32
  // for the int8 16x16 form).
  static_assert(!kNN || B_RPP % nn_swizzle_period<BMODE, MS>() == 0,
                "B swizzle period");
  static_assert(MS == 32 || !AT || A_RPP % 16 == 0, "16x16 swizzle period");
  static_assert(BMODE != kBNN8 || sizeof(T) == 1, "int8 NN takes int8 A");
  // k rows of a staged row-major operand per MFMA K step
  constexpr int KROWS = KSB / (int)sizeof(T);
  // Reads allowed in flight while the previous step's are collected. LDS
  // reads return in issue order and lgkmcnt has 4 bits: with more than 15
  // new reads the wait also takes the oldest of them (still correct).
  constexpr int RDW = RD < 16 ? RD : 15;
  // Unsplit 256x256 16x16 tiles: the waves of wave row 0 issue the copies
  // of their SIMD partner (wave w + 4) too, and the partner none. Issuing a
  // stage's copies stalls a wave for a while (the address unit drains them
  // at its own rate); this way one wave of each SIMD keeps the matrix core
  // fed meanwhile, instead of both stalling at every hand-off. Measured
  // 1.6-3 % faster on these tiles; on the 256x128 and 128x256 tiles, with
  // half the MFMAs a stage, 2-4.5 % slower, so they keep their own copies.
  constexpr bool kCopyPair = !SPLIT && !AT && WM == 2 && WN == 4 &&
                             BM == 256 && BN == 256 && MS == 16;
  constexpr int CPM = kCopyPair ? 2 : 1;  // copies per stage, as a multiple
  static_assert(STAGES >= 2 && (STAGES - 1) * LOADS_PER_STAGE * CPM < 64,
                "vmcnt range");
  // Unsplit 16x16 tiles issue each MFMA with its operands swapped (the B
  // fragment as the row operand; both share one lane layout): the fragment
  // then comes out transposed, lane l holding 4 consecutive columns of row
  // l % 16. An i32 output stores that run as one 16-byte chunk straight from
  // registers; f16 / f32 outputs stage it through LDS as one 8- / 16-byte
  // write instead of four. (W8A16 and transposed-A tiles keep the plain
  // order: not measured.)
  constexpr bool kSwapAB = MS == 16 && !SPLIT && BMODE != kBW8 && !AT;
  static_assert(STAGES * STAGE_BYTES <= 160 * 1024, "LDS budget");

  __shared__ __attribute__((aligned(1024))) char smem[STAGES * STAGE_BYTES];

  // Batch z: this workgroup's matrices, partials and counters. No branch on
  // a kernel argument here: each one would serialize another round of
  // kernel-argument loads ahead of the first copy. (s_mul is 0 without a
  // multiplier; one split has no partials, so zs only keeps those pointers
  // unmoved.)
  {
    const int64_t z = blockIdx.z;
    A += z * sa;
    Bv = (const char *)Bv + z * sb * TBB;
    C += z * sc;
    epi.mul += z * s_mul;
    if constexpr (SPLIT) {
      const int64_t zs = gridDim.y > 1 ? z : 0;
      partials += zs * (int64_t)gridDim.y * M * N;
      counters += zs * gridDim.x * kCounterStride;
    }
  }

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // Wave-uniform (SGPR): the copies' LDS addresses derive from it.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int tiles_m = SPLIT ? (M + BM - 1) / BM : M / BM;

  // One tile's K range [k_begin, k_begin + k_len): partial `part` of the
  // tile's `parts` (a single part stores C directly).
  auto tile_body = [&](int tile, int tiles, int64_t k_begin, int64_t k_len,
                       int part, int parts) __attribute__((always_inline)) {
  int tm, tn;
  xcd_tile_order(tile, tiles, tiles_m, N / BN, 4, &tm, &tn);
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;

  // Copy side: lane -> (row in the wave's slab, physical chunk); the global
  // chunk it fetches is the logical chunk that belongs in that slot. The
  // address is a wave-uniform base plus a 32-bit lane offset.
  const int ld_row = lane / CH;
  const int ld_chunk =
      (lane % CH) ^ chunk_swizzle<CH>(wave * ROWS_PER_WAVE + ld_row);
  const int64_t lda_b = lda * (int64_t)sizeof(T);
  const int64_t ldb_b = ldb * (int64_t)TBB;
  // A row of each copy pass, clamped to the last row of A (split mode).
  uint32_t a_lane[A_PASSES];
  if constexpr (AT) {
    // Same copy shape as row-major B: lane -> (k row, swizzled chunk).
    const int krow = wave * A_RPW + lane / ACH;
    const int chunk = (lane % ACH) ^ nn_swizzle<kBNN16, MS>(krow);
#pragma unroll
    for (int p = 0; p < A_PASSES; ++p)
      a_lane[p] = (uint32_t)((p * A_RPP + krow) * lda_b + chunk * 16);
  } else {
#pragma unroll
  for (int p = 0; p < A_PASSES; ++p) {
    int64_t row = m0 + p * ROWS_PER_PASS + wave * ROWS_PER_WAVE + ld_row;
    if (SPLIT && row > M - 1)
      row = M - 1;
    a_lane[p] = (uint32_t)((row - m0) * lda_b + ld_chunk * 16);
  }
  }
  const char *a_base =
      AT ? (const char *)A + m0 * (int64_t)sizeof(T) + k_begin * lda_b
         : (const char *)A + m0 * lda_b + k_begin * (int64_t)sizeof(T);
  uint32_t b_lane;
  const char *b_base;
  uint32_t b_lane_p = 0;  // the SIMD partner's rows (kCopyPair)
  if constexpr (kNN) {
    const int krow = wave * B_RPW + lane / BCH;
    const int chunk = (lane % BCH) ^ nn_swizzle<BMODE, MS>(krow);
    b_lane = (uint32_t)(krow * ldb_b + chunk * 16);
    if constexpr (kCopyPair) {
      const int krow_p = krow + 4 * B_RPW;
      const int chunk_p = (lane % BCH) ^ nn_swizzle<BMODE, MS>(krow_p);
      b_lane_p = (uint32_t)(krow_p * ldb_b + chunk_p * 16);
    }
    b_base = (const char *)Bv + n0 * TBB + k_begin * ldb_b;
  } else {
    b_lane = (uint32_t)((wave * ROWS_PER_WAVE + ld_row) * ldb_b +
                        ld_chunk * 16);
    b_base = (const char *)Bv + n0 * ldb_b + k_begin * (int64_t)sizeof(T);
  }
  IHP_LDS char *lds = (IHP_LDS char *)smem;

  // Copy pass p of stage kt into `slot` (A passes first, then B passes):
  // this wave's rows, or with PARTNER those of wave + 4 (kCopyPair). A
  // partner's K-contiguous rows are 4 ROWS_PER_WAVE further (same chunk
  // swizzle: it repeats every 16 rows); its row-major B rows have their
  // own lane offset.
  auto load_pass = [&](int kt, int slot, int p, auto partner_c) {
    constexpr bool PARTNER = decltype(partner_c)::value;
    constexpr int DW = PARTNER ? 4 : 0;
    IHP_LDS char *dst = lds + slot * STAGE_BYTES;
    const int64_t ka = (int64_t)kt * BKB;
    if (p < A_PASSES) {
      if constexpr (AT)
        global_to_lds_16s(a_base + (int64_t)kt * KE * lda_b, a_lane[p],
                          dst + wave * A_RPW * AROW + p * A_RPP * AROW);
      else
        global_to_lds_16s(a_base + ka + (int64_t)DW * ROWS_PER_WAVE * lda_b,
                          a_lane[p],
                          dst + (wave + DW) * ROWS_PER_WAVE * BKB +
                              p * ROWS_PER_PASS * BKB);
    } else {
      const int q = p - A_PASSES;
      if constexpr (kNN) {
        const int64_t kb = (int64_t)kt * KE * ldb_b;
        global_to_lds_16s(b_base + kb + (int64_t)q * B_RPP * ldb_b,
                          PARTNER ? b_lane_p : b_lane,
                          dst + A_BYTES + (wave + DW) * B_RPW * BROW +
                              q * B_RPP * BROW);
      } else {
        global_to_lds_16s(b_base + ka + (int64_t)q * ROWS_PER_PASS * ldb_b +
                              (int64_t)DW * ROWS_PER_WAVE * ldb_b,
                          b_lane,
                          dst + A_BYTES + (wave + DW) * ROWS_PER_WAVE * BKB +
                              q * ROWS_PER_PASS * BKB);
      }
    }
  };
  // Passes [LO, HI) of stage kt (kCopyPair: wave row 0 issues both waves'
  // passes, wave row 1 none).
  auto load_passes = [&](auto lo, auto hi, int kt, int slot) {
    using Own = std::false_type;
    using Partner = std::true_type;
    if constexpr (kCopyPair) {
      if (wave < 4)
        static_for<decltype(hi)::value - decltype(lo)::value>([&](auto i) {
          load_pass(kt, slot, decltype(lo)::value + decltype(i)::value, Own());
          load_pass(kt, slot, decltype(lo)::value + decltype(i)::value,
                    Partner());
        });
    } else {
      static_for<decltype(hi)::value - decltype(lo)::value>([&](auto i) {
        load_pass(kt, slot, decltype(lo)::value + decltype(i)::value, Own());
      });
    }
  };
  using First = std::integral_constant<int, 0>;
  using All = std::integral_constant<int, LOADS_PER_STAGE>;

  // Read side, A (and TN B): lane reads row (lane % MS) of each MS-row
  // fragment, logical chunk KCH*ks + lane/MS of the staged row (the swizzle
  // repeats every 16 rows, so it depends on the row in the fragment only).
  const int rd_row = lane & (MS - 1);
  const int rd_sw = chunk_swizzle<CH>(rd_row) ^ (lane / MS);
  int koff[KSTEPS];
#pragma unroll
  for (int ks = 0; ks < KSTEPS; ++ks)
    koff[ks] = ((KCH * ks) ^ rd_sw) * 16;
  const int a_rd = (wm * WTM + rd_row) * BKB;
  const int b_rd = A_BYTES + (wn * WTN + rd_row) * BKB;
  // Read side, transposed A: the row-major B offsets below with M for N.
  int a_nn[FM];
  if constexpr (AT) {
    const int blk = lane >> 4, jj = lane & 15;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      // 32x32: block reads k rows 8 (blk / 2) + jj / 4, columns 16 (blk % 2)
      // + 4 (jj % 4) .. +3; 16x16: k rows 8 blk + jj / 4, columns 4 (jj % 4)
      const int k = MS == 32 ? 8 * (blk >> 1) + (jj >> 2) : 8 * blk + (jj >> 2);
      const int byte =
          2 * (wm * WTM + i * MS + (MS == 32 ? 16 * (blk & 1) : 0) +
               4 * (jj & 3));
      a_nn[i] = k * AROW +
                (((byte >> 4) ^ nn_swizzle<kBNN16, MS>(k)) << 4) + (byte & 15);
    }
  }
  // Read side, NN B: per-lane byte offset of fragment j within a stage for
  // K step 0 (a K step adds 16 rows; the swizzle repeats every 4 or 8).
  int b_nn[FN];
  if constexpr (kNN) {
    const int blk = lane >> 4, jj = lane & 15;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      // 32x32: the block's k rows start at 8 (blk / 2), its columns at
      // 16 (blk % 2); 16x16: k rows from 8 blk, all 16 columns.
      const int krow0 = MS == 32 ? 8 * (blk >> 1) : 8 * blk;
      const int col0 = wn * WTN + j * MS + (MS == 32 ? 16 * (blk & 1) : 0);
      if constexpr (BMODE == kBNN16) {
        // block reads k rows krow0 + jj/4 (+4), columns col0 + 4*(jj%4) ..
        // +3
        const int k = krow0 + (jj >> 2);
        const int byte = 2 * (col0 + 4 * (jj & 3));
        b_nn[j] = A_BYTES + k * BROW +
                  (((byte >> 4) ^ nn_swizzle<BMODE, MS>(k)) << 4) +
                  (byte & 15);
      } else if constexpr (BMODE == kBNN8) {
        // int8 MFMA: 16 k rows per block (k rows 16 (blk / 2) for 32x32,
        // 16 blk for 16x16), read as rows krow0 + jj/2 and krow0 + 8 + jj/2,
        // columns col0 + 8*(jj%2) .. +7 (bytes)
        const int k = (MS == 32 ? 16 * (blk >> 1) : 16 * blk) + (jj >> 1);
        const int byte = col0 + 8 * (jj & 1);
        b_nn[j] = A_BYTES + k * BROW +
                  (((byte >> 4) ^ nn_swizzle<BMODE, MS>(k)) << 4) +
                  (byte & 15);
      } else {
        // block reads k rows krow0 + jj/2, columns col0 + 8*(jj%2) .. +7
        // (bytes)
        const int k = krow0 + (jj >> 1);
        const int byte = col0 + 8 * (jj & 1);
        b_nn[j] = A_BYTES + k * BROW +
                  (((byte >> 4) ^ nn_swizzle<BMODE, MS>(k)) << 4) +
                  (byte & 15);
      }
    }
  }

  // Raw fragment registers: A (and TN B) 16 bytes; NN B two or one 8-byte
  // transposed reads.
  struct Frags {
    i32x4 a[FM];
    i32x4 b[FN];
    i32x2 t[kTwoReadB ? 2 * FN : FN];
    i32x2 ta[AT ? 2 * FM : 1];
  };
  auto read_frags = [&](int slot, int ks, Frags &f) {
    const IHP_LDS char *st = lds + slot * STAGE_BYTES;
    if constexpr (AT) {
      const IHP_LDS char *pa = st + ks * KROWS * AROW;
      static_for<FM>([&](auto i) {
        constexpr int I = decltype(i)::value;
        f.ta[2 * I] = lds_read_tr16_async<0>(pa + a_nn[I]);
        f.ta[2 * I + 1] = lds_read_tr16_async<4 * AROW>(pa + a_nn[I]);
      });
    } else {
      const IHP_LDS char *pa = st + a_rd + koff[ks];
      static_for<FM>([&](auto i) {
        f.a[i] = lds_read_16_async<decltype(i)::value * MS * BKB>(pa);
      });
    }
    if constexpr (BMODE == kBTN) {
      const IHP_LDS char *pb = st + b_rd + koff[ks];
      static_for<FN>([&](auto j) {
        f.b[j] = lds_read_16_async<decltype(j)::value * MS * BKB>(pb);
      });
    } else {
      const IHP_LDS char *pb = st + ks * KROWS * BROW;
      static_for<FN>([&](auto j) {
        constexpr int J = decltype(j)::value;
        if constexpr (BMODE == kBNN16) {
          f.t[2 * J] = lds_read_tr16_async<0>(pb + b_nn[J]);
          f.t[2 * J + 1] = lds_read_tr16_async<4 * BROW>(pb + b_nn[J]);
        } else if constexpr (BMODE == kBNN8) {
          f.t[2 * J] = lds_read_tr8_async<0>(pb + b_nn[J]);
          f.t[2 * J + 1] = lds_read_tr8_async<8 * BROW>(pb + b_nn[J]);
        } else {
          f.t[J] = lds_read_tr8_async<0>(pb + b_nn[J]);
        }
      });
    }
  };
  // Wait until at most N reads are outstanding, pin the fragments, and
  // assemble NN B operands from the transposed reads.
  auto frags_ready = [&](auto n, Frags &f) {
    lgkm_wait<decltype(n)::value>();
    if constexpr (AT) {
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        lgkm_tie2(f.ta[2 * i]);
        lgkm_tie2(f.ta[2 * i + 1]);
        f.a[i] = i32x4{f.ta[2 * i][0], f.ta[2 * i][1], f.ta[2 * i + 1][0],
                       f.ta[2 * i + 1][1]};
      }
    } else {
#pragma unroll
      for (int i = 0; i < FM; ++i)
        lgkm_tie(f.a[i]);
    }
    if constexpr (BMODE == kBTN) {
#pragma unroll
      for (int j = 0; j < FN; ++j)
        lgkm_tie(f.b[j]);
    } else if constexpr (kTwoReadB) {
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        lgkm_tie2(f.t[2 * j]);
        lgkm_tie2(f.t[2 * j + 1]);
        f.b[j] = i32x4{f.t[2 * j][0], f.t[2 * j][1], f.t[2 * j + 1][0],
                       f.t[2 * j + 1][1]};
      }
    } else {
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        lgkm_tie2(f.t[j]);
        f.b[j] = i8x8_to_f16x8(f.t[j]);
      }
    }
  };

  Acc acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < AR; ++r)
        acc[i][j][r] = 0;

  const int nk = (int)((k_len * (int64_t)sizeof(T)) / BKB);
  // Prologue: fill every slot of the ring, wait for stage 0.
#pragma unroll
  for (int s = 0; s < STAGES; ++s)
    if (s < nk)
      load_passes(First(), All(), s, s);
  if (STAGES - 1 < nk)
    wait_vmcnt<(STAGES - 1) * LOADS_PER_STAGE * CPM>();
  else
    wait_vmcnt<0>();
  block_barrier();

  Frags fr[2];
  read_frags(0, 0, fr[0]);

  // One stage. Per K step: issue the next step's fragment reads, wait only
  // for this step's (issued one step earlier), then this step's MFMAs, which
  // run while the new reads are in flight. The copies of stage kt+STAGES are
  // issued whole at the handoff (COPY): their addresses cost no vector
  // instructions, and issuing them in two halves, the second after the next
  // stage's first K step, measured ~1 % slower. The flags are compile-time
  // constants, so each phase of the K loop below is free of branches: with
  // them the loop-carried fragment registers had to be copied at every stage.
  auto stage = [&](int kt, auto copy, auto handoff, auto exact)
      __attribute__((always_inline)) {
    const int slot = kt % STAGES;
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      const int cur = ks & 1, nxt = cur ^ 1;
      if (ks + 1 < KSTEPS) {
        read_frags(slot, ks + 1, fr[nxt]);
        frags_ready(std::integral_constant<int, RDW>(), fr[cur]);
      } else if constexpr (decltype(handoff)::value) {
        // Stage handoff: this step's fragments are in registers (all LDS
        // reads done), stage kt+1 must have landed for every wave, and every
        // wave must be done reading stage kt before its slot is refilled
        // with stage kt+STAGES. With EXACT this wave has issued every copy
        // up to stage kt+STAGES-1, so stage kt+1 has landed once at most
        // STAGES-2 stages of copies remain in flight; otherwise wait for all.
        frags_ready(std::integral_constant<int, 0>(), fr[cur]);
        if constexpr (decltype(exact)::value)
          wait_vmcnt<(STAGES - 2) * LOADS_PER_STAGE * CPM>();
        else
          wait_vmcnt<0>();
        block_barrier();
        if constexpr (decltype(copy)::value)
          load_passes(First(), All(), kt + STAGES, slot);
        read_frags((kt + 1) % STAGES, 0, fr[nxt]);
      } else {
        frags_ready(std::integral_constant<int, 0>(), fr[cur]);
      }
      // Issue order. With 16x16 fragments and FN >= 4 the A index runs
      // innermost, boustrophedon, so the B operand changes once per FM
      // MFMAs and not on every one (the two waves of a SIMD hold the same B
      // fragments): fewer operand bits switch in the matrix core, which on
      // random data runs power-limited. Measured 1.5-2 % faster on the
      // 256x256 TN tiles, ~0.7 % slower on 256x128 NN (FN = 2).
      if constexpr (MS == 16 && FN >= 4) {
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int ii = 0; ii < FM; ++ii) {
            const int i = (j & 1) ? FM - 1 - ii : ii;
            acc[i][j] = kSwapAB
                            ? MF::mma(fr[cur].b[j], fr[cur].a[i], acc[i][j])
                            : MF::mma(fr[cur].a[i], fr[cur].b[j], acc[i][j]);
          }
      } else {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            acc[i][j] = kSwapAB
                            ? MF::mma(fr[cur].b[j], fr[cur].a[i], acc[i][j])
                            : MF::mma(fr[cur].a[i], fr[cur].b[j], acc[i][j]);
      }
    }
  };
  using Yes = std::true_type;
  using No = std::false_type;
  // Phases: a later stage to copy (kt < nk-STAGES); the first stage with
  // every copy issued (kt == nk-STAGES, still an exact wait); the rest with
  // a handoff; the last stage, without one.
  int kt = 0;
  for (; kt < nk - STAGES; ++kt)
    stage(kt, Yes(), Yes(), Yes());
  if (kt == nk - STAGES) {
    stage(kt, No(), Yes(), Yes());
    ++kt;
  }
  for (; kt < nk - 1; ++kt)
    stage(kt, No(), Yes(), No());
  if (kt < nk)
    stage(kt, No(), No(), No());

  // Epilogue: C_out = [C_init +] acc (W8A16: acc * scale[n]), one rounding
  // for f16 outputs. Lane l holds column l % MS of a fragment; register r
  // holds row row_l + frow(r).
  const int col_l = lane & (MS - 1);
  const int row_l = 4 * (lane / MS);
  auto frow = [](int r) { return MS == 32 ? 8 * (r >> 2) + (r & 3) : r; };
  // Position of accumulator element r of fragment (i, j) in the wave tile.
  auto fr_row = [&](int i, int r) {
    return kSwapAB ? i * MS + (lane & 15) : i * MS + row_l + frow(r);
  };
  auto fr_col = [&](int j, int r) {
    return kSwapAB ? j * MS + 4 * (lane >> 4) + r : j * MS + col_l;
  };
  constexpr bool kIntOut = std::is_same<OutT, int32_t>::value;
  if constexpr (kSwapAB && kIntOut) {
    // Transposed fragments: lane l holds C[row l % 16][4 (l / 16) .. +3] of
    // each 16 x 16 fragment, so every fragment is one 16-byte store per
    // lane (16 rows x 64 bytes per instruction), no LDS staging. Per-element
    // stores serve accumulation and a C or pitch not 16-byte aligned.
    const int64_t r0 = m0 + wm * WTM + (lane & 15);
    const int64_t c0 = n0 + wn * WTN + 4 * (lane >> 4);
    const bool vec = store_mode != kStoreAccumulate &&
                     (uintptr_t)C % 16 == 0 && ldc % 4 == 0;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        OutT *dst = C + (r0 + i * MS) * ldc + c0 + j * MS;
        if (vec) {
          if (store_mode == kStoreThrough)
            store_through16(dst, acc[i][j]);
          else
            *(i32x4 *)dst = acc[i][j];
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            store_out(dst + r, acc[i][j][r], store_mode);
        }
      }
    return;
  }
  if constexpr (!kIntOut) {
    if ((!SPLIT || parts == 1) && !epi_plain(epi)) {
      // Fused epilogue: each 32-row fragment band of a wave goes through
      // LDS (the idle stage ring) column-major with a 33-float pitch, then
      // one rolled loop applies scale / bias / activation / multiplier and
      // stores whole rows, so the epilogue is instanced once per band
      // instead of once per accumulator register.
      constexpr int PITCH = MS + 1;
      static_assert(WM * WN * WTN * PITCH * 4 <= STAGES * STAGE_BYTES,
                    "epilogue staging");
      float *stage = (float *)smem + wave * WTN * PITCH;
      const int64_t row0 = m0 + wm * WTM, col0 = n0 + wn * WTN;
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        __syncthreads();  // LDS ring (or the previous band) fully read
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int r = 0; r < AR; ++r)
            if constexpr (kSwapAB)
              stage[fr_col(j, r) * PITCH + (lane & 15)] = (float)acc[i][j][r];
            else
              stage[(j * MS + col_l) * PITCH + row_l + frow(r)] =
                  (float)acc[i][j][r];
        __syncthreads();
        for (int t = lane; t < MS * WTN; t += 64) {
          const int rr = t / WTN, cc = t % WTN;
          const int64_t row = row0 + i * MS + rr, col = col0 + cc;
          if (SPLIT && row >= M)
            continue;
          float v = stage[cc * PITCH + rr];
          if constexpr (BMODE == kBW8)
            v *= (float)scale[col];
          store_out(C + row * ldc + col, epi_apply(v, row, col, epi),
                    store_mode);
        }
      }
      return;
    }
  }
  // Full tiles, plain or written-through stores: each wave stages its
  // WTM x WTN tile through its share of the idle LDS ring and stores whole
  // 16-byte row chunks, a quarter of the store instructions of one store
  // per accumulator element (issuing those took 4-7 us of the int8 4096^3
  // kernel) and full row segments. 16-byte chunks are XOR-swizzled by row,
  // so the fragment writes (16 lanes per row) and the chunk reads are
  // conflict free. Needs a 16-byte aligned C and row pitch; otherwise, and
  // when accumulating (one rounding of C_init + acc), the per-element
  // stores below run.
  if constexpr (!SPLIT && MS * WTN * sizeof(OutT) <=
                              STAGES * STAGE_BYTES / (WM * WN)) {
    constexpr int OB = (int)sizeof(OutT);
    constexpr int ROWB = WTN * OB;  // bytes of one wave-tile row
    constexpr int NCH = ROWB / 16;  // 16-byte chunks per row
    constexpr int SHARE = STAGES * STAGE_BYTES / (WM * WN);
    // fragment rows per band: the most that divide FM and fit the share
    constexpr int BAND = [] {
      int f = FM;
      while (f > 1 && (f * MS * ROWB > SHARE || FM % f != 0))
        --f;
      return f;
    }();
    static_assert(NCH >= 1 && (NCH & (NCH - 1)) == 0, "row chunks");
    if (store_mode != kStoreAccumulate && (uintptr_t)C % 16 == 0 &&
        ((int64_t)ldc * OB) % 16 == 0) {
      __syncthreads();  // every wave is done reading the ring
      char *ws = smem + wave * SHARE;
      const int64_t grow0 = m0 + wm * WTM, gcol0 = n0 + wn * WTN;
#pragma unroll
      for (int b = 0; b < FM; b += BAND) {
#pragma unroll
        for (int i = b; i < b + BAND; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j) {
            float sc = 1.0f;
            if constexpr (BMODE == kBW8)
              sc = (float)scale[gcol0 + j * MS + col_l];
            if constexpr (kSwapAB && !kIntOut) {
              // four consecutive columns of one row: one 8- or 16-byte write
              const int row = (i - b) * MS + (lane & 15);
              const int byte = fr_col(j, 0) * OB;
              const int off = row * ROWB +
                              (((byte >> 4) ^ (row & (NCH - 1))) << 4) +
                              (byte & 15);
              if constexpr (std::is_same<OutT, float>::value) {
                *(f32x4 *)(ws + off) = acc[i][j];
              } else {
                f16x4 h;
#pragma unroll
                for (int r = 0; r < 4; ++r)
                  h[r] = (f16)acc[i][j][r];
                *(f16x4 *)(ws + off) = h;
              }
              continue;
            }
#pragma unroll
            for (int r = 0; r < AR; ++r) {
              const int row = (i - b) * MS + row_l + frow(r);
              const int byte = (j * MS + col_l) * OB;
              const int off = row * ROWB +
                              (((byte >> 4) ^ (row & (NCH - 1))) << 4) +
                              (byte & 15);
              if constexpr (kIntOut) {
                *(OutT *)(ws + off) = acc[i][j][r];
              } else {
                float v = (float)acc[i][j][r];
                if constexpr (BMODE == kBW8)
                  v *= sc;
                *(OutT *)(ws + off) = (OutT)v;
              }
            }
          }
        for (int t = lane; t < BAND * MS * NCH; t += 64) {
          const int row = t / NCH, ch = t % NCH;
          const i32x4 v = *(const i32x4 *)(
              ws + row * ROWB + ((ch ^ (row & (NCH - 1))) << 4));
          char *dst = (char *)(C + (grow0 + b * MS + row) * ldc + gcol0) +
                      ch * 16;
          if (store_mode == kStoreThrough)
            store_through16(dst, v);
          else
            *(i32x4 *)dst = v;
        }
      }
      return;
    }
  }
  // One split (a ragged-M shape whose tiles alone cover the CUs): store
  // directly, rows past M masked, no partials.
  if (!SPLIT || parts == 1) {
    if constexpr (kIntOut && !SPLIT) {
      // Large i32 outputs: written through past the L2, tested once here.
      if (store_mode == kStoreThrough) {
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          OutT *crow = C + (m0 + wm * WTM + i * MS + row_l) * ldc + n0 +
                       wn * WTN + col_l;
#pragma unroll
          for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < AR; ++r)
              store_through(crow + frow(r) * ldc + j * MS, acc[i][j][r]);
        }
        return;
      }
    }
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      OutT *crow = C + (m0 + wm * WTM + i * MS + row_l) * ldc + n0 +
                   wn * WTN + col_l;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        float sc = 1.0f;
        if constexpr (BMODE == kBW8)
          sc = (float)scale[n0 + wn * WTN + j * MS + col_l];
#pragma unroll
        for (int r = 0; r < AR; ++r) {
          OutT *dst = kSwapAB ? C + (m0 + wm * WTM + fr_row(i, r)) * ldc + n0 +
                                    wn * WTN + fr_col(j, r)
                              : crow + frow(r) * ldc + j * MS;
          const int64_t row = m0 + wm * WTM + fr_row(i, r);
          if (SPLIT && row >= M)
            continue;
          if constexpr (kIntOut) {
            store_out(dst, acc[i][j][r], store_mode);
          } else {
            float v = (float)acc[i][j][r];
            if constexpr (BMODE == kBW8)
              v *= sc;
            store_out(dst, v, store_mode);
          }
        }
      }
    }
  } else {
    typedef typename MF::AccScalar P;
    // Publish this split's partial tile (rows < M only) with device-scope
    // stores; the last workgroup of the tile reads them with device-scope
    // loads. Only partials and the counter are shared, so no L2 write-back /
    // invalidate fence is needed, only the stores drained before arriving.
    P *part_out = partials + (int64_t)part * M * N;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int64_t col = n0 + wn * WTN + j * MS + col_l;
#pragma unroll
        for (int r = 0; r < AR; ++r) {
          const int64_t row = m0 + wm * WTM + i * MS + row_l + frow(r);
          if (row < M)
            store_device(part_out + row * N + col, (P)acc[i][j][r]);
        }
      }
    }
    // The LDS ring is idle once every wave passed the barrier below; its
    // first word carries the arrival result to the workgroup.
    unsigned *last_split = (unsigned *)smem;
    wait_vmcnt<0>();
    __syncthreads();
    if (tid == 0) {
      const unsigned prev =
          __hip_atomic_fetch_add(&counters[tile * kCounterStride], 1u,
                                 __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
      *last_split = prev == (unsigned)parts - 1;
    }
    __syncthreads();
    if (!*last_split)
      return;
    // The tile's valid rows, G elements per thread at a time, each summed
    // over the splits in split order: G x SB device-scope loads in flight
    // per wait instead of one element's splits.
    const int splits = parts;
    const int rows_valid = (int)(M - m0 < BM ? M - m0 : BM);
    const int count = rows_valid * BN;
    // L device-scope loads in flight per wait (64, or 32 where 512 threads
    // leave 256 registers a lane): SB split slots for each of G = L / SB
    // elements, SB the smallest of 2, 4, 8 that covers the splits (more
    // splits loop in steps of 8). Each element is summed in split order
    // whatever SB is. The epilogue choice is made once, outside the loop: a
    // per-element test of the epilogue fields costs the plain reduction ~10%.
    constexpr int L = NT > 256 ? 32 : 64;
    auto reduce = [&](auto with_epi, auto sb) {
      constexpr int SB = decltype(sb)::value;
      constexpr int G = L / SB;
      for (int base = 0; base < count; base += NT * G) {
        P sum[G];
#pragma unroll
        for (int e = 0; e < G; ++e)
          sum[e] = 0;
        for (int s0 = 0; s0 < splits; s0 += SB) {
          P v[G][SB];
#pragma unroll
          for (int e = 0; e < G; ++e) {
            const int idx = base + e * NT + tid;
            const int64_t row = m0 + idx / BN, col = n0 + idx % BN;
            const P *src = partials + ((int64_t)s0 * M + row) * N + col;
#pragma unroll
            for (int u = 0; u < SB; ++u)
              v[e][u] = idx < count && s0 + u < splits
                            ? load_device(src + (int64_t)u * M * N)
                            : (P)0;
          }
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
          for (int e = 0; e < G; ++e)
#pragma unroll
            for (int u = 0; u < SB; ++u) {
              vm_tie(v[e][u]);
              sum[e] += v[e][u];
            }
        }
#pragma unroll
        for (int e = 0; e < G; ++e) {
          const int idx = base + e * NT + tid;
          if (idx >= count)
            continue;
          const int64_t row = m0 + idx / BN, col = n0 + idx % BN;
          if constexpr (kIntOut) {
            store_out(C + row * ldc + col, sum[e], store_mode);
          } else {
            float v = (float)sum[e];
            if constexpr (BMODE == kBW8)
              v *= (float)scale[col];
            if constexpr (decltype(with_epi)::value)
              v = epi_apply(v, row, col, epi);
            store_out(C + row * ldc + col, v, store_mode);
          }
        }
      }
    };
    auto reduce_sb = [&](auto with_epi) {
      if (splits <= 2)
        reduce(with_epi, std::integral_constant<int, 2>());
      else if (splits <= 4)
        reduce(with_epi, std::integral_constant<int, 4>());
      else
        reduce(with_epi, std::integral_constant<int, 8>());
    };
    if (kIntOut || epi_plain(epi))
      reduce_sb(std::false_type());
    else
      reduce_sb(std::true_type());
    if (tid == 0)  // re-arm for the next call on this workspace
      __hip_atomic_store(&counters[tile * kCounterStride], 0u,
                         __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }
  };

  const int tiles = tiles_m * (N / BN);
  if (!SPLIT || sk_steps == 0) {
    // One tile per workgroup; split-K: K split `blockIdx.y` of gridDim.y.
    const int64_t k_begin = SPLIT ? (int64_t)blockIdx.y * k_split : 0;
    const int64_t k_len =
        SPLIT ? (K - k_begin < k_split ? K - k_begin : k_split) : K;
    tile_body((int)blockIdx.x, (int)gridDim.x, k_begin, k_len,
              SPLIT ? (int)blockIdx.y : 0, SPLIT ? (int)gridDim.y : 1);
    return;
  }
  if constexpr (SPLIT) {
    // Stream-K: the (tile, K stage) pairs in tile order are cut into runs of
    // sk_steps stages, one run per workgroup. The runs of one XCD's
    // workgroups are consecutive (workgroups go to XCDs round-robin), so a
    // tile's contributors mostly share an L2. A run covers the end of one
    // tile, whole tiles, and the start of another; a tile covered by c runs
    // gets partials 0 .. c-1 in K order, summed in that order by the last
    // to arrive.
    const int ksteps = (int)(K / KE);
    const int nwg = (int)gridDim.x, w = (int)blockIdx.x;
    const int run = nwg % 8 == 0 ? (w % 8) * (nwg / 8) + w / 8 : w;
    const int64_t total = (int64_t)tiles * ksteps;
    int64_t g = (int64_t)run * sk_steps;
    const int64_t g_end = g + sk_steps < total ? g + sk_steps : total;
    while (g < g_end) {
      const int tile = (int)(g / ksteps);
      const int64_t t0 = (int64_t)tile * ksteps;
      const int a = (int)(g - t0);
      const int b = g_end - t0 < ksteps ? (int)(g_end - t0) : ksteps;
      const int c0 = (int)(t0 / sk_steps);
      const int c1 = (int)((t0 + ksteps - 1) / sk_steps);
      // tile order without the XCD remap (the runs already follow the XCDs)
      tile_body(tile, 1, (int64_t)a * KE, (int64_t)(b - a) * KE, run - c0,
                c1 - c0 + 1);
      g = t0 + b;
      if (g < g_end)
        __syncthreads();  // the next tile's copies reuse the LDS ring
    }
  }
}

// ----------------------------------------------------------------------------
// General path: any extents, strides, A and B layout; bounds-checked element
// loads staged through registers into LDS (B converted to the MFMA input type
// on the way, which is where W8A16 dequantizes), 64x64 tiles, 4 waves of
// 32x32 fragments, optional per-column scale in the epilogue.
// ----------------------------------------------------------------------------

template <typename TA, typename TB, typename OutT, bool kScale>
__global__ __launch_bounds__(256) void gemm_general_kernel(
    const TA *__restrict__ A, const TB *__restrict__ B, OutT *__restrict__ C,
    const f16 *__restrict__ scale, int M, int N, int K, int64_t lda,
    int64_t ldb, int64_t ldc, int b_transposed, int accumulate, int64_t sa,
    int64_t sb, int64_t sc, Epi epi, int64_t s_mul, int a_transposed) {
  {
    const int64_t z = blockIdx.z;
    A += z * sa;
    B += z * sb;
    C += z * sc;
    epi.mul += z * s_mul;  // s_mul is 0 without a multiplier
  }
  // MFMA input type: f16 unless both operands are int8.
  typedef typename MfmaInput<TA, TB>::type TM;
  typedef Mfma32<TM> MF;
  constexpr int KE = 64 / (int)sizeof(TM);  // K elements per 64-byte slab
  constexpr int ROWB = 64 + 16;             // padded staged row (bytes)
  __shared__ __attribute__((aligned(16))) char As[64 * ROWB];
  __shared__ __attribute__((aligned(16))) char Bs[64 * ROWB];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t m0 = (int64_t)blockIdx.y * 64, n0 = (int64_t)blockIdx.x * 64;
  typename MF::Acc acc;
#pragma unroll
  for (int r = 0; r < 16; ++r)
    acc[r] = 0;

  constexpr int EPT = 16 / (int)sizeof(TM);  // elements per thread per slab
  const int ld_r = tid / 4, ld_c = (tid % 4) * EPT;

  for (int k0 = 0; k0 < K; k0 += KE) {
    if (!a_transposed) {  // A rows are M
      TM *dst = (TM *)(As + ld_r * ROWB) + ld_c;
      const int64_t m = m0 + ld_r;
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        const int k = k0 + ld_c + e;
        dst[e] = (m < M && k < K) ? (TM)A[m * lda + k] : (TM)0;
      }
    } else {  // A [K,M]: m fastest across threads, staged transposed
      const int mm = tid & 63, kq = tid >> 6;
      constexpr int KPT = KE / 4;
      TM *dst = (TM *)(As + mm * ROWB) + kq * KPT;
      const int64_t m = m0 + mm;
#pragma unroll
      for (int e = 0; e < KPT; ++e) {
        const int k = k0 + kq * KPT + e;
        dst[e] = (m < M && k < K) ? (TM)A[(int64_t)k * lda + m] : (TM)0;
      }
    }
    if (b_transposed) {  // B rows are N
      TM *dst = (TM *)(Bs + ld_r * ROWB) + ld_c;
      const int64_t n = n0 + ld_r;
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        const int k = k0 + ld_c + e;
        dst[e] = (n < N && k < K) ? (TM)B[n * ldb + k] : (TM)0;
      }
    } else {  // B [K,N]: n fastest across threads, staged transposed
      const int nn = tid & 63, kq = tid >> 6;
      constexpr int KPT = KE / 4;
      TM *dst = (TM *)(Bs + nn * ROWB) + kq * KPT;
      const int64_t n = n0 + nn;
#pragma unroll
      for (int e = 0; e < KPT; ++e) {
        const int k = k0 + kq * KPT + e;
        dst[e] = (n < N && k < K) ? (TM)B[(int64_t)k * ldb + n] : (TM)0;
      }
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int ch = 2 * ks + (lane >> 5);
      i32x4 af = *(const i32x4 *)(As + (wm * 32 + (lane & 31)) * ROWB + ch * 16);
      i32x4 bf = *(const i32x4 *)(Bs + (wn * 32 + (lane & 31)) * ROWB + ch * 16);
      acc = MF::mma(af, bf, acc);
    }
    __syncthreads();
  }

  const int64_t col = n0 + wn * 32 + (lane & 31);
  if (col >= N)
    return;
  float s = 1.0f;
  if (kScale)
    s = (float)scale[col];
  const int mode = accumulate ? kStoreAccumulate : kStorePlain;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int64_t row = m0 + wm * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
    if (row < M) {
      if constexpr (std::is_same<OutT, int32_t>::value) {
        store_out(C + row * ldc + col, acc[r], mode);
      } else {
        float v = (float)acc[r];
        if (kScale)
          v *= s;
        store_out(C + row * ldc + col, epi_apply(v, row, col, epi), mode);
      }
    }
  }
}

// ----------------------------------------------------------------------------
// Host launchers.
// ----------------------------------------------------------------------------

template <typename T, typename OutT, int BM, int BN, int BKB, int WM, int WN,
          int STAGES, int BMODE, bool SPLIT, bool AT, int MS = 32>
static hipError_t launch_fast(const MatmulArgs &a) {
  typedef typename Mfma32<T>::AccScalar P;
  const int64_t tiles_m = SPLIT ? (a.m + BM - 1) / BM : a.m / BM;
  const int tiles = (int)(tiles_m * (a.n / BN));
  const int splits = SPLIT ? a.splits : 1;
  const int k_split = SPLIT ? a.k_split : (int)a.k;
  unsigned *counters = SPLIT ? (unsigned *)a.workspace : nullptr;
  P *partials = SPLIT ? (P *)((char *)a.workspace +
                              split_counter_bytes(tiles))
                      : nullptr;
  const bool stream_k = SPLIT && a.sk_steps > 0;
  const dim3 grid = stream_k ? dim3((unsigned)a.sk_workgroups, 1, 1)
                             : dim3(tiles, splits, (unsigned)a.batch);
  const int store_mode =
      a.accumulate ? kStoreAccumulate
      : !SPLIT &&
              a.m * a.n * a.batch * (int64_t)sizeof(OutT) >= kStoreThroughBytes
          ? kStoreThrough
          : kStorePlain;
  hipLaunchKernelGGL(
      (gemm_lds_kernel<T, OutT, BM, BN, BKB, WM, WN, STAGES, BMODE, SPLIT,
                       AT, MS>),
      grid, dim3(64 * WM * WN), 0, (hipStream_t)a.stream, (const T *)a.a, a.b,
      (OutT *)a.c, (const f16 *)a.scale, (int)a.m, (int)a.n, (int)a.k, a.lda,
      a.ldb, a.ldc, store_mode, k_split, stream_k ? a.sk_steps : 0,
      partials, counters, a.sa, a.sb, a.sc, make_epi(a), epi_batch_stride(a));
  return hipGetLastError();
}

// Column split: the head configuration's grid over columns [0, n_head),
// whole rounds of the chip's CUs, then the tail configuration's grid over
// the rest, as two launches on the caller's stream. The tail launch sees a
// plain M x (N - n_head) product: every column-indexed operand (B, C, the
// W8A16 scale, the epilogue's bias and multiplier) starts n_head columns
// on, pitches unchanged. Each output element is computed by one tile of
// either grid in the same K order, so the result is that of the head
// configuration alone.
template <typename T, typename OutT, int BMODE, FastLaunchFn HEAD,
          FastLaunchFn TAIL, int HBM, int HBN, int TBM, int TBN>
static hipError_t launch_column_split(const MatmulArgs &a) {
  const int64_t n_head =
      column_split_head(a.m, a.n, HBM, HBN, TBM, TBN, kColumnSplitCus);
  if (n_head <= 0 || a.batch != 1)
    return hipErrorInvalidValue;
  MatmulArgs h = a;
  h.n = n_head;
  const hipError_t e = HEAD(h);
  if (e != hipSuccess)
    return e;
  constexpr int64_t TBB = BMODE == kBW8 ? 1 : (int64_t)sizeof(T);
  MatmulArgs t = a;
  t.n = a.n - n_head;
  t.b = (const char *)a.b + (BMODE == kBTN ? n_head * a.ldb : n_head) * TBB;
  t.c = (OutT *)a.c + n_head;
  if (a.scale)
    t.scale = (const f16 *)a.scale + n_head;
  if (a.bias)
    t.bias = (const f16 *)a.bias + n_head;
  if (a.mul)
    t.mul = (const f16 *)a.mul + n_head;
  return TAIL(t);
}

#define IHP_FAST_CONFIG(NAME, MODE, T, OUT, BM, BN, BKB, WM, WN, ST)           \
  IHP_FAST_CONFIG_X(NAME, MODE, T, OUT, BM, BN, BKB, WM, WN, ST, false, false, 32)
#define IHP_FAST_CONFIG_16(NAME, MODE, T, OUT, BM, BN, BKB, WM, WN, ST)        \
  IHP_FAST_CONFIG_X(NAME, MODE, T, OUT, BM, BN, BKB, WM, WN, ST, false, false, 16)
#define IHP_FAST_CONFIG_S(NAME, MODE, T, OUT, BM, BN, BKB, WM, WN, ST, SPLIT)  \
  IHP_FAST_CONFIG_X(NAME, MODE, T, OUT, BM, BN, BKB, WM, WN, ST, SPLIT, false, 32)
#define IHP_FAST_CONFIG_AT(NAME, MODE, T, OUT, BM, BN, BKB, WM, WN, ST)        \
  IHP_FAST_CONFIG_X(NAME, MODE, T, OUT, BM, BN, BKB, WM, WN, ST, false, true, 32)
#define IHP_FAST_CONFIG_AT16(NAME, MODE, T, OUT, BM, BN, BKB, WM, WN, ST)      \
  IHP_FAST_CONFIG_X(NAME, MODE, T, OUT, BM, BN, BKB, WM, WN, ST, false, true, 16)
#define IHP_FAST_CONFIG_X(NAME, MODE, T, OUT, BM, BN, BKB, WM, WN, ST, SPLIT,  \
                          AT, MS)                                             \
  IHP_FAST_CONFIG_XT(NAME, MODE, T, OUT, BM, BN, BKB, WM, WN, ST, SPLIT, AT,  \
                     MS, 0)
// A split-K configuration the planner takes only from its measured table.
#define IHP_FAST_CONFIG_S_TABLE(NAME, MODE, T, OUT, BM, BN, BKB, WM, WN, ST)   \
  IHP_FAST_CONFIG_XT(NAME, MODE, T, OUT, BM, BN, BKB, WM, WN, ST, true, false, \
                     32, 1)
#define IHP_FAST_CONFIG_XT(NAME, MODE, T, OUT, BM, BN, BKB, WM, WN, ST, SPLIT, \
                           AT, MS, TABLE)                                     \
  {NAME,                                                                      \
   MODE,                                                                      \
   SPLIT,                                                                     \
   AT,                                                                        \
   (const void *)&gemm_lds_kernel<T, OUT, BM, BN, BKB, WM, WN, ST, MODE,      \
                                  SPLIT, AT, MS>,                             \
   sizeof(T) == 1 ? kElemI8 : kElemF16,                                       \
   sizeof(OUT) == 4 && sizeof(T) == 2,                                        \
   BM,                                                                        \
   BN,                                                                        \
   BKB / (int)sizeof(T),                                                      \
   64 * WM * WN,                                                              \
   ST,                                                                        \
   ST * (BM * BKB + (MODE == kBTN ? BN * BKB                                  \
                                  : (BKB / (int)sizeof(T)) * BN *             \
                                        (MODE == kBW8 ? 1 : (int)sizeof(T)))),\
   &launch_fast<T, OUT, BM, BN, BKB, WM, WN, ST, MODE, SPLIT, AT, MS>,      \
   MS,                                                                        \
   TABLE}

// A column split of two listed 8-wave configurations (head H*, tail T*,
// both unsplit, one K stage size, one type and B form prefix PRE), named
// "<head>+<tail without PRE>" (within the plan's 63-character name). Its
// tile is the head's rows by the tail's columns (the shape's
// divisibility), its LDS the head's (the larger ring), its kernel entry
// the head's.
#define IHP_COLUMN_SPLIT(PRE, HEAD, TAIL, MODE, T, OUT, BKB, AT, HBM, HBN,    \
                         HST, HMS, TBM, TBN, TST, TMS)                        \
  {PRE HEAD "+" TAIL,                                                         \
   MODE,                                                                      \
   false,                                                                     \
   AT,                                                                        \
   (const void *)&gemm_lds_kernel<T, OUT, HBM, HBN, BKB, 2, 4, HST, MODE,     \
                                  false, AT, HMS>,                            \
   sizeof(T) == 1 ? kElemI8 : kElemF16,                                       \
   sizeof(OUT) == 4 && sizeof(T) == 2,                                        \
   HBM,                                                                       \
   TBN,                                                                       \
   BKB / (int)sizeof(T),                                                      \
   512,                                                                       \
   HST,                                                                       \
   HST * (HBM * BKB + (MODE == kBTN ? HBN * BKB                               \
                                    : (BKB / (int)sizeof(T)) * HBN *          \
                                          (MODE == kBW8 ? 1                   \
                                                        : (int)sizeof(T)))),  \
   &launch_column_split<                                                      \
       T, OUT, MODE,                                                          \
       &launch_fast<T, OUT, HBM, HBN, BKB, 2, 4, HST, MODE, false, AT, HMS>,  \
       &launch_fast<T, OUT, TBM, TBN, BKB, 2, 4, TST, MODE, false, AT, TMS>,  \
       HBM, HBN, TBM, TBN>,                                                   \
   HMS,                                                                       \
   0,                                                                         \
   PRE HEAD,                                                                  \
   PRE TAIL}

// Every compiled fast-path configuration (none spills registers: the
// 4-wave 256x256 tiles, 128 x 128 per wave, did and were dropped). The
// planner picks among these by
// its LDS-budget ranking or a measured table entry; bench.py --tune times
// them. Names: <types>_<b form>_<BM>x<BN>x<BK in elements>_w<wave grid>_s<LDS
// stages>.
static const FastConfig kFastConfigs[] = {
    IHP_FAST_CONFIG("i8_tn_256x256x128_w2x4_s2", kBTN, int8_t, int32_t, 256, 256, 128, 2, 4, 2),
    IHP_FAST_CONFIG("i8_tn_256x256x64_w2x4_s4", kBTN, int8_t, int32_t, 256, 256, 64, 2, 4, 4),
    IHP_FAST_CONFIG("i8_tn_256x128x128_w2x4_s2", kBTN, int8_t, int32_t, 256, 128, 128, 2, 4, 2),
    IHP_FAST_CONFIG("i8_tn_128x128x128_w2x2_s4", kBTN, int8_t, int32_t, 128, 128, 128, 2, 2, 4),
    IHP_FAST_CONFIG("f16_tn_256x256x64_w2x4_s2", kBTN, f16, f16, 256, 256, 128, 2, 4, 2),
    IHP_FAST_CONFIG("f16_tn_256x256x32_w2x4_s4", kBTN, f16, f16, 256, 256, 64, 2, 4, 4),
    IHP_FAST_CONFIG("f16_tn_256x128x64_w2x4_s2", kBTN, f16, f16, 256, 128, 128, 2, 4, 2),
    IHP_FAST_CONFIG("f16_tn_128x128x64_w2x2_s4", kBTN, f16, f16, 128, 128, 128, 2, 2, 4),
    IHP_FAST_CONFIG("f16f32_tn_256x256x64_w2x4_s2", kBTN, f16, float, 256, 256, 128, 2, 4, 2),
    IHP_FAST_CONFIG("f16f32_tn_128x128x64_w2x2_s4", kBTN, f16, float, 128, 128, 128, 2, 2, 4),
    // 16x16 MFMA forms of the TN macro-tiles
    IHP_FAST_CONFIG_16("i8_tn_256x256x128_w2x4_s2_m16", kBTN, int8_t, int32_t, 256, 256, 128, 2, 4, 2),
    IHP_FAST_CONFIG_16("i8_tn_256x128x128_w2x4_s2_m16", kBTN, int8_t, int32_t, 256, 128, 128, 2, 4, 2),
    IHP_FAST_CONFIG_16("f16_tn_256x256x64_w2x4_s2_m16", kBTN, f16, f16, 256, 256, 128, 2, 4, 2),
    IHP_FAST_CONFIG_16("f16_tn_256x128x64_w2x4_s2_m16", kBTN, f16, f16, 256, 128, 128, 2, 4, 2),
    IHP_FAST_CONFIG_16("f16f32_tn_256x256x64_w2x4_s2_m16", kBTN, f16, float, 256, 256, 128, 2, 4, 2),
    IHP_FAST_CONFIG_16("f16f32_tn_256x128x64_w2x4_s2_m16", kBTN, f16, float, 256, 128, 128, 2, 4, 2),
    IHP_FAST_CONFIG("f16_nn_256x256x64_w2x4_s2", kBNN16, f16, f16, 256, 256, 128, 2, 4, 2),
    IHP_FAST_CONFIG("f16_nn_256x128x64_w2x4_s2", kBNN16, f16, f16, 256, 128, 128, 2, 4, 2),
    IHP_FAST_CONFIG("f16_nn_128x128x64_w2x2_s4", kBNN16, f16, f16, 128, 128, 128, 2, 2, 4),
    IHP_FAST_CONFIG("f16f32_nn_256x256x64_w2x4_s2", kBNN16, f16, float, 256, 256, 128, 2, 4, 2),
    IHP_FAST_CONFIG("f16f32_nn_128x128x64_w2x2_s4", kBNN16, f16, float, 128, 128, 128, 2, 2, 4),
    IHP_FAST_CONFIG("w8a16_nn_256x256x64_w2x4_s3", kBW8, f16, f16, 256, 256, 128, 2, 4, 3),
    IHP_FAST_CONFIG("w8a16_nn_128x256x64_w2x4_s4", kBW8, f16, f16, 128, 256, 128, 2, 4, 4),
    IHP_FAST_CONFIG("w8a16_nn_128x256x64_w2x2_s4", kBW8, f16, f16, 128, 256, 128, 2, 2, 4),
    // 16x16 MFMA forms of the row-major f16 B macro-tiles (the W8A16 ones
    // measured 0-5 % slower than their 32x32 forms and are not built)
    IHP_FAST_CONFIG_16("f16_nn_256x256x64_w2x4_s2_m16", kBNN16, f16, f16, 256, 256, 128, 2, 4, 2),
    IHP_FAST_CONFIG_16("f16_nn_256x128x64_w2x4_s2_m16", kBNN16, f16, f16, 256, 128, 128, 2, 4, 2),
    IHP_FAST_CONFIG_16("f16f32_nn_256x256x64_w2x4_s2_m16", kBNN16, f16, float, 256, 256, 128, 2, 4, 2),
    IHP_FAST_CONFIG_16("f16f32_nn_256x128x64_w2x4_s2_m16", kBNN16, f16, float, 256, 128, 128, 2, 4, 2),
    // split-K skinny tiles (M < tile rows allowed; partials in workspace)
    // (measured on M = 16..128 with N, K in {4096, 11008}: 32x128 beats
    // 32x256 / 64x256 at every point, 64x128 is best for some M = 64..128)
    IHP_FAST_CONFIG_S("f16_nn_32x128x64_w1x4_s4_sk", kBNN16, f16, f16, 32, 128, 128, 1, 4, 4, true),
    IHP_FAST_CONFIG_S("f16_nn_64x128x64_w2x2_s4_sk", kBNN16, f16, f16, 64, 128, 128, 2, 2, 4, true),
    IHP_FAST_CONFIG_S("f16_nn_128x128x64_w2x2_s4_sk", kBNN16, f16, f16, 128, 128, 128, 2, 2, 4, true),
    IHP_FAST_CONFIG_S("f16f32_nn_32x128x64_w1x4_s4_sk", kBNN16, f16, float, 32, 128, 128, 1, 4, 4, true),
    IHP_FAST_CONFIG_S("f16_tn_32x128x64_w1x4_s4_sk", kBTN, f16, f16, 32, 128, 128, 1, 4, 4, true),
    IHP_FAST_CONFIG_S("f16_tn_128x128x64_w2x2_s4_sk", kBTN, f16, f16, 128, 128, 128, 2, 2, 4, true),
    IHP_FAST_CONFIG_S("w8a16_nn_32x256x64_w1x4_s4_sk", kBW8, f16, f16, 32, 256, 128, 1, 4, 4, true),
    IHP_FAST_CONFIG_S("w8a16_nn_128x256x64_w2x4_s4_sk", kBW8, f16, f16, 128, 256, 128, 2, 4, 4, true),
    // int8 with row-major B ([K,N], linalg.matmul's default map): the int8
    // weights are staged as they lie and read with ds_read_b64_tr_b8
    IHP_FAST_CONFIG("i8_nn_256x256x128_w2x4_s2", kBNN8, int8_t, int32_t, 256, 256, 128, 2, 4, 2),
    IHP_FAST_CONFIG_16("i8_nn_256x256x128_w2x4_s2_m16", kBNN8, int8_t, int32_t, 256, 256, 128, 2, 4, 2),
    IHP_FAST_CONFIG("i8_nn_128x256x128_w2x4_s2", kBNN8, int8_t, int32_t, 128, 256, 128, 2, 4, 2),
    // int8 split-K tiles for skinny and ragged M, either B form
    IHP_FAST_CONFIG_S("i8_tn_32x128x128_w1x4_s4_sk", kBTN, int8_t, int32_t, 32, 128, 128, 1, 4, 4, true),
    IHP_FAST_CONFIG_S("i8_tn_128x128x128_w2x2_s4_sk", kBTN, int8_t, int32_t, 128, 128, 128, 2, 2, 4, true),
    IHP_FAST_CONFIG_S("i8_nn_32x256x128_w1x4_s4_sk", kBNN8, int8_t, int32_t, 32, 256, 128, 1, 4, 4, true),
    IHP_FAST_CONFIG_S("i8_nn_128x256x128_w2x4_s3_sk", kBNN8, int8_t, int32_t, 128, 256, 128, 2, 4, 3, true),
    // transposed A ([K,M], M-contiguous), either B form
    IHP_FAST_CONFIG_AT("f16at_nn_256x256x64_w2x4_s2", kBNN16, f16, f16, 256, 256, 128, 2, 4, 2),
    IHP_FAST_CONFIG_AT("f16at_nn_256x128x64_w2x4_s2", kBNN16, f16, f16, 256, 128, 128, 2, 4, 2),
    IHP_FAST_CONFIG_AT("f16at_nn_128x128x64_w2x2_s4", kBNN16, f16, f16, 128, 128, 128, 2, 2, 4),
    IHP_FAST_CONFIG_AT("f16at_tn_256x256x64_w2x4_s2", kBTN, f16, f16, 256, 256, 128, 2, 4, 2),
    IHP_FAST_CONFIG_AT("f16at_tn_256x128x64_w2x4_s2", kBTN, f16, f16, 256, 128, 128, 2, 4, 2),
    IHP_FAST_CONFIG_AT("f16at_tn_128x128x64_w2x2_s4", kBTN, f16, f16, 128, 128, 128, 2, 2, 4),
    IHP_FAST_CONFIG_AT("f16f32at_nn_128x128x64_w2x2_s4", kBNN16, f16, float, 128, 128, 128, 2, 2, 4),
    IHP_FAST_CONFIG_AT("f16f32at_tn_128x128x64_w2x2_s4", kBTN, f16, float, 128, 128, 128, 2, 2, 4),
    IHP_FAST_CONFIG_AT("f16f32at_nn_256x128x64_w2x4_s2", kBNN16, f16, float, 256, 128, 128, 2, 4, 2),
    IHP_FAST_CONFIG_AT("f16f32at_tn_256x128x64_w2x4_s2", kBTN, f16, float, 256, 128, 128, 2, 4, 2),
    IHP_FAST_CONFIG_AT16("f16at_nn_256x256x64_w2x4_s2_m16", kBNN16, f16, f16, 256, 256, 128, 2, 4, 2),
    IHP_FAST_CONFIG_AT16("f16at_tn_256x256x64_w2x4_s2_m16", kBTN, f16, f16, 256, 256, 128, 2, 4, 2),
    IHP_FAST_CONFIG_AT16("f16f32at_nn_256x256x64_w2x4_s2_m16", kBNN16, f16, float, 256, 256, 128, 2, 4, 2),
    IHP_FAST_CONFIG_AT16("f16f32at_tn_256x256x64_w2x4_s2_m16", kBTN, f16, float, 256, 256, 128, 2, 4, 2),
    // 8-wave skinny split-K tile (512-byte weight rows, twice the copies in
    // flight of the 4-wave 32x128 tile per CU). Measured ahead only on the
    // shape the planner's table names it for (slower at M = 16 with N =
    // 4096, M = 128 and K = 11008), so the cost model does not rank it.
    IHP_FAST_CONFIG_S_TABLE("f16_nn_64x256x64_w2x4_s4_sk", kBNN16, f16, f16, 64, 256, 128, 2, 4, 4),
    // The same for C3 M=128 N=11008: 8 waves of 64x32 on a 128x128 tile.
    IHP_FAST_CONFIG_S_TABLE("f16_nn_128x128x64_w2x4_s4_sk", kBNN16, f16, f16, 128, 128, 128, 2, 4, 4),
    // And 8 waves of 32x32 on a 64x128 tile (4 stages of 24 KiB).
    IHP_FAST_CONFIG_S_TABLE("f16_nn_64x128x64_w2x4_s4_sk", kBNN16, f16, f16, 64, 128, 128, 2, 4, 4),
    // Column splits: a ragged last round of 256x256 tiles (C3 M=2048
    // N=11008: 344 tiles, a round of 256 and one of 88) re-tiled as one
    // round of half-size tiles after the whole rounds.
    IHP_COLUMN_SPLIT("f16_nn_", "256x256x64_w2x4_s2_m16", "256x128x64_w2x4_s2_m16",
                     kBNN16, f16, f16, 128, false, 256, 256, 2, 16, 256, 128, 2, 16),
    IHP_COLUMN_SPLIT("f16_tn_", "256x256x64_w2x4_s2_m16", "256x128x64_w2x4_s2_m16",
                     kBTN, f16, f16, 128, false, 256, 256, 2, 16, 256, 128, 2, 16),
    IHP_COLUMN_SPLIT("i8_tn_", "256x256x128_w2x4_s2_m16", "256x128x128_w2x4_s2_m16",
                     kBTN, int8_t, int32_t, 128, false, 256, 256, 2, 16, 256, 128, 2, 16),
    IHP_COLUMN_SPLIT("i8_nn_", "256x256x128_w2x4_s2_m16", "128x256x128_w2x4_s2",
                     kBNN8, int8_t, int32_t, 128, false, 256, 256, 2, 16, 128, 256, 2, 32),
    IHP_COLUMN_SPLIT("w8a16_nn_", "256x256x64_w2x4_s3", "128x256x64_w2x4_s4",
                     kBW8, f16, f16, 128, false, 256, 256, 3, 32, 128, 256, 4, 32),
    IHP_COLUMN_SPLIT("f16at_nn_", "256x256x64_w2x4_s2_m16", "256x128x64_w2x4_s2",
                     kBNN16, f16, f16, 128, true, 256, 256, 2, 16, 256, 128, 2, 32),
    IHP_COLUMN_SPLIT("f16at_tn_", "256x256x64_w2x4_s2_m16", "256x128x64_w2x4_s2",
                     kBTN, f16, f16, 128, true, 256, 256, 2, 16, 256, 128, 2, 32),
    IHP_COLUMN_SPLIT("f16f32at_nn_", "256x256x64_w2x4_s2_m16", "256x128x64_w2x4_s2",
                     kBNN16, f16, float, 128, true, 256, 256, 2, 16, 256, 128, 2, 32),
    IHP_COLUMN_SPLIT("f16f32at_tn_", "256x256x64_w2x4_s2_m16", "256x128x64_w2x4_s2",
                     kBTN, f16, float, 128, true, 256, 256, 2, 16, 256, 128, 2, 32),
    IHP_COLUMN_SPLIT("f16f32_nn_", "256x256x64_w2x4_s2_m16", "256x128x64_w2x4_s2_m16",
                     kBNN16, f16, float, 128, false, 256, 256, 2, 16, 256, 128, 2, 16),
    IHP_COLUMN_SPLIT("f16f32_tn_", "256x256x64_w2x4_s2_m16", "256x128x64_w2x4_s2_m16",
                     kBTN, f16, float, 128, false, 256, 256, 2, 16, 256, 128, 2, 16),
};

const FastConfig *fast_configs(int *count) {
  *count = (int)(sizeof(kFastConfigs) / sizeof(kFastConfigs[0]));
  return kFastConfigs;
}

// Every GEMM kernel: the macro-tile configurations, then the general kernel's
// four instances.
const KernelEntry *gemm_kernels(int *count) {
  static const std::vector<KernelEntry> all = [] {
    std::vector<KernelEntry> v;
    for (const FastConfig &c : kFastConfigs) {
      if (c.head)
        continue;  // a column split launches two listed kernels
      const uint32_t ex = c.elem == kElemI8 ? kExportMatmulI8
                          : c.b_mode == kBW8
                              ? kExportW8A16
                              : kExportMatmulF16 | kExportBatchMatmulF16;
      v.push_back({c.name, c.kernel, c.threads, ex});
    }
    const uint32_t f16x = kExportMatmulF16 | kExportBatchMatmulF16;
    v.push_back({"general_f16", (const void *)&gemm_general_kernel<f16, f16, f16, false>, 256, f16x});
    v.push_back({"general_f16f32", (const void *)&gemm_general_kernel<f16, f16, float, false>, 256, f16x});
    v.push_back({"general_i8", (const void *)&gemm_general_kernel<int8_t, int8_t, int32_t, false>, 256, kExportMatmulI8});
    v.push_back({"general_w8a16", (const void *)&gemm_general_kernel<f16, int8_t, f16, true>, 256, kExportW8A16});
    return v;
  }();
  *count = (int)all.size();
  return all.data();
}

template <typename TA, typename TB, typename OutT, bool kScale>
static hipError_t launch_general_t(const MatmulArgs &a, const void *scale) {
  dim3 grid((unsigned)((a.n + 63) / 64), (unsigned)((a.m + 63) / 64),
            (unsigned)a.batch);
  hipLaunchKernelGGL((gemm_general_kernel<TA, TB, OutT, kScale>), grid,
                     dim3(256), 0, (hipStream_t)a.stream, (const TA *)a.a,
                     (const TB *)a.b, (OutT *)a.c, (const f16 *)scale,
                     (int)a.m, (int)a.n, (int)a.k, a.lda, a.ldb, a.ldc,
                     a.b_transposed, a.accumulate, a.sa, a.sb, a.sc,
                     make_epi(a), epi_batch_stride(a), a.a_transposed);
  return hipGetLastError();
}

hipError_t launch_general(const MatmulArgs &a, GeneralKind kind,
                          const void *scale) {
  switch (kind) {
    case kGeneralF16F16:
      return launch_general_t<f16, f16, f16, false>(a, nullptr);
    case kGeneralF16F32:
      return launch_general_t<f16, f16, float, false>(a, nullptr);
    case kGeneralI8I32:
      return launch_general_t<int8_t, int8_t, int32_t, false>(a, nullptr);
    case kGeneralW8A16:
      return launch_general_t<f16, int8_t, f16, true>(a, scale);
  }
  return hipErrorInvalidValue;
}

}  // namespace ihp
