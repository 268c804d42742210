// Dispatch classification and gfx950 macro-tile planning (host only).
// See include/iree_mi355x_planner.h for the reference functions each entry
// point replaces.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <tuple>

#include "../../include/iree_mi355x_kernels.h"
#include "../../include/iree_mi355x_planner.h"
#include "kernels_internal.h"

namespace ihp {

int fail(int status, const char *fmt, ...);
int require_workspace(const char *who, size_t need, const void *workspace,
                      size_t workspace_bytes);

namespace {

constexpr int64_t kDefaultLdsBudget = 160 * 1024;
constexpr int32_t kDefaultCus = 256;

// Measured choices (bench.py --tune writes the candidates' timings; the
// winners are recorded here). Keyed by element types, exact shape and flags.
struct TunedEntry {
  int32_t a_elem, b_elem, c_elem;
  int64_t m, n, k;
  uint32_t flags;
  const char *config;
  int32_t splits;  // K splits of a split-K configuration (0: the model's)
};
// Measured on MI355X with random inputs (bench.py --tune): the 8-wave
// 256x256 tile wins for int8 and f16 (two waves per SIMD hide each other's
// stage hand-off waits; int8 2098 against 1930 TOPS for the 4-wave tile),
// in its 16x16 MFMA form (int8 61.6 against 65.1 us, f16 109.9 against
// 115.2 us on one box).
const TunedEntry kTuned[] = {
    {IREE_MI355X_ELEM_I8, IREE_MI355X_ELEM_I8, IREE_MI355X_ELEM_I32, 4096, 4096,
     4096,
     IREE_MI355X_MATMUL_B_TRANSPOSED, "i8_tn_256x256x128_w2x4_s2_m16", 0},
    {IREE_MI355X_ELEM_F16, IREE_MI355X_ELEM_F16, IREE_MI355X_ELEM_F16, 4096,
     4096, 4096, IREE_MI355X_MATMUL_B_TRANSPOSED,
     "f16_tn_256x256x64_w2x4_s2_m16", 0},
    {IREE_MI355X_ELEM_F16, IREE_MI355X_ELEM_F16, IREE_MI355X_ELEM_F32, 4096,
     4096, 4096, IREE_MI355X_MATMUL_B_TRANSPOSED,
     "f16f32_tn_256x256x64_w2x4_s2_m16", 0},
    // Skinny shapes where the model's pick measured slower than a sweep of
    // every tile and split count (random inputs, rotating weights).
    {IREE_MI355X_ELEM_F16, IREE_MI355X_ELEM_F16, IREE_MI355X_ELEM_F16, 16,
     4096, 11008, 0, "f16_nn_64x128x64_w2x4_s4_sk", 8},
    // C3 M=16 N=11008: the 8-wave 64x256 tile, 4 splits (172 workgroups),
    // 20.7 against 22.3 us for the best 32x128 split count.
    {IREE_MI355X_ELEM_F16, IREE_MI355X_ELEM_F16, IREE_MI355X_ELEM_F16, 16,
     11008, 4096, 0, "f16_nn_64x256x64_w2x4_s4_sk", 4},
    // C5 W8A16 M=128: stream-K runs of the 32x256 tile, 37.8 / 38.4 against
    // 42.9 / 43.3 us for its single split in two sweeps.
    {IREE_MI355X_ELEM_F16, IREE_MI355X_ELEM_I8, IREE_MI355X_ELEM_F16, 128,
     11008, 4096, 0, "w8a16_nn_32x256x64_w1x4_s4_sk", -1},
    // C3 M=16 and M=128 at N=K=4096 and M=128 at K=11008: the 8-wave 64x128
    // tile, 12.2 against 12.9 us (x6), 18.5 against 21.2 us (x4) and 33.1
    // against 35.2 us (x4) for the model's picks; at M=16 K=11008 (the
    // entry above) 21.3 against 21.8 us for the 4-wave 32x128 tile, x8.
    {IREE_MI355X_ELEM_F16, IREE_MI355X_ELEM_F16, IREE_MI355X_ELEM_F16, 16,
     4096, 4096, 0, "f16_nn_64x128x64_w2x4_s4_sk", 6},
    {IREE_MI355X_ELEM_F16, IREE_MI355X_ELEM_F16, IREE_MI355X_ELEM_F16, 128,
     4096, 4096, 0, "f16_nn_64x128x64_w2x4_s4_sk", 4},
    {IREE_MI355X_ELEM_F16, IREE_MI355X_ELEM_F16, IREE_MI355X_ELEM_F16, 128,
     4096, 11008, 0, "f16_nn_64x128x64_w2x4_s4_sk", 4},
    // C3 M=128 N=11008: the 8-wave 128x128 tile, 2 splits (172 workgroups),
    // 32.8 against 37.8 us for 64x128 x1 and 35.5 us for the 4-wave 128x128.
    {IREE_MI355X_ELEM_F16, IREE_MI355X_ELEM_F16, IREE_MI355X_ELEM_F16, 128,
     11008, 4096, 0, "f16_nn_128x128x64_w2x4_s4_sk", 2},
    // C1 (128x512x256, latency-bound): 16 workgroups of 32x128 with one
    // split (rows stored directly) beat 4 of 128x128 (4.0 against 5.7 us),
    // each workgroup streaming a quarter of the operand bytes.
    {IREE_MI355X_ELEM_F16, IREE_MI355X_ELEM_F16, IREE_MI355X_ELEM_F16, 128,
     512, 256, 0, "f16_nn_32x128x64_w1x4_s4_sk", 1},
    // M=192 N=11008 (86 tiles of 128x128): the 8-wave tile, one split,
    // 39.7 / 40.5 against 41.3 / 41.9 us for the 4-wave one in two sweeps.
    {IREE_MI355X_ELEM_F16, IREE_MI355X_ELEM_F16, IREE_MI355X_ELEM_F16, 192,
     11008, 4096, 0, "f16_nn_128x128x64_w2x4_s4_sk", 1},
    // Stream-K (splits -1) where it measured fastest.
    {IREE_MI355X_ELEM_F16, IREE_MI355X_ELEM_I8, IREE_MI355X_ELEM_F16, 192,
     11008, 11008, 0, "w8a16_nn_128x256x64_w2x4_s4_sk", -1},
    {0, 0, 0, 0, 0, 0, 0, nullptr, 0},  // sentinel
};

int elem_bytes(int32_t e) {
  switch (e) {
    case IREE_MI355X_ELEM_I8:
      return 1;
    case IREE_MI355X_ELEM_F16:
      return 2;
    default:
      return 4;
  }
}

bool types_supported(const iree_mi355x_matmul_desc_t &d) {
  const bool f16 = d.a_elem == IREE_MI355X_ELEM_F16 &&
                   d.b_elem == IREE_MI355X_ELEM_F16 &&
                   (d.c_elem == IREE_MI355X_ELEM_F16 ||
                    d.c_elem == IREE_MI355X_ELEM_F32) &&
                   !d.has_scale;
  const bool i8 = d.a_elem == IREE_MI355X_ELEM_I8 &&
                  d.b_elem == IREE_MI355X_ELEM_I8 &&
                  d.c_elem == IREE_MI355X_ELEM_I32 && !d.has_scale;
  const bool w8a16 = d.a_elem == IREE_MI355X_ELEM_F16 &&
                     d.b_elem == IREE_MI355X_ELEM_I8 &&
                     d.c_elem == IREE_MI355X_ELEM_F16 && d.has_scale;
  return f16 || i8 || w8a16;
}

bool gemv_eligible(const iree_mi355x_matmul_desc_t &d) {
  if (d.m < 1 || d.k < 1 || (d.flags & IREE_MI355X_MATMUL_A_TRANSPOSED) ||
      !d.b_aligned16)
    return false;
  if (d.flags & IREE_MI355X_MATMUL_B_TRANSPOSED) {
    // Row-dot form (W [N,K]): whole 16-byte segments of each row of W (K a
    // multiple of 16 covers f16 and int8), x rows copied into LDS in
    // 16-byte pieces, a launch's x (at most 4 rows) within the LDS it
    // stages in. int8 weights only in the W8A16 form, which also takes up
    // to kRowdotMaxRowsW8A16 rows as launches of 4.
    const bool w8 = d.b_elem == IREE_MI355X_ELEM_I8;
    const int64_t rows = w8 ? rowdot_w8a16_rows(d.m, d.k) : d.m;
    if (d.m > (w8 ? kRowdotMaxRowsW8A16 : kGemvMaxRows) || d.k % 16 != 0 ||
        !d.a_aligned16 || rows < 1 || rows * d.k * 2 > kRowdotMaxXBytes)
      return false;
    return w8 ? d.has_scale != 0 : true;
  }
  if (d.m > kGemvMaxRows)
    return false;
  const int cols = 16 / elem_bytes(d.b_elem);
  if (d.n % cols != 0)
    return false;
  // one arrival counter per column block of 64 lanes x `cols` columns, per
  // batch (the full-wave form; the half-wave form's twice as many blocks are
  // planned only where they fit too)
  const int64_t batch = d.batch > 0 ? d.batch : 1;
  if ((d.n + 64 * cols - 1) / (64 * cols) * batch > kMaxWorkspaceCounters)
    return false;
  // int8 weights only in the W8A16 form; f16 with f16 or f32 output.
  if (d.b_elem == IREE_MI355X_ELEM_I8)
    return d.has_scale;
  return true;
}

// The B form a dispatch needs, or -1 if no fast kernel computes it.
int wanted_b_mode(const iree_mi355x_matmul_desc_t &d) {
  const bool bt = d.flags & IREE_MI355X_MATMUL_B_TRANSPOSED;
  if (d.has_scale)
    return (!bt && d.a_elem == IREE_MI355X_ELEM_F16 &&
            d.b_elem == IREE_MI355X_ELEM_I8 &&
            d.c_elem == IREE_MI355X_ELEM_F16 &&
            !(d.flags & IREE_MI355X_MATMUL_ACCUMULATE))
               ? kBW8
               : -1;
  if (d.a_elem != d.b_elem)
    return -1;
  if (bt)
    return kBTN;
  return d.a_elem == IREE_MI355X_ELEM_F16 ? kBNN16 : kBNN8;
}

// Fast-kernel candidates for the shape: N and K tile exactly; M tiles
// exactly unless the configuration splits K (its A copy clamps rows to M-1).
bool fast_fits(const iree_mi355x_matmul_desc_t &d, const FastConfig &c) {
  if (!d.a_aligned16 || !d.b_aligned16 || d.k <= 0 || d.m <= 0)
    return false;
  if (c.b_mode != wanted_b_mode(d))
    return false;
  if (c.a_trans != ((d.flags & IREE_MI355X_MATMUL_A_TRANSPOSED) ? 1 : 0))
    return false;
  const int want_elem = d.a_elem == IREE_MI355X_ELEM_I8 ? kElemI8 : kElemF16;
  if (c.elem != want_elem)
    return false;
  if (want_elem == kElemF16 && c.out_f32 != (d.c_elem == IREE_MI355X_ELEM_F32))
    return false;
  if (d.n % c.bn != 0 || d.k % c.bk != 0)
    return false;
  return c.split_k ? true : d.m % c.bm == 0;
}

// One ranked candidate: a configuration plus its K split.
struct Candidate {
  int index = -1;
  int splits = 1;       // stream-K: the most runs one tile spans
  int k_split = 0;
  int sk_steps = 0;     // stream-K: K stages per workgroup run (0: off)
  int64_t sk_wgs = 0;   // stream-K: workgroups
  int64_t tiles = 0;
  int64_t critical = 0;  // per-CU critical-path MACs
  int64_t traffic = 0;   // modeled global->LDS bytes (operands + partials)
  int64_t workspace = 0;
  int64_t est_ns = 0;    // modeled time, the ranking key
};

// MI355X rates the cost model uses (measured on the box where noted):
// dense MFMA per CU at 2.4 GHz; the LDS-DMA operand feed of all CUs (about
// 16 TB/s measured with the copy-only variant of the MFMA kernel); HBM at
// about three quarters of its 8 TB/s peak.
constexpr double kMacsPerCuNsF16 = 2048.0 * 2.4;  // 4096 flop/clk
constexpr double kMacsPerCuNsI8 = 4096.0 * 2.4;   // 8192 op/clk
// The 16x16 MFMAs sustain this much more on random operands (the
// calibration loop: 1.145x int8, 1.112x f16).
constexpr double kMfma16Speedup = 1.1;
constexpr double kFeedBytesPerNs = 16000.0;
constexpr double kHbmBytesPerNs = 6000.0;
// Fixed latencies: each round of workgroups (one per CU) pays the pipeline
// fill and the epilogue; a split-K tile also pays the partial publish, the
// arrival count and the last arriver's reduction.
constexpr double kRoundNs = 1500.0;
constexpr double kSplitNs = 2000.0;
constexpr double kRoundTripNs = 700.0;  // one dependent device-scope access
constexpr double kStageNs = 500.0;      // per K stage of one workgroup
// A split covers at least this many K stages, so its copy pipeline overlaps.
constexpr int64_t kMinStagesPerSplit = 2;

// Stream-K's forced split value: equal runs of (tile, K stage) pairs.
constexpr int kStreamK = -1;

// Stream-K: one workgroup per CU, each taking an equal run of the (tile, K
// stage) pairs in tile order (at least kMinStagesPerSplit stages). Priced
// like split-K: the busiest CU's MACs, the operand feed and HBM (plus the
// partial tiles of tiles split across runs), one pipeline fill per tile a
// run touches, and the last arriver's reduction of the most runs a tile
// spans.
bool evaluate_stream_k(const iree_mi355x_matmul_desc_t &d, const FastConfig &c,
                       int index, int64_t cus, int64_t tiles, int64_t tiles_m,
                       Candidate *out) {
  const int64_t ks = d.k / c.bk;
  const int64_t total = tiles * ks;
  int64_t run = (total + cus - 1) / cus;
  if (run < kMinStagesPerSplit)
    run = kMinStagesPerSplit;
  if (run >= ((int64_t)1 << 31) / 2)
    return false;
  const int64_t wgs = (total + run - 1) / run;
  int layers = 1;
  int64_t split_parts = 0;  // partial tiles published
  for (int64_t t = 0; t < tiles; ++t) {
    const int64_t c0 = t * ks / run, c1 = (t * ks + ks - 1) / run;
    const int n = (int)(c1 - c0 + 1);
    if (n > layers)
      layers = n;
    if (n > 1)
      split_parts += n;
  }
  const int64_t segs = (run + ks - 1) / ks + 1;  // most tiles one run touches
  const int64_t ab = elem_bytes(d.a_elem), bb = elem_bytes(d.b_elem);
  Candidate r;
  r.index = index;
  r.splits = layers;
  r.k_split = 0;
  r.sk_steps = (int)run;
  r.sk_wgs = wgs;
  r.tiles = tiles;
  r.critical = run * c.bm * c.bn * c.bk;
  r.traffic = ab * (tiles_m * c.bm) * d.k * (d.n / c.bn) +
              bb * d.n * d.k * tiles_m;
  const int64_t partial_bytes = 2 * split_parts * c.bm * c.bn * 4;
  r.traffic += partial_bytes;
  r.workspace = layers > 1 ? (int64_t)split_counter_bytes(tiles) +
                                 layers * d.m * d.n * 4
                           : 0;
  // stream-K runs fill every CU (its configurations are 32x32 MFMAs)
  const double macs_per_ns =
      (d.a_elem == IREE_MI355X_ELEM_I8 ? kMacsPerCuNsI8 : kMacsPerCuNsF16) *
      (c.mfma == 16 ? kMfma16Speedup : 1.0);
  double t = (double)r.critical / macs_per_ns;
  const double t_feed = (double)r.traffic / kFeedBytesPerNs;
  const double t_hbm =
      (double)(ab * d.m * d.k + bb * d.n * d.k +
               elem_bytes(d.c_elem) * d.m * d.n + partial_bytes) /
      kHbmBytesPerNs;
  const double t_chain = (double)run * kStageNs;
  if (t_feed > t)
    t = t_feed;
  if (t_hbm > t)
    t = t_hbm;
  if (t_chain > t)
    t = t_chain;
  t += (double)segs * kRoundNs;
  if (layers > 1) {
    const int64_t rows = d.m < c.bm ? d.m : c.bm;
    const int64_t per_thread = (rows * c.bn + c.threads - 1) / c.threads;
    const int64_t loads = c.threads > 256 ? 32 : 64;
    const int64_t sb = layers <= 2 ? 2 : layers <= 4 ? 4 : 8;
    const int64_t g = loads / sb;
    t += kSplitNs + (double)((per_thread + g - 1) / g) *
                        (double)((layers + sb - 1) / sb) * kRoundTripNs;
  }
  r.est_ns = (int64_t)t;
  *out = r;
  return true;
}

// `explicit_config`: the caller named this configuration, so a split
// configuration runs even where one split is all the shape needs.
// `forced_splits` kStreamK asks for stream-K instead of a split count.
bool evaluate(const iree_mi355x_matmul_desc_t &d, const FastConfig &c,
              int index, int64_t cus, Candidate *out,
              bool explicit_config = false, int forced_splits = 0) {
  if (!fast_fits(d, c))
    return false;
  const int64_t batch = d.batch > 0 ? d.batch : 1;
  if (c.head) {
    // Column split: the head configuration over the columns its whole
    // rounds cover, then the tail over the rest, priced as the two
    // launches they are, one after the other. The launcher splits for the
    // chip's own CU count, so only that count plans one.
    if (batch != 1 || cus != kColumnSplitCus)
      return false;
    int count = 0;
    const FastConfig *cfgs = fast_configs(&count);
    int hi = -1, ti = -1;
    for (int i = 0; i < count; ++i) {
      if (strcmp(cfgs[i].name, c.head) == 0)
        hi = i;
      if (strcmp(cfgs[i].name, c.tail) == 0)
        ti = i;
    }
    if (hi < 0 || ti < 0)
      return false;
    const FastConfig &hc = cfgs[hi], &tc = cfgs[ti];
    const int64_t n_head =
        column_split_head(d.m, d.n, hc.bm, hc.bn, tc.bm, tc.bn, cus);
    if (n_head <= 0)
      return false;
    iree_mi355x_matmul_desc_t dh = d, dt = d;
    dh.n = n_head;
    dt.n = d.n - n_head;
    Candidate ch, ct;
    if (!evaluate(dh, hc, hi, cus, &ch) || !evaluate(dt, tc, ti, cus, &ct))
      return false;
    Candidate r;
    r.index = index;
    r.tiles = ch.tiles + ct.tiles;
    r.critical = ch.critical + ct.critical;
    r.traffic = ch.traffic + ct.traffic;
    r.est_ns = ch.est_ns + ct.est_ns;
    *out = r;
    return true;
  }
  const int64_t tiles_m = (d.m + c.bm - 1) / c.bm;
  const int64_t tiles = tiles_m * (d.n / c.bn);
  if (c.split_k && tiles * batch > kMaxWorkspaceCounters)
    return false;  // one arrival counter per tile of every batch
  int splits = 1;
  int64_t k_split = d.k;
  if (forced_splits == kStreamK) {
    if (!c.split_k || batch != 1)
      return false;
    return evaluate_stream_k(d, c, index, cus, tiles, tiles_m, out);
  }
  if (c.split_k) {
    // Enough workgroups to cover every CU; each split a multiple of BK.
    int64_t want = (cus + tiles * batch - 1) / (tiles * batch);
    const int64_t max_splits =
        explicit_config ? d.k / c.bk : d.k / (kMinStagesPerSplit * c.bk);
    if (forced_splits > 0)
      want = forced_splits;
    if (want > max_splits)
      want = max_splits;
    if (want < 1)
      want = 1;
    k_split = ((d.k + want - 1) / want + c.bk - 1) / c.bk * c.bk;
    splits = (int)((d.k + k_split - 1) / k_split);
    // One split stores directly (rows past M masked): worth it where M is
    // ragged, or where the shape's unsplit grid would leave most CUs idle
    // (short K: many small tiles, each a short chain); else an unsplit
    // configuration covers the shape better.
    if (splits < 2 && !explicit_config && d.m % c.bm == 0 &&
        tiles * batch * 2 >= cus)
      return false;
  }
  const int64_t ab = elem_bytes(d.a_elem), bb = elem_bytes(d.b_elem);
  const int64_t acc_bytes = 4;
  Candidate r;
  r.index = index;
  r.splits = splits;
  r.k_split = (int)k_split;
  r.tiles = tiles;
  r.critical =
      ((tiles * splits * batch + cus - 1) / cus) * c.bm * c.bn * k_split;
  // A rows past M (split configurations) are still copied, as clamped
  // duplicates of row M-1.
  r.traffic = batch * (ab * (tiles_m * c.bm) * d.k * (d.n / c.bn) +
                       bb * d.n * d.k * tiles_m);
  int64_t partial_bytes = 0;
  if (c.split_k && splits > 1) {
    r.workspace = (int64_t)split_counter_bytes(tiles) +
                  batch * splits * d.m * d.n * acc_bytes;
    partial_bytes = 2 * batch * splits * d.m * d.n * acc_bytes;
    r.traffic += partial_bytes;
  }
  // time = the slowest of MFMA work on the busiest CU, the operand feed, and
  // HBM (each operand and C once, plus split partials written and read)
  // The 16x16 rate only where the tiles fill every CU: the feed term is a
  // whole-chip aggregate, which a half-empty grid does not reach.
  const bool full = tiles * splits * batch >= cus;
  const double macs_per_ns =
      (d.a_elem == IREE_MI355X_ELEM_I8 ? kMacsPerCuNsI8 : kMacsPerCuNsF16) *
      (c.mfma == 16 && full ? kMfma16Speedup : 1.0);
  const double t_mfma = (double)r.critical / macs_per_ns;
  const double t_feed = (double)r.traffic / kFeedBytesPerNs;
  const double hbm = (double)(batch * (ab * d.m * d.k + bb * d.n * d.k +
                                       elem_bytes(d.c_elem) * d.m * d.n) +
                              partial_bytes);
  const double t_hbm = hbm / kHbmBytesPerNs;
  double t = t_mfma > t_feed ? t_mfma : t_feed;
  if (t_hbm > t)
    t = t_hbm;
  // A workgroup's K loop is a chain of stages, each at least a copy latency
  // apart once the ring's lookahead is spent.
  const int64_t rounds = (tiles * splits * batch + cus - 1) / cus;
  const double t_chain = (double)rounds * (double)(k_split / c.bk) * kStageNs;
  // An unsplit grid filling under half the CUs never reaches the copy /
  // MFMA overlap of a long K loop: its few stages pay both in turn. (Split
  // grids keep the overlapped form, so the split count is not pushed
  // across the half-grid boundary.)
  if (splits == 1 && tiles * batch * 2 < cus)
    t = t_mfma + t_chain > t ? t_mfma + t_chain : t;
  else if (t_chain > t)
    t = t_chain;
  t += (double)rounds * kRoundNs;
  if (c.split_k && splits > 1) {
    // the last arriver keeps L loads in flight per round trip: SB split
    // slots (2, 4 or 8) for each of L / SB elements
    const int64_t rows = d.m < c.bm ? d.m : c.bm;
    const int64_t per_thread = (rows * c.bn + c.threads - 1) / c.threads;
    const int64_t loads = c.threads > 256 ? 32 : 64;
    const int64_t sb = splits <= 2 ? 2 : splits <= 4 ? 4 : 8;
    const int64_t g = loads / sb;
    t += kSplitNs + (double)((per_thread + g - 1) / g) *
                        (double)((splits + sb - 1) / sb) * kRoundTripNs;
  }
  r.est_ns = (int64_t)t;
  *out = r;
  return true;
}

}  // namespace
}  // namespace ihp

using namespace ihp;

extern "C" {

void iree_mi355x_matmul_desc_init(iree_mi355x_matmul_desc_t *desc,
                                  int32_t a_elem, int32_t b_elem,
                                  int32_t c_elem, int64_t m, int64_t n,
                                  int64_t k, uint32_t flags) {
  memset(desc, 0, sizeof(*desc));
  desc->a_elem = a_elem;
  desc->b_elem = b_elem;
  desc->c_elem = c_elem;
  desc->m = m;
  desc->n = n;
  desc->k = k;
  desc->flags = flags;
  desc->a_aligned16 = 1;
  desc->b_aligned16 = 1;
  desc->lds_budget_bytes = kDefaultLdsBudget;
  desc->num_cus = kDefaultCus;
  desc->batch = 1;
}

int32_t iree_mi355x_classify_matmul(const iree_mi355x_matmul_desc_t *d) {
  if (!d || !types_supported(*d) || d->m < 0 || d->n < 0 || d->k < 0)
    return IREE_MI355X_FAMILY_NONE;
  if (gemv_eligible(*d))
    return IREE_MI355X_FAMILY_GEMV;
  int count = 0;
  const FastConfig *cfgs = fast_configs(&count);
  const int64_t cus = d->num_cus > 0 ? d->num_cus : kDefaultCus;
  for (int i = 0; i < count; ++i) {
    Candidate c;
    if (!cfgs[i].table_only && cfgs[i].lds_bytes <= d->lds_budget_bytes &&
        evaluate(*d, cfgs[i], i, cus, &c))
      return IREE_MI355X_FAMILY_MFMA;
  }
  return IREE_MI355X_FAMILY_GENERAL;
}

int iree_mi355x_plan_matmul(const iree_mi355x_matmul_desc_t *d,
                            iree_mi355x_matmul_plan_t *plan) {
  if (!d || !plan)
    return IREE_MI355X_INVALID_ARGUMENT;
  memset(plan, 0, sizeof(*plan));
  plan->config_index = -1;
  const int32_t family = iree_mi355x_classify_matmul(d);
  plan->family = family;
  if (family == IREE_MI355X_FAMILY_NONE)
    return IREE_MI355X_UNSUPPORTED;
  const int64_t budget =
      d->lds_budget_bytes > 0 ? d->lds_budget_bytes : kDefaultLdsBudget;
  const int64_t cus = d->num_cus > 0 ? d->num_cus : kDefaultCus;

  if (family == IREE_MI355X_FAMILY_GEMV &&
      (d->flags & IREE_MI355X_MATMUL_B_TRANSPOSED)) {
    // Row-dot form: one wave per output column at a time, K whole.
    const int wb = elem_bytes(d->b_elem);
    const int64_t batch = d->batch > 0 ? d->batch : 1;
    snprintf(plan->config_name, sizeof(plan->config_name),
             "gemv_rowdot_%s_r%lld",
             wb == 1 ? "w8a16"
                     : (d->c_elem == IREE_MI355X_ELEM_F32 ? "f16f32" : "f16"),
             (long long)d->m);
    plan->tile_m = d->m;
    plan->tile_n = 1;
    plan->tile_k = d->k;
    const int64_t rows = wb == 1 ? rowdot_w8a16_rows(d->m, d->k) : d->m;
    const int64_t launches = (d->m + rows - 1) / rows;
    plan->lds_bytes = rows * d->k * 2;
    plan->workgroups = rowdot_workgroups(d->n) * batch * launches;
    plan->threads = kGemvThreads;
    plan->splits = 1;
    plan->workspace_bytes = 0;
    plan->traffic_bytes =
        batch * (launches * d->n * d->k * wb + d->m * d->k * 2);
    return IREE_MI355X_OK;
  }
  if (family == IREE_MI355X_FAMILY_GEMV) {
    const int wb = elem_bytes(d->b_elem);
    const int64_t batch = d->batch > 0 ? d->batch : 1;
    GemvPlan g = gemv_plan(d->m, d->n, d->k, wb, batch);
    snprintf(plan->config_name, sizeof(plan->config_name), "gemv_%s_r%lld%s",
             wb == 1 ? "w8a16" : "f16", (long long)d->m,
             g.halves == 2 ? "_h2" : "");
    plan->tile_m = d->m;
    plan->tile_n = g.cols_per_wg;
    plan->tile_k = g.k_chunk;
    plan->workgroups = g.col_blocks * g.splits * batch;
    plan->threads = kGemvThreads;
    plan->splits = g.splits;
    plan->workspace_bytes =
        (int64_t)gemv_workspace_bytes(d->m, d->n, d->k, wb, batch);
    plan->traffic_bytes = batch * (d->n * d->k * wb + d->m * d->k * 2);
    return IREE_MI355X_OK;
  }

  if (family == IREE_MI355X_FAMILY_MFMA) {
    int count = 0;
    const FastConfig *cfgs = fast_configs(&count);
    Candidate best;
    // A measured entry wins when it fits. Entries were timed on one matrix:
    // a batch multiplies the grid, so batched calls take the model's pick.
    for (const TunedEntry &t : kTuned) {
      if (!t.config || d->batch > 1 || t.a_elem != d->a_elem ||
          t.b_elem != d->b_elem ||
          t.c_elem != d->c_elem ||
          t.m != d->m || t.n != d->n || t.k != d->k || t.flags != d->flags)
        continue;
      for (int i = 0; i < count; ++i) {
        Candidate c;
        if (strcmp(cfgs[i].name, t.config) == 0 &&
            cfgs[i].lds_bytes <= budget &&
            evaluate(*d, cfgs[i], i, cus, &c, t.splits != 0, t.splits)) {
          best = c;
          plan->from_tuned_table = 1;
        }
      }
    }
    // Otherwise rank: (modeled time, traffic, tiles, -N) over the
    // configurations within the LDS budget, each split-K configuration at
    // the split count that just covers the CUs and at a range of others
    // (more splits spread the work, fewer shorten the reduction).
    if (best.index < 0) {
      std::tuple<int64_t, int64_t, int64_t, int64_t, int64_t> best_rank;
      // Stream-K is not ranked: measured against the split counts it won
      // only where K is long (the partial tiles it publishes cost more
      // than the model prices); measured entries above select it.
      static const int kSplitChoices[] = {0, 1, 2, 3, 4, 5, 6, 8, 10, 12, 16};
      for (int i = 0; i < count; ++i) {
        // Column splits are not ranked: they replace their head below.
        if (cfgs[i].lds_bytes > budget || cfgs[i].table_only ||
            cfgs[i].head)
          continue;
        for (int forced : kSplitChoices) {
          if (forced && !cfgs[i].split_k)
            break;
          Candidate c;
          if (!evaluate(*d, cfgs[i], i, cus, &c, false, forced))
            continue;
          // Between equal modeled times (feed- or HBM-bound models) the
          // 16x16 MFMA form comes first where its tiles fill every CU: it
          // measured faster on every such f16 shape (4096^3 TN 6-8 %, C3
          // M = 2048 row-major B 1-4.5 %, transposed A 1-2 %).
          const int64_t wgs = c.tiles * c.splits * (d->batch > 0 ? d->batch : 1);
          const int64_t mfma16 = cfgs[i].mfma == 16 && wgs >= cus ? 1 : 0;
          auto rank = std::make_tuple(c.est_ns, -mfma16, c.traffic, c.tiles,
                                      -(int64_t)cfgs[i].bn);
          if (best.index < 0 || rank < best_rank) {
            best = c;
            best_rank = rank;
          }
        }
      }
      // A ranked unsplit pick gives way to the column split of its form
      // wherever one applies (the shape's 256x256 grid ends in a ragged
      // round that one round of half-size tiles covers): measured 7-11 %
      // faster at 2048 x 11008 than the head alone in every form (K = 4096
      // and 11008) and 2 % at M = 8192; for W8A16 at 2048 x 11008 also 7 %
      // faster than the ranked 128x256 tile (171.6 against 185.2 us). The
      // results are identical to the head's alone. The cost model's
      // aggregate operand feed
      // cannot see that gain (the tail grid fills 176 of the 256 CUs), so
      // the rule is measured, not modeled.
      if (best.index >= 0 && !cfgs[best.index].split_k) {
        for (int i = 0; i < count; ++i) {
          Candidate c;
          if (cfgs[i].head && cfgs[i].lds_bytes <= budget &&
              evaluate(*d, cfgs[i], i, cus, &c)) {
            best = c;
            break;
          }
        }
      }
    }
    if (best.index < 0)
      return IREE_MI355X_UNSUPPORTED;
    const FastConfig &c = cfgs[best.index];
    plan->config_index = best.index;
    snprintf(plan->config_name, sizeof(plan->config_name), "%s", c.name);
    plan->tile_m = c.bm;
    plan->tile_n = c.bn;
    plan->tile_k = c.bk;
    plan->lds_bytes = c.lds_bytes;
    plan->workgroups =
        best.sk_steps > 0
            ? best.sk_wgs
            : best.tiles * best.splits * (d->batch > 0 ? d->batch : 1);
    plan->threads = c.threads;
    plan->splits = best.splits;
    plan->k_split = best.k_split;
    plan->stream_k_steps = best.sk_steps;
    plan->workspace_bytes = best.workspace;
    plan->traffic_bytes = best.traffic;
    return IREE_MI355X_OK;
  }

  // General kernel: 64x64 tiles, 256 threads, 10 KiB LDS.
  snprintf(plan->config_name, sizeof(plan->config_name), "general_64x64");
  plan->tile_m = 64;
  plan->tile_n = 64;
  plan->tile_k = 64 / (d->a_elem == IREE_MI355X_ELEM_I8 &&
                               d->b_elem == IREE_MI355X_ELEM_I8
                           ? 1
                           : 2);
  plan->lds_bytes = 2 * 64 * 80;
  plan->workgroups = ((d->m + 63) / 64) * ((d->n + 63) / 64);
  plan->threads = 256;
  const int64_t ab = elem_bytes(d->a_elem), bb = elem_bytes(d->b_elem);
  plan->traffic_bytes = ab * d->m * d->k * ((d->n + 63) / 64) +
                        bb * d->n * d->k * ((d->m + 63) / 64);
  return IREE_MI355X_OK;
}

int iree_mi355x_mfma_config_count(void) {
  int count = 0;
  fast_configs(&count);
  return count;
}

int iree_mi355x_mfma_config_info(int index, const char **name,
                                 int32_t *b_form, int32_t *a_elem,
                                 int32_t *c_elem, int64_t *tile_m,
                                 int64_t *tile_n, int64_t *tile_k,
                                 int64_t *lds_bytes, int32_t *threads) {
  int count = 0;
  const FastConfig *cfgs = fast_configs(&count);
  if (index < 0 || index >= count)
    return IREE_MI355X_INVALID_ARGUMENT;
  const FastConfig &c = cfgs[index];
  if (name)
    *name = c.name;
  if (b_form)
    *b_form = c.b_mode;
  if (a_elem)
    *a_elem = c.elem == kElemI8 ? IREE_MI355X_ELEM_I8 : IREE_MI355X_ELEM_F16;
  if (c_elem)
    *c_elem = c.elem == kElemI8 ? IREE_MI355X_ELEM_I32
                                : (c.out_f32 ? IREE_MI355X_ELEM_F32
                                             : IREE_MI355X_ELEM_F16);
  if (tile_m)
    *tile_m = c.bm;
  if (tile_n)
    *tile_n = c.bn;
  if (tile_k)
    *tile_k = c.bk;
  if (lds_bytes)
    *lds_bytes = c.lds_bytes;
  if (threads)
    *threads = c.threads;
  return IREE_MI355X_OK;
}

int32_t iree_mi355x_mfma_config_layout_flags(int index) {
  int count = 0;
  const FastConfig *cfgs = fast_configs(&count);
  if (index < 0 || index >= count)
    return -1;
  return (int32_t)((cfgs[index].b_mode == kBTN
                        ? IREE_MI355X_MATMUL_B_TRANSPOSED
                        : 0u) |
                   (cfgs[index].a_trans ? IREE_MI355X_MATMUL_A_TRANSPOSED
                                        : 0u));
}

}  // extern "C"

namespace {

// The checks and the plan of one configuration run (the candidate it would
// launch), shared by the run and its workspace query.
int config_candidate(int index, int32_t splits, const void *a, const void *b,
                     const void *scale, const void *c, int64_t m, int64_t n,
                     int64_t k, int64_t lda, int64_t ldb, int64_t ldc,
                     uint32_t flags, Candidate *out) {
  int count = 0;
  const FastConfig *cfgs = fast_configs(&count);
  if (index < 0 || index >= count)
    return fail(IREE_MI355X_INVALID_ARGUMENT, "mfma_config: bad index %d",
                index);
  const FastConfig &cfg = cfgs[index];
  const int32_t ae = cfg.elem == kElemI8 ? IREE_MI355X_ELEM_I8
                                         : IREE_MI355X_ELEM_F16;
  const int32_t be = cfg.b_mode == kBW8 ? IREE_MI355X_ELEM_I8 : ae;
  const int32_t ce = cfg.elem == kElemI8
                         ? IREE_MI355X_ELEM_I32
                         : (cfg.out_f32 ? IREE_MI355X_ELEM_F32
                                        : IREE_MI355X_ELEM_F16);
  iree_mi355x_matmul_desc_t d;
  iree_mi355x_matmul_desc_init(&d, ae, be, ce, m, n, k, flags);
  d.has_scale = cfg.b_mode == kBW8;
  const int64_t aeb = elem_bytes(ae), beb = elem_bytes(be);
  d.a_aligned16 = a && fast_operand(a, lda * aeb);
  d.b_aligned16 = b && fast_operand(b, ldb * beb);
  const bool bt = flags & IREE_MI355X_MATMUL_B_TRANSPOSED;
  const bool at = flags & IREE_MI355X_MATMUL_A_TRANSPOSED;
  if (flags & ~(IREE_MI355X_MATMUL_B_TRANSPOSED | IREE_MI355X_MATMUL_ACCUMULATE |
                IREE_MI355X_MATMUL_OUT_F32 | IREE_MI355X_MATMUL_A_TRANSPOSED))
    return fail(IREE_MI355X_INVALID_ARGUMENT, "mfma_config: unknown flags");
  if (!c || (uintptr_t)c % elem_bytes(ce) != 0 || lda < (at ? m : k) ||
      ldb < (bt ? k : n) || ldc < n || m >= ((int64_t)1 << 31) ||
      n >= ((int64_t)1 << 31) || k >= ((int64_t)1 << 31) ||
      (d.has_scale && (!scale || (uintptr_t)scale % 2 != 0)))
    return fail(IREE_MI355X_INVALID_ARGUMENT, "mfma_config: bad arguments");
  if (splits < kStreamK || ((splits > 1 || splits == kStreamK) &&
                            !cfg.split_k))
    return fail(IREE_MI355X_INVALID_ARGUMENT,
                "mfma_config %s: %d splits", cfg.name, splits);
  if (!evaluate(d, cfg, index, kDefaultCus, out, true, splits))
    return fail(IREE_MI355X_UNSUPPORTED,
                "mfma_config %s: shape or layout does not fit", cfg.name);
  return IREE_MI355X_OK;
}

}  // namespace

extern "C" {

size_t iree_mi355x_matmul_mfma_config_workspace_bytes(int index,
                                                      int32_t splits,
                                                      int64_t m, int64_t n,
                                                      int64_t k,
                                                      uint32_t flags) {
  // Any 256-byte aligned operands with natural pitches plan alike.
  const void *p = (const void *)(uintptr_t)256;
  const bool bt = flags & IREE_MI355X_MATMUL_B_TRANSPOSED;
  const bool at = flags & IREE_MI355X_MATMUL_A_TRANSPOSED;
  Candidate cand;
  if (config_candidate(index, splits, p, p, p, p, m, n, k, at ? m : k,
                       bt ? k : n, n, flags, &cand) != IREE_MI355X_OK)
    return 0;
  return cand.workspace > 0 ? (size_t)cand.workspace : 0;
}

int iree_mi355x_matmul_mfma_config_split(
    int index, int32_t splits, const void *a, const void *b, const void *scale,
    void *c, int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb,
    int64_t ldc, uint32_t flags, void *workspace, size_t workspace_bytes,
    void *stream) {
  Candidate cand;
  int st = config_candidate(index, splits, a, b, scale, c, m, n, k, lda, ldb,
                            ldc, flags, &cand);
  if (st != IREE_MI355X_OK)
    return st;
  int count = 0;
  const FastConfig &cfg = fast_configs(&count)[index];
  if ((st = require_workspace(cfg.name, (size_t)cand.workspace, workspace,
                              workspace_bytes)) != IREE_MI355X_OK)
    return st;
  const bool bt = flags & IREE_MI355X_MATMUL_B_TRANSPOSED;
  const bool at = flags & IREE_MI355X_MATMUL_A_TRANSPOSED;
  MatmulArgs args{a, b, c, m, n, k, lda, ldb, ldc, bt ? 1 : 0,
                  (flags & IREE_MI355X_MATMUL_ACCUMULATE) ? 1 : 0, stream,
                  scale, cand.splits, cand.k_split,
                  cand.workspace > 0 ? workspace : nullptr};
  args.a_transposed = at ? 1 : 0;
  args.sk_steps = cand.sk_steps;
  args.sk_workgroups = (int)cand.sk_wgs;
  hipError_t e = cfg.launch(args);
  if (e != hipSuccess)
    return fail(IREE_MI355X_LAUNCH_FAILED, "%s: %s", cfg.name,
                hipGetErrorString(e));
  return IREE_MI355X_OK;
}

int iree_mi355x_matmul_mfma_config(int index, const void *a, const void *b,
                                   const void *scale, void *c, int64_t m,
                                   int64_t n, int64_t k, int64_t lda,
                                   int64_t ldb, int64_t ldc, uint32_t flags,
                                   void *workspace, size_t workspace_bytes,
                                   void *stream) {
  return iree_mi355x_matmul_mfma_config_split(index, 0, a, b, scale, c, m, n,
                                              k, lda, ldb, ldc, flags,
                                              workspace, workspace_bytes,
                                              stream);
}

}  // extern "C"
