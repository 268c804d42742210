// Dispatch classification and gfx950 tile planning for matched matmul
// dispatches. Host-only: no HIP call, usable without a GPU.
//
// Replaces the reference's HMX strategy selection and VTCM tile search:
//  * iree_mi355x_classify_matmul  <- isHmxCandidateContraction /
//    hasHmxElementTypes / isHmxLowerableMatmul / selectHmxStrategy
//    (CG/Strategy/Planning/Strategies/ContractionStrategy.cpp:133-213),
//    extended to the int8 and W8A16 dispatches HMX does not take (:141);
//  * iree_mi355x_plan_matmul      <- selectHmxTileSizes + planVTCMTiling
//    (CG/Strategy/Planning/VTCMPlanning.cpp:156-329) with the 2 MiB VTCM
//    budget (CG/Pipelines/TranslationPipeline.cpp:28-34) replaced by the
//    160 KiB LDS of one gfx950 CU, and the candidates by the compiled MFMA
//    macro-tiles. The ranking keeps the reference's tie-breaks (in budget,
//    least global traffic, fewest tiles, larger N) behind one key added
//    first: a modeled time, the slowest of MFMA work on the busiest CU, the
//    LDS-DMA operand feed and HBM traffic, plus fixed latencies per round of
//    workgroups and per K split, since 256 CUs run the tiles in parallel
//    where the DSP ran them in sequence (RT/dsp/command_buffer.c:670-719).
//    Split-K candidates divide K so that the tiles times splits cover the
//    CUs. A measured table (autotuner) is consulted before the ranking.
#ifndef IREE_MI355X_PLANNER_H_
#define IREE_MI355X_PLANNER_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum iree_mi355x_elem_e {
  IREE_MI355X_ELEM_F16 = 0,
  IREE_MI355X_ELEM_I8 = 1,
  IREE_MI355X_ELEM_I32 = 2,
  IREE_MI355X_ELEM_F32 = 3,
} iree_mi355x_elem_t;

typedef enum iree_mi355x_family_e {
  IREE_MI355X_FAMILY_NONE = 0,     // not a dispatch this library takes
  IREE_MI355X_FAMILY_MFMA = 1,     // LDS-DMA MFMA macro-tile kernel
  IREE_MI355X_FAMILY_GENERAL = 2,  // bounds-checked MFMA kernel, any shape
  IREE_MI355X_FAMILY_GEMV = 3,     // HBM-streaming skinny kernel (M <= 4)
} iree_mi355x_family_t;

typedef struct iree_mi355x_matmul_desc_t {
  int32_t a_elem, b_elem, c_elem;  // iree_mi355x_elem_t
  int64_t m, n, k;
  uint32_t flags;            // IREE_MI355X_MATMUL_* (kernels header)
  int32_t a_aligned16;       // A base and row pitch are 16-byte aligned
  int32_t b_aligned16;       // B base and row pitch are 16-byte aligned
  int32_t has_scale;         // per-column f16 scale (W8A16)
  int64_t lds_budget_bytes;  // per-workgroup LDS budget (default 160 KiB)
  int32_t num_cus;           // CUs the tiles spread over (default 256)
  int64_t batch;             // matrices per dispatch (default 1)
} iree_mi355x_matmul_desc_t;

typedef struct iree_mi355x_matmul_plan_t {
  int32_t family;        // iree_mi355x_family_t
  int32_t config_index;  // MFMA: index into the compiled config table
  // "<head>+<tail>": a column split, two launches on the call's stream (the
  // head configuration over whole rounds of the CUs, then the tail over the
  // remaining columns); the tail is named without the type and B form
  // prefix it shares with the head ("f16_nn_256x256x64_w2x4_s2_m16+
  // 256x128x64_w2x4_s2_m16"); `workgroups` counts both grids.
  char config_name[64];
  int64_t tile_m, tile_n, tile_k;  // workgroup macro-tile (the VTCM tile)
  int64_t lds_bytes;               // LDS per workgroup
  int64_t workgroups;
  int32_t threads;                 // threads per workgroup
  int32_t splits;                  // K splits (GEMV, split-K MFMA)
  int32_t k_split;                 // K elements per split (split-K MFMA)
  int64_t workspace_bytes;
  int64_t traffic_bytes;           // modeled global->LDS bytes of the plan
  int32_t from_tuned_table;        // 1 if a measured entry chose it
  // Stream-K (split-K configuration, batch 1): K stages per workgroup; the
  // workgroups take equal runs of the (tile, K stage) pairs and `splits`
  // is the most runs one tile spans. 0: one tile (split) per workgroup.
  int32_t stream_k_steps;
} iree_mi355x_matmul_plan_t;

// Fills defaults: both operands assumed 16-byte aligned, no scale, 160 KiB
// LDS, 256 CUs, batch 1.
void iree_mi355x_matmul_desc_init(iree_mi355x_matmul_desc_t *desc,
                                  int32_t a_elem, int32_t b_elem,
                                  int32_t c_elem, int64_t m, int64_t n,
                                  int64_t k, uint32_t flags);

// Which kernel family takes the dispatch (FAMILY_NONE for element types no
// kernel computes). Mirrors the HMX eligibility rules, see above.
int32_t iree_mi355x_classify_matmul(const iree_mi355x_matmul_desc_t *desc);

// Full plan: family, macro-tile, resources. Returns 0 (IREE_MI355X_OK) or
// IREE_MI355X_UNSUPPORTED.
int iree_mi355x_plan_matmul(const iree_mi355x_matmul_desc_t *desc,
                            iree_mi355x_matmul_plan_t *plan);

// B operand forms of the MFMA family.
typedef enum iree_mi355x_b_form_e {
  IREE_MI355X_B_FORM_TN = 0,     // B [N,K], element type of A
  IREE_MI355X_B_FORM_NN = 1,     // B [K,N] f16
  IREE_MI355X_B_FORM_W8A16 = 2,  // B [K,N] int8 + per-column f16 scale
} iree_mi355x_b_form_t;

// The compiled MFMA configurations (for the autotuner and the library export
// table): name, operand forms, macro-tile and resources of entry `index`.
int iree_mi355x_mfma_config_count(void);
int iree_mi355x_mfma_config_info(int index, const char **name,
                                 int32_t *b_form, int32_t *a_elem,
                                 int32_t *c_elem, int64_t *tile_m,
                                 int64_t *tile_n, int64_t *tile_k,
                                 int64_t *lds_bytes, int32_t *threads);

// The layout flags (IREE_MI355X_MATMUL_B_TRANSPOSED, _A_TRANSPOSED) a
// configuration's operands must carry, or -1 for a bad index.
int32_t iree_mi355x_mfma_config_layout_flags(int index);

// Launch one compiled MFMA configuration by index on an eligible shape
// (autotuner entry). Arguments as iree_mi355x_matmul_f16 / _i8 /
// _w8a16_matmul (scale is read only by the W8A16 form); flags must match the
// configuration's B form. A split-K run takes its partials and counters
// from `workspace` (sized by iree_mi355x_matmul_mfma_config_workspace_bytes,
// zero-filled before its first use; IREE_MI355X_WORKSPACE_TOO_SMALL when
// absent or short). Returns IREE_MI355X_UNSUPPORTED if the shape does not
// tile exactly.
int iree_mi355x_matmul_mfma_config(int index, const void *a, const void *b,
                                   const void *scale, void *c, int64_t m,
                                   int64_t n, int64_t k, int64_t lda,
                                   int64_t ldb, int64_t ldc, uint32_t flags,
                                   void *workspace, size_t workspace_bytes,
                                   void *stream);

// As iree_mi355x_matmul_mfma_config, with the K split count of a split-K
// configuration forced (0: the planner's; clamped to one K stage per split;
// IREE_MI355X_SPLITS_STREAM_K: stream-K runs, batch 1), so the autotuner can
// time every split.
#define IREE_MI355X_SPLITS_STREAM_K (-1)
int iree_mi355x_matmul_mfma_config_split(
    int index, int32_t splits, const void *a, const void *b, const void *scale,
    void *c, int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb,
    int64_t ldc, uint32_t flags, void *workspace, size_t workspace_bytes,
    void *stream);

// Workspace bytes a configuration run of this shape and split count needs
// with 16-byte aligned operands of natural pitch (0: none, or the run is
// refused). No counterpart in the reference, whose tile search has no
// run-time scratch; it sizes the autotuner's workspace.
size_t iree_mi355x_matmul_mfma_config_workspace_bytes(int index,
                                                      int32_t splits,
                                                      int64_t m, int64_t n,
                                                      int64_t k,
                                                      uint32_t flags);

#ifdef __cplusplus
}  // extern "C"
#endif

#endif  // IREE_MI355X_PLANNER_H_
