// Executable-library ABI of the MI355X dispatch library: what a HAL driver
// loads (dlopen + dlsym of IREE_MI355X_EXECUTABLE_LIBRARY_EXPORT_NAME) to find
// the dispatch functions of matched dispatch regions.
//
// Same shape as the reference's Hexagon executable library
// (plugins/runtime/hexagon/dsp/rt/executable_library.h:40-250): a versioned
// header, an import table and a struct-of-arrays export table with per-export
// resource attributes. Differences, each forced by the GPU:
//  * the workgroup loop the DSP scheduler runs on the host
//    (RT/dsp/command_buffer.c:670-719) is the GPU grid, so a dispatch function
//    is called once per dispatch and has no workgroup_state argument;
//  * the dispatch state carries the hipStream_t the work is enqueued on;
//  * resource attributes report LDS bytes and threads per workgroup where the
//    reference reports VTCM bytes and HVX thread counts (:180-219).
#ifndef IREE_MI355X_EXECUTABLE_LIBRARY_H_
#define IREE_MI355X_EXECUTABLE_LIBRARY_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint32_t iree_mi355x_executable_library_version_t;

// 'MI' in the upper half, like the reference's 'HX' (0x48580001,
// executable_library.h:49-52), so it cannot be mistaken for an upstream IREE
// version.
#define IREE_MI355X_EXECUTABLE_LIBRARY_VERSION_1 0x4D490001u
#define IREE_MI355X_EXECUTABLE_LIBRARY_VERSION_LATEST \
  IREE_MI355X_EXECUTABLE_LIBRARY_VERSION_1
#define IREE_MI355X_EXECUTABLE_LIBRARY_EXPORT_NAME \
  "iree_mi355x_executable_library_query"

typedef struct iree_mi355x_executable_library_header_t {
  iree_mi355x_executable_library_version_t version;
  const char *name;
} iree_mi355x_executable_library_header_t;

typedef struct iree_mi355x_executable_environment_t {
  const uint32_t *constants;  // executable-level constants (unused: NULL)
} iree_mi355x_executable_environment_t;

// Per-dispatch state. `constants` are the push constants (u32), whose layout
// each export documents below; 64-bit extents are passed as lo/hi pairs.
//
// `workspace` is the split-K / GEMV scratch of this dispatch, sized by a
// workspace query (below); a dispatch that needs one and gets NULL, or a
// short one, returns IREE_MI355X_WORKSPACE_TOO_SMALL before anything is
// enqueued (the library allocates no device memory). Its counter region
// must be zero before first use, and the kernels leave it zero. Dispatches
// that may run concurrently need disjoint ones.
//
// `workspace_query`, when non-NULL, turns the call into a validation: every
// check and the plan run, nothing is allocated or enqueued, and the bytes of
// workspace the dispatch needs are written there. A runtime validates a whole
// command buffer this way before enqueuing any of it (where the reference's
// DSP scheduler sizes VTCM partitions, RT/dsp/command_buffer.c:807-913).
typedef struct iree_mi355x_executable_dispatch_state_t {
  uint32_t constant_count;
  const uint32_t *constants;
  uint32_t binding_count;
  void *const *binding_ptrs;       // device pointers
  const size_t *binding_lengths;   // bytes, 1:1 with binding_ptrs
  void *stream;                    // hipStream_t
  void *workspace;
  size_t workspace_bytes;
  size_t *workspace_query;
} iree_mi355x_executable_dispatch_state_t;

// Returns 0 on success. Unlike the reference (where non-zero means device
// loss, executable_library.h:168-173) the value is an iree_mi355x_status_t and
// nothing has been enqueued when it is non-zero: binding ranges that do not
// cover the accessed extents are rejected before launch.
typedef int (*iree_mi355x_executable_dispatch_fn_t)(
    const iree_mi355x_executable_environment_t *environment,
    const iree_mi355x_executable_dispatch_state_t *dispatch_state);

enum iree_mi355x_dispatch_flag_bits_e {
  IREE_MI355X_DISPATCH_FLAG_NONE = 0ull,
  IREE_MI355X_DISPATCH_FLAG_RESOURCES_VALID = 1ull << 0,
  IREE_MI355X_DISPATCH_FLAG_USES_MFMA = 1ull << 1,
  IREE_MI355X_DISPATCH_FLAG_USES_LDS_DMA = 1ull << 2,
  IREE_MI355X_DISPATCH_FLAG_USES_WORKSPACE = 1ull << 3,
};

// 24 bytes, field for field the size of the reference's attrs.
typedef struct iree_mi355x_executable_dispatch_attrs_t {
  uint64_t flags;      // iree_mi355x_dispatch_flag_bits_e
  uint64_t lds_bytes;  // largest static LDS of any kernel the export launches
  uint64_t threads;    // largest workgroup size it launches
} iree_mi355x_executable_dispatch_attrs_t;

typedef struct iree_mi355x_executable_import_table_t {
  uint32_t count;
  const char *const *symbols;
} iree_mi355x_executable_import_table_t;

typedef struct iree_mi355x_executable_export_table_t {
  uint32_t count;
  const iree_mi355x_executable_dispatch_fn_t *ptrs;
  const iree_mi355x_executable_dispatch_attrs_t *attrs;
  const char *const *names;
} iree_mi355x_executable_export_table_t;

typedef struct iree_mi355x_executable_library_t {
  const iree_mi355x_executable_library_header_t *header;
  iree_mi355x_executable_import_table_t imports;
  iree_mi355x_executable_export_table_t exports;
} iree_mi355x_executable_library_t;

// Returns the library (as a pointer to its header pointer, like the
// reference's query) or NULL if max_version is not the version it was built
// with. `environment` is not read.
const iree_mi355x_executable_library_header_t **
iree_mi355x_executable_library_query(
    iree_mi355x_executable_library_version_t max_version,
    const iree_mi355x_executable_environment_t *environment);

// Resources of one compiled kernel: the measured side of the export
// attributes above, which must cover every kernel an export may launch (the
// reference annotates each export with the VTCM, HVX threads and HMX use of
// its dispatch, CG/Transforms/HexagonAnnotateDispatchResources.cpp).
typedef struct iree_mi355x_kernel_resources_t {
  const char *name;           // MFMA configuration or kernel name
  uint32_t exports;           // bit i: export ordinal i may launch it
  int32_t threads;            // workgroup size it is launched with
  int32_t vgprs;              // registers per lane (hipFuncGetAttributes)
  int32_t lds_bytes;          // static LDS per workgroup
  int32_t scratch_bytes;      // private memory per lane (register spills)
  int32_t max_threads;        // the kernel's launch bound
  int32_t workgroups_per_cu;  // resident workgroups per CU at `threads`
} iree_mi355x_kernel_resources_t;

// Number of compiled kernels (MFMA configurations, general, GEMV, attention
// and runtime kernels).
int iree_mi355x_kernel_count(void);

// Fills name, exports and threads always; the other fields load the kernel
// and need a device (IREE_MI355X_NO_DEVICE without one).
int iree_mi355x_kernel_resources(int index,
                                 iree_mi355x_kernel_resources_t *out);

// Export push-constant layouts (u32 words):
//  "matmul_f16"   constants: m_lo m_hi n_lo n_hi k_lo k_hi lda_lo lda_hi
//                 ldb_lo ldb_hi ldc_lo ldc_hi flags   bindings: a b c
//  "matmul_i8"    same constants and bindings as matmul_f16
//  "w8a16_matmul" same constants   bindings: x w scale y
//  "attention_f16" constants: batch heads seq_q seq_kv head_dim
//                 scale_bits(f32) flags [kv_heads q_stride_batch_lo/hi
//                 q_stride_head_lo/hi q_stride_row_lo/hi, then the same
//                 three for k, v and o [head_dim_v mask_stride_batch_lo/hi
//                 mask_stride_head_lo/hi mask_stride_row_lo/hi
//                 mask_stride_key_lo/hi]] (7, 32 or 41 words); flags
//                 IREE_MI355X_ATTENTION_CAUSAL, _OUT_F32, _MASK (41 words)
//                 bindings: q k v o [mask]
//  "batch_matmul_f16" constants: the matmul_f16 ones, then batch_lo batch_hi
//                 stride_a_lo/hi stride_b_lo/hi stride_c_lo/hi activation
//                 epilogue_bindings (bit 0 bias, bit 1 multiplier)
//                 ld_multiplier_lo/hi batch_stride_multiplier_lo/hi
//                 bindings: a b c [bias] [multiplier]

#ifdef __cplusplus
}  // extern "C"
#endif

#endif  // IREE_MI355X_EXECUTABLE_LIBRARY_H_
