// Runtime caller of the MI355X dispatch library: command buffers that record
// dispatches of an executable library, fills, copies and barriers, and submit
// them onto HIP streams, running the dispatches between two barriers
// concurrently on up to N streams.
//
// Replaces the Hexagon HAL command buffer and its DSP-side scheduler:
//  * recording (RT/command_buffer.c:586-665 serializes each dispatch with its
//    constants and buffer references; binding-table slots are resolved at
//    submission) is kept on the host, constants copied at record time;
//  * execution (RT/dsp/command_buffer.c:807-913: up to
//    --hexagon_max_concurrent_dispatches dispatches in flight between
//    barriers, RT/registration/driver_module.c:20-23, each in its own VTCM
//    partition) becomes up to `max_concurrent` lane streams: the commands of
//    one barrier segment go round-robin over the lanes, a barrier joins every
//    lane (events) and the end joins them back into the caller's stream;
//  * the VTCM partition of a dispatch becomes a split-K / GEMV workspace
//    slice per lane, sized by validating every dispatch of the command buffer
//    (its workspace query) before any of it is enqueued.
//
// Every enqueue goes through the executable library's export functions on the
// caller's stream or a lane stream; nothing here allocates device memory
// except the runtime's own lane workspace (when the caller passes none) and
// the lane streams and events, created on first use and kept for the process.
// A submission with max_concurrent = 1 enqueues in order on the caller's
// stream only, so it can be captured into a HIP graph; a submission with more
// lanes into a capturing stream is refused (UNSUPPORTED).
#ifndef IREE_MI355X_RUNTIME_H_
#define IREE_MI355X_RUNTIME_H_

#include <stddef.h>
#include <stdint.h>

#include "iree_mi355x_executable_library.h"

#ifdef __cplusplus
extern "C" {
#endif

// A buffer reference: a direct device pointer, or a slot of the binding table
// given at submission (the reference's binding-table slots, resolved by the
// DSP at execution, RT/dsp/command_buffer.c:600-633).
#define IREE_MI355X_BINDING_DIRECT 0xFFFFFFFFu
#define IREE_MI355X_WHOLE_BUFFER UINT64_MAX

typedef struct iree_mi355x_buffer_ref_t {
  uint32_t binding_slot;  // binding-table slot, or IREE_MI355X_BINDING_DIRECT
  void *buffer;           // the device pointer when direct
  uint64_t offset;        // bytes into the slot or buffer
  uint64_t length;        // bytes; IREE_MI355X_WHOLE_BUFFER: rest of the slot
} iree_mi355x_buffer_ref_t;

typedef struct iree_mi355x_binding_t {
  void *buffer;     // device pointer
  uint64_t length;  // bytes
} iree_mi355x_binding_t;

typedef struct iree_mi355x_command_buffer_t iree_mi355x_command_buffer_t;

// Lanes used when a submission asks for 0: one (in order). Lane 0 is the
// caller's stream; every further lane is a stream on another hardware queue,
// and a fork / join across hardware queues costs ~35-40 us of GPU time per
// submission on MI355X. The planner already spreads a dispatch over every CU
// (split-K for skinny shapes), so lanes pay only for long dispatches that
// leave most CUs idle, and are requested explicitly.
#define IREE_MI355X_DEFAULT_CONCURRENCY 1u
#define IREE_MI355X_MAX_CONCURRENCY 8u

// New, empty command buffer recording against `library` (NULL: this
// library's own table, iree_mi355x_executable_library_query).
int iree_mi355x_command_buffer_create(
    const iree_mi355x_executable_library_t *library,
    iree_mi355x_command_buffer_t **out_command_buffer);

void iree_mi355x_command_buffer_release(
    iree_mi355x_command_buffer_t *command_buffer);

// Record a dispatch of export `ordinal` with its push constants (copied) and
// bindings (as the export documents them).
int iree_mi355x_command_buffer_dispatch(
    iree_mi355x_command_buffer_t *command_buffer, uint32_t ordinal,
    const uint32_t *constants, uint32_t constant_count,
    const iree_mi355x_buffer_ref_t *bindings, uint32_t binding_count);

// Fill `target` with a 1-, 2- or 4-byte pattern; offset and length must be
// multiples of the pattern length. Runs as a kernel, not a memset, so a
// captured graph holds no memset node.
int iree_mi355x_command_buffer_fill(
    iree_mi355x_command_buffer_t *command_buffer,
    iree_mi355x_buffer_ref_t target, const void *pattern,
    uint32_t pattern_length);

// Copy `length` bytes from `source` to `target` (device to device; the ranges
// must not overlap).
int iree_mi355x_command_buffer_copy(
    iree_mi355x_command_buffer_t *command_buffer,
    iree_mi355x_buffer_ref_t source, iree_mi355x_buffer_ref_t target,
    uint64_t length);

// Every command recorded before completes before any recorded after starts
// (the reference's execution barrier, RT/dsp/command_buffer.c:915-933).
int iree_mi355x_command_buffer_barrier(
    iree_mi355x_command_buffer_t *command_buffer);

// Ends recording; a command buffer is submitted only after this.
int iree_mi355x_command_buffer_end(
    iree_mi355x_command_buffer_t *command_buffer);

// Bytes of workspace a submission with this binding table and concurrency
// needs (one slice per lane, each the largest any dispatch asks for), after
// validating every command; 0 on error (see iree_mi355x_last_error).
size_t iree_mi355x_command_buffer_workspace_bytes(
    const iree_mi355x_command_buffer_t *command_buffer,
    const iree_mi355x_binding_t *binding_table, uint32_t binding_count,
    uint32_t max_concurrent);

// Submit on `stream` (hipStream_t; NULL = the null stream): resolves the
// binding table, validates every command (a failing one enqueues nothing),
// then enqueues. max_concurrent: 0 = IREE_MI355X_DEFAULT_CONCURRENCY, 1 = in
// order on `stream` alone, at most IREE_MI355X_MAX_CONCURRENCY. `workspace`
// holds the lane slices, sized by iree_mi355x_command_buffer_workspace_bytes
// (one slice is that query at concurrency 1); a submission that needs one
// and has none, or a short one, returns IREE_MI355X_WORKSPACE_TOO_SMALL
// before enqueueing anything (the runtime allocates no device memory). Lane
// l's slice starts at l slices and opens with its arrival counters: a
// workspace must be zero-filled before its first use and then serve
// submissions of one slice size only (its flat calls' counters likewise sit
// at its start), after each of which the kernels leave every lane's
// counters zero again. Submissions that overlap must not share a
// workspace. Work is stream-ordered after `stream`'s prior work, and
// `stream`'s later work is ordered after it.
int iree_mi355x_command_buffer_submit(
    const iree_mi355x_command_buffer_t *command_buffer,
    const iree_mi355x_binding_t *binding_table, uint32_t binding_count,
    uint32_t max_concurrent, void *workspace, size_t workspace_bytes,
    void *stream);

// Recorded commands (for inspection and tests).
uint32_t iree_mi355x_command_buffer_count(
    const iree_mi355x_command_buffer_t *command_buffer);

// One stream operation of a submission's lane schedule, in issue order.
// Lane 0 is the caller's stream, lanes 1.. the runtime's lane streams.
// Event 0 is the fork event (recorded on the caller's stream first); event
// 1 + l is lane l's event.
typedef enum iree_mi355x_lane_op_kind_e {
  IREE_MI355X_LANE_OP_RECORD = 0,   // record `event` on `lane`
  IREE_MI355X_LANE_OP_WAIT = 1,     // `lane` waits for `event`
  IREE_MI355X_LANE_OP_ENQUEUE = 2,  // command `command` on `lane`
} iree_mi355x_lane_op_kind_t;
typedef struct iree_mi355x_lane_op_t {
  uint32_t kind;
  uint32_t lane;
  uint32_t event;
  uint32_t command;
} iree_mi355x_lane_op_t;

// The lane schedule a submission with this concurrency issues (the same
// rules as iree_mi355x_command_buffer_submit: commands of a barrier segment
// dealt round-robin over the lanes, each lane's first command of a segment
// after a wait on the previous segment's other lanes, the other lanes
// joined back into the caller's stream at the end). Writes at most
// `capacity` operations to `ops` and returns how many the schedule has; no
// device is touched. The reference's DSP scheduler has no such query
// (RT/dsp/command_buffer.c:807-913 schedules inside its submit).
uint32_t iree_mi355x_command_buffer_lane_schedule(
    const iree_mi355x_command_buffer_t *command_buffer,
    uint32_t max_concurrent, iree_mi355x_lane_op_t *ops, uint32_t capacity);

#ifdef __cplusplus
}  // extern "C"
#endif

#endif  // IREE_MI355X_RUNTIME_H_
