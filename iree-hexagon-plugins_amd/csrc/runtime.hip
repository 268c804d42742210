// Runtime caller of the dispatch library (include/iree_mi355x_runtime.h):
// command buffers recorded on the host and submitted onto HIP streams.
//
// The reference records serialized commands on the host
// (RT/command_buffer.c:586-665) and its DSP scheduler runs the dispatches
// between barriers with up to max_concurrent in flight, each on a worker
// thread with its own VTCM partition (RT/dsp/command_buffer.c:807-913). Here a
// submission first validates every command through the export functions'
// workspace query (so a bad command enqueues nothing and the largest split-K
// workspace is known), then deals the commands of each barrier segment
// round-robin onto up to N lane streams, each lane with its own workspace
// slice, and joins the lanes with events at every barrier and at the end.
#include <hip/hip_runtime.h>
#include <rocprofiler-sdk-roctx/roctx.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/iree_mi355x_kernels.h"
#include "../../include/iree_mi355x_runtime.h"
#include "kernels_internal.h"

namespace ihp {

int fail(int status, const char *fmt, ...);

// Fill [dst, dst + length) with a pattern whose byte i is byte i % 4 of
// `word` (the 1-, 2- or 4-byte pattern repeated to four bytes). Whole 16-byte
// chunks are written as vectors, the unaligned head and tail bytewise.
__global__ __launch_bounds__(256) void fill_kernel(unsigned char *dst,
                                                   uint64_t length,
                                                   uint32_t word) {
  const uintptr_t base = (uintptr_t)dst;
  const uintptr_t a0 = (base + 15) & ~(uintptr_t)15;
  const uintptr_t end = base + length;
  const uintptr_t a1 = end & ~(uintptr_t)15;
  const uint64_t tid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t nthreads = (uint64_t)gridDim.x * blockDim.x;
  auto byte_at = [&](uint64_t i) {
    return (unsigned char)(word >> (8 * (i & 3)));
  };
  if (a0 >= a1) {  // no whole chunk
    for (uint64_t i = tid; i < length; i += nthreads)
      dst[i] = byte_at(i);
    return;
  }
  const uint64_t head = a0 - base, tail = end - a1;
  if (tid < head)
    dst[tid] = byte_at(tid);
  if (tid < tail)
    dst[(a1 - base) + tid] = byte_at((a1 - base) + tid);
  // Every chunk starts at the same pattern phase (16 is a multiple of 4).
  const uint32_t rot = (uint32_t)(head & 3);
  const uint32_t w = rot ? (word >> (8 * rot)) | (word << (32 - 8 * rot)) : word;
  const uint4 v = make_uint4(w, w, w, w);
  uint4 *body = (uint4 *)a0;
  const uint64_t chunks = (a1 - a0) / 16;
  for (uint64_t j = tid; j < chunks; j += nthreads)
    body[j] = v;
}

const KernelEntry *runtime_kernels(int *count) {
  static const KernelEntry all[] = {
      {"runtime_fill", (const void *)&fill_kernel, 256, 0u},
  };
  *count = 1;
  return all;
}

namespace {

struct Ref {
  uint32_t slot = IREE_MI355X_BINDING_DIRECT;
  void *ptr = nullptr;
  uint64_t offset = 0;
  uint64_t length = 0;
};

Ref to_ref(const iree_mi355x_buffer_ref_t &r) {
  Ref out;
  out.slot = r.binding_slot;
  out.ptr = r.buffer;
  out.offset = r.offset;
  out.length = r.length;
  return out;
}

enum Kind { kDispatch, kFill, kCopy, kBarrier };

struct Command {
  Kind kind = kBarrier;
  uint32_t ordinal = 0;             // dispatch
  std::vector<uint32_t> constants;  // dispatch
  std::vector<Ref> bindings;        // dispatch
  Ref target, source;               // fill / copy
  uint64_t length = 0;              // copy
  uint32_t word = 0;                // fill: pattern repeated to 4 bytes
  uint32_t pattern_length = 0;      // fill
};

}  // namespace
}  // namespace ihp

struct iree_mi355x_command_buffer_t {
  const iree_mi355x_executable_library_t *library = nullptr;
  std::vector<ihp::Command> commands;
  bool ended = false;
};

namespace ihp {
namespace {

const iree_mi355x_executable_library_t *own_library() {
  return (const iree_mi355x_executable_library_t *)
      iree_mi355x_executable_library_query(
          IREE_MI355X_EXECUTABLE_LIBRARY_VERSION_LATEST, nullptr);
}

int recording(const iree_mi355x_command_buffer_t *cb, const char *who) {
  if (!cb)
    return fail(IREE_MI355X_INVALID_ARGUMENT, "%s: null command buffer", who);
  if (cb->ended)
    return fail(IREE_MI355X_INVALID_ARGUMENT,
                "%s: command buffer already ended", who);
  return IREE_MI355X_OK;
}

// A reference resolved against the binding table: device range [ptr, +len).
int resolve(const Ref &r, const iree_mi355x_binding_t *table, uint32_t count,
            uint32_t index, const char *what, char **ptr, uint64_t *len) {
  if (r.slot == IREE_MI355X_BINDING_DIRECT) {
    if (!r.ptr)
      return fail(IREE_MI355X_INVALID_ARGUMENT, "command %u: %s: null buffer",
                  index, what);
    if (r.length == IREE_MI355X_WHOLE_BUFFER)
      return fail(IREE_MI355X_INVALID_ARGUMENT,
                  "command %u: %s: a direct buffer needs a length", index,
                  what);
    *ptr = (char *)r.ptr + r.offset;
    *len = r.length;
    return IREE_MI355X_OK;
  }
  if (!table || r.slot >= count)
    return fail(IREE_MI355X_INVALID_ARGUMENT,
                "command %u: %s: slot %u outside the binding table (%u)",
                index, what, r.slot, count);
  const iree_mi355x_binding_t &b = table[r.slot];
  if (!b.buffer)
    return fail(IREE_MI355X_INVALID_ARGUMENT,
                "command %u: %s: slot %u is unbound", index, what, r.slot);
  if (r.offset > b.length)
    return fail(IREE_MI355X_INVALID_ARGUMENT,
                "command %u: %s: offset %llu past slot %u (%llu bytes)", index,
                what, (unsigned long long)r.offset, r.slot,
                (unsigned long long)b.length);
  const uint64_t avail = b.length - r.offset;
  const uint64_t l = r.length == IREE_MI355X_WHOLE_BUFFER ? avail : r.length;
  if (l > avail)
    return fail(IREE_MI355X_INVALID_ARGUMENT,
                "command %u: %s: %llu bytes from offset %llu overrun slot %u "
                "(%llu bytes)",
                index, what, (unsigned long long)l,
                (unsigned long long)r.offset, r.slot,
                (unsigned long long)b.length);
  *ptr = (char *)b.buffer + r.offset;
  *len = l;
  return IREE_MI355X_OK;
}

// One command with every reference resolved, ready to enqueue.
struct Ready {
  std::vector<void *> ptrs;     // dispatch bindings
  std::vector<size_t> lengths;  // dispatch binding lengths
  char *target = nullptr, *source = nullptr;
  uint64_t target_length = 0;
};

// Resolve and validate every command; the largest workspace any dispatch
// asks for goes to *max_workspace. Enqueues nothing.
int prepare(const iree_mi355x_command_buffer_t *cb,
            const iree_mi355x_binding_t *table, uint32_t count,
            std::vector<Ready> *out, size_t *max_workspace) {
  *max_workspace = 0;
  out->assign(cb->commands.size(), Ready());
  const iree_mi355x_executable_export_table_t &ex = cb->library->exports;
  for (uint32_t i = 0; i < (uint32_t)cb->commands.size(); ++i) {
    const Command &c = cb->commands[i];
    Ready &r = (*out)[i];
    int st;
    switch (c.kind) {
      case kDispatch: {
        r.ptrs.resize(c.bindings.size());
        r.lengths.resize(c.bindings.size());
        for (size_t b = 0; b < c.bindings.size(); ++b) {
          char *p;
          uint64_t l;
          if ((st = resolve(c.bindings[b], table, count, i, "binding", &p,
                            &l)))
            return st;
          r.ptrs[b] = p;
          r.lengths[b] = (size_t)l;
        }
        size_t need = 0;
        iree_mi355x_executable_dispatch_state_t s = {};
        s.constant_count = (uint32_t)c.constants.size();
        s.constants = c.constants.data();
        s.binding_count = (uint32_t)r.ptrs.size();
        s.binding_ptrs = r.ptrs.data();
        s.binding_lengths = r.lengths.data();
        s.workspace_query = &need;
        if ((st = ex.ptrs[c.ordinal](nullptr, &s))) {
          const std::string why = iree_mi355x_last_error();
          return fail(st, "command %u (%s): %s", i, ex.names[c.ordinal],
                      why.c_str());
        }
        *max_workspace = std::max(*max_workspace, need);
        break;
      }
      case kFill:
        if ((st = resolve(c.target, table, count, i, "fill target", &r.target,
                          &r.target_length)))
          return st;
        if (c.target.offset % c.pattern_length ||
            r.target_length % c.pattern_length)
          return fail(IREE_MI355X_INVALID_ARGUMENT,
                      "command %u: fill range not a multiple of the %u-byte "
                      "pattern",
                      i, c.pattern_length);
        break;
      case kCopy: {
        uint64_t sl = 0;
        if ((st = resolve(c.source, table, count, i, "copy source", &r.source,
                          &sl)) ||
            (st = resolve(c.target, table, count, i, "copy target", &r.target,
                          &r.target_length)))
          return st;
        if (sl < c.length || r.target_length < c.length)
          return fail(IREE_MI355X_INVALID_ARGUMENT,
                      "command %u: copy of %llu bytes overruns its ranges", i,
                      (unsigned long long)c.length);
        if (r.source < r.target + c.length && r.target < r.source + c.length &&
            c.length > 0)
          return fail(IREE_MI355X_INVALID_ARGUMENT,
                      "command %u: copy ranges overlap", i);
        r.target_length = c.length;
        break;
      }
      case kBarrier:
        break;
    }
  }
  return IREE_MI355X_OK;
}

// Lanes a submission uses: the requested concurrency, but no more than the
// largest barrier segment holds.
uint32_t lanes_for(const iree_mi355x_command_buffer_t *cb, uint32_t requested) {
  uint32_t widest = 0, run = 0;
  for (const Command &c : cb->commands) {
    if (c.kind == kBarrier) {
      run = 0;
    } else {
      widest = std::max(widest, ++run);
    }
  }
  return std::max(1u, std::min(requested, widest));
}

size_t slice_bytes(size_t need) { return (need + 255) & ~(size_t)255; }

// The stream operations of a concurrent submission, in issue order: fork
// record on the caller's stream; per barrier segment, each lane's first
// command after waits on the previous segment's events of the other lanes
// (a lane's own earlier work is already ahead of it in stream order), then
// one record per lane used; at the end, each other lane used records its
// event and the caller's stream waits on it.
std::vector<iree_mi355x_lane_op_t> lane_schedule(
    const iree_mi355x_command_buffer_t *cb, uint32_t lanes) {
  std::vector<iree_mi355x_lane_op_t> ops;
  auto op = [&](uint32_t kind, uint32_t lane, uint32_t event,
                uint32_t command) {
    ops.push_back({kind, lane, event, command});
  };
  const uint32_t n = (uint32_t)cb->commands.size();
  if (lanes <= 1) {
    for (uint32_t j = 0; j < n; ++j)
      if (cb->commands[j].kind != kBarrier)
        op(IREE_MI355X_LANE_OP_ENQUEUE, 0, 0, j);
    return ops;
  }
  struct Prior {
    uint32_t event, lane;
  };
  std::vector<Prior> prior = {{0, 0}};
  bool used_ever[IREE_MI355X_MAX_CONCURRENCY] = {};
  op(IREE_MI355X_LANE_OP_RECORD, 0, 0, 0);
  uint32_t i = 0;
  while (i < n) {
    uint32_t end = i;
    while (end < n && cb->commands[end].kind != kBarrier)
      ++end;
    bool used[IREE_MI355X_MAX_CONCURRENCY] = {};
    for (uint32_t j = i; j < end; ++j) {
      const uint32_t l = (j - i) % lanes;
      if (!used[l]) {
        used[l] = used_ever[l] = true;
        for (const Prior &e : prior)
          if (e.lane != l)
            op(IREE_MI355X_LANE_OP_WAIT, l, e.event, 0);
      }
      op(IREE_MI355X_LANE_OP_ENQUEUE, l, 0, j);
    }
    if (end > i) {
      prior.clear();
      for (uint32_t l = 0; l < lanes; ++l)
        if (used[l]) {
          op(IREE_MI355X_LANE_OP_RECORD, l, 1 + l, 0);
          prior.push_back({1 + l, l});
        }
    }
    i = end + 1;  // past the barrier
  }
  for (uint32_t l = 1; l < lanes; ++l) {
    if (!used_ever[l])
      continue;
    op(IREE_MI355X_LANE_OP_RECORD, l, 1 + l, 0);
    op(IREE_MI355X_LANE_OP_WAIT, 0, 1 + l, 0);
  }
  return ops;
}

// Per device: the lane streams and events (default priority, non-blocking,
// kept for the process), and a lock that makes
// submissions on one device enqueue one at a time.
struct DeviceLanes {
  std::mutex lock;
  hipStream_t streams[IREE_MI355X_MAX_CONCURRENCY] = {};
  hipEvent_t lane_done[IREE_MI355X_MAX_CONCURRENCY] = {};
  hipEvent_t fork = nullptr;
};

std::mutex g_devices_lock;
std::vector<DeviceLanes *> g_devices;

DeviceLanes *device_lanes(int dev) {
  std::lock_guard<std::mutex> guard(g_devices_lock);
  if ((int)g_devices.size() <= dev)
    g_devices.resize(dev + 1, nullptr);
  if (!g_devices[dev])
    g_devices[dev] = new DeviceLanes();
  return g_devices[dev];
}

// Lane 0 is the caller's stream; lanes 1.. are the device's lane streams
// streams[0..lanes-2]. Every lane has an event.
int ensure_lanes(DeviceLanes *d, uint32_t lanes) {
  if (!d->fork &&
      hipEventCreateWithFlags(&d->fork, hipEventDisableTiming) != hipSuccess)
    return fail(IREE_MI355X_LAUNCH_FAILED, "submit: hipEventCreate failed");
  for (uint32_t l = 0; l < lanes; ++l) {
    if (l + 1 < lanes && !d->streams[l] &&
        hipStreamCreateWithFlags(&d->streams[l], hipStreamNonBlocking) !=
            hipSuccess)
      return fail(IREE_MI355X_LAUNCH_FAILED, "submit: hipStreamCreate failed");
    if (!d->lane_done[l] &&
        hipEventCreateWithFlags(&d->lane_done[l], hipEventDisableTiming) !=
            hipSuccess)
      return fail(IREE_MI355X_LAUNCH_FAILED, "submit: hipEventCreate failed");
  }
  return IREE_MI355X_OK;
}

// Enqueue one prepared command on `stream`, with `ws` as its workspace.
int enqueue(const iree_mi355x_command_buffer_t *cb, uint32_t index,
            const Ready &r, hipStream_t stream, void *ws, size_t ws_bytes) {
  const Command &c = cb->commands[index];
  const iree_mi355x_executable_export_table_t &ex = cb->library->exports;
  char zone[96];
  int st = IREE_MI355X_OK;
  switch (c.kind) {
    case kDispatch: {
      snprintf(zone, sizeof(zone), "dispatch %s", ex.names[c.ordinal]);
      roctxRangePushA(zone);
      iree_mi355x_executable_dispatch_state_t s = {};
      s.constant_count = (uint32_t)c.constants.size();
      s.constants = c.constants.data();
      s.binding_count = (uint32_t)r.ptrs.size();
      s.binding_ptrs = r.ptrs.data();
      s.binding_lengths = r.lengths.data();
      s.stream = stream;
      s.workspace = ws;
      s.workspace_bytes = ws_bytes;
      if ((st = ex.ptrs[c.ordinal](nullptr, &s))) {
        const std::string why = iree_mi355x_last_error();
        st = fail(st, "command %u (%s): %s", index, ex.names[c.ordinal],
                  why.c_str());
      }
      roctxRangePop();
      return st;
    }
    case kFill: {
      roctxRangePushA("fill");
      if (r.target_length > 0) {
        const uint64_t chunks = r.target_length / 16 + 1;
        const uint64_t blocks =
            std::min<uint64_t>(1024, std::max<uint64_t>(1, (chunks + 255) / 256));
        hipLaunchKernelGGL(fill_kernel, dim3((unsigned)blocks), dim3(256), 0,
                           stream, (unsigned char *)r.target, r.target_length,
                           c.word);
        if (hipGetLastError() != hipSuccess)
          st = fail(IREE_MI355X_LAUNCH_FAILED, "command %u: fill launch failed",
                    index);
      }
      roctxRangePop();
      return st;
    }
    case kCopy:
      roctxRangePushA("copy");
      if (c.length > 0 &&
          hipMemcpyAsync(r.target, r.source, c.length,
                         hipMemcpyDeviceToDevice, stream) != hipSuccess)
        st = fail(IREE_MI355X_LAUNCH_FAILED, "command %u: copy failed", index);
      roctxRangePop();
      return st;
    case kBarrier:
      return IREE_MI355X_OK;
  }
  return IREE_MI355X_OK;
}

int hip_ok(hipError_t e, const char *what) {
  return e == hipSuccess
             ? IREE_MI355X_OK
             : fail(IREE_MI355X_LAUNCH_FAILED, "submit: %s: %s", what,
                    hipGetErrorString(e));
}

}  // namespace
}  // namespace ihp

using namespace ihp;

extern "C" {

int iree_mi355x_command_buffer_create(
    const iree_mi355x_executable_library_t *library,
    iree_mi355x_command_buffer_t **out_command_buffer) {
  if (!out_command_buffer)
    return fail(IREE_MI355X_INVALID_ARGUMENT, "create: null output");
  *out_command_buffer = nullptr;
  if (!library)
    library = own_library();
  if (!library || !library->header || !library->exports.ptrs ||
      !library->exports.names)
    return fail(IREE_MI355X_INVALID_ARGUMENT, "create: no executable library");
  iree_mi355x_command_buffer_t *cb = new iree_mi355x_command_buffer_t();
  cb->library = library;
  *out_command_buffer = cb;
  return IREE_MI355X_OK;
}

void iree_mi355x_command_buffer_release(
    iree_mi355x_command_buffer_t *command_buffer) {
  delete command_buffer;
}

int iree_mi355x_command_buffer_dispatch(
    iree_mi355x_command_buffer_t *cb, uint32_t ordinal,
    const uint32_t *constants, uint32_t constant_count,
    const iree_mi355x_buffer_ref_t *bindings, uint32_t binding_count) {
  int st;
  if ((st = recording(cb, "dispatch")))
    return st;
  if (ordinal >= cb->library->exports.count)
    return fail(IREE_MI355X_INVALID_ARGUMENT,
                "dispatch: export %u of %u", ordinal,
                cb->library->exports.count);
  if ((constant_count && !constants) || (binding_count && !bindings))
    return fail(IREE_MI355X_INVALID_ARGUMENT,
                "dispatch: null constants or bindings");
  Command c;
  c.kind = kDispatch;
  c.ordinal = ordinal;
  c.constants.assign(constants, constants + constant_count);
  for (uint32_t b = 0; b < binding_count; ++b)
    c.bindings.push_back(to_ref(bindings[b]));
  cb->commands.push_back(std::move(c));
  return IREE_MI355X_OK;
}

int iree_mi355x_command_buffer_fill(iree_mi355x_command_buffer_t *cb,
                                    iree_mi355x_buffer_ref_t target,
                                    const void *pattern,
                                    uint32_t pattern_length) {
  int st;
  if ((st = recording(cb, "fill")))
    return st;
  if (!pattern || (pattern_length != 1 && pattern_length != 2 &&
                   pattern_length != 4))
    return fail(IREE_MI355X_INVALID_ARGUMENT,
                "fill: pattern of 1, 2 or 4 bytes expected");
  Command c;
  c.kind = kFill;
  c.target = to_ref(target);
  c.pattern_length = pattern_length;
  unsigned char bytes[4];
  for (int i = 0; i < 4; ++i)
    bytes[i] = ((const unsigned char *)pattern)[i % pattern_length];
  memcpy(&c.word, bytes, 4);
  cb->commands.push_back(std::move(c));
  return IREE_MI355X_OK;
}

int iree_mi355x_command_buffer_copy(iree_mi355x_command_buffer_t *cb,
                                    iree_mi355x_buffer_ref_t source,
                                    iree_mi355x_buffer_ref_t target,
                                    uint64_t length) {
  int st;
  if ((st = recording(cb, "copy")))
    return st;
  Command c;
  c.kind = kCopy;
  c.source = to_ref(source);
  c.target = to_ref(target);
  c.length = length;
  cb->commands.push_back(std::move(c));
  return IREE_MI355X_OK;
}

int iree_mi355x_command_buffer_barrier(iree_mi355x_command_buffer_t *cb) {
  int st;
  if ((st = recording(cb, "barrier")))
    return st;
  Command c;
  c.kind = kBarrier;
  cb->commands.push_back(std::move(c));
  return IREE_MI355X_OK;
}

int iree_mi355x_command_buffer_end(iree_mi355x_command_buffer_t *cb) {
  int st;
  if ((st = recording(cb, "end")))
    return st;
  cb->ended = true;
  return IREE_MI355X_OK;
}

uint32_t iree_mi355x_command_buffer_count(
    const iree_mi355x_command_buffer_t *cb) {
  return cb ? (uint32_t)cb->commands.size() : 0;
}

uint32_t iree_mi355x_command_buffer_lane_schedule(
    const iree_mi355x_command_buffer_t *cb, uint32_t max_concurrent,
    iree_mi355x_lane_op_t *ops, uint32_t capacity) {
  if (!cb || max_concurrent > IREE_MI355X_MAX_CONCURRENCY)
    return 0;
  const uint32_t lanes = lanes_for(
      cb, max_concurrent ? max_concurrent : IREE_MI355X_DEFAULT_CONCURRENCY);
  const std::vector<iree_mi355x_lane_op_t> s = lane_schedule(cb, lanes);
  for (uint32_t i = 0; i < capacity && i < s.size(); ++i)
    ops[i] = s[i];
  return (uint32_t)s.size();
}

size_t iree_mi355x_command_buffer_workspace_bytes(
    const iree_mi355x_command_buffer_t *cb,
    const iree_mi355x_binding_t *binding_table, uint32_t binding_count,
    uint32_t max_concurrent) {
  if (!cb || max_concurrent > IREE_MI355X_MAX_CONCURRENCY)
    return 0;
  std::vector<Ready> ready;
  size_t need = 0;
  if (prepare(cb, binding_table, binding_count, &ready, &need) !=
      IREE_MI355X_OK)
    return 0;
  const uint32_t lanes = lanes_for(
      cb, max_concurrent ? max_concurrent : IREE_MI355X_DEFAULT_CONCURRENCY);
  return need ? slice_bytes(need) * lanes : 0;
}

int iree_mi355x_command_buffer_submit(
    const iree_mi355x_command_buffer_t *cb,
    const iree_mi355x_binding_t *binding_table, uint32_t binding_count,
    uint32_t max_concurrent, void *workspace, size_t workspace_bytes,
    void *stream) {
  if (!cb)
    return fail(IREE_MI355X_INVALID_ARGUMENT, "submit: null command buffer");
  if (!cb->ended)
    return fail(IREE_MI355X_INVALID_ARGUMENT,
                "submit: command buffer not ended");
  if (max_concurrent > IREE_MI355X_MAX_CONCURRENCY)
    return fail(IREE_MI355X_INVALID_ARGUMENT,
                "submit: concurrency %u > %u", max_concurrent,
                IREE_MI355X_MAX_CONCURRENCY);
  std::vector<Ready> ready;
  size_t need = 0;
  int st = prepare(cb, binding_table, binding_count, &ready, &need);
  if (st)
    return st;
  if (cb->commands.empty())
    return IREE_MI355X_OK;
  const uint32_t lanes = lanes_for(
      cb, max_concurrent ? max_concurrent : IREE_MI355X_DEFAULT_CONCURRENCY);
  const size_t slice = need ? slice_bytes(need) : 0;
  // The caller provides the lane slices: the runtime allocates no device
  // memory.
  if (slice && (!workspace || workspace_bytes < slice * lanes))
    return fail(IREE_MI355X_WORKSPACE_TOO_SMALL,
                "submit: workspace %zu < %zu (%u lanes x %zu; size it with "
                "iree_mi355x_command_buffer_workspace_bytes)",
                workspace ? workspace_bytes : (size_t)0, slice * lanes, lanes,
                slice);

  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess)
    return fail(IREE_MI355X_NO_DEVICE, "submit: hipGetDevice failed");
  DeviceLanes *d = device_lanes(dev);
  std::lock_guard<std::mutex> guard(d->lock);
  char *ws = (char *)workspace;
  hipStream_t caller = (hipStream_t)stream;
  roctxRangePushA("iree_mi355x submit");
  const uint32_t n = (uint32_t)cb->commands.size();

  if (lanes == 1) {
    // In order on the caller's stream: barriers hold by stream order.
    for (uint32_t i = 0; i < n && !st; ++i)
      st = enqueue(cb, i, ready[i], caller, slice ? ws : nullptr, slice);
    roctxRangePop();
    return st;
  }

  // Concurrent lanes are not submitted into a stream capture: such a
  // capture (4 lanes, fork / join through events) ended in a host crash in
  // hipStreamEndCapture whose cause is not established, so a capture takes
  // the in-order path above (max_concurrent = 1) or is refused here.
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(caller, &capture) != hipSuccess ||
      capture != hipStreamCaptureStatusNone) {
    roctxRangePop();
    return fail(IREE_MI355X_UNSUPPORTED,
                "submit: %u concurrent lanes inside a stream capture; capture "
                "with max_concurrent = 1",
                lanes);
  }
  if ((st = ensure_lanes(d, lanes))) {
    roctxRangePop();
    return st;
  }
  // Lane 0 is the caller's stream itself, lanes 1.. the device's lane
  // streams; event 0 is the fork event, 1 + l lane l's event.
  hipStream_t lane_stream[IREE_MI355X_MAX_CONCURRENCY];
  lane_stream[0] = caller;
  for (uint32_t l = 1; l < lanes; ++l)
    lane_stream[l] = d->streams[l - 1];
  auto event = [&](uint32_t e) { return e == 0 ? d->fork : d->lane_done[e - 1]; };
  // After a failure the remaining records and waits still run (no more
  // commands), so every lane is joined back into the caller's stream; the
  // first error is returned.
  for (const iree_mi355x_lane_op_t &o : lane_schedule(cb, lanes)) {
    int r = IREE_MI355X_OK;
    switch (o.kind) {
      case IREE_MI355X_LANE_OP_RECORD:
        r = hip_ok(hipEventRecord(event(o.event), lane_stream[o.lane]),
                   "lane record");
        break;
      case IREE_MI355X_LANE_OP_WAIT:
        r = hip_ok(hipStreamWaitEvent(lane_stream[o.lane], event(o.event), 0),
                   "lane wait");
        break;
      default:
        if (st)
          continue;
        r = enqueue(cb, o.command, ready[o.command], lane_stream[o.lane],
                    slice ? ws + (size_t)o.lane * slice : nullptr, slice);
    }
    if (r && !st)
      st = r;
  }
  roctxRangePop();
  return st;
}

}  // extern "C"
