"""MI355X (gfx950) matmul / attention dispatch library: Python host binding.

A thin ctypes layer over ``lib/libiree_mi355x.so``, the C-ABI declared in
``include/iree_mi355x_kernels.h``, ``include/iree_mi355x_planner.h`` and
``include/iree_mi355x_executable_library.h``. Device buffers are torch tensors
(torch is the device-memory and stream plumbing); every op enqueues on the
current torch stream and returns without synchronizing.

There is no fallback: if the native library is missing the import of a
binding raises, and every call goes to the HIP kernels.
"""
from __future__ import annotations

import ctypes
import functools
import os
import struct
from dataclasses import dataclass

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libiree_mi355x.so")

# Status codes (iree_mi355x_status_t).
OK = 0
INVALID_ARGUMENT = 1
MISALIGNED = 2
UNSUPPORTED = 3
LAUNCH_FAILED = 4
NO_DEVICE = 5
WORKSPACE_TOO_SMALL = 6
STATUS_NAMES = {
    OK: "OK", INVALID_ARGUMENT: "INVALID_ARGUMENT", MISALIGNED: "MISALIGNED",
    UNSUPPORTED: "UNSUPPORTED", LAUNCH_FAILED: "LAUNCH_FAILED",
    NO_DEVICE: "NO_DEVICE", WORKSPACE_TOO_SMALL: "WORKSPACE_TOO_SMALL",
}

# Flags.
B_TRANSPOSED = 0x1
ACCUMULATE = 0x2
OUT_F32 = 0x4
A_TRANSPOSED = 0x8
SPLITS_STREAM_K = -1  # matmul_mfma_config: stream-K runs of (tile, K stage)
CAUSAL = 0x1
ATTENTION_OUT_F32 = 0x2
ATTENTION_MASK = 0x4

# Element kinds (iree_mi355x_elem_t) and kernel families.
ELEM_F16, ELEM_I8, ELEM_I32, ELEM_F32 = 0, 1, 2, 3
FAMILY_NONE, FAMILY_MFMA, FAMILY_GENERAL, FAMILY_GEMV = 0, 1, 2, 3
B_FORM_TN, B_FORM_NN, B_FORM_W8A16, B_FORM_NN8 = 0, 1, 2, 3
FAMILY_NAMES = {FAMILY_NONE: "none", FAMILY_MFMA: "mfma",
                FAMILY_GENERAL: "general", FAMILY_GEMV: "gemv"}

EXECUTABLE_LIBRARY_VERSION = 0x4D490001

# Every symbol the C-ABI headers declare (checked by the CPU tests).
EXPORTED_SYMBOLS = (
    "iree_mi355x_matmul_f16", "iree_mi355x_matmul_i8",
    "iree_mi355x_w8a16_matmul", "iree_mi355x_attention_f16",
    "iree_mi355x_attention_f16_strided", "iree_mi355x_attention",
    "iree_mi355x_matmul_workspace_bytes", "iree_mi355x_last_error",
    "iree_mi355x_version", "iree_mi355x_device_count",
    "iree_mi355x_matmul_desc_init", "iree_mi355x_classify_matmul",
    "iree_mi355x_plan_matmul", "iree_mi355x_mfma_config_count",
    "iree_mi355x_mfma_config_info", "iree_mi355x_matmul_mfma_config",
    "iree_mi355x_executable_library_query", "iree_mi355x_batch_matmul_f16",
    "iree_mi355x_batch_matmul_workspace_bytes",
    "iree_mi355x_matmul_mfma_config_workspace_bytes",
    "iree_mi355x_mfma_config_layout_flags",
    "iree_mi355x_matmul_mfma_config_split",
    "iree_mi355x_command_buffer_create", "iree_mi355x_command_buffer_release",
    "iree_mi355x_command_buffer_dispatch", "iree_mi355x_command_buffer_fill",
    "iree_mi355x_command_buffer_copy", "iree_mi355x_command_buffer_barrier",
    "iree_mi355x_command_buffer_end",
    "iree_mi355x_command_buffer_workspace_bytes",
    "iree_mi355x_command_buffer_submit", "iree_mi355x_command_buffer_count",
    "iree_mi355x_command_buffer_lane_schedule",
    "iree_mi355x_kernel_count", "iree_mi355x_kernel_resources",
    "iree_mi355x_executable_serialize", "iree_mi355x_executable_verify",
    "iree_mi355x_executable_load", "iree_mi355x_loaded_executable_library",
    "iree_mi355x_loaded_executable_release",
    "iree_mi355x_matmul_f16_no_alloc",
    "iree_mi355x_match_linalg_op", "iree_mi355x_match_dispatch_region",
)

# Activations of the fused matmul epilogue (include/iree_mi355x_kernels.h).
ACT_NONE, ACT_RELU, ACT_GELU_TANH, ACT_SILU = 0, 1, 2, 3
_ACT_NAMES = {None: ACT_NONE, "none": ACT_NONE, "relu": ACT_RELU,
              "gelu_tanh": ACT_GELU_TANH, "gelu": ACT_GELU_TANH,
              "silu": ACT_SILU}


class Epilogue(ctypes.Structure):
    """iree_mi355x_epilogue_t."""
    _fields_ = [("bias", ctypes.c_void_p), ("multiplier", ctypes.c_void_p),
                ("ld_multiplier", ctypes.c_int64),
                ("batch_stride_multiplier", ctypes.c_int64),
                ("activation", ctypes.c_uint32)]


class MI355XError(RuntimeError):
    def __init__(self, status: int, message: str):
        self.status = status
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")


class MatmulDesc(ctypes.Structure):
    _fields_ = [("a_elem", ctypes.c_int32), ("b_elem", ctypes.c_int32),
                ("c_elem", ctypes.c_int32), ("m", ctypes.c_int64),
                ("n", ctypes.c_int64), ("k", ctypes.c_int64),
                ("flags", ctypes.c_uint32), ("a_aligned16", ctypes.c_int32),
                ("b_aligned16", ctypes.c_int32), ("has_scale", ctypes.c_int32),
                ("lds_budget_bytes", ctypes.c_int64),
                ("num_cus", ctypes.c_int32), ("batch", ctypes.c_int64)]


class MatmulPlan(ctypes.Structure):
    _fields_ = [("family", ctypes.c_int32), ("config_index", ctypes.c_int32),
                ("config_name", ctypes.c_char * 64), ("tile_m", ctypes.c_int64),
                ("tile_n", ctypes.c_int64), ("tile_k", ctypes.c_int64),
                ("lds_bytes", ctypes.c_int64), ("workgroups", ctypes.c_int64),
                ("threads", ctypes.c_int32), ("splits", ctypes.c_int32),
                ("k_split", ctypes.c_int32),
                ("workspace_bytes", ctypes.c_int64),
                ("traffic_bytes", ctypes.c_int64),
                ("from_tuned_table", ctypes.c_int32),
                ("stream_k_steps", ctypes.c_int32)]


class DispatchState(ctypes.Structure):
    _fields_ = [("constant_count", ctypes.c_uint32),
                ("constants", ctypes.POINTER(ctypes.c_uint32)),
                ("binding_count", ctypes.c_uint32),
                ("binding_ptrs", ctypes.POINTER(ctypes.c_void_p)),
                ("binding_lengths", ctypes.POINTER(ctypes.c_size_t)),
                ("stream", ctypes.c_void_p),
                ("workspace", ctypes.c_void_p),
                ("workspace_bytes", ctypes.c_size_t),
                ("workspace_query", ctypes.POINTER(ctypes.c_size_t))]


DISPATCH_FN = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p,
                               ctypes.POINTER(DispatchState))


class DispatchAttrs(ctypes.Structure):
    _fields_ = [("flags", ctypes.c_uint64), ("lds_bytes", ctypes.c_uint64),
                ("threads", ctypes.c_uint64)]


class ExportTable(ctypes.Structure):
    _fields_ = [("count", ctypes.c_uint32),
                ("ptrs", ctypes.POINTER(ctypes.c_void_p)),
                ("attrs", ctypes.POINTER(DispatchAttrs)),
                ("names", ctypes.POINTER(ctypes.c_char_p))]


class ImportTable(ctypes.Structure):
    _fields_ = [("count", ctypes.c_uint32),
                ("symbols", ctypes.POINTER(ctypes.c_char_p))]


class LibraryHeader(ctypes.Structure):
    _fields_ = [("version", ctypes.c_uint32), ("name", ctypes.c_char_p)]


class Library(ctypes.Structure):
    _fields_ = [("header", ctypes.POINTER(LibraryHeader)),
                ("imports", ImportTable), ("exports", ExportTable)]


class KernelResources(ctypes.Structure):
    """iree_mi355x_kernel_resources_t."""
    _fields_ = [("name", ctypes.c_char_p), ("exports", ctypes.c_uint32),
                ("threads", ctypes.c_int32), ("vgprs", ctypes.c_int32),
                ("lds_bytes", ctypes.c_int32), ("scratch_bytes", ctypes.c_int32),
                ("max_threads", ctypes.c_int32),
                ("workgroups_per_cu", ctypes.c_int32)]


# Runtime (include/iree_mi355x_runtime.h).
BINDING_DIRECT = 0xFFFFFFFF
WHOLE_BUFFER = (1 << 64) - 1
DEFAULT_CONCURRENCY = 1
MAX_CONCURRENCY = 8


class LaneOp(ctypes.Structure):
    """iree_mi355x_lane_op_t: one stream operation of a lane schedule."""
    _fields_ = [("kind", ctypes.c_uint32), ("lane", ctypes.c_uint32),
                ("event", ctypes.c_uint32), ("command", ctypes.c_uint32)]


LANE_OP_RECORD, LANE_OP_WAIT, LANE_OP_ENQUEUE = 0, 1, 2


class BufferRef(ctypes.Structure):
    """iree_mi355x_buffer_ref_t: a binding-table slot or a direct pointer."""
    _fields_ = [("binding_slot", ctypes.c_uint32), ("buffer", ctypes.c_void_p),
                ("offset", ctypes.c_uint64), ("length", ctypes.c_uint64)]


class Binding(ctypes.Structure):
    """iree_mi355x_binding_t: one binding-table entry."""
    _fields_ = [("buffer", ctypes.c_void_p), ("length", ctypes.c_uint64)]


# Dispatch matcher (include/iree_mi355x_matcher.h).
MAX_LOOPS, MAX_OPERANDS, MAX_BODY = 8, 6, 24
OP_GENERIC, OP_MATMUL, OP_BATCH_MATMUL, OP_QUANTIZED_MATMUL = 0, 1, 2, 3
OP_FILL, OP_TRANSPOSE, OP_ATTENTION = 4, 5, 6
TYPES = {"f16": 1, "bf16": 2, "f32": 3, "f64": 4, "i1": 5, "i8": 6,
         "i32": 7, "i64": 8, "index": 9}
MAP_ZERO = -1
FROM_ARGUMENT, FROM_CONSTANT = -1, -2
BODY_OPS = {"yield": 0, "const": 1, "extf": 2, "truncf": 3, "extsi": 4,
            "sitofp": 5, "mulf": 6, "addf": 7, "subf": 8, "divf": 9,
            "maximumf": 10, "exp": 11, "muli": 12, "addi": 13, "subi": 14,
            "index": 15, "index_cast": 16, "cmpf": 17, "cmpi": 18,
            "select": 19, "andi": 20}
PREDICATES = {"oeq": 1, "eq": 1, "ogt": 2, "sgt": 2, "ugt": 3}
MATCH_NAMED_ONLY = 0x1


class BodyOp(ctypes.Structure):
    """iree_mi355x_body_op_t."""
    _fields_ = [("opcode", ctypes.c_uint32), ("operands", ctypes.c_int32 * 3),
                ("type", ctypes.c_int32), ("constant", ctypes.c_double)]


class LinalgOp(ctypes.Structure):
    """iree_mi355x_linalg_op_t."""
    _fields_ = [("kind", ctypes.c_uint32), ("num_loops", ctypes.c_uint32),
                ("reduction_loops", ctypes.c_uint32),
                ("loop_extent", ctypes.c_int64 * MAX_LOOPS),
                ("num_inputs", ctypes.c_uint32),
                ("num_outputs", ctypes.c_uint32),
                ("elem_type", ctypes.c_int32 * MAX_OPERANDS),
                ("map_rank", ctypes.c_uint32 * MAX_OPERANDS),
                ("map", (ctypes.c_int32 * MAX_LOOPS) * MAX_OPERANDS),
                ("producer", ctypes.c_int32 * MAX_OPERANDS),
                ("producer_result", ctypes.c_int32 * MAX_OPERANDS),
                ("scalar", ctypes.c_double * MAX_OPERANDS),
                ("num_body_ops", ctypes.c_uint32),
                ("body", BodyOp * MAX_BODY)]


class MatchResult(ctypes.Structure):
    """iree_mi355x_match_t."""
    _fields_ = [("taken", ctypes.c_int32), ("export_name", ctypes.c_char * 32),
                ("flags", ctypes.c_uint32), ("batch_loop", ctypes.c_int32),
                ("m_loop", ctypes.c_int32), ("n_loop", ctypes.c_int32),
                ("k_loop", ctypes.c_int32), ("root", ctypes.c_int32),
                ("scale", ctypes.c_float), ("head_loop", ctypes.c_int32),
                ("reason", ctypes.c_char * 160),
                ("init_fill", ctypes.c_int32), ("init_value", ctypes.c_double),
                ("head_dim_loop", ctypes.c_int32)]


_lib = None


def _share_hip_runtime() -> None:
    # torch ships its own libamdhip64; importing it first makes the native
    # library bind to that same runtime, so one process has one HIP runtime
    # and torch's device pointers and streams are valid in both.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass


def library():
    """Load (once) and return the native library; raise if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"native library {LIB_PATH} is not built; run "
            "`python -c 'import __graft_entry__ as g; g.build()'`")
    _share_hip_runtime()
    lib = ctypes.CDLL(LIB_PATH)
    p, i64, u32, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_uint32, ctypes.c_size_t
    lib.iree_mi355x_matmul_f16.argtypes = [p, p, p, i64, i64, i64, i64, i64,
                                           i64, u32, p, sz, p]
    lib.iree_mi355x_matmul_i8.argtypes = [p, p, p, i64, i64, i64, i64, i64,
                                          i64, u32, p, sz, p]
    lib.iree_mi355x_matmul_f16_no_alloc.argtypes = [p, p, p, i64, i64, i64,
                                                    i64, i64, i64, u32, p]
    lib.iree_mi355x_w8a16_matmul.argtypes = [p, p, p, p, i64, i64, i64, i64,
                                             i64, i64, u32, p, sz, p]
    lib.iree_mi355x_attention_f16.argtypes = [p, p, p, p, i64, i64, i64, i64,
                                              i64, ctypes.c_float, u32, p]
    lib.iree_mi355x_attention_f16_strided.argtypes = [
        p, p, p, p, i64, i64, i64, i64, i64, i64, ctypes.c_float, u32, p, p]
    lib.iree_mi355x_attention.argtypes = [p, p]
    lib.iree_mi355x_matmul_workspace_bytes.restype = sz
    lib.iree_mi355x_matmul_workspace_bytes.argtypes = [i64, i64, i64, u32]
    lib.iree_mi355x_batch_matmul_f16.argtypes = [
        p, p, p, i64, i64, i64, i64, i64, i64, i64, i64, i64, i64, u32,
        ctypes.POINTER(Epilogue), p, sz, p]
    lib.iree_mi355x_batch_matmul_workspace_bytes.restype = sz
    lib.iree_mi355x_batch_matmul_workspace_bytes.argtypes = [i64, i64, i64,
                                                             i64, u32]
    lib.iree_mi355x_last_error.restype = ctypes.c_char_p
    lib.iree_mi355x_version.restype = ctypes.c_char_p
    lib.iree_mi355x_matmul_desc_init.restype = None
    lib.iree_mi355x_matmul_desc_init.argtypes = [
        ctypes.POINTER(MatmulDesc), ctypes.c_int32, ctypes.c_int32,
        ctypes.c_int32, i64, i64, i64, u32]
    lib.iree_mi355x_classify_matmul.argtypes = [ctypes.POINTER(MatmulDesc)]
    lib.iree_mi355x_plan_matmul.argtypes = [ctypes.POINTER(MatmulDesc),
                                            ctypes.POINTER(MatmulPlan)]
    lib.iree_mi355x_mfma_config_info.argtypes = [
        ctypes.c_int, ctypes.POINTER(ctypes.c_char_p),
        ctypes.POINTER(ctypes.c_int32),
        ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32),
        ctypes.POINTER(i64), ctypes.POINTER(i64), ctypes.POINTER(i64),
        ctypes.POINTER(i64), ctypes.POINTER(ctypes.c_int32)]
    lib.iree_mi355x_mfma_config_layout_flags.restype = ctypes.c_int32
    lib.iree_mi355x_mfma_config_layout_flags.argtypes = [ctypes.c_int]
    lib.iree_mi355x_matmul_mfma_config_split.argtypes = [
        ctypes.c_int, ctypes.c_int32, p, p, p, p, i64, i64, i64, i64, i64, i64,
        u32, p, sz, p]
    lib.iree_mi355x_matmul_mfma_config.argtypes = [ctypes.c_int, p, p, p, p,
                                                   i64, i64, i64, i64, i64,
                                                   i64, u32, p, sz, p]
    lib.iree_mi355x_matmul_mfma_config_workspace_bytes.restype = sz
    lib.iree_mi355x_matmul_mfma_config_workspace_bytes.argtypes = [
        ctypes.c_int, ctypes.c_int32, i64, i64, i64, u32]
    cbp = ctypes.c_void_p
    lib.iree_mi355x_command_buffer_create.argtypes = [p, ctypes.POINTER(cbp)]
    lib.iree_mi355x_command_buffer_release.argtypes = [cbp]
    lib.iree_mi355x_command_buffer_release.restype = None
    lib.iree_mi355x_command_buffer_dispatch.argtypes = [
        cbp, u32, ctypes.POINTER(u32), u32, ctypes.POINTER(BufferRef), u32]
    lib.iree_mi355x_command_buffer_fill.argtypes = [cbp, BufferRef, p, u32]
    lib.iree_mi355x_command_buffer_copy.argtypes = [cbp, BufferRef, BufferRef,
                                                    ctypes.c_uint64]
    lib.iree_mi355x_command_buffer_barrier.argtypes = [cbp]
    lib.iree_mi355x_command_buffer_end.argtypes = [cbp]
    lib.iree_mi355x_command_buffer_count.argtypes = [cbp]
    lib.iree_mi355x_command_buffer_count.restype = u32
    lib.iree_mi355x_command_buffer_workspace_bytes.argtypes = [
        cbp, ctypes.POINTER(Binding), u32, u32]
    lib.iree_mi355x_command_buffer_workspace_bytes.restype = sz
    lib.iree_mi355x_command_buffer_submit.argtypes = [
        cbp, ctypes.POINTER(Binding), u32, u32, p, sz, p]
    lib.iree_mi355x_command_buffer_lane_schedule.argtypes = [
        cbp, u32, ctypes.POINTER(LaneOp), u32]
    lib.iree_mi355x_command_buffer_lane_schedule.restype = u32
    lib.iree_mi355x_kernel_resources.argtypes = [ctypes.c_int,
                                                 ctypes.POINTER(KernelResources)]
    lib.iree_mi355x_executable_serialize.restype = sz
    lib.iree_mi355x_executable_serialize.argtypes = [ctypes.c_char_p, p, sz]
    lib.iree_mi355x_executable_verify.argtypes = [p, sz]
    lib.iree_mi355x_executable_load.argtypes = [p, sz, ctypes.POINTER(p)]
    lib.iree_mi355x_loaded_executable_library.restype = p
    lib.iree_mi355x_loaded_executable_library.argtypes = [p]
    lib.iree_mi355x_loaded_executable_release.restype = None
    lib.iree_mi355x_loaded_executable_release.argtypes = [p]
    lib.iree_mi355x_executable_library_query.restype = ctypes.c_void_p
    lib.iree_mi355x_executable_library_query.argtypes = [u32, p]
    lib.iree_mi355x_match_linalg_op.argtypes = [
        ctypes.POINTER(LinalgOp), u32, ctypes.POINTER(MatchResult)]
    lib.iree_mi355x_match_dispatch_region.argtypes = [
        ctypes.POINTER(LinalgOp), u32, u32, ctypes.POINTER(MatchResult)]
    _lib = lib
    return lib


def last_error() -> str:
    return library().iree_mi355x_last_error().decode()


def _check(status: int) -> None:
    if status != OK:
        raise MI355XError(status, last_error())


# ------------------------------------------------------------------ planner --

def make_desc(a_elem, b_elem, c_elem, m, n, k, flags=0, *, has_scale=False,
              aligned=True, lds_budget_bytes=None, batch=1) -> MatmulDesc:
    d = MatmulDesc()
    library().iree_mi355x_matmul_desc_init(ctypes.byref(d), a_elem, b_elem,
                                           c_elem, m, n, k, flags)
    d.batch = batch
    d.has_scale = int(has_scale)
    d.a_aligned16 = d.b_aligned16 = int(aligned)
    if lds_budget_bytes is not None:
        d.lds_budget_bytes = lds_budget_bytes
    return d


def classify(desc: MatmulDesc) -> int:
    return library().iree_mi355x_classify_matmul(ctypes.byref(desc))


def plan(desc: MatmulDesc) -> MatmulPlan:
    out = MatmulPlan()
    _check(library().iree_mi355x_plan_matmul(ctypes.byref(desc),
                                             ctypes.byref(out)))
    return out


@dataclass
class MfmaConfig:
    index: int
    name: str
    b_form: int
    a_elem: int
    c_elem: int
    tile_m: int
    tile_n: int
    tile_k: int
    lds_bytes: int
    threads: int
    layout_flags: int = 0  # B_TRANSPOSED / A_TRANSPOSED the operands carry

    @property
    def a_transposed(self) -> bool:
        return bool(self.layout_flags & A_TRANSPOSED)


def mfma_configs() -> list[MfmaConfig]:
    lib = library()
    out = []
    for i in range(lib.iree_mi355x_mfma_config_count()):
        name = ctypes.c_char_p()
        bf, ae, ce, th = (ctypes.c_int32() for _ in range(4))
        tm, tn, tk, lds = (ctypes.c_int64() for _ in range(4))
        _check(lib.iree_mi355x_mfma_config_info(
            i, ctypes.byref(name), ctypes.byref(bf), ctypes.byref(ae),
            ctypes.byref(ce), ctypes.byref(tm), ctypes.byref(tn),
            ctypes.byref(tk), ctypes.byref(lds), ctypes.byref(th)))
        out.append(MfmaConfig(i, name.value.decode(), bf.value, ae.value,
                              ce.value, tm.value, tn.value, tk.value,
                              lds.value, th.value,
                              lib.iree_mi355x_mfma_config_layout_flags(i)))
    return out


# ----------------------------------------------------------------- matcher --

def linalg_op(kind, loops, maps, types, *, inputs, reductions=(),
              extents=None, args=None, body=(), producers=None,
              scalars=None) -> LinalgOp:
    """Describe one linalg op for the matcher.

    loops: loop names in order ("m n k" or a list); reductions: the
    reduction loops' names; maps: one per operand (inputs, then outputs),
    each the loop names of its dimensions with "0" for a broadcast
    dimension ("m k", "b m 0"); types: element type names per operand;
    inputs: how many operands are inputs; extents: {loop: extent}
    (missing: dynamic); args: names of the body's block arguments (default:
    in0.., out0..); body: SSA ops in order, each (name, op, operand names,
    type[, attribute]) with the attribute a constant's value, an index op's
    loop name or a comparison predicate, ending with ("yield", [names]);
    producers: per operand, an earlier op's index (or (index, result)),
    "arg" (default) or ("const", value).
    """
    loop_names = loops.split() if isinstance(loops, str) else list(loops)
    pos = {n: i for i, n in enumerate(loop_names)}
    op = LinalgOp()
    op.kind = kind
    op.num_loops = len(loop_names)
    op.reduction_loops = sum(1 << pos[r] for r in reductions)
    for i in range(MAX_LOOPS):
        op.loop_extent[i] = -1
    for name, ext in (extents or {}).items():
        op.loop_extent[pos[name]] = ext
    op.num_inputs = inputs
    op.num_outputs = len(maps) - inputs
    for i, (m, t) in enumerate(zip(maps, types)):
        dims = m.split() if isinstance(m, str) else list(m)
        op.elem_type[i] = TYPES[t]
        op.map_rank[i] = len(dims)
        for r, d in enumerate(dims):
            op.map[i][r] = MAP_ZERO if d == "0" else pos[d]
        op.producer[i] = FROM_ARGUMENT
    for i, prod in enumerate(producers or ()):
        if prod == "arg" or prod is None:
            op.producer[i] = FROM_ARGUMENT
        elif isinstance(prod, tuple) and prod[0] == "const":
            op.producer[i] = FROM_CONSTANT
            op.scalar[i] = prod[1]
        elif isinstance(prod, tuple):
            op.producer[i], op.producer_result[i] = prod
        else:
            op.producer[i] = prod
    for i, v in (scalars or {}).items():
        op.scalar[i] = v
    values = {}
    names = args or ([f"in{i}" for i in range(inputs)] +
                     [f"out{i}" for i in range(len(maps) - inputs)])
    for i, n in enumerate(names):
        values[n] = i
    op.num_body_ops = len(body)
    for b, entry in enumerate(body):
        if entry[0] == "yield":
            bo = op.body[b]
            bo.opcode = BODY_OPS["yield"]
            ids = [values[n] for n in entry[1]] + [-1, -1, -1]
            bo.operands[:] = ids[:3]
            continue
        name, code, operand_names, typ = entry[:4]
        attr = entry[4] if len(entry) > 4 else 0.0
        bo = op.body[b]
        bo.opcode = BODY_OPS[code]
        ids = [values[n] for n in operand_names] + [-1, -1, -1]
        bo.operands[:] = ids[:3]
        bo.type = TYPES[typ]
        if code == "index":
            bo.constant = pos[attr]
        elif code in ("cmpf", "cmpi"):
            bo.constant = PREDICATES[attr]
        else:
            bo.constant = float(attr)
        values[name] = len(names) + b
    return op


@dataclass
class Match:
    taken: bool
    export: str
    flags: int
    batch_loop: int
    m_loop: int
    n_loop: int
    k_loop: int
    root: int
    scale: float
    head_loop: int
    reason: str
    # ACCUMULATE over a constant fill: fill the output with init_value first
    init_fill: bool = False
    init_value: float = 0.0
    # attention: the loop of Q's / K's head dim (n_loop is V's)
    head_dim_loop: int = -1


def _match_result(r: MatchResult) -> Match:
    return Match(bool(r.taken), r.export_name.decode(), r.flags, r.batch_loop,
                 r.m_loop, r.n_loop, r.k_loop, r.root, r.scale, r.head_loop,
                 r.reason.decode(), bool(r.init_fill), r.init_value,
                 r.head_dim_loop)


def match(op: LinalgOp, *, named_only=False) -> Match:
    """Which export computes one linalg op (iree_mi355x_match_linalg_op)."""
    out = MatchResult()
    _check(library().iree_mi355x_match_linalg_op(
        ctypes.byref(op), MATCH_NAMED_ONLY if named_only else 0,
        ctypes.byref(out)))
    return _match_result(out)


def match_region(ops, *, named_only=False) -> Match:
    """Which export computes a dispatch region (ops in program order, the
    last one's result is the region's)."""
    arr = (LinalgOp * len(ops))(*ops)
    out = MatchResult()
    _check(library().iree_mi355x_match_dispatch_region(
        arr, len(ops), MATCH_NAMED_ONLY if named_only else 0,
        ctypes.byref(out)))
    return _match_result(out)


# ----------------------------------------------------------- library table --

def executable_library(version: int = EXECUTABLE_LIBRARY_VERSION):
    """The export table (or None if `version` does not match)."""
    addr = library().iree_mi355x_executable_library_query(version, None)
    if not addr:
        return None
    return ctypes.cast(addr, ctypes.POINTER(Library)).contents


def export_names() -> list[str]:
    lib = executable_library()
    return [lib.exports.names[i].decode() for i in range(lib.exports.count)]


def call_export(name: str, constants, bindings, binding_lengths, stream=None,
                workspace=None, workspace_bytes=0, query=False):
    """Invoke an export's dispatch function; returns the status code, or with
    ``query`` (validate only, nothing enqueued) (status, workspace bytes)."""
    lib = executable_library()
    names = export_names()
    idx = names.index(name)
    fn = DISPATCH_FN(lib.exports.ptrs[idx])
    consts = (ctypes.c_uint32 * len(constants))(*constants)
    ptrs = (ctypes.c_void_p * len(bindings))(*bindings)
    lens = (ctypes.c_size_t * len(binding_lengths))(*binding_lengths)
    need = ctypes.c_size_t(0)
    state = DispatchState(len(constants), consts, len(bindings), ptrs, lens,
                          stream, workspace, workspace_bytes,
                          ctypes.pointer(need) if query else None)
    st = fn(None, ctypes.byref(state))
    return (st, need.value) if query else st


def matmul_constants(m, n, k, lda, ldb, ldc, flags):
    words = []
    for v in (m, n, k, lda, ldb, ldc):
        words += [v & 0xFFFFFFFF, (v >> 32) & 0xFFFFFFFF]
    return words + [flags]


def batch_matmul_constants(m, n, k, lda, ldb, ldc, flags, batch, stride_a,
                           stride_b, stride_c, activation=ACT_NONE,
                           has_bias=False, has_multiplier=False,
                           ld_multiplier=0, batch_stride_multiplier=0):
    words = matmul_constants(m, n, k, lda, ldb, ldc, flags)
    for v in (batch, stride_a, stride_b, stride_c):
        words += [v & 0xFFFFFFFF, (v >> 32) & 0xFFFFFFFF]
    words += [activation, (1 if has_bias else 0) | (2 if has_multiplier else 0)]
    for v in (ld_multiplier, batch_stride_multiplier):
        words += [v & 0xFFFFFFFF, (v >> 32) & 0xFFFFFFFF]
    return words


def attention_constants(batch, heads, seq_q, seq_kv, head_dim, scale, flags,
                        kv_heads=None, strides=None, head_dim_v=None,
                        mask_strides=None):
    """Push constants of "attention_f16"; with `strides` (12 element strides:
    batch, head, row of q, k, v, o) the 32-word strided form; with
    `head_dim_v` or `mask_strides` (batch, head, row, key of the mask,
    binding 4, flag ATTENTION_MASK) the 41-word general form, whose strides
    default to contiguous ones."""
    scale_bits = struct.unpack("<I", struct.pack("<f", scale))[0]
    words = [batch, heads, seq_q, seq_kv, head_dim, scale_bits, flags]
    general = head_dim_v is not None or mask_strides is not None
    dv = head_dim if head_dim_v is None else head_dim_v
    if general and strides is None:
        hk = heads if kv_heads is None else kv_heads
        strides = [heads * seq_q * head_dim, seq_q * head_dim, head_dim,
                   hk * seq_kv * head_dim, seq_kv * head_dim, head_dim,
                   hk * seq_kv * dv, seq_kv * dv, dv,
                   heads * seq_q * dv, seq_q * dv, dv]
    if strides is not None:
        words.append(heads if kv_heads is None else kv_heads)
        for v in strides:
            words += [v & 0xFFFFFFFF, (v >> 32) & 0xFFFFFFFF]
    if general:
        words.append(dv)
        for v in (mask_strides or (0, 0, 0, 0)):
            words += [v & 0xFFFFFFFF, (v >> 32) & 0xFFFFFFFF]
    return words


# --------------------------------------------------------------- workspace --

# The C-ABI allocates no device memory: calls whose plan splits K take their
# partials and arrival counters from a workspace. For calls made without
# one, the wrapper keeps one zero-filled buffer per (device, stream),
# allocated through torch's allocator in that stream's order, grown
# geometrically and never released: a graph captured earlier may hold an
# older buffer, so the ones a larger buffer replaces stay alive too. Two
# streams never share a buffer (their arrival counters would collide).
_STREAM_WORKSPACES: dict = {}
_MIN_WORKSPACE = 64 << 20


def _torch_stream(stream, dev):
    import torch
    if stream is None:
        return torch.cuda.current_stream(dev)
    if isinstance(stream, int):
        return (torch.cuda.ExternalStream(stream, device=dev) if stream
                else torch.cuda.default_stream(dev))
    return stream


def stream_workspace(need: int, device=None, stream=None, layout=None):
    """(pointer, bytes) of the wrapper's workspace for `stream` (None: the
    current one; an int: a raw hipStream_t) on `device`, holding at least
    `need` bytes; (None, 0) when `need` is 0. `layout` keeps apart buffers
    whose arrival counters sit at different offsets (a command buffer's lane
    slices): None for flat calls, whose counters open the buffer. Under graph
    capture a buffer that is too small is not grown:
    MI355XError(WORKSPACE_TOO_SMALL)."""
    import torch
    if need <= 0:
        return None, 0
    dev = torch.device("cuda") if device is None else torch.device(device)
    if dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    s = _torch_stream(stream, dev)
    bufs = _STREAM_WORKSPACES.setdefault((dev.index, s.cuda_stream, layout),
                                         [])
    have = bufs[-1].numel() if bufs else 0
    if have >= need:
        return bufs[-1].data_ptr(), have
    if torch.cuda.is_current_stream_capturing():
        raise MI355XError(
            WORKSPACE_TOO_SMALL,
            f"the stream is capturing and its workspace holds {have} < "
            f"{need} bytes: make one call of this shape on the stream "
            "before capture, or pass a workspace")
    size = max(_MIN_WORKSPACE, 2 * have, need)
    with torch.cuda.stream(s):
        buf = torch.zeros(size, dtype=torch.uint8, device=dev)
    bufs.append(buf)
    return buf.data_ptr(), size


@functools.lru_cache(maxsize=4096)
def _matmul_workspace_need(m, n, k, flags) -> int:
    return library().iree_mi355x_matmul_workspace_bytes(m, n, k, flags)


@functools.lru_cache(maxsize=4096)
def _batch_workspace_need(batch, m, n, k, flags) -> int:
    return library().iree_mi355x_batch_matmul_workspace_bytes(batch, m, n, k,
                                                              flags)


# --------------------------------------------------------------- operators --

def _stream_ptr(stream=None):
    """hipStream_t of a torch stream (None: the current one); an int is taken
    as the raw handle (0: the null stream)."""
    if isinstance(stream, int):
        return stream
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def _unit_col(t) -> bool:
    """Elements of a row are adjacent (a one-element row has any stride)."""
    return t.shape[-1] == 1 or t.stride(-1) == 1


def _require(t, dtype, name, dims=(2,)):
    """Type, rank and layout of one operand (the device is checked last, by
    _on_device, so that every shape error is reported first)."""
    import torch
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if t.dim() not in dims or not _unit_col(t):
        raise ValueError(f"{name} must be {'/'.join(map(str, dims))}-D with "
                         "unit column stride")


def _shape(t, expected, name):
    if tuple(t.shape) != tuple(expected):
        raise ValueError(f"{name} must be {list(expected)}, got {list(t.shape)}")


def _on_device(*named):
    """Every operand is a device tensor on the same GPU: the C-ABI sees only
    pointers, and a host or foreign-device pointer would fault the kernel."""
    device = None
    for t, name in named:
        if t is None:
            continue
        if not t.is_cuda:
            raise TypeError(f"{name} must be a device tensor")
        if device is None:
            device = t.device
        elif t.device != device:
            raise ValueError(f"{name} is on {t.device}, expected {device}")


def matmul(a, b, c=None, *, b_transposed=False, accumulate=False,
           out_dtype=None, a_transposed=False, stream=None):
    """linalg.matmul dispatch: C = [C +] A . B on the MI355X kernels.

    f16 inputs accumulate in f32 and write f16 (or f32 with
    out_dtype=torch.float32); int8 inputs accumulate exactly into int32.
    ``b_transposed``: B is stored [N, K]. ``a_transposed`` (f16 only): A is
    stored [K, M]. ``c`` (required with ``accumulate``) must be [M, N].
    """
    import torch
    if a.dtype == torch.int8:
        if a_transposed:
            raise ValueError("a_transposed is an f16 layout")
        _require(a, torch.int8, "a")
        _require(b, torch.int8, "b")
        if out_dtype not in (None, torch.int32):
            raise TypeError("int8 matmul writes int32")
        out_dtype = torch.int32
    else:
        _require(a, torch.float16, "a")
        _require(b, torch.float16, "b")
        out_dtype = out_dtype or torch.float16
        if out_dtype not in (torch.float16, torch.float32):
            raise TypeError("f16 matmul writes float16 or float32")
    k, m = a.shape if a_transposed else a.shape[::-1]
    n = b.shape[0] if b_transposed else b.shape[1]
    if (b.shape[1] if b_transposed else b.shape[0]) != k:
        raise ValueError("contraction extents differ")
    if c is None:
        if accumulate:
            raise ValueError("accumulate needs an init tensor c")
    else:
        _require(c, out_dtype, "c")
        _shape(c, (m, n), "c")
    _on_device((a, "a"), (b, "b"), (c, "c"))
    lib = library()
    if c is None:
        c = torch.empty((m, n), dtype=out_dtype, device=a.device)
    flags = ((B_TRANSPOSED if b_transposed else 0) |
             (ACCUMULATE if accumulate else 0) |
             (A_TRANSPOSED if a_transposed else 0))
    s = _stream_ptr(stream)
    if a.dtype != torch.int8 and out_dtype == torch.float32:
        flags |= OUT_F32
    ws, wsb = stream_workspace(_matmul_workspace_need(m, n, k, flags),
                               a.device, s)
    if a.dtype == torch.int8:
        _check(lib.iree_mi355x_matmul_i8(a.data_ptr(), b.data_ptr(),
                                         c.data_ptr(), m, n, k, a.stride(0),
                                         b.stride(0), c.stride(0), flags, ws,
                                         wsb, s))
    else:
        _check(lib.iree_mi355x_matmul_f16(a.data_ptr(), b.data_ptr(),
                                          c.data_ptr(), m, n, k, a.stride(0),
                                          b.stride(0), c.stride(0), flags,
                                          ws, wsb, s))
    return c


def _epilogue(bias, activation, multiplier, m, n, batch):
    import torch
    if isinstance(activation, int):
        if activation not in _ACT_NAMES.values():
            raise ValueError(f"unknown activation {activation}")
        act = activation
    else:
        if activation not in _ACT_NAMES:
            raise ValueError(f"unknown activation {activation!r}")
        act = _ACT_NAMES[activation]
    if bias is None and multiplier is None and act == ACT_NONE:
        return None
    e = Epilogue()
    e.activation = act
    if bias is not None:
        _require(bias, torch.float16, "bias", (1,))
        if bias.numel() != n or not bias.is_contiguous():
            raise ValueError("bias must be a contiguous f16 vector of N")
        e.bias = bias.data_ptr()
    if multiplier is not None:
        _require(multiplier, torch.float16, "multiplier", (2, 3))
        if tuple(multiplier.shape[-2:]) != (m, n):
            raise ValueError(f"multiplier must be [.., {m}, {n}]")
        if multiplier.dim() == 3 and multiplier.shape[0] != batch:
            raise ValueError("multiplier batch differs")
        e.multiplier = multiplier.data_ptr()
        e.ld_multiplier = multiplier.stride(-2)
        e.batch_stride_multiplier = (multiplier.stride(0)
                                     if multiplier.dim() == 3 and batch > 1
                                     else 0)
    return e


def batch_matmul(a, b, c=None, *, b_transposed=False, accumulate=False,
                 out_dtype=None, bias=None, activation=None, multiplier=None,
                 a_transposed=False, stream=None):
    """linalg.batch_matmul (f16, f32 accumulation) with a fused epilogue:
    C[z] = [C[z] +] multiplier[z] * act(A[z] . B[z] + bias).

    a: [Z, M, K] (or [M, K] shared; [Z, K, M] / [K, M] with
    ``a_transposed``); b: [Z, K, N] / [Z, N, K] with ``b_transposed`` (or
    2-D, shared by the batch); bias [N]; multiplier
    [Z, M, N] or [M, N]; activation None / "relu" / "gelu_tanh" / "silu".
    c is [Z, M, N] when either operand is 3-D, else [M, N].
    Every matrix needs a unit column stride; batch strides may be 0.
    """
    import torch
    _require(a, torch.float16, "a", (2, 3))
    _require(b, torch.float16, "b", (2, 3))
    out_dtype = out_dtype or torch.float16
    if out_dtype not in (torch.float16, torch.float32):
        raise TypeError("batch_matmul writes float16 or float32")
    a3 = a if a.dim() == 3 else a.unsqueeze(0)
    b3 = b if b.dim() == 3 else b.unsqueeze(0)
    batched = a.dim() == 3 or b.dim() == 3
    batch = max(a3.shape[0], b3.shape[0])
    k, m = (a3.shape[1], a3.shape[2]) if a_transposed else (a3.shape[2], a3.shape[1])
    n = b3.shape[1] if b_transposed else b3.shape[2]
    if (b3.shape[2] if b_transposed else b3.shape[1]) != k:
        raise ValueError("contraction extents differ")
    for t, name in ((a3, "a"), (b3, "b")):
        if t.shape[0] not in (1, batch):
            raise ValueError(f"{name}: batch extent {t.shape[0]} is neither 1 "
                             f"nor {batch}")
    sa = 0 if a3.shape[0] == 1 else a3.stride(0)
    sb = 0 if b3.shape[0] == 1 else b3.stride(0)
    out_shape = (batch, m, n) if batched else (m, n)
    if c is None:
        if accumulate:
            raise ValueError("accumulate needs an init tensor c")
    else:
        _require(c, out_dtype, "c", (3,) if batched else (2,))
        _shape(c, out_shape, "c")
    e = _epilogue(bias, activation, multiplier, m, n, batch)
    _on_device((a, "a"), (b, "b"), (c, "c"), (bias, "bias"),
               (multiplier, "multiplier"))
    lib = library()
    if c is None:
        c = torch.empty(out_shape, dtype=out_dtype, device=a.device)
    c3 = c if c.dim() == 3 else c.unsqueeze(0)
    sc = c3.stride(0) if batch > 1 else m * n
    flags = ((B_TRANSPOSED if b_transposed else 0) |
             (ACCUMULATE if accumulate else 0) |
             (OUT_F32 if out_dtype == torch.float32 else 0) |
             (A_TRANSPOSED if a_transposed else 0))
    st = _stream_ptr(stream)
    ws, wsb = stream_workspace(_batch_workspace_need(batch, m, n, k, flags),
                               a.device, st)
    _check(lib.iree_mi355x_batch_matmul_f16(
        a3.data_ptr(), b3.data_ptr(), c3.data_ptr(), batch, m, n, k,
        a3.stride(1), b3.stride(1), c3.stride(1), sa, sb, sc, flags,
        ctypes.byref(e) if e is not None else None, ws, wsb, st))
    return c


def linear(x, w, bias=None, *, activation=None, multiplier=None,
           w_transposed=False, out=None, stream=None):
    """y = multiplier * act(x . W + bias) for x [M, K], W [K, N] (or [N, K]
    with ``w_transposed``): one dispatch, epilogue fused into the store."""
    return batch_matmul(x, w, out, b_transposed=w_transposed, bias=bias,
                        activation=activation, multiplier=multiplier,
                        stream=stream)


def quantized_matmul(x, w, scale, y=None, *, w_transposed=False, stream=None):
    """W8A16 linear: y = f16((x . w_int8) * scale[n]), zero point 0.
    x [M, K] f16, w [K, N] int8 (or [N, K] with ``w_transposed``), scale [N]
    f16, y [M, N] f16."""
    import torch
    _require(x, torch.float16, "x")
    _require(w, torch.int8, "w")
    m, k = x.shape
    n = w.shape[0] if w_transposed else w.shape[1]
    if (w.shape[1] if w_transposed else w.shape[0]) != k:
        raise ValueError("w does not contract over K")
    _require(scale, torch.float16, "scale", (1,))
    if scale.numel() != n or not scale.is_contiguous():
        raise ValueError("scale must be a contiguous f16 vector of N")
    if y is not None:
        _require(y, torch.float16, "y")
        _shape(y, (m, n), "y")
    _on_device((x, "x"), (w, "w"), (scale, "scale"), (y, "y"))
    lib = library()
    if y is None:
        y = torch.empty((m, n), dtype=torch.float16, device=x.device)
    flags = B_TRANSPOSED if w_transposed else 0
    st = _stream_ptr(stream)
    ws, wsb = stream_workspace(_matmul_workspace_need(m, n, k, flags),
                               x.device, st)
    _check(lib.iree_mi355x_w8a16_matmul(
        x.data_ptr(), w.data_ptr(), scale.data_ptr(), y.data_ptr(), m, n, k,
        x.stride(0), w.stride(0), y.stride(0), flags, ws, wsb, st))
    return y


class AttentionStrides(ctypes.Structure):
    """iree_mi355x_attention_strides_t: (batch, head, row) element strides of
    q, k, v and o."""
    _fields_ = [("q", ctypes.c_int64 * 3), ("k", ctypes.c_int64 * 3),
                ("v", ctypes.c_int64 * 3), ("o", ctypes.c_int64 * 3)]


class AttentionArgs(ctypes.Structure):
    """iree_mi355x_attention_t."""
    _fields_ = [("q", ctypes.c_void_p), ("k", ctypes.c_void_p),
                ("v", ctypes.c_void_p), ("o", ctypes.c_void_p),
                ("mask", ctypes.c_void_p), ("batch", ctypes.c_int64),
                ("heads", ctypes.c_int64), ("kv_heads", ctypes.c_int64),
                ("seq_q", ctypes.c_int64), ("seq_kv", ctypes.c_int64),
                ("head_dim", ctypes.c_int64), ("head_dim_v", ctypes.c_int64),
                ("scale", ctypes.c_float), ("flags", ctypes.c_uint32),
                ("strides", AttentionStrides),
                ("mask_strides", ctypes.c_int64 * 4)]


def attention(q, k, v, o=None, *, causal=True, scale=None, mask=None,
              out_dtype=None, stream=None):
    """Fused attention forward: q [B, Hq, Sq, D], k [B, Hkv, Skv, D],
    v [B, Hkv, Skv, Dv] f16 with Hq a multiple of Hkv (query head h reads KV
    head h // (Hq // Hkv)); o [B, Hq, Sq, Dv], f16 or f32 (``out_dtype``
    when o is not given). ``mask``, an f16 tensor that broadcasts to
    [B, Hq, Sq, Skv], is added to the scaled scores; a row whose keys are all
    -inf is 0. Any operand may be a strided view whose last dimension is
    contiguous (a slice of a longer KV cache, o a permuted view of a
    [B, Sq, Hq, Dv] buffer). Equal head dims of 64 or 128 with no mask and
    an f16 o run the MFMA kernel; the rest the general one (head dims up to
    256)."""
    import torch
    for t, nm in ((q, "q"), (k, "k"), (v, "v")):
        if (not isinstance(t, torch.Tensor) or t.dtype != torch.float16
                or t.dim() != 4 or not _unit_col(t)):
            raise TypeError(f"{nm} must be a 4-D f16 tensor with unit "
                            "stride along head_dim")
    if o is not None:
        if (not isinstance(o, torch.Tensor)
                or o.dtype not in (torch.float16, torch.float32)
                or o.dim() != 4 or not _unit_col(o)):
            raise TypeError("o must be a 4-D f16 or f32 tensor with unit "
                            "stride along head_dim")
        if out_dtype is not None and out_dtype != o.dtype:
            raise TypeError(f"o is {o.dtype}, out_dtype {out_dtype}")
    out_dtype = o.dtype if o is not None else (out_dtype or torch.float16)
    if out_dtype not in (torch.float16, torch.float32):
        raise TypeError("out_dtype must be torch.float16 or torch.float32")
    b, h, sq, d = q.shape
    hkv, skv = k.shape[1], k.shape[2]
    dv = v.shape[3]
    if hkv < 1 or h % hkv:
        raise ValueError(f"k must be [{b}, Hkv, Skv, {d}] with Hkv dividing "
                         f"the {h} query heads, got {list(k.shape)}")
    _shape(k, (b, hkv, skv, d), "k")
    _shape(v, (b, hkv, skv, dv), "v")
    if o is not None:
        _shape(o, (b, h, sq, dv), "o")
    if mask is not None:
        if not isinstance(mask, torch.Tensor) or mask.dtype != torch.float16:
            raise TypeError("mask must be an f16 tensor")
        try:
            mask = mask.expand(b, h, sq, skv)
        except RuntimeError:
            raise ValueError(f"mask {list(mask.shape)} does not broadcast to "
                             f"{[b, h, sq, skv]}") from None
    _on_device((q, "q"), (k, "k"), (v, "v"), (o, "o"), (mask, "mask"))
    lib = library()
    if scale is None:
        scale = d ** -0.5
    if o is None:
        o = torch.empty(b, h, sq, dv, dtype=out_dtype, device=q.device)
    flags = CAUSAL if causal else 0
    fast = (mask is None and out_dtype == torch.float16 and d == dv
            and d in (64, 128))
    if fast and hkv == h and all(t.is_contiguous() for t in (q, k, v, o)):
        _check(lib.iree_mi355x_attention_f16(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), b, h, sq,
            skv, d, float(scale), flags, _stream_ptr(stream)))
        return o
    st = AttentionStrides()
    for field, t in (("q", q), ("k", k), ("v", v), ("o", o)):
        getattr(st, field)[:] = list(t.stride()[:3])
    if fast:
        _check(lib.iree_mi355x_attention_f16_strided(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), b, h,
            hkv, sq, skv, d, float(scale), flags, ctypes.byref(st),
            _stream_ptr(stream)))
        return o
    a = AttentionArgs(q=q.data_ptr(), k=k.data_ptr(), v=v.data_ptr(),
                      o=o.data_ptr(), batch=b, heads=h, kv_heads=hkv,
                      seq_q=sq, seq_kv=skv, head_dim=d, head_dim_v=dv,
                      scale=float(scale), strides=st)
    if out_dtype == torch.float32:
        flags |= ATTENTION_OUT_F32
    if mask is not None:
        flags |= ATTENTION_MASK
        a.mask = mask.data_ptr()
        a.mask_strides[:] = list(mask.stride())
    a.flags = flags
    _check(lib.iree_mi355x_attention(ctypes.byref(a), _stream_ptr(stream)))
    return o


def matmul_mfma_config(index, a, b, c, *, scale=None, splits=0, accumulate=False,
                       stream=None):
    """Run one compiled MFMA configuration (autotuner entry point).

    The configuration's B form decides how `b` is read: TN takes B [N, K],
    NN takes B [K, N] of the A type (f16, or int8 for the int8 row-major
    form), W8A16 takes B [K, N] int8 plus `scale`; a
    transposed-A configuration takes A [K, M]. `splits` forces a split-K
    configuration's K split count (0: the planner's; SPLITS_STREAM_K:
    stream-K runs). With `accumulate` the result is added into `c`."""
    import torch
    cfg = mfma_configs()[index]
    a_dtype = torch.int8 if cfg.a_elem == ELEM_I8 else torch.float16
    b_dtype = torch.int8 if cfg.b_form == B_FORM_W8A16 else a_dtype
    c_dtype = {ELEM_I32: torch.int32, ELEM_F32: torch.float32}.get(
        cfg.c_elem, torch.float16)
    _require(a, a_dtype, "a")
    _require(b, b_dtype, "b")
    _require(c, c_dtype, "c")
    k, m = a.shape if cfg.a_transposed else a.shape[::-1]
    if cfg.b_form == B_FORM_TN:
        n, flags = b.shape[0], B_TRANSPOSED
    else:
        n, flags = b.shape[1], 0
    if cfg.a_transposed:
        flags |= A_TRANSPOSED
    # The C-ABI sees only pointers: the extents it is given must be the
    # tensors' own, or the kernel would stream past a buffer.
    if (b.shape[1] if cfg.b_form == B_FORM_TN else b.shape[0]) != k:
        raise ValueError(f"{cfg.name}: b does not contract over K = {k}")
    _shape(c, (m, n), "c")
    if cfg.b_form == B_FORM_W8A16:
        if scale is None:
            raise ValueError(f"{cfg.name}: needs a scale")
        _require(scale, torch.float16, "scale", (1,))
        if scale.numel() != n or not scale.is_contiguous():
            raise ValueError("scale must be a contiguous f16 vector of N")
    _on_device((a, "a"), (b, "b"), (c, "c"), (scale, "scale"))
    if c.dtype == torch.float32 and a.dtype == torch.float16:
        flags |= OUT_F32
    if accumulate:
        flags |= ACCUMULATE
    lib = library()
    s = _stream_ptr(stream)
    ws, wsb = stream_workspace(
        lib.iree_mi355x_matmul_mfma_config_workspace_bytes(index, splits, m, n,
                                                           k, flags),
        a.device, s)
    _check(lib.iree_mi355x_matmul_mfma_config_split(
        index, splits, a.data_ptr(), b.data_ptr(),
        scale.data_ptr() if scale is not None else None, c.data_ptr(), m, n,
        k, a.stride(0), b.stride(0), c.stride(0), flags, ws, wsb, s))
    return c


# ----------------------------------------------------------------- runtime --

def slot(index: int, offset: int = 0, length: int = WHOLE_BUFFER) -> BufferRef:
    """Reference to binding-table slot `index` (bytes [offset, +length))."""
    return BufferRef(index, None, offset, length)


def direct(t, offset: int = 0, length: int | None = None) -> BufferRef:
    """Reference to a device tensor (or (pointer, bytes)) directly."""
    ptr, nbytes = _ptr_len(t)
    return BufferRef(BINDING_DIRECT, ptr, offset,
                     nbytes - offset if length is None else length)


def _ptr_len(t):
    if isinstance(t, tuple):
        return t
    return t.data_ptr(), t.numel() * t.element_size()


def binding_table(entries):
    """A binding table from device tensors or (pointer, bytes) pairs."""
    arr = (Binding * max(1, len(entries)))()
    for i, e in enumerate(entries):
        arr[i] = Binding(*_ptr_len(e))
    return arr, len(entries)


class CommandBuffer:
    """Recorded dispatches, fills, copies and barriers of an executable
    library (this library's own, or a `LoadedExecutable`'s), submitted onto
    HIP streams with the dispatches of each barrier segment spread over up to
    `max_concurrent` streams."""

    def __init__(self, executable=None):
        lib = library()
        self._lib = lib
        self._exe = executable          # keeps a loaded library alive
        table = executable.table_ptr if executable is not None else None
        h = ctypes.c_void_p()
        _check(lib.iree_mi355x_command_buffer_create(table, ctypes.byref(h)))
        self._h = h
        self._names = (executable.export_names() if executable is not None
                       else export_names())

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            self._lib.iree_mi355x_command_buffer_release(h)
            self._h = None

    def __len__(self):
        return self._lib.iree_mi355x_command_buffer_count(self._h)

    def dispatch(self, export, constants, bindings):
        ordinal = self._names.index(export) if isinstance(export, str) else export
        consts = (ctypes.c_uint32 * max(1, len(constants)))(*constants)
        refs = (BufferRef * max(1, len(bindings)))(*bindings)
        _check(self._lib.iree_mi355x_command_buffer_dispatch(
            self._h, ordinal, consts, len(constants), refs, len(bindings)))
        return self

    def fill(self, target: BufferRef, pattern: bytes):
        buf = ctypes.create_string_buffer(bytes(pattern), len(pattern))
        _check(self._lib.iree_mi355x_command_buffer_fill(
            self._h, target, buf, len(pattern)))
        return self

    def copy(self, source: BufferRef, target: BufferRef, length: int):
        _check(self._lib.iree_mi355x_command_buffer_copy(
            self._h, source, target, length))
        return self

    def barrier(self):
        _check(self._lib.iree_mi355x_command_buffer_barrier(self._h))
        return self

    def end(self):
        _check(self._lib.iree_mi355x_command_buffer_end(self._h))
        return self

    def workspace_bytes(self, table=(), max_concurrent=0) -> int:
        arr, n = binding_table(list(table))
        return self._lib.iree_mi355x_command_buffer_workspace_bytes(
            self._h, arr, n, max_concurrent)

    def lane_schedule(self, max_concurrent=0) -> list[tuple]:
        """The stream operations a submission at this concurrency issues,
        in order: (kind, lane, event, command) with kind one of LANE_OP_*;
        lane 0 is the caller's stream, event 0 the fork event and event
        1 + l lane l's event. Host-only: no device is touched."""
        n = self._lib.iree_mi355x_command_buffer_lane_schedule(
            self._h, max_concurrent, None, 0)
        ops = (LaneOp * max(n, 1))()
        got = self._lib.iree_mi355x_command_buffer_lane_schedule(
            self._h, max_concurrent, ops, n)
        assert got == n
        return [(o.kind, o.lane, o.event, o.command) for o in ops[:n]]

    def submit(self, table=(), max_concurrent=0, workspace=None, stream=None):
        """Submit on `stream`; without a `workspace` the lane slices come
        from the wrapper's workspace of that stream for this slice size
        (lane l's counters sit at l slices: a buffer serves one slice size)."""
        arr, n = binding_table(list(table))
        s = _stream_ptr(stream)
        if workspace is None:
            need = self._lib.iree_mi355x_command_buffer_workspace_bytes(
                self._h, arr, n, max_concurrent)
            slice_ = self._lib.iree_mi355x_command_buffer_workspace_bytes(
                self._h, arr, n, 1) if need else 0
            ws, wsb = stream_workspace(need, None, s, ("lanes", slice_))
        else:
            ws, wsb = _ptr_len(workspace)
        _check(self._lib.iree_mi355x_command_buffer_submit(
            self._h, arr, n, max_concurrent, ws, wsb, s))


def kernel_resources(device: bool = True) -> list[dict]:
    """Every compiled kernel: name, the exports that may launch it (a list
    of export names) and its launch threads; with ``device``, also the VGPRs,
    static LDS, scratch per lane, launch bound and resident workgroups per
    CU that the loaded code object reports."""
    lib = library()
    names = export_names()
    out = []
    for i in range(lib.iree_mi355x_kernel_count()):
        r = KernelResources()
        st = lib.iree_mi355x_kernel_resources(i, ctypes.byref(r))
        if st != OK and (device or st != NO_DEVICE):
            _check(st)
        rec = {"name": r.name.decode(), "threads": r.threads,
               "exports": [n for b, n in enumerate(names) if r.exports >> b & 1]}
        if st == OK:
            rec.update(vgprs=r.vgprs, lds_bytes=r.lds_bytes,
                       scratch_bytes=r.scratch_bytes, max_threads=r.max_threads,
                       workgroups_per_cu=r.workgroups_per_cu)
        out.append(rec)
    return out


# ------------------------------------------------------------- executables --

def serialize_executable(library_path: str | None = None) -> bytes:
    """The versioned container of an ELF dispatch library (default: this
    one) with its export table and checksum."""
    lib = library()
    path = library_path.encode() if library_path else None
    need = lib.iree_mi355x_executable_serialize(path, None, 0)
    if need == 0:
        raise MI355XError(INVALID_ARGUMENT, last_error())
    buf = ctypes.create_string_buffer(need)
    got = lib.iree_mi355x_executable_serialize(path, buf, need)
    if got != need:
        raise MI355XError(INVALID_ARGUMENT, last_error())
    return buf.raw


def verify_executable(data: bytes) -> int:
    """Status of the container's header / version / arch / checksum check."""
    return library().iree_mi355x_executable_verify(data, len(data))


class LoadedExecutable:
    """A container loaded into this process (its ELF dlopened privately)."""

    def __init__(self, data: bytes):
        lib = library()
        self._lib = lib
        h = ctypes.c_void_p()
        _check(lib.iree_mi355x_executable_load(data, len(data), ctypes.byref(h)))
        self._h = h
        self.table_ptr = lib.iree_mi355x_loaded_executable_library(h)

    def export_names(self) -> list[str]:
        table = ctypes.cast(self.table_ptr, ctypes.POINTER(Library)).contents
        return [table.exports.names[i].decode()
                for i in range(table.exports.count)]

    def release(self):
        """Unload (every dispatch of it must have completed)."""
        if self._h is not None and self._h.value:
            self._lib.iree_mi355x_loaded_executable_release(self._h)
        self._h = None
