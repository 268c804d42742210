"""The runtime's command buffers without a GPU: recording, and every
validation a submission runs before it enqueues anything (binding-table
resolution, each export's own checks through its workspace query, fill /
copy ranges, workspace sizing)."""
import pytest

FAKE = 0x10000  # aligned, never dereferenced: every call here fails or plans


def matmul_consts(pkg, m, n, k, flags=0):
    return pkg.matmul_constants(m, n, k, k, n, n, flags)


def skinny_cb(pkg, count=4, m=16, n=4096, k=4096):
    """`count` independent split-K matmuls (A_i, B, C_i from table slots)."""
    cb = pkg.CommandBuffer()
    for i in range(count):
        cb.dispatch("matmul_f16", matmul_consts(pkg, m, n, k),
                    [pkg.slot(3 * i), pkg.slot(3 * i + 1), pkg.slot(3 * i + 2)])
    return cb.end()


def skinny_table(count=4, m=16, n=4096, k=4096):
    t = []
    for i in range(count):
        base = FAKE * (1 + 3 * i) << 12
        t += [(base, m * k * 2), (base + (1 << 27), k * n * 2),
              (base + (2 << 27), m * n * 2)]
    return t


def test_record_and_end(pkg):
    cb = pkg.CommandBuffer()
    cb.fill(pkg.slot(0), b"\x00\x3c")
    cb.barrier()
    cb.copy(pkg.slot(0), pkg.slot(1), 64)
    assert len(cb) == 3
    cb.end()
    with pytest.raises(pkg.MI355XError) as e:
        cb.barrier()
    assert e.value.status == pkg.INVALID_ARGUMENT and "ended" in str(e.value)


def test_record_errors(pkg):
    cb = pkg.CommandBuffer()
    with pytest.raises(pkg.MI355XError) as e:
        cb.dispatch(99, [0], [pkg.slot(0)])
    assert e.value.status == pkg.INVALID_ARGUMENT
    with pytest.raises(pkg.MI355XError):
        cb.fill(pkg.slot(0), b"\x01\x02\x03")       # 3-byte pattern
    lib = pkg.library()
    # submit before end
    arr, n = pkg.binding_table([])
    assert lib.iree_mi355x_command_buffer_submit(cb._h, arr, n, 1, None, 0,
                                                 None) == pkg.INVALID_ARGUMENT
    assert "not ended" in pkg.last_error()


def test_submit_validation_enqueues_nothing(pkg):
    cb = skinny_cb(pkg)
    table = skinny_table()
    # slot outside the table
    with pytest.raises(pkg.MI355XError) as e:
        cb.submit(table[:5], max_concurrent=1, stream=0)
    assert e.value.status == pkg.INVALID_ARGUMENT and "slot 5" in str(e.value)
    # a binding too short for what the export reads: the export's own check,
    # reported with the command index and export name
    short = list(table)
    short[4] = (short[4][0], 16)
    with pytest.raises(pkg.MI355XError) as e:
        cb.submit(short, max_concurrent=4, stream=0)
    assert "command 1 (matmul_f16)" in str(e.value)
    # too many lanes
    with pytest.raises(pkg.MI355XError) as e:
        cb.submit(table, max_concurrent=9, stream=0)
    assert e.value.status == pkg.INVALID_ARGUMENT


def test_fill_and_copy_validation(pkg):
    cb = pkg.CommandBuffer()
    cb.fill(pkg.slot(0, 2, 6), b"\x01\x02\x03\x04")   # offset 2 vs 4-byte pattern
    cb.end()
    with pytest.raises(pkg.MI355XError) as e:
        cb.submit([(FAKE, 64)], stream=0)
    assert "multiple" in str(e.value)
    cb = pkg.CommandBuffer()
    cb.copy(pkg.slot(0, 0, 64), pkg.slot(0, 32, 64), 64)  # overlapping
    cb.end()
    with pytest.raises(pkg.MI355XError) as e:
        cb.submit([(FAKE, 256)], stream=0)
    assert "overlap" in str(e.value)
    cb = pkg.CommandBuffer()
    cb.copy(pkg.slot(0), pkg.slot(1), 128)               # longer than slot 1
    cb.end()
    with pytest.raises(pkg.MI355XError) as e:
        cb.submit([(FAKE, 256), (FAKE * 16, 64)], stream=0)
    assert "overruns" in str(e.value)
    cb = pkg.CommandBuffer()
    cb.fill(pkg.BufferRef(pkg.BINDING_DIRECT, FAKE, 0, pkg.WHOLE_BUFFER), b"\x00")
    cb.end()
    with pytest.raises(pkg.MI355XError) as e:
        cb.submit([], stream=0)
    assert "needs a length" in str(e.value)


def test_workspace_sizing(pkg):
    """One slice per lane, each the largest split-K workspace of any
    dispatch (what the planner gives that shape), 256-byte aligned; lanes
    are capped by the widest barrier segment."""
    F16 = pkg.ELEM_F16
    need = pkg.plan(pkg.make_desc(F16, F16, F16, 16, 4096, 4096)).workspace_bytes
    assert need > 0
    slice_ = (need + 255) // 256 * 256
    cb = skinny_cb(pkg, count=4)
    table = skinny_table(4)
    assert cb.workspace_bytes(table, 1) == slice_
    assert cb.workspace_bytes(table, 2) == 2 * slice_
    assert cb.workspace_bytes(table, 0) == slice_         # default: in order
    assert cb.workspace_bytes(table, 8) == 4 * slice_     # 4 dispatches only
    # too small a caller workspace is refused before anything is enqueued
    with pytest.raises(pkg.MI355XError) as e:
        cb.submit(table, max_concurrent=4, workspace=(FAKE, slice_), stream=0)
    assert e.value.status == pkg.WORKSPACE_TOO_SMALL
    # full tiles: no workspace at all
    cb = pkg.CommandBuffer()
    cb.dispatch("matmul_f16", matmul_consts(pkg, 2048, 4096, 4096),
                [pkg.slot(0), pkg.slot(1), pkg.slot(2)]).end()
    assert cb.workspace_bytes([(FAKE, 2048 * 4096 * 2), (FAKE * 2, 4096 ** 2 * 2),
                               (FAKE * 4, 2048 * 4096 * 2)], 4) == 0


def test_workspace_query_through_export(pkg):
    """An export called with a workspace query validates and plans only."""
    st, need = pkg.call_export(
        "matmul_f16", matmul_consts(pkg, 16, 4096, 4096),
        [FAKE, FAKE << 8, FAKE << 9], [16 * 4096 * 2, 4096 * 4096 * 2,
                                       16 * 4096 * 2], stream=0, query=True)
    F16 = pkg.ELEM_F16
    assert st == pkg.OK
    assert need == pkg.plan(pkg.make_desc(F16, F16, F16, 16, 4096, 4096)).workspace_bytes
    st, need = pkg.call_export("matmul_i8", matmul_consts(pkg, 64, 64, 64),
                               [FAKE, FAKE, FAKE], [4096, 4096, 16384],
                               stream=0, query=True)
    assert st == pkg.OK and need == 0
    st, _ = pkg.call_export("matmul_f16", matmul_consts(pkg, 64, 64, 64),
                            [FAKE, FAKE, FAKE], [4096, 4096, 10],
                            stream=0, query=True)
    assert st == pkg.INVALID_ARGUMENT
