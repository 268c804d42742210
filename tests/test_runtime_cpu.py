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
    # and so is none at all: the runtime allocates no workspace of its own
    arr, n = pkg.binding_table(table)
    assert pkg.library().iree_mi355x_command_buffer_submit(
        cb._h, arr, n, 2, None, 0, None) == pkg.WORKSPACE_TOO_SMALL
    assert "workspace" in pkg.last_error()
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


# ------------------------------------------------------- lane schedule ----

def happens_before(pkg, ops):
    """Simulate a lane schedule: stream order within each lane plus
    record -> wait edges. Returns, per enqueued command, the set of
    commands that finish before it starts, and the set the caller's stream
    (lane 0) has waited for at the end. A wait takes the event's latest
    record at the time of the wait (the HIP / CUDA event semantics)."""
    lane_done = {}   # lane -> commands ordered before the lane's next op
    event_set = {}   # event -> commands covered by its latest record
    before = {}
    for kind, lane, event, command in ops:
        done = lane_done.setdefault(lane, set())
        if kind == pkg.LANE_OP_RECORD:
            event_set[event] = set(done)
        elif kind == pkg.LANE_OP_WAIT:
            assert event in event_set, f"wait on event {event} before a record"
            done |= event_set[event]
        else:
            assert command not in before, f"command {command} enqueued twice"
            before[command] = set(done)
            done.add(command)
    return before, lane_done.get(0, set())


def segments_of(pkg, kinds):
    """Command index -> barrier segment, for a list of 'd' / 'b' kinds."""
    seg, out = 0, {}
    for i, k in enumerate(kinds):
        if k == "b":
            seg += 1
        else:
            out[i] = seg
    return out


def build(pkg, kinds):
    cb = pkg.CommandBuffer()
    for k in kinds:
        if k == "b":
            cb.barrier()
        else:
            cb.fill(pkg.slot(0), b"\x00\x00")
    return cb.end()


@pytest.mark.parametrize("kinds", [
    "ddddd", "ddddbddbd", "dbdbdbd", "dddddddddbdd", "ddbbddd", "bdddb",
    "d", "ddddddddddddddddd",
])
@pytest.mark.parametrize("lanes", [1, 2, 3, 4, 8])
def test_lane_schedule_orders_segments_and_joins_every_lane(pkg, kinds, lanes):
    """The schedule a submission issues (the same one submit executes):
    every command runs after every command of the earlier barrier
    segments; the caller's stream ends after every command (each lane
    joined back); no lane waits on its own event; each command is enqueued
    once; every wait follows a record of its event."""
    cb = build(pkg, kinds)
    ops = cb.lane_schedule(lanes)
    seg = segments_of(pkg, kinds)
    before, caller_end = happens_before(pkg, ops)
    assert set(before) == set(seg)
    for c, s in seg.items():
        for p_, ps in seg.items():
            if ps < s:
                assert p_ in before[c], (kinds, lanes, p_, c)
    assert caller_end | {c for c in seg
                         if any(o[0] == pkg.LANE_OP_ENQUEUE and o[1] == 0
                                and o[3] == c for o in ops)} >= set(seg)
    # every lane's last command is ordered before the caller's end
    last_on_lane = {}
    for kind, lane, _, command in ops:
        if kind == pkg.LANE_OP_ENQUEUE:
            last_on_lane[lane] = command
    for lane, c in last_on_lane.items():
        assert lane == 0 or c in caller_end, (kinds, lanes, lane)
    # no self-waits: a lane never waits on the event it records
    for kind, lane, event, _ in ops:
        if kind == pkg.LANE_OP_WAIT:
            assert event != 1 + lane
    # lanes used: the request, capped by the widest barrier segment; a
    # single lane runs in order with no events
    widest = max(len(r) for r in kinds.split("b"))
    eff = max(1, min(lanes, widest))
    used = {o[1] for o in ops if o[0] == pkg.LANE_OP_ENQUEUE}
    assert used == set(range(eff))
    if eff == 1:
        assert all(o[0] == pkg.LANE_OP_ENQUEUE for o in ops)
    else:
        assert ops[0][:3] == (pkg.LANE_OP_RECORD, 0, 0)


def test_lane_schedule_in_order_has_no_events(pkg):
    cb = build(pkg, "ddbdd")
    ops = cb.lane_schedule(1)
    assert [o[0] for o in ops] == [pkg.LANE_OP_ENQUEUE] * 4
    assert [o[3] for o in ops] == [0, 1, 3, 4] and {o[1] for o in ops} == {0}


def test_lane_schedule_deals_round_robin(pkg):
    # 5 commands on 4 lanes: lanes 0..3 then lane 0 again; the fork event
    # is waited on by lanes 1..3 only
    ops = build(pkg, "ddddd").lane_schedule(4)
    enq = [(o[1], o[3]) for o in ops if o[0] == pkg.LANE_OP_ENQUEUE]
    assert enq == [(0, 0), (1, 1), (2, 2), (3, 3), (0, 4)]
    fork_waits = sorted(o[1] for o in ops
                        if o[0] == pkg.LANE_OP_WAIT and o[2] == 0)
    assert fork_waits == [1, 2, 3]
