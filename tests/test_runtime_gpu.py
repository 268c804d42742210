"""The runtime's command buffers on the GPU: concurrent dispatches between
barriers on lane streams with their own workspace slices, fills and copies,
ordering across barriers, validation that enqueues nothing, and replay of a
captured submission."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

FP16_BOUND = 2e-3


def consts(pkg, m, n, k, flags=0):
    return pkg.matmul_constants(m, n, k, k, n, n, flags)


class Program:
    """Segment 1: C_i = A_i.B for four skinny (split-K) matmuls, and a fill
    of F. Segment 2: D = copy(C_0), C_1 += A_1.B. Segment 3: E = copy(C_1).
    Binding table: A_0..A_3, B, C_0..C_3, D, E, F."""

    M, N, K = 16, 4096, 2048

    def __init__(self, pkg, dev, seed=0):
        g = torch.Generator().manual_seed(seed)
        m, n, k = self.M, self.N, self.K
        self.a = [(torch.randn(m, k, generator=g) * 0.5).half() for _ in range(4)]
        self.b = torch.randn(k, n, generator=g).half()
        self.dev = dev
        self.da = [x.to(dev) for x in self.a]
        self.db = self.b.to(dev)
        self.dc = [torch.full((m, n), 9.0, dtype=torch.float16, device=dev)
                   for _ in range(4)]
        self.dd = torch.full((m, n), 9.0, dtype=torch.float16, device=dev)
        self.de = torch.full((m, n), 9.0, dtype=torch.float16, device=dev)
        self.df = torch.zeros(1000, dtype=torch.int16, device=dev)
        cb = pkg.CommandBuffer()
        for i in range(4):
            cb.dispatch("matmul_f16", consts(pkg, m, n, k),
                        [pkg.slot(i), pkg.slot(4), pkg.slot(5 + i)])
        cb.fill(pkg.slot(11, 6, 1990), b"\x34\x12")
        cb.barrier()
        cb.copy(pkg.slot(5), pkg.slot(9), m * n * 2)
        cb.dispatch("matmul_f16", consts(pkg, m, n, k, pkg.ACCUMULATE),
                    [pkg.slot(1), pkg.slot(4), pkg.slot(6)])
        cb.barrier()
        cb.copy(pkg.slot(6), pkg.slot(10), m * n * 2)
        self.cb = cb.end()

    def table(self):
        return self.da + [self.db] + self.dc + [self.dd, self.de, self.df]

    def reset_outputs(self):
        for t in self.dc + [self.dd, self.de]:
            t.fill_(9.0)
        self.df.zero_()

    def check(self, oracle):
        torch.cuda.synchronize()
        refs = [oracle.matmul_f16(x.numpy(), self.b.numpy()) for x in self.a]
        for i in (0, 2, 3):
            assert oracle.fp16_parity(self.dc[i].cpu().numpy(), refs[i]) <= FP16_BOUND
        c1 = oracle.matmul_f16(self.a[1].numpy(), self.b.numpy(), refs[1])
        assert oracle.fp16_parity(self.dc[1].cpu().numpy(), c1) <= FP16_BOUND
        assert torch.equal(self.dd.cpu(), self.dc[0].cpu())
        assert torch.equal(self.de.cpu(), self.dc[1].cpu())
        f = self.df.cpu().numpy()
        assert (f[:3] == 0).all() and (f[3:998] == 0x1234).all() and (f[998:] == 0).all()


@pytest.mark.parametrize("lanes", [1, 2, 4, 8])
def test_program_every_concurrency(pkg, oracle, dev, lanes):
    p = Program(pkg, dev, seed=lanes)
    p.cb.submit(p.table(), max_concurrent=lanes)
    p.check(oracle)
    # a second submission re-uses the lane workspaces (counters re-armed)
    p.reset_outputs()
    p.cb.submit(p.table(), max_concurrent=lanes)
    p.check(oracle)


def test_lane_slices_of_different_sizes_on_one_stream(pkg, oracle, dev):
    """Two command buffers whose lane slices differ, submitted at 2 lanes
    between flat split-K calls on one stream: lane l's counters sit at l
    slices, where a buffer used with another slice (or by flat calls) holds
    partials, so each slice size needs its own zeroed workspace.
    (Regression: sharing one buffer gave the second lane dirty counters.)"""
    g = torch.Generator().manual_seed(41)
    k = 4096
    x = (torch.randn(16, k, generator=g) * 0.5).half()
    xd = x.to(dev)
    progs = []
    for n in (4096, 11008):
        ws = [(torch.randn(k, n, generator=g) * 0.02).half() for _ in range(2)]
        ys = [torch.empty(16, n, dtype=torch.float16, device=dev)
              for _ in range(2)]
        cb = pkg.CommandBuffer()
        for i in range(2):
            cb.dispatch("matmul_f16", consts(pkg, 16, n, k),
                        [pkg.slot(0), pkg.slot(1 + i), pkg.slot(3 + i)])
        cb.end()
        table = [xd] + [w.to(dev) for w in ws] + ys
        refs = [oracle.matmul_f16(x.numpy(), w.numpy()) for w in ws]
        progs.append((cb, table, ys, refs))
    slices = {p[0].workspace_bytes(p[1], 1) for p in progs}
    assert len(slices) == 2, slices
    wf = (torch.randn(k, 11008, generator=g) * 0.02).half()
    ref_f = oracle.matmul_f16(x.numpy(), wf.numpy())
    wfd = wf.to(dev)
    for order in (0, 1, 0, 1):
        cb, table, ys, refs = progs[order]
        for y in ys:
            y.fill_(7.0)
        cb.submit(table, max_concurrent=2)
        yf = pkg.matmul(xd, wfd)  # flat split-K on the stream's own buffer
        torch.cuda.synchronize()
        for y, ref in zip(ys, refs):
            assert oracle.fp16_parity(y.cpu().numpy(), ref) <= FP16_BOUND
        assert oracle.fp16_parity(yf.cpu().numpy(), ref_f) <= FP16_BOUND


def test_program_caller_workspace(pkg, oracle, dev):
    p = Program(pkg, dev, seed=11)
    need = p.cb.workspace_bytes(p.table(), 4)
    assert need > 0
    ws = torch.zeros(need, dtype=torch.uint8, device=dev)
    p.cb.submit(p.table(), max_concurrent=4, workspace=ws)
    p.check(oracle)
    assert int(ws[:64 * 1024].count_nonzero()) == 0   # lane 0's counters re-armed


def test_failed_validation_enqueues_nothing(pkg, dev):
    m, n, k = 128, 512, 256
    a = torch.randn(m, k, device=dev).half()
    b = torch.randn(k, n, device=dev).half()
    c = torch.full((m, n), 5.0, dtype=torch.float16, device=dev)
    cb = pkg.CommandBuffer()
    cb.dispatch("matmul_f16", consts(pkg, m, n, k), [pkg.slot(0), pkg.slot(1), pkg.slot(2)])
    cb.dispatch("matmul_f16", consts(pkg, m, n, k), [pkg.slot(0), pkg.slot(1), pkg.slot(3)])
    cb.end()
    short = torch.empty(16, dtype=torch.float16, device=dev)
    with pytest.raises(pkg.MI355XError) as e:
        cb.submit([a, b, c, short], max_concurrent=2)
    assert "command 1" in str(e.value)
    torch.cuda.synchronize()
    assert bool((c == 5.0).all()), "a command before the failing one ran"


def test_direct_references_and_attention(pkg, oracle, dev):
    """Direct buffer references, and an attention dispatch next to a
    matmul in one segment."""
    g = torch.Generator().manual_seed(5)
    q, k_, v = (torch.randn(1, 2, 256, 64, generator=g).half() for _ in range(3))
    o = torch.empty(1, 2, 256, 64, dtype=torch.float16, device=dev)
    a = torch.randn(256, 128, generator=g).half()
    b = torch.randn(128, 256, generator=g).half()
    c = torch.empty(256, 256, dtype=torch.float16, device=dev)
    dq, dk, dv, da, db = (t.to(dev) for t in (q, k_, v, a, b))
    scale = 64 ** -0.5
    import struct
    sbits = struct.unpack("<I", struct.pack("<f", scale))[0]
    cb = pkg.CommandBuffer()
    cb.dispatch("attention_f16", [1, 2, 256, 256, 64, sbits, pkg.CAUSAL],
                [pkg.direct(dq), pkg.direct(dk), pkg.direct(dv), pkg.direct(o)])
    cb.dispatch("matmul_f16", consts(pkg, 256, 256, 128),
                [pkg.direct(da), pkg.direct(db), pkg.direct(c)])
    cb.end()
    cb.submit([], max_concurrent=2)
    torch.cuda.synchronize()
    ref_o = oracle.attention_f16(q.numpy(), k_.numpy(), v.numpy(), scale=scale,
                                 causal=True)
    assert oracle.fp16_parity(o.cpu().numpy(), ref_o) <= FP16_BOUND
    assert oracle.fp16_parity(c.cpu().numpy(),
                              oracle.matmul_f16(a.numpy(), b.numpy())) <= FP16_BOUND


def test_general_attention_in_a_command_buffer(pkg, oracle, dev):
    """The 41-word attention_f16 form through a command buffer: a mask in
    binding 4 taken from the binding table, head dims 96 / 96 with an f32
    result (the MFMA kernel's f32 mask instance) and 24 / 40 (the general
    kernel), in one segment on two lanes."""
    g = torch.Generator().manual_seed(9)
    b, h, s = 1, 2, 192
    cases = []
    for d, dv in ((96, 96), (24, 40)):
        q, k_ = (torch.randn(b, h, s, d, generator=g).half() for _ in range(2))
        v = torch.randn(b, h, s, dv, generator=g).half()
        o = torch.full((b, h, s, dv), float("nan"), device=dev)
        cases.append((d, dv, q, k_, v, o))
    mask = (2 * torch.randn(s, s, generator=g)).half()
    mask[torch.rand(s, s, generator=g) < 0.1] = float("-inf")
    dm = mask.to(dev)
    flags = pkg.ATTENTION_MASK | pkg.ATTENTION_OUT_F32 | pkg.CAUSAL
    cb = pkg.CommandBuffer()
    table = [dm]
    held = []  # the device copies must outlive the submission
    for d, dv, q, k_, v, o in cases:
        consts = pkg.attention_constants(b, h, s, s, d, 0.25, flags,
                                         head_dim_v=dv,
                                         mask_strides=[0, 0, s, 1])
        dq, dk, dvv = q.to(dev), k_.to(dev), v.to(dev)
        held += [dq, dk, dvv]
        cb.dispatch("attention_f16", consts,
                    [pkg.direct(dq), pkg.direct(dk), pkg.direct(dvv),
                     pkg.direct(o), pkg.slot(0)])
    cb.end()
    cb.submit(table, max_concurrent=2)
    torch.cuda.synchronize()
    for d, dv, q, k_, v, o in cases:
        ref = oracle.attention(q.numpy(), k_.numpy(), v.numpy(), scale=0.25,
                               causal=True, mask=mask.numpy(), out_f32=True)
        # both attention kernels round the probabilities to f16: 4e-4
        bound = 4e-4
        assert oracle.fp16_parity(o.cpu().numpy(), ref) <= bound, (d, dv)


@pytest.mark.skip(reason="a 4-lane submission captured into a HIP graph ended "
                  "in a host segmentation fault in hipStreamEndCapture; the "
                  "cause is not established, so the runtime refuses "
                  "concurrent lanes under capture")
def test_captured_submission_replays(pkg, oracle, dev):
    """A 4-lane submission captured into a HIP graph from the caller's
    stream (fork/join through events): every replay, with eager work that
    changes the inputs and clobbers the outputs in between, matches."""
    p = Program(pkg, dev, seed=21)
    need = p.cb.workspace_bytes(p.table(), 4)
    ws = torch.zeros(need, dtype=torch.uint8, device=dev)
    p.cb.submit(p.table(), max_concurrent=4, workspace=ws)   # lanes created
    p.check(oracle)
    s = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        p.cb.submit(p.table(), max_concurrent=4, workspace=ws, stream=s)
    for rep in range(3):
        p.reset_outputs()
        for i in range(4):
            p.a[i] = (-p.a[i]) if rep % 2 == 0 else (p.a[i] * 0.5).half()
            p.da[i].copy_(p.a[i].to(dev))
        torch.cuda.synchronize()
        graph.replay()
        p.check(oracle)


def test_captured_in_order_submission_replays(pkg, oracle, dev):
    """A submission with max_concurrent = 1 (in order on the capturing
    stream: dispatches, a fill kernel and copies) captured into a HIP graph:
    every replay, with eager work that changes the inputs and clobbers the
    outputs in between, matches."""
    p = Program(pkg, dev, seed=31)
    need = p.cb.workspace_bytes(p.table(), 1)
    ws = torch.zeros(need, dtype=torch.uint8, device=dev)
    p.cb.submit(p.table(), max_concurrent=1, workspace=ws)
    p.check(oracle)
    s = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        p.cb.submit(p.table(), max_concurrent=1, workspace=ws, stream=s)
    for rep in range(3):
        p.reset_outputs()
        for i in range(4):
            p.a[i] = (-p.a[i]) if rep % 2 == 0 else (p.a[i] * 0.5).half()
            p.da[i].copy_(p.a[i].to(dev))
        torch.cuda.synchronize()
        graph.replay()
        p.check(oracle)


def test_loaded_executable_dispatches(pkg, oracle, dev):
    """A serialized executable loaded into a private copy of the library:
    its exports run a macro-tile and a split-K matmul through a command
    buffer, matching the oracle."""
    exe = pkg.LoadedExecutable(pkg.serialize_executable())
    try:
        g = torch.Generator().manual_seed(41)
        cases = [(256, 512, 128), (16, 4096, 2048)]
        ts, refs = [], []
        cb = pkg.CommandBuffer(executable=exe)
        for i, (m, n, k) in enumerate(cases):
            a = (torch.randn(m, k, generator=g) * 0.5).half()
            b = torch.randn(k, n, generator=g).half()
            refs.append(oracle.matmul_f16(a.numpy(), b.numpy()))
            c = torch.full((m, n), 3.0, dtype=torch.float16, device=dev)
            ts += [a.to(dev), b.to(dev), c]
            cb.dispatch("matmul_f16", consts(pkg, m, n, k),
                        [pkg.slot(3 * i), pkg.slot(3 * i + 1), pkg.slot(3 * i + 2)])
        cb.end()
        cb.submit(ts, max_concurrent=1)
        torch.cuda.synchronize()
        for i, ref in enumerate(refs):
            assert oracle.fp16_parity(ts[3 * i + 2].cpu().numpy(), ref) <= FP16_BOUND
        del cb
    finally:
        torch.cuda.synchronize()
        exe.release()
