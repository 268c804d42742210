"""The general attention path on the GPU against the oracle: head dims
other than 64 / 128 (Q/K and V may differ), an additive f16 mask with
broadcast strides, f32 output, grouped KV heads and strided views, through
the Python wrapper, the C-ABI descriptor and the executable library's
41-word attention_f16 dispatch.

The reference lowers iree_linalg_ext.attention whatever its head dims, mask
and output type (CG/Pipelines/LoweringPipelines.cpp:561-595); its pipeline
test test/codegen/pipelines/hexagon_lower_executable_target.mlir:195-233
runs Q/K head dim 4, V head dim 5, scale 0.5 and an f32 accumulator, the
first case here. Tolerances: f16 output within the 2e-3 fp16 parity bound
(max |got - ref| / max |ref|); f32 output within 4e-4 of the f32 oracle:
both attention kernels round the probabilities to f16 before PV, as their
f16 output does (measured about 1e-4).
"""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

F16_BOUND = 2e-3
F32_BOUND = 4e-4


def rand(g, *shape):
    return torch.randn(*shape, generator=g).half()


def random_mask(g, shape, dead=0.2):
    m = 2 * torch.randn(*shape, generator=g)
    m[torch.rand(*shape, generator=g) < dead] = float("-inf")
    return m.half()


CASES = [
    # b, hq, hkv, sq, skv, dqk, dv, mask shape (None: none), causal, out
    (1, 1, 1, 2, 3, 4, 5, None, False, "f32"),
    (2, 3, 3, 37, 53, 24, 40, (2, 1, 37, 53), False, "f32"),
    (2, 4, 2, 100, 130, 96, 96, (1, 130), True, "f16"),
    (1, 8, 8, 129, 257, 80, 80, None, True, "f16"),
    (2, 2, 1, 64, 64, 128, 64, (2, 2, 64, 64), False, "f16"),
    (1, 2, 2, 70, 90, 256, 256, None, False, "f32"),
    (1, 3, 1, 1, 500, 160, 200, (1, 1, 1, 500), False, "f16"),
    (1, 2, 2, 300, 40, 8, 16, (300, 40), True, "f32"),
    (1, 2, 2, 128, 128, 64, 64, (128, 128), True, "f16"),
    (1, 2, 2, 128, 128, 128, 128, None, False, "f32"),
]


@pytest.mark.parametrize("case", CASES, ids=[
    "b{}h{}/{}q{}k{}d{}x{}_m{}_c{}_{}".format(
        *c[:7], "x".join(map(str, c[7])) if c[7] else "none", int(c[8]), c[9])
    for c in CASES])
def test_attention_general_vs_oracle(pkg, oracle, dev, case):
    b, hq, hkv, sq, skv, dqk, dv, mshape, causal, out = case
    print(f"attention general {case}", flush=True)
    g = torch.Generator().manual_seed(sq * 31 + skv * 7 + dqk + dv)
    q, k = rand(g, b, hq, sq, dqk), rand(g, b, hkv, skv, dqk)
    v = rand(g, b, hkv, skv, dv)
    mask = random_mask(g, mshape) if mshape else None
    scale = 0.5 if dqk == 4 else dqk ** -0.5
    out_dtype = torch.float32 if out == "f32" else torch.float16
    o = pkg.attention(q.to(dev), k.to(dev), v.to(dev), causal=causal,
                      scale=scale, out_dtype=out_dtype,
                      mask=None if mask is None else mask.to(dev))
    torch.cuda.synchronize()
    assert o.dtype == out_dtype and tuple(o.shape) == (b, hq, sq, dv)
    ref = oracle.attention(q.numpy(), k.numpy(), v.numpy(), scale=scale,
                           causal=causal, out_f32=out == "f32",
                           mask=None if mask is None else mask.numpy())
    got = o.cpu().numpy()
    assert np.isfinite(got).all()
    err = oracle.fp16_parity(got, ref)
    assert err <= (F32_BOUND if out == "f32" else F16_BOUND), err


def test_attention_general_fully_masked_rows(pkg, oracle, dev):
    # rows whose keys are all -inf write exactly 0 (the all-masked guard)
    g = torch.Generator().manual_seed(4)
    q, k, v = rand(g, 1, 2, 70, 32), rand(g, 1, 2, 45, 32), rand(g, 1, 2, 45, 32)
    mask = torch.zeros(70, 45, dtype=torch.float16)
    mask[[0, 13, 69]] = float("-inf")
    o = pkg.attention(q.to(dev), k.to(dev), v.to(dev), causal=False,
                      mask=mask.to(dev), out_dtype=torch.float32)
    got = o.cpu().numpy()
    assert (got[:, :, [0, 13, 69]] == 0).all()
    ref = oracle.attention(q.numpy(), k.numpy(), v.numpy(), scale=32 ** -0.5,
                           mask=mask.numpy(), out_f32=True)
    assert oracle.fp16_parity(got, ref) <= F32_BOUND
    # causal with more queries than keys: every row sees key 0 at least
    o2 = pkg.attention(q.to(dev), k[:, :, :1].to(dev), v[:, :, :1].to(dev),
                       causal=True, scale=0.3)
    assert np.array_equal(o2.cpu().numpy(),
                          np.broadcast_to(v[:, :, :1].numpy(), (1, 2, 70, 32)))
    # no keys at all: every row sees none and writes 0, over a NaN-filled
    # output (head dims 24 / 40 take the general kernel)
    for out_dtype in (torch.float16, torch.float32):
        o3 = torch.full((1, 2, 70, 40), float("nan"), dtype=out_dtype,
                        device=dev)
        pkg.attention(q[..., :24].contiguous().to(dev),
                      torch.empty(1, 2, 0, 24, dtype=torch.float16, device=dev),
                      torch.empty(1, 2, 0, 40, dtype=torch.float16, device=dev),
                      o3)
        assert (o3.cpu() == 0).all()


def test_attention_general_strided_views(pkg, oracle, dev):
    # K / V the first rows of a longer cache, o a permuted view of a
    # [B, S, H, Dv] buffer, q a head-major view of [B, S, H, D], a mask
    # broadcast over heads: the same values as contiguous copies
    g = torch.Generator().manual_seed(8)
    b, h, hkv, sq, ctx, cache, d, dv = 2, 6, 2, 90, 70, 128, 48, 80
    q_bshd = rand(g, b, sq, h, d).to(dev)
    kc, vc = rand(g, b, hkv, cache, d).to(dev), rand(g, b, hkv, cache, dv).to(dev)
    mask = random_mask(g, (b, 1, sq, ctx), 0.1).to(dev)
    out = torch.full((b, sq, h, dv), float("nan"), dtype=torch.float16,
                     device=dev)
    q = q_bshd.permute(0, 2, 1, 3)
    pkg.attention(q, kc[:, :, :ctx], vc[:, :, :ctx], out.permute(0, 2, 1, 3),
                  causal=True, mask=mask)
    want = pkg.attention(q.contiguous(), kc[:, :, :ctx].contiguous(),
                         vc[:, :, :ctx].contiguous(), causal=True,
                         mask=mask.expand(b, h, sq, ctx).contiguous())
    got = out.permute(0, 2, 1, 3)
    assert torch.equal(got, want)
    ref = oracle.attention(q.cpu().numpy(), kc[:, :, :ctx].cpu().numpy(),
                           vc[:, :, :ctx].cpu().numpy(), scale=d ** -0.5,
                           causal=True, mask=mask.cpu().numpy())
    assert oracle.fp16_parity(got.cpu().numpy(), ref) <= F16_BOUND


def test_attention_general_routing(pkg, oracle, dev):
    # equal head dims of 64 / 128, no mask, f16 out: the MFMA kernel, the
    # same bits through the descriptor as through attention_f16. A zero mask
    # with contiguous keys takes the MFMA kernel's mask instance; the same
    # zeros read with a key stride of 2 take the general kernel: both within
    # the fp16 bound of the unmasked result, and not the same bits (two
    # kernels ran)
    g = torch.Generator().manual_seed(12)
    q, k, v = (rand(g, 2, 4, 256, 128).to(dev) for _ in range(3))
    fast = pkg.attention(q, k, v, causal=True)
    lib = pkg.library()
    o = torch.empty_like(q)
    a = pkg.AttentionArgs(q=q.data_ptr(), k=k.data_ptr(), v=v.data_ptr(),
                          o=o.data_ptr(), batch=2, heads=4, kv_heads=4,
                          seq_q=256, seq_kv=256, head_dim=128,
                          head_dim_v=128, scale=128 ** -0.5,
                          flags=pkg.CAUSAL)
    for f, t in (("q", q), ("k", k), ("v", v), ("o", o)):
        getattr(a.strides, f)[:] = list(t.stride()[:3])
    assert lib.iree_mi355x_attention(
        ctypes.byref(a), torch.cuda.current_stream().cuda_stream) == pkg.OK
    torch.cuda.synchronize()
    assert torch.equal(o, fast)
    zero = torch.zeros(1, 256, dtype=torch.float16, device=dev)
    masked = pkg.attention(q, k, v, causal=True, mask=zero)
    zero2 = torch.zeros(1, 512, dtype=torch.float16, device=dev)[:, ::2]
    general = pkg.attention(q, k, v, causal=True, mask=zero2)
    for got in (masked, general):
        assert oracle.fp16_parity(got.cpu().numpy(),
                                  fast.cpu().numpy()) <= F16_BOUND
    assert not torch.equal(general, masked)


def test_attention_general_through_export_table(pkg, oracle, dev):
    # the 41-word attention_f16 constants: unequal head dims, a row mask
    # shared by every (batch, head) in binding 4, f32 o
    g = torch.Generator().manual_seed(15)
    b, h, sq, skv, d, dv = 2, 3, 40, 50, 24, 40
    q, k = rand(g, b, h, sq, d).to(dev), rand(g, b, h, skv, d).to(dev)
    v = rand(g, b, h, skv, dv).to(dev)
    mask = random_mask(g, (sq, skv), 0.1).to(dev)
    o = torch.full((b, h, sq, dv), float("nan"), device=dev)
    flags = pkg.ATTENTION_MASK | pkg.ATTENTION_OUT_F32 | pkg.CAUSAL
    consts = pkg.attention_constants(b, h, sq, skv, d, 0.5, flags,
                                     head_dim_v=dv, mask_strides=[0, 0, skv, 1])
    ts = [q, k, v, o, mask]
    s = torch.cuda.current_stream().cuda_stream
    st = pkg.call_export("attention_f16", consts, [t.data_ptr() for t in ts],
                         [t.numel() * t.element_size() for t in ts], s)
    assert st == pkg.OK, pkg.last_error()
    torch.cuda.synchronize()
    ref = oracle.attention(q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy(),
                           scale=0.5, causal=True, mask=mask.cpu().numpy(),
                           out_f32=True)
    assert oracle.fp16_parity(o.cpu().numpy(), ref) <= F32_BOUND


def test_attention_general_wrapper_checks(pkg, dev):
    q = torch.zeros(1, 2, 16, 32, dtype=torch.float16, device=dev)
    v = torch.zeros(1, 2, 16, 40, dtype=torch.float16, device=dev)
    with pytest.raises(ValueError, match="broadcast"):
        pkg.attention(q, q, v, mask=torch.zeros(3, 16, dtype=torch.float16,
                                                device=dev))
    with pytest.raises(TypeError, match="mask"):
        pkg.attention(q, q, v, mask=torch.zeros(16, 16, device=dev))
    with pytest.raises(ValueError, match="o must be"):
        pkg.attention(q, q, v, torch.empty_like(q))  # o needs Dv = 40
    with pytest.raises(pkg.MI355XError) as e:
        big = torch.zeros(1, 1, 4, 300, dtype=torch.float16, device=dev)
        pkg.attention(big, big, big)
    assert e.value.status == pkg.UNSUPPORTED


MFMA_MASK_CASES = [
    # b, hq, hkv, sq, skv, d, mask shape, causal
    (1, 4, 4, 256, 256, 128, (256, 256), True),
    (2, 4, 2, 200, 300, 128, (2, 1, 200, 300), False),
    (1, 2, 2, 130, 516, 64, (1, 2, 130, 516), True),
    (2, 3, 3, 64, 64, 64, (64,), False),
    (1, 8, 2, 1, 1024, 128, (1, 8, 1, 1024), False),
    (1, 2, 2, 333, 128, 128, (333, 128), True),
]


@pytest.mark.parametrize("case", MFMA_MASK_CASES, ids=[
    "b{}h{}/{}q{}k{}d{}_m{}_c{}".format(*c[:6], "x".join(map(str, c[6])),
                                        int(c[7])) for c in MFMA_MASK_CASES])
def test_attention_mask_mfma_path(pkg, oracle, dev, case):
    # head dims 64 / 128 with an additive mask whose keys are contiguous run
    # the MFMA kernel's mask instance: ragged lengths (tails of query rows and
    # key blocks), grouped heads, masks broadcast over batch, heads or rows,
    # -inf entries, with and without the causal mask
    b, hq, hkv, sq, skv, d, mshape, causal = case
    print(f"attention mask mfma {case}", flush=True)
    g = torch.Generator().manual_seed(sq + skv + d + hq)
    q, k, v = rand(g, b, hq, sq, d), rand(g, b, hkv, skv, d), rand(g, b, hkv, skv, d)
    mask = random_mask(g, mshape, 0.15)
    o = pkg.attention(q.to(dev), k.to(dev), v.to(dev), causal=causal,
                      mask=mask.to(dev), scale=0.11)
    torch.cuda.synchronize()
    ref = oracle.attention(q.numpy(), k.numpy(), v.numpy(), scale=0.11,
                           causal=causal, mask=mask.numpy())
    got = o.cpu().numpy()
    assert np.isfinite(got).all()
    err = oracle.fp16_parity(got, ref)
    assert err <= F16_BOUND, err


def test_attention_mask_mfma_rows_and_views(pkg, oracle, dev):
    # fully masked rows write 0; a mask that is a view of a wider buffer
    # (row stride past seq_kv) over a KV-cache slice, o in [B, S, H, D]
    g = torch.Generator().manual_seed(31)
    b, h, sq, ctx, cache, d = 2, 4, 160, 192, 256, 128
    q = rand(g, b, h, sq, d).to(dev)
    kc, vc = rand(g, b, h, cache, d).to(dev), rand(g, b, h, cache, d).to(dev)
    wide = random_mask(g, (b, 1, sq, cache), 0.1)
    wide[:, :, [0, 77, 159]] = float("-inf")
    wide = wide.to(dev)
    mask = wide[..., :ctx]
    out = torch.full((b, sq, h, d), float("nan"), dtype=torch.float16,
                     device=dev)
    pkg.attention(q, kc[:, :, :ctx], vc[:, :, :ctx], out.permute(0, 2, 1, 3),
                  causal=False, mask=mask)
    got = out.permute(0, 2, 1, 3).cpu().numpy()
    assert (got[:, :, [0, 77, 159]] == 0).all()
    ref = oracle.attention(q.cpu().numpy(), kc[:, :, :ctx].cpu().numpy(),
                           vc[:, :, :ctx].cpu().numpy(), scale=d ** -0.5,
                           mask=mask.cpu().numpy())
    assert oracle.fp16_parity(got, ref) <= F16_BOUND


HEAD_DIM_CASES = [
    # b, hq, hkv, sq, skv, d, mask shape (None: none), causal
    (1, 4, 4, 256, 256, 96, None, True),
    (2, 4, 2, 200, 300, 80, (300,), False),
    (1, 2, 2, 130, 516, 32, (1, 2, 130, 516), True),
    (2, 3, 3, 64, 64, 16, None, False),
    (1, 8, 2, 1, 1024, 112, None, False),
    (1, 2, 2, 333, 128, 48, (333, 128), True),
    (1, 6, 3, 512, 512, 96, (512, 512), True),
]


@pytest.mark.parametrize("case", HEAD_DIM_CASES, ids=[
    "b{}h{}/{}q{}k{}d{}_m{}_c{}".format(
        *c[:6], "x".join(map(str, c[6])) if c[6] else "none", int(c[7]))
    for c in HEAD_DIM_CASES])
def test_attention_head_dims_mfma_path(pkg, oracle, dev, case):
    # head dims that are multiples of 16 up to 128 run the MFMA kernel with
    # the 64- or 128-wide LDS layout, reading only their own chunks: with
    # and without masks, grouped heads, ragged lengths, causal or not; the
    # columns past the head dim of the output's buffer stay untouched
    b, hq, hkv, sq, skv, d, mshape, causal = case
    print(f"attention head dim {case}", flush=True)
    g = torch.Generator().manual_seed(sq * 3 + skv + d)
    q, k, v = rand(g, b, hq, sq, d), rand(g, b, hkv, skv, d), rand(g, b, hkv, skv, d)
    mask = random_mask(g, mshape, 0.1) if mshape else None
    # o inside a wider buffer: a canary past the head dim of every row
    wide = torch.full((b, hq, sq, d + 16), 7.0, dtype=torch.float16,
                      device=dev)
    o = wide[..., :d]
    pkg.attention(q.to(dev), k.to(dev), v.to(dev), o, causal=causal,
                  mask=None if mask is None else mask.to(dev))
    torch.cuda.synchronize()
    ref = oracle.attention(q.numpy(), k.numpy(), v.numpy(), scale=d ** -0.5,
                           causal=causal,
                           mask=None if mask is None else mask.numpy())
    got = o.cpu().numpy()
    assert np.isfinite(got).all()
    assert oracle.fp16_parity(got, ref) <= F16_BOUND
    assert (wide[..., d:].cpu() == 7.0).all()


F32_MFMA_CASES = [
    # b, hq, hkv, sq, skv, d, mask shape, causal
    (1, 2, 2, 300, 300, 96, None, True),
    (2, 4, 4, 256, 256, 128, (256,), False),
    (1, 6, 2, 520, 260, 64, (1, 6, 520, 260), True),
    (2, 2, 2, 129, 64, 32, None, False),
]


@pytest.mark.parametrize("case", F32_MFMA_CASES, ids=[
    "b{}h{}/{}q{}k{}d{}_m{}_c{}".format(
        *c[:6], "x".join(map(str, c[6])) if c[6] else "none", int(c[7]))
    for c in F32_MFMA_CASES])
def test_attention_f32_mfma_path(pkg, oracle, dev, case):
    # f32 outputs on the MFMA kernel, stored from registers: several query
    # blocks per workgroup (the second block's rows must not take the
    # first's values), ragged lengths, masks, grouped heads, and a canary
    # past the head dim
    b, hq, hkv, sq, skv, d, mshape, causal = case
    print(f"attention f32 mfma {case}", flush=True)
    g = torch.Generator().manual_seed(sq + 2 * skv + d)
    q, k, v = rand(g, b, hq, sq, d), rand(g, b, hkv, skv, d), rand(g, b, hkv, skv, d)
    mask = random_mask(g, mshape, 0.1) if mshape else None
    wide = torch.full((b, hq, sq, d + 16), 7.0, device=dev)
    o = wide[..., :d]
    pkg.attention(q.to(dev), k.to(dev), v.to(dev), o, causal=causal,
                  mask=None if mask is None else mask.to(dev))
    torch.cuda.synchronize()
    ref = oracle.attention(q.numpy(), k.numpy(), v.numpy(), scale=d ** -0.5,
                           causal=causal, out_f32=True,
                           mask=None if mask is None else mask.numpy())
    got = o.cpu().numpy()
    assert np.isfinite(got).all()
    assert oracle.fp16_parity(got, ref) <= F32_BOUND
    assert (wide[..., d:].cpu() == 7.0).all()
