"""Size-independent properties at the BASELINE configs' full sizes, where
the CPU oracle would take too long to compare element by element.

  * C2 int8 4096^3: negating A (clamped to -127 .. 127) negates C, bit for
    bit (i32, no overflow at |a|, |b| <= 128 and K = 4096); B with its
    columns permuted gives C with the same columns permuted.
  * fp16 4096^3: A (its subnormals set to 0) doubled gives C doubled bit
    for bit wherever C is safely normal (scaling by 2 is exact in f16 and
    f32 and commutes with the one rounding there; near and below the
    subnormal range the rounding of 2c may pick the neighbour of
    2 round(c), 2^-24 away). The f32 result doubles exactly everywhere.
  * C4 attention (B1 H32 S2048 D128, causal): V doubled gives O doubled bit
    for bit where O is a normal f16 (O is P V / l with P independent of
    V); queries are independent rows, so O of a row subset equals the same
    rows of O.
  * C5 W8A16 M=1: the per-column scale is applied after the sum: scale
    doubled gives y doubled bit for bit.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu

F16_MIN_NORMAL = 2.0 ** -14


def doubled(got2, got):
    """got2 == 2 got bit for bit where got is at least twice the smallest
    normal f16 (the value it rounds is then normal, and so is twice it);
    below that, where got is or came from a subnormal (rounded on the 2^-24
    grid), 2 got may have been rounded on the same grid: they may differ by
    2^-24."""
    want = got * 2
    normal = got.abs() >= 2 * F16_MIN_NORMAL
    assert torch.equal(got2[normal], want[normal])
    if (~normal).any():
        assert (got2[~normal].float() - want[~normal].float()).abs().max() \
            .item() <= 2.0 ** -24


def test_c2_int8_negation_and_column_permutation(pkg, inputs, dev):
    print("C2 properties", flush=True)
    a, bt = (t.to(dev) for t in inputs.c2_matmul_i8())
    a = a.clamp(min=-127)  # -(-128) does not exist in int8
    c = pkg.matmul(a, bt, b_transposed=True)
    c_neg = pkg.matmul(-a, bt, b_transposed=True)
    torch.cuda.synchronize()
    assert torch.equal(c_neg, -c)
    perm = torch.randperm(4096, generator=torch.Generator().manual_seed(1))
    perm = perm.to(dev)
    c_perm = pkg.matmul(a, bt[perm].contiguous(), b_transposed=True)
    torch.cuda.synchronize()
    assert torch.equal(c_perm, c[:, perm])


def test_fp16_4096_scaling_is_exact(pkg, inputs, dev):
    print("fp16 4096^3 scaling", flush=True)
    x, w = inputs.c3_linear_f16(4096, 4096, 4096)
    # subnormal inputs (|x| < 2^-14) set to 0: whether the matrix core
    # flushes them or not, x and 2 x then multiply alike
    x = torch.where(x.abs() < 2.0 ** -13, torch.zeros_like(x), x)
    x, bt = x.to(dev), w.t().contiguous().to(dev)
    c = pkg.matmul(x, bt, b_transposed=True)
    c2 = pkg.matmul(x * 2, bt, b_transposed=True)
    torch.cuda.synchronize()
    doubled(c2, c)
    c32 = pkg.matmul(x, bt, b_transposed=True, out_dtype=torch.float32)
    c32_2 = pkg.matmul(x * 2, bt, b_transposed=True, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(c32_2, c32 * 2)
    assert torch.equal(c32.half(), c)  # one rounding, the same one


def test_c4_attention_linearity_in_v_and_row_independence(pkg, inputs, dev):
    print("C4 properties", flush=True)
    q, k, v = (t.to(dev) for t in inputs.c4_attention_f16())
    v = torch.where(v.abs() < 2.0 ** -13, torch.zeros_like(v), v)
    o = pkg.attention(q, k, v, causal=True)
    o2 = pkg.attention(q, k, v * 2, causal=True)
    torch.cuda.synchronize()
    doubled(o2, o)
    # a head's first 640 query rows attend to the same (causal) keys
    o_part = pkg.attention(q[:, :, :640].contiguous(), k, v, causal=True)
    torch.cuda.synchronize()
    assert (o_part - o[:, :, :640]).abs().max().item() <= \
        2e-3 * o.abs().max().item()


def test_c5_w8a16_scale_is_applied_after_the_sum(pkg, inputs, dev):
    print("C5 M=1 scale", flush=True)
    x, w, s = (t.to(dev) for t in inputs.c5_w8a16(1))
    y = pkg.quantized_matmul(x, w, s)
    y2 = pkg.quantized_matmul(x, w, s * 2)
    torch.cuda.synchronize()
    doubled(y2, y)
