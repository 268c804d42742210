"""Operand checks of the Python operator mirror, on host tensors.

The C-ABI sees only pointers and the extents it is given, so a wrapper that
passed an output or secondary operand of the wrong extent would make the
kernel read or write past a buffer. Every shape and dtype error must be
raised before the device check (host tensors with consistent shapes reach
the device check and stop there: nothing is launched)."""
import pytest
import torch

H, I8 = torch.float16, torch.int8


def z(*shape, dtype=H):
    return torch.zeros(*shape, dtype=dtype)


def test_matmul_output_shape_and_dtype(pkg):
    a, b = z(8, 16), z(16, 4)
    with pytest.raises(ValueError, match="c must be"):
        pkg.matmul(a, b, z(8, 5))
    with pytest.raises(ValueError, match="c must be"):
        pkg.matmul(a, b, z(4, 8))
    with pytest.raises(TypeError):
        pkg.matmul(a, b, z(8, 4, dtype=torch.float32))
    with pytest.raises(TypeError):
        pkg.matmul(a, b, out_dtype=torch.int32)
    with pytest.raises(ValueError, match="contraction"):
        pkg.matmul(a, z(15, 4))
    with pytest.raises(ValueError, match="contraction"):
        pkg.matmul(a, z(4, 15), b_transposed=True)
    with pytest.raises(ValueError, match="accumulate"):
        pkg.matmul(a, b, accumulate=True)
    # consistent shapes on the host stop at the device check
    with pytest.raises(TypeError, match="device"):
        pkg.matmul(a, b, z(8, 4))
    with pytest.raises(TypeError, match="device"):
        pkg.matmul(z(16, 8), b, z(8, 4), a_transposed=True)


def test_matmul_i8_output(pkg):
    a, bt = z(8, 32, dtype=I8), z(4, 32, dtype=I8)
    with pytest.raises(TypeError):
        pkg.matmul(a, bt, z(8, 4, dtype=torch.float32), b_transposed=True)
    with pytest.raises(ValueError, match="c must be"):
        pkg.matmul(a, bt, z(8, 3, dtype=torch.int32), b_transposed=True)
    with pytest.raises(ValueError, match="f16 layout"):
        pkg.matmul(a, bt, a_transposed=True, b_transposed=True)
    with pytest.raises(TypeError):
        pkg.matmul(a, z(32, 4), b_transposed=False)  # f16 B with int8 A


def test_batch_matmul_output_rank_and_batch(pkg):
    a, b = z(3, 8, 16), z(16, 4)
    # batch 3: a 2-D c would take 3 * 8 * 4 elements
    with pytest.raises(ValueError):
        pkg.batch_matmul(a, b, z(8, 4))
    with pytest.raises(ValueError, match="c must be"):
        pkg.batch_matmul(a, b, z(2, 8, 4))
    with pytest.raises(ValueError, match="c must be"):
        pkg.batch_matmul(a, b, z(3, 8, 5))
    with pytest.raises(ValueError, match="batch extent"):
        pkg.batch_matmul(a, z(2, 16, 4))
    with pytest.raises(ValueError, match="contraction"):
        pkg.batch_matmul(a, z(3, 15, 4))
    with pytest.raises(ValueError, match="bias"):
        pkg.batch_matmul(a, b, bias=z(5))
    with pytest.raises(ValueError, match="multiplier"):
        pkg.batch_matmul(a, b, multiplier=z(3, 8, 5))
    with pytest.raises(ValueError, match="multiplier batch"):
        pkg.batch_matmul(a, b, multiplier=z(2, 8, 4))
    with pytest.raises(ValueError, match="activation"):
        pkg.batch_matmul(a, b, activation="tanh")
    with pytest.raises(TypeError, match="device"):
        pkg.batch_matmul(a, b, z(3, 8, 4), bias=z(4), activation="silu")
    # unbatched operands take a 2-D c
    with pytest.raises(ValueError):
        pkg.batch_matmul(z(8, 16), b, z(1, 8, 4))
    with pytest.raises(TypeError, match="device"):
        pkg.linear(z(8, 16), b, z(4))


def test_quantized_matmul_operands(pkg):
    x, w, s = z(2, 64), z(64, 32, dtype=I8), z(32)
    with pytest.raises(ValueError, match="contract"):
        pkg.quantized_matmul(x, z(63, 32, dtype=I8), s)
    with pytest.raises(ValueError, match="contract"):
        pkg.quantized_matmul(x, z(32, 63, dtype=I8), s, w_transposed=True)
    with pytest.raises(ValueError, match="scale"):
        pkg.quantized_matmul(x, w, z(31))
    with pytest.raises(TypeError):
        pkg.quantized_matmul(x, w, z(32, dtype=torch.float32))
    with pytest.raises(ValueError, match="y must be"):
        pkg.quantized_matmul(x, w, s, z(2, 31))
    with pytest.raises(TypeError):
        pkg.quantized_matmul(x, w, s, z(2, 32, dtype=torch.float32))
    with pytest.raises(TypeError, match="device"):
        pkg.quantized_matmul(x, w, s, z(2, 32))


def test_attention_operands(pkg):
    q = z(1, 2, 16, 64)
    kv = z(1, 2, 24, 64)
    with pytest.raises(ValueError, match="k must be"):
        pkg.attention(q, z(1, 3, 24, 64), kv)
    with pytest.raises(ValueError, match="k must be"):
        pkg.attention(q, z(1, 2, 24, 128), kv)
    with pytest.raises(ValueError, match="v must be"):
        pkg.attention(q, kv, z(1, 2, 20, 64))
    with pytest.raises(ValueError, match="o must be"):
        pkg.attention(q, kv, kv, z(1, 2, 24, 64))
    with pytest.raises(TypeError):
        pkg.attention(q, kv, kv, z(1, 2, 16, 64, dtype=torch.float32))
    with pytest.raises(TypeError):
        pkg.attention(q, kv, kv, z(1, 2, 64, 16).transpose(2, 3))
    with pytest.raises(TypeError, match="device"):
        pkg.attention(q, kv, kv, z(1, 2, 16, 64))


def test_mfma_config_operands(pkg):
    cfgs = pkg.mfma_configs()
    tn = next(c for c in cfgs if c.name == "f16_tn_128x128x64_w2x2_s4")
    w8 = next(c for c in cfgs if c.b_form == pkg.B_FORM_W8A16)
    a, bt = z(128, 64), z(128, 64)
    with pytest.raises(ValueError, match="c must be"):
        pkg.matmul_mfma_config(tn.index, a, bt, z(128, 64))
    with pytest.raises(TypeError):
        pkg.matmul_mfma_config(tn.index, a, bt, z(128, 128, dtype=torch.float32))
    with pytest.raises(TypeError):
        pkg.matmul_mfma_config(tn.index, a.to(I8), bt, z(128, 128))
    with pytest.raises(ValueError, match="scale"):
        pkg.matmul_mfma_config(w8.index, z(128, 128), z(128, 256, dtype=I8),
                               z(128, 256))
    with pytest.raises(TypeError, match="device"):
        pkg.matmul_mfma_config(tn.index, a, bt, z(128, 128))
