"""The ScaledMMLinear drop-in on the GPU: `nn.Linear` relabelled by `to_scaled_mm_linear` runs the fp8 scaled
matmul. Its output equals `scaled_mm_hip` on the module's own buffers bit for bit, meets the oracle's bar
on those buffers, and stays close to the unquantized fp32 Linear (the quantization error of an fp8 weight,
checked loosely)."""

import pytest
import torch
from torch import nn

from gpu_helpers import check_against_oracle, sample_rows

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def fo():
    import feather_ops

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return feather_ops


def _linear(k, n, bias=True, seed=0):
    torch.manual_seed(seed)
    return nn.Linear(k, n, bias=bias).cuda()


@pytest.mark.parametrize("fp8,per_channel,dtype,bias", [
    (torch.float8_e5m2, False, torch.float16, True),
    (torch.float8_e5m2, True, torch.bfloat16, False),
    (torch.float8_e4m3fn, True, torch.bfloat16, True),
    (torch.float8_e4m3fn, False, torch.float16, False),
])
def test_forward_matches_the_kernel_and_the_oracle(fo, fp8, per_channel, dtype, bias):
    lin = _linear(640, 264, bias)
    ref_fp32 = nn.Linear(640, 264, bias=bias).cuda()
    ref_fp32.load_state_dict(lin.state_dict())
    assert fo.to_scaled_mm_linear(lin, fp8, per_channel) == 1
    x = torch.randn(3, 37, 640, device="cuda").to(dtype)
    y = lin(x)
    assert y.shape == (3, 37, 264) and y.dtype == dtype
    x2 = x.reshape(-1, 640)
    b = None if lin.bias is None else lin.bias.to(dtype)
    direct = fo.scaled_mm_hip(x2, lin.weight_fp8, lin.weight_scale, b, dtype)
    assert torch.equal(y.reshape(-1, 264).view(torch.int16), direct.view(torch.int16))
    check_against_oracle(direct, x2, lin.weight_fp8, lin.weight_scale, b)
    want = ref_fp32(x.float())
    rel = ((y.float() - want).norm() / want.norm()).item()
    assert rel < (0.08 if fp8 == torch.float8_e5m2 else 0.04), rel


def test_inference_path_matches_the_op(fo):
    """Under no_grad the layer skips the custom op's dispatch; the output is the op's bit for bit."""
    lin = _linear(512, 320)
    fo.to_scaled_mm_linear(lin, torch.float8_e4m3fn, per_channel=True)
    x = torch.randn(5, 7, 512, device="cuda").to(torch.bfloat16)
    with torch.no_grad():
        fast = lin(x)
    via_op = torch.ops.feather_ops.scaled_mm_linear(x, lin.weight_fp8, lin.weight_scale, lin.bias.to(x.dtype))
    assert torch.equal(fast.view(torch.int16), via_op.view(torch.int16))
    with torch.inference_mode():
        assert torch.equal(lin(x).view(torch.int16), via_op.view(torch.int16))


def test_misaligned_input_view(fo):
    """An input view that starts 2 bytes into its buffer is copied once, not refused."""
    lin = _linear(256, 128)
    fo.to_scaled_mm_linear(lin)
    buf = torch.randn(1 + 50 * 256, device="cuda").to(torch.float16)
    x = buf[1:].view(50, 256)
    assert x.data_ptr() % 16 != 0
    assert torch.equal(lin(x).view(torch.int16), lin(x.clone()).view(torch.int16))


def test_split_k_sized_layer(fo):
    """A 5120 -> 5376 layer on 512 tokens: the heuristic splits K; checked on a row sample."""
    lin = _linear(5120, 5376)
    fo.to_scaled_mm_linear(lin)
    x = torch.randn(512, 5120, device="cuda").to(torch.float16)
    y = lin(x)
    check_against_oracle(y, x, lin.weight_fp8, lin.weight_scale, lin.bias.to(torch.float16), rows=sample_rows(512))


def test_compiled_model_matches_eager(fo):
    """A model of ScaledMMLinear layers under torch.compile: the kernel stays one opaque node per layer."""
    torch.manual_seed(3)
    model = nn.Sequential(nn.Linear(512, 1024), nn.GELU(), nn.Linear(1024, 256)).cuda()
    assert fo.to_scaled_mm_linear(model) == 2
    x = torch.randn(4, 50, 512, device="cuda").to(torch.bfloat16)
    eager = model(x)
    compiled = torch.compile(model, fullgraph=True)(x)
    assert torch.equal(compiled.view(torch.int16), eager.view(torch.int16))


def test_backward_gives_input_and_bias_gradients(fo):
    """dX = dY @ (Wq * scale)^T and dbias = sum(dY) on the dequantized weight; the fp8 weight is frozen."""
    lin = _linear(256, 192)
    fo.to_scaled_mm_linear(lin, torch.float8_e5m2, per_channel=True)
    x = torch.randn(2, 30, 256, device="cuda").to(torch.bfloat16).requires_grad_()
    y = lin(x)
    g = torch.randn_like(y)
    y.backward(g)
    w = lin.weight_fp8.permute(0, 2, 1).reshape(-1, 192)[:256].float() * lin.weight_scale[None, :]
    want_x = (g.reshape(-1, 192).float() @ w.t()).reshape(2, 30, 256)
    assert x.grad.dtype == torch.bfloat16
    assert torch.allclose(x.grad.float(), want_x.to(torch.bfloat16).float(), rtol=0, atol=0)
    # the bias enters the op cast to the input dtype, so its gradient arrives through that cast (bf16)
    want_bias = g.float().sum((0, 1))
    assert torch.allclose(lin.bias.grad, want_bias, rtol=2**-7, atol=1e-3)
    assert lin.weight.grad is None
