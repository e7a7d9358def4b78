"""GPU parity of the W8A8 gate_up GEMM with the SiLU-and-mul epilogue
(tvq_w8a8_gemm_glu): bit-identical to tvq_w8a8_gemm of the same gate_up
weights followed by tvq_silu_mul, the two-kernel path it replaces, on
ragged M (partial 256-row tiles), partial 256-column tiles and both output
dtypes; plus its use in the model's MLP at prefill size."""
from __future__ import annotations

import pytest
import torch

from nanovllm.quantization.utils import quantize_int8_per_channel
from tests.helpers import make_activations

pytestmark = pytest.mark.gpu


def _case(m, i, k, dtype, seed):
    from nanovllm.quantization import _hip
    print(f"CASE gemm_glu m={m} i={i} k={k} dtype={dtype}", flush=True)
    g = torch.Generator().manual_seed(seed)
    x = make_activations(m, k, seed=seed, dtype=dtype).cuda()
    w = torch.randn(2 * i, k, generator=g) * 0.02
    qw, ws = quantize_int8_per_channel(w)
    qw, ws = qw.cuda(), ws.float().cuda()
    xq, xs = _hip.act_quant(x)
    ref = _hip.w8a8_gemm(xq, xs, qw, ws, out_dtype=dtype, split_k=False)
    yref, _ = _hip.silu_mul(ref, out=True, quant=False)
    q2, s2 = _hip.glu_interleave(qw, ws)
    y = _hip.w8a8_gemm_glu(xq, xs, q2, s2, out_dtype=dtype)
    torch.cuda.synchronize()
    assert y.shape == (m, i)
    assert torch.equal(y, yref)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,i,k", [(1, 64, 128), (300, 3072, 1024), (4133, 3072, 1024), (513, 96, 256),
                                   (2048, 160, 384)])
def test_gemm_glu_matches_gemm_then_silu_mul(hiplib, m, i, k, dtype):
    _case(m, i, k, dtype, seed=m + i + k)


def test_gemm_glu_back_to_back_calls_with_smaller_input(hiplib):
    _case(4096, 3072, 1024, torch.bfloat16, seed=1)
    _case(257, 3072, 1024, torch.bfloat16, seed=2)


def test_mlp_glu_path_matches_unfused_and_follows_weight_updates(hiplib):
    """The engine MLP at >= GLU_MIN_TOKENS tokens (fused gate_up + SiLU-and-mul)
    equals the unfused path, also after the weights change in place."""
    from nanovllm.models.qwen3 import Qwen3Config, Qwen3MLP
    from nanovllm.quantization import _hip
    from nanovllm.quantization.activation import QuantizedActivation
    print("CASE mlp glu path", flush=True)
    cfg = Qwen3Config(hidden_size=256, intermediate_size=512)
    mlp = Qwen3MLP(cfg, "w8a8").cuda()
    g = torch.Generator().manual_seed(7)

    def draw():
        for lin in (mlp.gate_up_proj, mlp.down_proj):
            q, s = quantize_int8_per_channel(torch.randn(lin.qweight.shape, generator=g) * 0.02)
            lin.qweight.copy_(q.cuda())
            lin.w_scales.copy_(s.float().cuda())

    def unfused(qa):
        keep = Qwen3MLP.GLU_MIN_TOKENS
        Qwen3MLP.GLU_MIN_TOKENS = 1 << 40
        try:
            return mlp(qa)
        finally:
            Qwen3MLP.GLU_MIN_TOKENS = keep

    m = Qwen3MLP.GLU_MIN_TOKENS
    xq, xs = _hip.act_quant(make_activations(m, 256, seed=3).cuda())
    qa = QuantizedActivation(xq, xs, torch.bfloat16, (m, 256))
    with torch.no_grad():
        draw()
        assert torch.equal(mlp(qa), unfused(qa))
        draw()  # in place: the regrouped copy must follow
        assert torch.equal(mlp(qa), unfused(qa))
        # through the layer's weight_loader hooks (they write via .data, which
        # does not advance _version): the copy must follow
        lin = mlp.gate_up_proj
        q, s = quantize_int8_per_channel(torch.randn(lin.qweight.shape, generator=g) * 0.02)
        lin.qweight.weight_loader(lin.qweight, q)
        lin.w_scales.weight_loader(lin.w_scales, s.float())
        assert torch.equal(mlp(qa), unfused(qa))
        # re-assigned parameters (new tensors, possibly at a reused address)
        q, s = quantize_int8_per_channel(torch.randn(lin.qweight.shape, generator=g) * 0.02)
        lin.qweight = torch.nn.Parameter(q.cuda(), requires_grad=False)
        lin.w_scales = torch.nn.Parameter(s.float().cuda(), requires_grad=False)
        assert torch.equal(mlp(qa), unfused(qa))
