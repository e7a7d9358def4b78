"""GPU tests of the engine counterpart of LLM.generate with the quantized
projections on the gfx950 kernels.

* every quantized projection of a model step goes through the C-ABI library
  (calls into the ctypes binding are counted; the torch path is never taken);
* every quantized projection inside a GPU forward matches the oracle on the
  activations it received (the reference's torch path, cuda.py:293-300,
  455-465, and the kernels' fp32-scale numerics); whole-model logits are not
  compared across devices, since the CPU and GPU attention / norm rounding
  differences are amplified by W8A8's activation rounding;
* greedy KV-cache decoding on the GPU equals a cache-free recomputation;
* W8A16 / W8A8 engines stay close to the bf16 engine built from the same
  random weights.
"""
from __future__ import annotations

import pytest
import torch

from nanovllm import LLM, SamplingParams
from nanovllm.engine.model_runner import random_init_
from nanovllm.models.qwen3 import Qwen3Config
from nanovllm.quantization import _hip
from nanovllm.utils.context import step_context

pytestmark = pytest.mark.gpu

SMALL = dict(vocab_size=1024, hidden_size=256, intermediate_size=768, num_hidden_layers=3, num_attention_heads=4,
             num_key_value_heads=2, head_dim=128, max_position_embeddings=512)
# The real Qwen3-0.6B architecture: 28 layers, hidden 1024,
# intermediate 3072, 16 q / 8 kv heads, head_dim 128, vocab 151936.
QWEN3_06B = dict(vocab_size=151936, hidden_size=1024, intermediate_size=3072, num_hidden_layers=28,
                 num_attention_heads=16, num_key_value_heads=8, head_dim=128, max_position_embeddings=4096)


def _engine(quantization, device="cuda", std=0.08, eager=True, arch=SMALL):
    llm = LLM(Qwen3Config(**arch), device=device, quantization=quantization, max_model_len=256,
              max_num_batched_tokens=512, max_num_seqs=8, enforce_eager=eager)
    random_init_(llm.model_runner.model, seed=3, std=std, device=device)
    return llm


def _prefill_logits(model, ids: list[int], device) -> torch.Tensor:
    """Cache-free prefill of one sequence (no KV slot written)."""
    n = len(ids)
    if device == "cuda":
        meta = dict(attn_blocks=_hip.prefill_blocks([(0, n)]).cuda())
    else:
        meta = {}
    with torch.no_grad(), step_context(True, cu_seqlens_q=torch.tensor([0, n]), max_seqlen_q=n, **meta):
        x = torch.tensor(ids, device=device)
        return model.compute_logits(model(x, torch.arange(len(ids), device=device))).float().cpu()


def _rel_l2(a: torch.Tensor, b: torch.Tensor) -> float:
    return float((a - b).norm() / b.norm())


@pytest.mark.parametrize("mode", ["int8", "w8a8"])
def test_quantized_projections_run_native(gpu, hiplib, monkeypatch, mode):
    calls = {"n": 0}
    # W8A16: every projection is one tvq_w8a16_gemm. W8A8: every projection
    # receives int8 codes from a producer with the quantization fused in
    # (qkv / gate_up / down from the norm and SiLU kernels, o_proj from the
    # attention kernel) and runs tvq_w8a8_gemm.
    names = ["w8a16_gemm"] if mode == "int8" else ["w8a8_linear", "w8a8_gemm"]

    def counting(orig):
        def counted(*a, **k):
            calls["n"] += 1
            return orig(*a, **k)
        return counted

    llm = _engine(mode)  # its warm-up prefill runs before the counting starts
    for name in names:
        monkeypatch.setattr(_hip, name, counting(getattr(_hip, name)))
    llm.generate([[1, 2, 3, 4, 5, 6]], SamplingParams(temperature=0.0, max_tokens=3, ignore_eos=True),
                 use_tqdm=False)
    # 1 prefill + 2 decode steps, 4 projections x 3 layers each
    assert calls["n"] == 3 * 4 * 3


def _check_projections_against_oracle(llm, mode, arch, prompt):
    """Every quantized projection of one GPU prefill, on the activations it
    actually received, against the oracle on those same activations: the
    act-quant codes and scales are bit-exact, the outputs within the bf16
    tolerance of the reference's torch path and of the kernels' own
    fp32-scale numerics."""
    import oracle
    from nanovllm.layers.linear import LinearBase
    from nanovllm.quantization.activation import QuantizedActivation
    model = llm.model_runner.model
    seen = []

    def grab(mod, inp, out):
        x = inp[0]
        x = QuantizedActivation(x.xq.cpu(), x.scales.cpu(), x.dtype, x.shape) \
            if isinstance(x, QuantizedActivation) else x.detach().cpu()
        seen.append((mod, x, out.detach().cpu()))

    hooks = [m.register_forward_hook(grab) for m in model.modules() if isinstance(m, LinearBase)]
    _prefill_logits(model, prompt, "cuda")
    for h in hooks:
        h.remove()
    layers = arch["num_hidden_layers"]
    assert len(seen) == 4 * layers
    fused = 0
    for mod, x, y in seen:
        q = mod.qweight.cpu()
        if mode == "int8":
            s = mod.scales.cpu()
            ref_path = oracle.w8a16_torch_path(x, q, s)
            ref_own = oracle.w8a16_fp32_scale_torch(x, q, s)
        else:
            s = mod.w_scales.cpu()
            if isinstance(x, QuantizedActivation):   # codes from a fused producer
                xq, a_s = x.xq, x.scales
                fused += 1
            else:
                xq, a_s = oracle.quantize_rows_torch(x)
                gq, ga = _hip.act_quant(x.cuda())
                assert torch.equal(gq.cpu(), xq) and torch.equal(ga.cpu(), a_s)
            ref_path = oracle.w8a8_torch_path(xq, a_s, q, s, None, torch.bfloat16)
            ref_own = oracle.w8a8_fp32_scale_torch(xq, a_s, q, s, None, torch.bfloat16)
        yf = y.float().numpy()
        for ref in (ref_path, ref_own):
            rf = ref.float().numpy()
            assert oracle.rel_l2(yf, rf) <= oracle.REL_L2_TOL
            assert oracle.max_abs_ratio(yf, rf) <= oracle.MAX_ABS_TOL
        # against its own numerics the kernel is far tighter than the tolerance
        assert oracle.rel_l2(yf, ref_own.float().numpy()) < 2e-3
    assert fused == (4 * layers if mode == "w8a8" else 0)  # o_proj's codes come from the attention kernel


@pytest.mark.parametrize("mode", ["int8", "w8a8"])
def test_projections_inside_model_match_oracle(gpu, hiplib, mode):
    _check_projections_against_oracle(_engine(mode), mode, SMALL, list(range(7, 7 + 200, 3)) + [5] * 31)


@pytest.mark.parametrize("mode", ["int8", "w8a8"])
def test_qwen3_06b_architecture_projections_match_oracle(gpu, hiplib, mode):
    """The full 28-layer Qwen3-0.6B architecture (random init): all 112
    projections of a 2-prompt prefill against the oracle."""
    print(f"CASE qwen3_06b projections mode={mode}", flush=True)
    llm = _engine(mode, std=0.02, arch=QWEN3_06B)
    _check_projections_against_oracle(llm, mode, QWEN3_06B, list(range(100, 100 + 7 * 60, 7)) + [9] * 37)


@pytest.mark.parametrize("mode", [None, "int8", "w8a8"])
def test_qwen3_06b_architecture_graph_decode_matches_eager(gpu, hiplib, mode):
    """Qwen3-0.6B architecture: greedy decode through the captured HIP graphs
    gives the same tokens as eager execution."""
    print(f"CASE qwen3_06b graph-vs-eager mode={mode}", flush=True)
    prompts = [list(range(1000, 1000 + 90)), [5, 17, 33, 2, 90, 41], [77] * 31]
    sp = SamplingParams(temperature=0.0, max_tokens=10, ignore_eos=True)
    outs = {}
    for eager in (True, False):
        llm = _engine(mode, std=0.02, eager=eager, arch=QWEN3_06B)
        assert bool(llm.model_runner.graphs) == (not eager)
        outs[eager] = [o["token_ids"] for o in llm.generate(prompts, sp, use_tqdm=False)]
        del llm
        torch.cuda.empty_cache()
    assert outs[True] == outs[False]


def test_bf16_kv_cache_decode_matches_recompute(gpu):
    llm = _engine(None, eager=False)
    prompts = [[5, 17, 33, 2, 90, 41], [100, 3], list(range(40, 160))]
    outs = llm.generate(prompts, SamplingParams(temperature=0.0, max_tokens=12, ignore_eos=True), use_tqdm=False)
    model = llm.model_runner.model
    for p, o in zip(prompts, outs):
        full = p + o["token_ids"]
        pred = _prefill_logits(model, full, "cuda")[len(p) - 1: len(full) - 1]
        top2 = pred.topk(2, dim=-1).values
        clear = (top2[:, 0] - top2[:, 1]) > 0.05
        got = torch.tensor(o["token_ids"])
        assert torch.equal(pred.argmax(-1)[clear], got[clear])


@pytest.mark.parametrize("mode", ["int8", "w8a8"])
def test_quantized_engine_close_to_bf16(gpu, hiplib, mode):
    ids = list(range(11, 11 + 150))
    ref = _prefill_logits(_engine(None).model_runner.model, ids, "cuda")
    got = _prefill_logits(_engine(mode).model_runner.model, ids, "cuda")
    # int8 weights (and int8 activations for w8a8) perturb every projection;
    # across 3 layers the logits stay within a few percent.
    assert _rel_l2(got, ref) < (0.05 if mode == "int8" else 0.08), _rel_l2(got, ref)


@pytest.mark.parametrize("mode", [None, "int8", "w8a8"])
def test_decode_graph_replay_matches_eager(gpu, hiplib, mode):
    """Decode through captured HIP graphs (batch padded to its bucket) gives
    the same greedy tokens as eager execution, over many replays."""
    prompts = [[5, 17, 33, 2, 90, 41], [100, 3], list(range(40, 160)), [7] * 30, [1, 2, 3]]
    sp = SamplingParams(temperature=0.0, max_tokens=12, ignore_eos=True)
    outs = {}
    for eager in (True, False):
        llm = LLM(Qwen3Config(**SMALL), quantization=mode, max_model_len=256, max_num_batched_tokens=512,
                  max_num_seqs=8, enforce_eager=eager)
        random_init_(llm.model_runner.model, seed=3, std=0.08)
        assert bool(llm.model_runner.graphs) == (not eager)
        outs[eager] = [o["token_ids"] for o in llm.generate(prompts, sp, use_tqdm=False)]
    assert outs[True] == outs[False]
