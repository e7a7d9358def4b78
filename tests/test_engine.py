"""CPU tests of the engine counterpart of LLM.generate: scheduler policy
(reference scheduler.py:25-73), sampling-parameter checks, the engine loop's
outputs and statistics (reference llm_engine.py:86-163), KV-cache decode
against full recomputation, and loading a quantized artifact made by the
quantize CLI. The quantized layers run the reference's torch path here
(CPU tensors); the GPU counterpart of these checks is test_gpu_engine.py.
"""
from __future__ import annotations

import json

import pytest
import torch
from safetensors.torch import save_file

from nanovllm import LLM, SamplingParams
from nanovllm.engine.model_runner import random_init_
from nanovllm.engine.scheduler import Scheduler
from nanovllm.engine.sequence import Sequence
from nanovllm.models.qwen3 import Qwen3Config
from nanovllm.utils.context import step_context

TINY = dict(vocab_size=256, hidden_size=64, intermediate_size=128, num_hidden_layers=2, num_attention_heads=4,
            num_key_value_heads=2, head_dim=16, max_position_embeddings=256)


def _engine(quantization=None, std=0.3, **kw):
    args = dict(max_model_len=96, max_num_batched_tokens=128, max_num_seqs=4)
    args.update(kw)
    llm = LLM(Qwen3Config(**TINY), device="cpu", quantization=quantization, **args)
    random_init_(llm.model_runner.model, seed=0, std=std, device="cpu")
    return llm


def test_sampling_params_checks():
    assert SamplingParams().temperature == 1.0 and SamplingParams().max_tokens == 64
    SamplingParams(temperature=0.0)  # greedy
    with pytest.raises(ValueError):
        SamplingParams(temperature=-1.0)
    with pytest.raises(ValueError):
        SamplingParams(max_tokens=0)


def test_scheduler_prefill_first_limits_and_slots():
    sp = SamplingParams(max_tokens=2, ignore_eos=True)
    sch = Scheduler(max_num_seqs=2, max_num_batched_tokens=10, num_slots=3, eos=0)
    seqs = [Sequence([1] * n, sp) for n in (4, 5, 3, 2)]
    for s in seqs:
        sch.add(s)
    batch, prefill = sch.schedule()              # 4 + 5 tokens fit, third would exceed 10
    assert prefill and batch == seqs[:2] and [s.slot for s in batch] == [0, 1]
    batch, prefill = sch.schedule()              # max_num_seqs running: decode them
    assert not prefill and batch == seqs[:2]
    sch.postprocess(batch, [7, 7])
    sch.postprocess(seqs[:1], [7])               # seqs[0] reaches max_tokens=2 -> finished, slot freed
    assert seqs[0].is_finished and not seqs[1].is_finished and sch.free_slots == [2, 0]
    batch, prefill = sch.schedule()              # 3 tokens fit; lowest free slot first
    assert prefill and batch == [seqs[2]] and seqs[2].slot == 0
    batch, prefill = sch.schedule()
    assert not prefill and batch == [seqs[1], seqs[2]]
    sch.postprocess(batch, [7, 7])
    assert seqs[1].is_finished and sorted(sch.free_slots) == [1, 2]
    batch, prefill = sch.schedule()
    assert prefill and batch == [seqs[3]] and seqs[3].slot == 1


def test_scheduler_eos_and_ignore_eos():
    sch = Scheduler(4, 64, 4, eos=9)
    a, b = Sequence([1, 2], SamplingParams(max_tokens=5)), Sequence([1, 2], SamplingParams(max_tokens=5, ignore_eos=True))
    sch.add(a)
    sch.add(b)
    sch.schedule()
    sch.postprocess([a, b], [9, 9])
    assert a.is_finished and not b.is_finished and a.completion_token_ids == [9]


@pytest.mark.parametrize("quantization", [None, "int8", "w8a8"])
def test_generate_outputs_and_stats(quantization):
    llm = _engine(quantization)
    prompts = [[1, 2, 3, 4, 5], [7] * 20, [9, 8, 7], list(range(30)), [3, 3]]
    sps = [SamplingParams(temperature=0.0, max_tokens=m, ignore_eos=True) for m in (6, 3, 8, 1, 5)]
    outs, st = llm.generate_with_stats(prompts, sps)
    assert [len(o["token_ids"]) for o in outs] == [6, 3, 8, 1, 5]
    assert st["prefill_tokens"] == sum(map(len, prompts))
    assert st["decode_tokens"] == sum(sp.max_tokens for sp in sps) - len(prompts)
    assert st["prefill_steps"] == 2  # 4 seqs (max_num_seqs) then the fifth
    assert st["ttft_seconds_approx"] is not None and st["decode_tokens_per_second"] > 0
    assert llm.scheduler.is_finished() and sorted(llm.scheduler.free_slots) == [0, 1, 2, 3]


def test_kv_cache_decode_matches_recompute():
    """Every greedy token equals the argmax of a cache-free prefill over the
    prompt plus the tokens generated before it."""
    llm = _engine(None)
    prompts = [[5, 17, 33, 2, 90, 41], [100, 3], list(range(40, 60))]
    outs = llm.generate(prompts, SamplingParams(temperature=0.0, max_tokens=10, ignore_eos=True), use_tqdm=False)
    model = llm.model_runner.model
    distinct = 0
    for p, o in zip(prompts, outs):
        full = p + o["token_ids"]
        with torch.no_grad(), step_context(True, cu_seqlens_q=torch.tensor([0, len(full)])):
            logits = model.compute_logits(model(torch.tensor(full), torch.arange(len(full))))
        pred = logits[len(p) - 1: len(full) - 1].float()
        top2 = pred.topk(2, dim=-1).values
        clear = (top2[:, 0] - top2[:, 1]) > 0.05  # skip near-ties: bf16 cache vs recompute rounding
        got = torch.tensor(o["token_ids"])
        assert torch.equal(pred.argmax(-1)[clear], got[clear])
        distinct += len(set(o["token_ids"]))
    assert distinct > 3  # generations are not a single repeated token


def test_temperature_sampling_runs_and_respects_eos():
    llm = _engine(None)
    outs = llm.generate([[1, 2, 3]] * 3, SamplingParams(temperature=0.8, max_tokens=12), use_tqdm=False)
    for o in outs:
        assert 1 <= len(o["token_ids"]) <= 12


def test_add_request_validation():
    llm = _engine(None)
    with pytest.raises(ValueError):
        llm.add_request([1] * 90, SamplingParams(max_tokens=10))  # exceeds max_model_len 96
    with pytest.raises(ValueError):
        llm.add_request("text prompt", SamplingParams())          # no tokenizer in a random model


def _checkpoint(tmp_path):
    cfg = Qwen3Config(**TINY)
    g = torch.Generator().manual_seed(1)

    def w(*shape, std=0.2):
        return (torch.randn(*shape, generator=g) * std).to(torch.bfloat16)

    H, D, I = cfg.hidden_size, cfg.head_dim, cfg.intermediate_size
    t = {"model.embed_tokens.weight": w(cfg.vocab_size, H), "model.norm.weight": torch.ones(H, dtype=torch.bfloat16)}
    for i in range(cfg.num_hidden_layers):
        p = f"model.layers.{i}."
        t[p + "self_attn.q_proj.weight"] = w(cfg.num_attention_heads * D, H)
        t[p + "self_attn.k_proj.weight"] = w(cfg.num_key_value_heads * D, H)
        t[p + "self_attn.v_proj.weight"] = w(cfg.num_key_value_heads * D, H)
        t[p + "self_attn.o_proj.weight"] = w(H, cfg.num_attention_heads * D)
        t[p + "self_attn.q_norm.weight"] = torch.ones(D, dtype=torch.bfloat16)
        t[p + "self_attn.k_norm.weight"] = torch.ones(D, dtype=torch.bfloat16)
        t[p + "mlp.gate_proj.weight"] = w(I, H)
        t[p + "mlp.up_proj.weight"] = w(I, H)
        t[p + "mlp.down_proj.weight"] = w(H, I)
        t[p + "input_layernorm.weight"] = torch.ones(H, dtype=torch.bfloat16)
        t[p + "post_attention_layernorm.weight"] = torch.ones(H, dtype=torch.bfloat16)
    d = tmp_path / "model"
    d.mkdir()
    save_file(t, d / "model.safetensors")
    (d / "config.json").write_text(json.dumps({**TINY, "eos_token_id": 255, "tie_word_embeddings": True}))
    return d


@pytest.mark.parametrize("mode", ["int8", "w8a8"])
def test_engine_loads_checkpoint_and_quantized_artifact(tmp_path, mode):
    from nanovllm.quantization.quantize import main
    src = _checkpoint(tmp_path)
    main(["--model", str(src), "--output", str(tmp_path / mode), "--quantization", mode])
    kw = dict(device="cpu", max_model_len=64, max_num_batched_tokens=64, max_num_seqs=2)
    ref = LLM(str(src), **kw)
    q = LLM(str(src), quantization=mode, quantized_model_path=str(tmp_path / mode), **kw)
    assert ref.config.eos == 255
    layer = q.model_runner.model.model.layers[0].mlp.down_proj
    assert layer.qweight.dtype == torch.int8 and int(layer.qweight.abs().max()) == 127
    prompts = [[1, 2, 3, 4], [50, 60, 70]]
    sp = SamplingParams(temperature=0.0, max_tokens=8, ignore_eos=True)
    a = [o["token_ids"] for o in ref.generate(prompts, sp, use_tqdm=False)]
    b = [o["token_ids"] for o in q.generate(prompts, sp, use_tqdm=False)]
    assert a[0][0] == b[0][0] and a[1][0] == b[1][0]  # first tokens agree under int8 weights


def test_glu_cache_key_follows_every_kind_of_weight_change():
    """The fused gate_up path's regrouped-weight cache key changes on in-place
    updates, on loader writes through .data and on re-assignment."""
    from nanovllm.models.qwen3 import Qwen3MLP
    mlp = Qwen3MLP(Qwen3Config(hidden_size=256, intermediate_size=512), "w8a8")
    lin = mlp.gate_up_proj
    keys = [mlp._glu_key()]
    with torch.no_grad():
        lin.qweight.copy_(torch.ones_like(lin.qweight))
    keys.append(mlp._glu_key())
    lin.qweight.weight_loader(lin.qweight, torch.zeros_like(lin.qweight))
    keys.append(mlp._glu_key())
    lin.w_scales.weight_loader(lin.w_scales, torch.ones(lin.w_scales.shape))
    keys.append(mlp._glu_key())
    lin.qweight = torch.nn.Parameter(torch.zeros_like(lin.qweight), requires_grad=False)
    keys.append(mlp._glu_key())
    assert len(set(keys)) == len(keys)


def test_glu_fused_path_shape_gate():
    from nanovllm.models.qwen3 import Qwen3MLP
    assert Qwen3MLP(Qwen3Config(hidden_size=1024, intermediate_size=3072), "w8a8").glu_shape_ok()
    assert not Qwen3MLP(Qwen3Config(hidden_size=1000, intermediate_size=3072), "w8a8").glu_shape_ok()
    assert not Qwen3MLP(Qwen3Config(hidden_size=1024, intermediate_size=3000), "w8a8").glu_shape_ok()


def test_step_context_nesting_and_validation():
    from nanovllm.utils.context import get_context, step_context
    assert not get_context().is_prefill
    with step_context(True, max_seqlen_q=7) as outer:
        assert get_context() is outer
        with step_context(False, context_lens=torch.ones(2)):
            assert not get_context().is_prefill
        assert get_context() is outer
    assert not get_context().is_prefill and get_context().max_seqlen_q == 0
    with pytest.raises(TypeError, match="do not belong to a prefill"):
        with step_context(True, context_lens=torch.ones(2)):
            pass
    with pytest.raises(TypeError, match="unknown step metadata"):
        with step_context(False, bogus=1):
            pass
    with pytest.raises(RuntimeError):
        with step_context(True):
            raise RuntimeError("inside")
    assert not get_context().is_prefill


def test_sequence_keeps_prompt_and_output_apart():
    s = Sequence([4, 5, 6], SamplingParams(max_tokens=3))
    assert len(s) == 3 and s.last_token == 6 and s.num_completion_tokens == 0
    s.append_token(9)
    assert s.token_ids == [4, 5, 6, 9] and s.completion_token_ids == [9] and s.last_token == 9
    assert s.num_prompt_tokens == 3 and len(s) == 4 and s.max_tokens == 3
    t = Sequence([1])
    assert t.seq_id > s.seq_id
    with pytest.raises(ValueError):
        Sequence([])
