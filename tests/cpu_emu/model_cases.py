"""The Qwen3 model's device path (the HIP kernels the GPU engine runs) on the
CPU emulation of those kernels: test infrastructure, run by
tests/test_cpu_emu_model.py in a child process, because it makes every
torch tensor of this process report is_cuda=True (so that the model takes
its device path) and points nanovllm.quantization._hip at the emulated
library built from the same kernel sources.

Cases (prints "all cases passed" at the end):
  * every quantized projection of a prefill, on the activations it actually
    received, against the oracle (W8A16 and W8A8; in W8A8 all four
    projections receive fused codes: qkv / gate_up / down from the norm and
    SiLU kernels, o_proj from the attention kernel); the 3-layer test
    architecture, and for W8A8 the 28-layer Qwen3-0.6B one (every layer's
    input kinds, three layers' outputs);
  * the W8A8 MLP's gate_up GEMM with the SiLU-and-mul epilogue (>= 4096
    tokens) gives the same hidden states, bit for bit, as the unfused path;
  * greedy decode through the KV cache (prompt K/V stored by the fused
    q/k-norm + rotary kernel, decode attention appending one row per step)
    equals a cache-free recomputation wherever the top-2 logits are clear;
  * the device path's logits stay close to the host (torch) path's.

With --race (and EMU_DMA=late) it runs on the race-checking build
(tests/cpu_emu/racecheck.h) and fails on any report.
"""
from __future__ import annotations

import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path[:0] = [str(ROOT), str(ROOT / "tiny-vllm_amd"), str(HERE)]

import torch  # noqa: E402

import emu  # noqa: E402
import oracle  # noqa: E402
from nanovllm.engine.model_runner import random_init_  # noqa: E402
from nanovllm.layers.linear import LinearBase  # noqa: E402
from nanovllm.models.qwen3 import Attention, Qwen3Config, Qwen3ForCausalLM, Qwen3MLP  # noqa: E402
from nanovllm.quantization import _hip  # noqa: E402
from nanovllm.quantization.activation import QuantizedActivation  # noqa: E402
from nanovllm.utils.context import step_context  # noqa: E402

SMALL = dict(vocab_size=1024, hidden_size=256, intermediate_size=768, num_hidden_layers=3, num_attention_heads=4,
             num_key_value_heads=2, head_dim=128, max_position_embeddings=512)
QWEN3_06B = dict(vocab_size=151936, hidden_size=1024, intermediate_size=3072, num_hidden_layers=28,
                 num_attention_heads=16, num_key_value_heads=8, head_dim=128, max_position_embeddings=4096)
MAX_LEN, SLOTS = 256, 4


def case(name):
    print("CASE", name, flush=True)


def build(mode, arch, std):
    torch.set_default_dtype(torch.bfloat16)
    model = Qwen3ForCausalLM(Qwen3Config(**arch), quantization=mode).eval()
    torch.set_default_dtype(torch.float32)
    random_init_(model, seed=3, std=std, device="cpu")
    attns = [m for m in model.modules() if isinstance(m, Attention)]
    kv = torch.zeros(2, len(attns), SLOTS, attns[0].num_kv_heads, MAX_LEN, 128, dtype=torch.bfloat16)
    for i, a in enumerate(attns):
        a.k_cache, a.v_cache = kv[0, i], kv[1, i]
    return model


class _NoDevice:
    def __init__(self, *a, **k):
        pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        return False


def device_path_on_emulation():
    """From here on the model takes its device path, on the emulated kernels."""
    lib = emu.load(race="--race" in sys.argv)
    n = lib.tvq_gemm_workspace_bytes()
    raw = torch.zeros(n + 256, dtype=torch.uint8)
    off = (-raw.data_ptr()) % 256
    ws = raw[off:off + n]
    cnt = torch.zeros(_hip.ATTN_COUNTERS, dtype=torch.int32)
    _hip.load_library = lambda: lib
    _hip._stream = lambda dev: None
    _hip.gemm_workspace = lambda dev: ws
    _hip.attn_counters = lambda dev: cnt
    _hip._keep = (raw, cnt)
    torch.cuda.device = _NoDevice
    torch.Tensor.is_cuda = property(lambda self: True)


def prefill(model, prompts, slots, device_path=True):
    """Packed prefill of the prompts into their KV slots; last hidden row of each."""
    lens = [len(p) for p in prompts]
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    ids = torch.tensor([t for p in prompts for t in p])
    pos = torch.cat([torch.arange(n) for n in lens])
    meta = dict(cu_seqlens_q=torch.tensor(cu), max_seqlen_q=max(lens), slot_mapping=torch.tensor(slots))
    if device_path:
        meta.update(attn_blocks=_hip.prefill_blocks([(cu[i], n) for i, n in enumerate(lens)]),
                    token_slots=torch.repeat_interleave(torch.tensor(slots), torch.tensor(lens)))
    with torch.no_grad(), step_context(True, **meta):
        h = model(ids, pos)
    return h[torch.tensor(cu[1:]) - 1]


def decode(model, tokens, slots, lens):
    with torch.no_grad(), step_context(False, max_seqlen_k=max(lens), slot_mapping=torch.tensor(slots, dtype=torch.int32),
                                       context_lens=torch.tensor(lens, dtype=torch.int32), kv_lo=min(slots),
                                       kv_hi=max(slots) + 1):
        return model(torch.tensor(tokens), torch.tensor([n - 1 for n in lens]))


def check_projections(model, mode, layers, prompt, sample_layers=None):
    """Every projection's count and input kind; the outputs of all layers, or
    of `sample_layers`, against the oracle."""
    seen = []

    def grab(mod, inp, out):
        x = inp[0]
        x = QuantizedActivation(x.xq.clone(), x.scales.clone(), x.dtype, x.shape) \
            if isinstance(x, QuantizedActivation) else x.detach().clone()
        seen.append((mod, x, out.detach().clone()))

    hooks = [m.register_forward_hook(grab) for m in model.modules() if isinstance(m, LinearBase)]
    prefill(model, [prompt], [0])
    for h in hooks:
        h.remove()
    assert len(seen) == 4 * layers, len(seen)
    fused = sum(isinstance(x, QuantizedActivation) for _, x, _ in seen)
    assert fused == (4 * layers if mode == "w8a8" else 0), fused
    for i, (mod, x, y) in enumerate(seen):
        if sample_layers is not None and i // 4 not in sample_layers:
            continue
        if mode == "int8":
            refs = (oracle.w8a16_torch_path(x, mod.qweight, mod.scales),
                    oracle.w8a16_fp32_scale_torch(x, mod.qweight, mod.scales))
        else:
            if isinstance(x, QuantizedActivation):
                xq, a_s = x.xq, x.scales
            else:
                xq, a_s = oracle.quantize_rows_torch(x)
            refs = (oracle.w8a8_torch_path(xq, a_s, mod.qweight, mod.w_scales, None, torch.bfloat16),
                    oracle.w8a8_fp32_scale_torch(xq, a_s, mod.qweight, mod.w_scales, None, torch.bfloat16))
        yf = y.float().numpy()
        for ref in refs:
            assert oracle.rel_l2(yf, ref.float().numpy()) <= oracle.REL_L2_TOL
            assert oracle.max_abs_ratio(yf, ref.float().numpy()) <= oracle.MAX_ABS_TOL
        assert oracle.rel_l2(yf, refs[1].float().numpy()) < 2e-3


def main() -> None:
    prompt = list(range(7, 7 + 200, 3)) + [5] * 31

    # host-path logits first (before the device path is switched on)
    host = {}
    for mode in (None, "int8", "w8a8"):
        m = build(mode, SMALL, 0.08)
        with torch.no_grad():
            host[mode] = m.compute_logits(prefill(m, [list(range(11, 11 + 150))], [0], device_path=False)).float()

    device_path_on_emulation()

    for mode in ("int8", "w8a8"):
        case(f"projections vs oracle, test architecture, {mode}")
        check_projections(build(mode, SMALL, 0.08), mode, 3, prompt)

    for mode in (None, "int8", "w8a8"):
        case(f"device path close to host path, {mode}")
        m = build(mode, SMALL, 0.08)
        with torch.no_grad():
            dev = m.compute_logits(prefill(m, [list(range(11, 11 + 150))], [0])).float()
        rel = float((dev - host[mode]).norm() / host[mode].norm())
        # W8A8's activation rounding amplifies the host path's bf16-rounded scales
        assert rel < (0.08 if mode == "w8a8" else 0.05), (mode, rel)

    case("w8a8 gate_up with the SiLU epilogue (>= 4096 tokens) equals the unfused path")
    m = build("w8a8", SMALL, 0.08)
    long = [list(range(1, 250)) * 5 for _ in range(4)]  # 4 x 1245 = 4980 tokens
    with torch.no_grad(), step_context(True, cu_seqlens_q=torch.tensor([0, 1245, 2490, 3735, 4980]), max_seqlen_q=1245,
                                       attn_blocks=_hip.prefill_blocks([(1245 * i, 1245) for i in range(4)])):
        ids = torch.tensor([t for p in long for t in p])
        pos = torch.cat([torch.arange(1245)] * 4)
        fused = m(ids, pos)
        old = Qwen3MLP.GLU_MIN_TOKENS
        Qwen3MLP.GLU_MIN_TOKENS = 1 << 30
        unfused = m(ids, pos)
        Qwen3MLP.GLU_MIN_TOKENS = old
    assert torch.equal(fused.view(torch.int16), unfused.view(torch.int16))

    for mode in (None, "int8", "w8a8"):
        case(f"greedy KV-cache decode equals recomputation, {mode}")
        m = build(mode, SMALL, 0.08)
        prompts = [[5, 17, 33, 2, 90, 41], [100, 3], list(range(40, 160))]
        slots = [2, 0, 3]
        with torch.no_grad():
            toks = m.compute_logits(prefill(m, prompts, slots)).float().argmax(-1).tolist()
        gen = [[t] for t in toks]
        lens = [len(p) + 1 for p in prompts]
        for _ in range(7):
            with torch.no_grad():
                toks = m.compute_logits(decode(m, toks, slots, lens)).float().argmax(-1).tolist()
            for g, t in zip(gen, toks):
                g.append(t)
            lens = [n + 1 for n in lens]
        for p, g in zip(prompts, gen):
            full = p + g
            n = len(full)
            with torch.no_grad(), step_context(True, cu_seqlens_q=torch.tensor([0, n]), max_seqlen_q=n,
                                               attn_blocks=_hip.prefill_blocks([(0, n)])):
                logits = m.compute_logits(m(torch.tensor(full), torch.arange(n))).float()
            pred = logits[len(p) - 1: n - 1]
            top2 = pred.topk(2, dim=-1).values
            clear = (top2[:, 0] - top2[:, 1]) > 0.05
            assert torch.equal(pred.argmax(-1)[clear], torch.tensor(g)[clear]), (mode, p[:4])

    case("projections vs oracle, Qwen3-0.6B architecture (28 layers), w8a8")
    check_projections(build("w8a8", QWEN3_06B, 0.02), "w8a8", 28, list(range(100, 100 + 7 * 60, 7)) + [9] * 37,
                      sample_layers=(0, 13, 27))

    if "--race" in sys.argv:
        n = _hip.load_library().tvq_emu_race_reports()
        assert n == 0, f"{n} race report(s)"
    print("all cases passed", flush=True)


if __name__ == "__main__":
    main()
