"""Qwen3 decoder for the end-to-end quantized-linear benchmark
(architecture of the reference's nanovllm/models/qwen3.py).

Every qkv / o / gate_up / down projection is a tensor-parallel Linear from
nanovllm.layers.linear, so with `quantization` = "int8" or "w8a8" the 4
projections of each layer run on the gfx950 quantized kernels (112 linears
for the 28-layer 0.6B model). RMSNorm (with the fused residual add) and
SiLU-and-multiply run on the fused HIP producer kernels, which for W8A8 also
emit the next projection's int8 codes and per-token scales. The rest is plain
PyTorch: rotary embedding (rotate-half, neox style), grouped-query attention
over the engine's KV cache (SDPA for prefill, batched matmuls for decode),
tied or separate LM head.

Attention reads its per-step metadata from nanovllm.utils.context, which the
engine sets before each forward:
  prefill: cu_seqlens_q (ragged packing of the prompts), slot ids
  decode : context_lens (tokens in cache incl. the new one), slot ids, the
           slot range [kv_lo, kv_hi) of the running batch, max_seqlen_k
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import nn

from nanovllm.layers.activation import SiluAndMul
from nanovllm.layers.layernorm import RMSNorm
from nanovllm.layers.linear import MergedColumnParallelLinear, QKVParallelLinear, RowParallelLinear
from nanovllm.quantization import _hip
from nanovllm.quantization.activation import QuantizedActivation
from nanovllm.quantization.cuda import _get_w8a8_backend_preference
from nanovllm.utils.context import get_context


@dataclass
class Qwen3Config:
    """The fields of a Hugging Face Qwen3 config this model reads."""
    vocab_size: int = 151936
    hidden_size: int = 1024
    intermediate_size: int = 3072
    num_hidden_layers: int = 28
    num_attention_heads: int = 16
    num_key_value_heads: int = 8
    head_dim: int = 128
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1000000.0
    max_position_embeddings: int = 40960
    tie_word_embeddings: bool = True
    attention_bias: bool = False
    hidden_act: str = "silu"


class RotaryEmbedding(nn.Module):
    def __init__(self, head_dim: int, max_position: int, base: float):
        super().__init__()
        inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float) / head_dim))
        freqs = torch.outer(torch.arange(max_position, dtype=torch.float), inv_freq)
        self.register_buffer("cos", freqs.cos(), persistent=False)
        self.register_buffer("sin", freqs.sin(), persistent=False)

    def forward(self, positions: torch.Tensor, q: torch.Tensor, k: torch.Tensor):
        cos = self.cos[positions].unsqueeze(1)
        sin = self.sin[positions].unsqueeze(1)

        def rot(x):
            x1, x2 = x.float().chunk(2, dim=-1)
            return torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), dim=-1).to(x.dtype)

        return rot(q), rot(k)


class Attention(nn.Module):
    """GQA attention over a per-sequence KV cache [slots, kv_heads, max_len, head_dim]."""

    def __init__(self, num_heads: int, num_kv_heads: int, head_dim: int):
        super().__init__()
        self.num_heads, self.num_kv_heads, self.head_dim = num_heads, num_kv_heads, head_dim
        self.scale = head_dim ** -0.5
        self.k_cache = self.v_cache = None  # set by the engine

    def _prefill_gpu(self, q, k, v, ctx, quant: bool):
        """HIP varlen causal attention over the packed prompts. The prompt
        tokens' K/V were already stored into their cache slots by the fused
        q/k-norm + rotary kernel (Qwen3Attention.forward)."""
        if quant:
            return self._quantized(*_hip.prefill_attention_quant(q, k, v, ctx.attn_blocks, self.scale))
        return _hip.prefill_attention(q, k, v, ctx.attn_blocks, self.scale)

    @staticmethod
    def _quantized(out: torch.Tensor, xq: torch.Tensor, scales: torch.Tensor) -> QuantizedActivation:
        return QuantizedActivation(xq, scales, out.dtype, tuple(xq.shape))

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, quant: bool = False):
        """softmax(scale q K^T) V; with `quant` (W8A8 o_proj on the GPU), the
        output comes back as o_proj's per-token int8 codes and scales,
        quantized inside the attention kernel (bit-identical to quantizing
        the bf16 output)."""
        ctx = get_context()
        group = self.num_heads // self.num_kv_heads
        if ctx.is_prefill:
            if q.is_cuda:
                return self._prefill_gpu(q, k, v, ctx, quant)
            # Host path (CPU tests): one causal attention per sequence
            # (host-side cu_seqlens_q), after writing its keys/values to its
            # cache slot.
            out = torch.empty_like(q)
            cu = ctx.cu_seqlens_q.tolist()
            slots = ctx.slot_mapping.tolist() if ctx.slot_mapping is not None else [None] * (len(cu) - 1)
            for i in range(len(cu) - 1):
                a, b = cu[i], cu[i + 1]
                kk, vv = k[a:b].transpose(0, 1), v[a:b].transpose(0, 1)
                if self.k_cache is not None and slots[i] is not None:
                    self.k_cache[slots[i], :, : b - a] = kk
                    self.v_cache[slots[i], :, : b - a] = vv
                if group > 1:
                    kk, vv = kk.repeat_interleave(group, 0), vv.repeat_interleave(group, 0)
                o = F.scaled_dot_product_attention(q[a:b].transpose(0, 1).unsqueeze(0), kk.unsqueeze(0),
                                                   vv.unsqueeze(0), is_causal=True, scale=self.scale)
                out[a:b] = o.squeeze(0).transpose(0, 1)
            return out
        # Decode: one new token per running sequence.
        slots, lens = ctx.slot_mapping, ctx.context_lens
        if q.is_cuda:
            # HIP kernel: appends k/v at position lens-1 of each slot and
            # attends over the valid prefix only; lengths are read on the
            # device (graph-capturable).
            if quant:
                return self._quantized(*_hip.decode_attention_quant(q, k, v, self.k_cache, self.v_cache, slots, lens,
                                                                     self.scale))
            return _hip.decode_attention(q, k, v, self.k_cache, self.v_cache, slots, lens, self.scale)
        # Host path (CPU tests): the running batch owns cache slots inside
        # [kv_lo, kv_hi); attention runs over that slice of the cache up to the
        # longest context, with a per-slot length mask. Idle slots inside the
        # range see one position and their rows are dropped.
        slots, lens = slots.long(), lens.long()
        self.k_cache[slots, :, lens - 1] = k
        self.v_cache[slots, :, lens - 1] = v
        lo, hi, lmax = ctx.kv_lo, ctx.kv_hi, int(ctx.max_seqlen_k)
        rel = slots - lo
        qf = q.new_zeros((hi - lo, self.num_kv_heads, group, self.head_dim))
        qf[rel] = q.view(-1, self.num_kv_heads, group, self.head_dim)
        lf = torch.ones(hi - lo, dtype=lens.dtype, device=lens.device)
        lf[rel] = lens
        kc = self.k_cache[lo:hi, :, :lmax]
        vc = self.v_cache[lo:hi, :, :lmax]
        s = torch.matmul(qf, kc.transpose(-1, -2)).float() * self.scale  # [S, Hkv, G, L]
        valid = torch.arange(lmax, device=q.device)[None, :] < lf[:, None]
        s.masked_fill_(~valid[:, None, None, :], float("-inf"))
        p = torch.softmax(s, dim=-1).to(q.dtype)
        o = torch.matmul(p, vc)  # [S, Hkv, G, D]
        return o[rel].reshape(-1, self.num_heads, self.head_dim)


class Qwen3Attention(nn.Module):
    def __init__(self, cfg: Qwen3Config, quantization: str | None):
        super().__init__()
        from nanovllm.layers.linear import _tp
        _, tp = _tp()
        self.num_heads = cfg.num_attention_heads // tp
        self.num_kv_heads = cfg.num_key_value_heads // tp
        self.head_dim = cfg.head_dim
        self.q_size = self.num_heads * self.head_dim
        self.kv_size = self.num_kv_heads * self.head_dim
        self.qkv_proj = QKVParallelLinear(cfg.hidden_size, cfg.head_dim, cfg.num_attention_heads,
                                          cfg.num_key_value_heads, bias=cfg.attention_bias, quantization=quantization)
        self.o_proj = RowParallelLinear(cfg.num_attention_heads * cfg.head_dim, cfg.hidden_size, bias=False,
                                        quantization=quantization)
        self.rotary_emb = RotaryEmbedding(cfg.head_dim, cfg.max_position_embeddings, cfg.rope_theta)
        self.attn = Attention(self.num_heads, self.num_kv_heads, self.head_dim)
        self.fuse_quant = quantization == "w8a8"
        self.qk_norm = not cfg.attention_bias
        if self.qk_norm:
            self.q_norm = RMSNorm(cfg.head_dim, cfg.rms_norm_eps)
            self.k_norm = RMSNorm(cfg.head_dim, cfg.rms_norm_eps)

    def forward(self, positions: torch.Tensor, x) -> torch.Tensor:
        qkv = self.qkv_proj(x)
        if qkv.is_cuda:
            # fused per-head q/k RMSNorm + rotary (one HIP launch); v stays a view
            qw = self.q_norm.weight if self.qk_norm else None
            kw = self.k_norm.weight if self.qk_norm else None
            eps = self.q_norm.eps if self.qk_norm else 0.0
            ctx = get_context()
            store = ctx.is_prefill and ctx.token_slots is not None and self.attn.k_cache is not None
            q, k = _hip.qk_norm_rope(qkv, positions, self.rotary_emb.cos, self.rotary_emb.sin, qw, kw, eps,
                                     self.num_heads, self.num_kv_heads, self.head_dim,
                                     self.attn.k_cache if store else None, self.attn.v_cache if store else None,
                                     ctx.token_slots if store else None)
            v = qkv[:, self.q_size + self.kv_size:].view(-1, self.num_kv_heads, self.head_dim)
        else:
            q, k, v = qkv.split([self.q_size, self.kv_size, self.kv_size], dim=-1)
            q = q.reshape(-1, self.num_heads, self.head_dim)
            k = k.reshape(-1, self.num_kv_heads, self.head_dim)
            v = v.reshape(-1, self.num_kv_heads, self.head_dim)
            if self.qk_norm:
                q, k = self.q_norm(q), self.k_norm(k)
            q, k = self.rotary_emb(positions, q, k)
        if self.fuse_quant and q.is_cuda and _get_w8a8_backend_preference() == "native":
            # W8A8: o_proj's per-token quantization happens inside the attention kernel
            return self.o_proj(self.attn(q, k, v, quant=True))
        o = self.attn(q, k, v)
        return self.o_proj(o.reshape(-1, self.q_size))


class Qwen3MLP(nn.Module):
    def __init__(self, cfg: Qwen3Config, quantization: str | None):
        super().__init__()
        assert cfg.hidden_act == "silu"
        self.gate_up_proj = MergedColumnParallelLinear(cfg.hidden_size, [cfg.intermediate_size] * 2,
                                                       quantization=quantization)
        self.down_proj = RowParallelLinear(cfg.intermediate_size, cfg.hidden_size, quantization=quantization)
        self.act_fn = SiluAndMul()
        self.fuse_quant = quantization == "w8a8"

    # W8A8 prefill: at this many tokens the gate_up GEMM runs its 256x256
    # tiles anyway, and the SiLU-and-mul moves into its epilogue (the [M, 2I]
    # gate_up output never reaches HBM; the result is bit-identical).
    GLU_MIN_TOKENS = 4096

    def glu_shape_ok(self) -> bool:
        """The fused gate_up kernel needs K % 128 == 0 (K <= 2^22) and the
        intermediate size a multiple of 32 (its 32-row gate/up blocks); other
        shapes take the unfused path."""
        n2, k = self.gate_up_proj.qweight.shape
        return k % 128 == 0 and k <= (1 << 22) and n2 % 64 == 0

    def forward(self, x) -> torch.Tensor:
        if (self.fuse_quant and isinstance(x, QuantizedActivation) and x.is_cuda and
                x.xq.shape[0] >= self.GLU_MIN_TOKENS and _get_w8a8_backend_preference() == "native"
                and self.glu_shape_ok()):
            return self.down_proj(self._glu_quant(x))
        return self.down_proj(self.act_fn(self.gate_up_proj(x), quant=self.fuse_quant))

    def _glu_key(self) -> tuple:
        """Identity of gate_up's current weights: the parameter objects
        themselves (re-assignment), their storage and in-place versions, and
        the layer's loader counter (loaders write through .data, which does
        not advance _version)."""
        lin = self.gate_up_proj
        return (id(lin.qweight), id(lin.w_scales), lin.qweight.data_ptr(), lin.w_scales.data_ptr(),
                lin.qweight._version, lin.w_scales._version, lin.weights_generation)

    def _glu_quant(self, x: "QuantizedActivation") -> "QuantizedActivation":
        lin = self.gate_up_proj
        # gate/up rows regrouped once per weight state (an extra copy of
        # gate_up's weights; the decode path keeps the original layout). The
        # cache holds the parameters it was built from, so their ids cannot
        # be reused by new tensors while it is alive; load_weights also drops it.
        key = self._glu_key()
        cache = getattr(self, "_glu_weights", None)
        if cache is None or cache[0] != key or cache[3] is not lin.qweight or cache[4] is not lin.w_scales:
            cache = (key, *_hip.glu_interleave(lin.qweight.data, lin.w_scales.data), lin.qweight, lin.w_scales)
            self._glu_weights = cache
        h = _hip.w8a8_gemm_glu(x.xq, x.scales, cache[1], cache[2], out_dtype=x.dtype)
        q, s = _hip.act_quant(h)
        return QuantizedActivation(q, s, x.dtype, (*x.shape[:-1], h.shape[-1]))


class Qwen3DecoderLayer(nn.Module):
    def __init__(self, cfg: Qwen3Config, quantization: str | None):
        super().__init__()
        self.self_attn = Qwen3Attention(cfg, quantization)
        self.mlp = Qwen3MLP(cfg, quantization)
        self.input_layernorm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        self.post_attention_layernorm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        # W8A8: the norms emit int8 codes + per-token scales for qkv_proj and
        # gate_up_proj directly (fused producer quantization).
        self.fuse_quant = quantization == "w8a8"

    def forward(self, positions, h, residual):
        q = self.fuse_quant
        if residual is None:
            h, residual = self.input_layernorm(h, quant=q), h
        else:
            h, residual = self.input_layernorm(h, residual, quant=q)
        h = self.self_attn(positions, h)
        h, residual = self.post_attention_layernorm(h, residual, quant=q)
        return self.mlp(h), residual


class Qwen3ForCausalLM(nn.Module):
    packed_modules_mapping = {
        "q_proj": ("qkv_proj", "q"), "k_proj": ("qkv_proj", "k"), "v_proj": ("qkv_proj", "v"),
        "gate_proj": ("gate_up_proj", 0), "up_proj": ("gate_up_proj", 1),
    }

    def __init__(self, cfg: Qwen3Config, quantization: str | None = None):
        super().__init__()
        self.config = cfg
        self.model = nn.Module()
        self.model.embed_tokens = nn.Embedding(cfg.vocab_size, cfg.hidden_size)
        self.model.layers = nn.ModuleList([Qwen3DecoderLayer(cfg, quantization) for _ in range(cfg.num_hidden_layers)])
        self.model.norm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        self.lm_head = nn.Linear(cfg.hidden_size, cfg.vocab_size, bias=False)
        if cfg.tie_word_embeddings:
            self.lm_head.weight = self.model.embed_tokens.weight

    def forward(self, input_ids: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        h = self.model.embed_tokens(input_ids)
        residual = None
        for layer in self.model.layers:
            h, residual = layer(positions, h, residual)
        h, _ = self.model.norm(h, residual)
        return h

    def compute_logits(self, hidden: torch.Tensor) -> torch.Tensor:
        return self.lm_head(hidden)
