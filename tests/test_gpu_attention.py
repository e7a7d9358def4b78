"""GPU tests of the decode-attention kernel (tvq_decode_attention) against a
plain PyTorch fp32 reference of the reference's decode step
(attention.py:59-88: store_kvcache, then flash_attn_with_kvcache with
cache_seqlens, causal): the appended K/V row is bit-exact, every other cache
entry is untouched, and the output is within bf16 rounding of the fp32
reference (max-abs <= 1e-2 * max|ref| + 1e-3)."""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def _ref(q, kc, vc, slots, lens, scale):
    out = []
    hq, hkv = q.shape[1], kc.shape[1]
    for b in range(q.shape[0]):
        n = int(lens[b])
        k = kc[int(slots[b]), :, :n].float().repeat_interleave(hq // hkv, 0)  # [Hq, n, D]
        v = vc[int(slots[b]), :, :n].float().repeat_interleave(hq // hkv, 0)
        p = torch.softmax((q[b].float()[:, None, :] @ k.transpose(1, 2)).squeeze(1) * scale, -1)  # [Hq, n]
        out.append((p[:, None, :] @ v).squeeze(1))
    return torch.stack(out)


@pytest.mark.parametrize("hq,hkv", [(16, 8), (32, 8), (8, 8)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_decode_attention_matches_fp32_reference(hiplib, hq, hkv, dtype):
    from nanovllm.quantization import _hip
    print(f"CASE decode_attention hq={hq} hkv={hkv} dtype={dtype}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(hq * 10 + hkv)
    n_slots, max_len, d = 12, 1100, 128
    kc = torch.randn(n_slots, hkv, max_len, d, device="cuda", generator=g).to(dtype)
    vc = torch.randn(n_slots, hkv, max_len, d, device="cuda", generator=g).to(dtype)
    lens_l = [1, 2, 17, 16, 33, 100, 1000, 1100, 257]
    slots_l = [3, 0, 11, 5, 7, 1, 2, 9, 10]
    b = len(lens_l)
    # q / k / v as strided views of a packed qkv row, as the model produces them
    qkv = torch.randn(b, (hq + 2 * hkv) * d, device="cuda", generator=g).to(dtype)
    q = qkv[:, : hq * d].view(b, hq, d)
    k = qkv[:, hq * d: (hq + hkv) * d].view(b, hkv, d)
    v = qkv[:, (hq + hkv) * d:].view(b, hkv, d)
    slots = torch.tensor(slots_l, dtype=torch.int32, device="cuda")
    lens = torch.tensor(lens_l, dtype=torch.int32, device="cuda")
    kc0, vc0 = kc.clone(), vc.clone()
    scale = d ** -0.5
    out = _hip.decode_attention(q, k, v, kc, vc, slots, lens, scale)
    torch.cuda.synchronize()
    # cache: new rows appended, everything else unchanged
    exp_k, exp_v = kc0.clone(), vc0.clone()
    for i in range(b):
        exp_k[slots_l[i], :, lens_l[i] - 1] = k[i]
        exp_v[slots_l[i], :, lens_l[i] - 1] = v[i]
    assert torch.equal(kc, exp_k) and torch.equal(vc, exp_v)
    ref = _ref(q, exp_k, exp_v, slots, lens, scale)
    err = (out.float() - ref).abs().max().item()
    assert err <= 1e-2 * ref.abs().max().item() + 1e-3, err


def test_decode_attention_invalid_metadata_is_inert(hiplib):
    from nanovllm.quantization import _hip
    kc = torch.randn(2, 8, 64, 128, device="cuda").bfloat16()
    vc = torch.randn(2, 8, 64, 128, device="cuda").bfloat16()
    kc0, vc0 = kc.clone(), vc.clone()
    q = torch.randn(3, 16, 128, device="cuda").bfloat16()
    k = torch.randn(3, 8, 128, device="cuda").bfloat16()
    slots = torch.tensor([0, 5, 1], dtype=torch.int32, device="cuda")   # slot 5 out of range
    lens = torch.tensor([65, 3, 0], dtype=torch.int32, device="cuda")   # 65 > max_len, 0 < 1
    out = _hip.decode_attention(q, k, k, kc, vc, slots, lens, 0.1)
    torch.cuda.synchronize()
    assert torch.equal(kc, kc0) and torch.equal(vc, vc0)
    assert torch.count_nonzero(out) == 0


def test_decode_attention_in_graph_replays(hiplib):
    """Captured once, replayed with new lengths written into the same buffers."""
    from nanovllm.quantization import _hip
    kc = torch.randn(4, 8, 256, 128, device="cuda").bfloat16()
    vc = torch.randn(4, 8, 256, 128, device="cuda").bfloat16()
    q = torch.randn(4, 16, 128, device="cuda").bfloat16()
    k = torch.randn(4, 8, 128, device="cuda").bfloat16()
    v = torch.randn(4, 8, 128, device="cuda").bfloat16()
    slots = torch.tensor([0, 1, 2, 3], dtype=torch.int32, device="cuda")
    lens = torch.tensor([5, 6, 7, 8], dtype=torch.int32, device="cuda")
    out = torch.empty_like(q)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        _hip.decode_attention(q, k, v, kc, vc, slots, lens, 0.088, out=out)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _hip.decode_attention(q, k, v, kc, vc, slots, lens, 0.088, out=out)
    for step in range(3):
        lens.copy_(torch.tensor([9 + step, 100 + step, 33, 200 + step], dtype=torch.int32))
        graph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        ref = _hip.decode_attention(q, k, v, kc.clone(), vc.clone(), slots, lens, 0.088)
        torch.cuda.synchronize()
        assert torch.equal(got, ref)


def _prefill_ref(q, k, v, lens, scale):
    out = torch.empty_like(q, dtype=torch.float32)
    hq, hkv = q.shape[1], k.shape[1]
    off = 0
    for n in lens:
        qq = q[off:off + n].float().transpose(0, 1)                                # [Hq, n, D]
        kk = k[off:off + n].float().transpose(0, 1).repeat_interleave(hq // hkv, 0)
        vv = v[off:off + n].float().transpose(0, 1).repeat_interleave(hq // hkv, 0)
        s = qq @ kk.transpose(1, 2) * scale
        s.masked_fill_(torch.ones(n, n, dtype=torch.bool, device=q.device).triu(1), float("-inf"))
        out[off:off + n] = (torch.softmax(s, -1) @ vv).transpose(0, 1)
        off += n
    return out


@pytest.mark.parametrize("hq,hkv", [(16, 8), (32, 8), (8, 8), (24, 4), (6, 2)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prefill_attention_matches_fp32_reference(hiplib, hq, hkv, dtype):
    from nanovllm.quantization import _hip
    print(f"CASE prefill_attention hq={hq} hkv={hkv} dtype={dtype}", flush=True)
    lens = [1, 5, 64, 65, 100, 300, 1024, 17, 128, 129, 255]
    t, d = sum(lens), 128
    g = torch.Generator(device="cuda").manual_seed(hq + hkv)
    q = torch.randn(t, hq, d, device="cuda", generator=g).to(dtype)
    k = torch.randn(t, hkv, d, device="cuda", generator=g).to(dtype)
    qkv = torch.randn(t, (hq + 2 * hkv) * d, device="cuda", generator=g).to(dtype)
    v = qkv[:, (hq + hkv) * d:].view(t, hkv, d)          # strided view, as the model passes it
    offs, o = [], 0
    for n in lens:
        offs.append((o, n))
        o += n
    blocks = _hip.prefill_blocks(offs).cuda()
    scale = d ** -0.5
    out = _hip.prefill_attention(q, k, v, blocks, scale)
    torch.cuda.synchronize()
    ref = _prefill_ref(q, k, v, lens, scale)
    err = (out.float() - ref).abs()
    # P is rounded to the input dtype before the value product (as flash attention does)
    tol = (1.5e-2 if dtype == torch.bfloat16 else 4e-3) * ref.abs().amax() + 1e-3
    assert err.max().item() <= tol, (err.max().item(), tol)
    assert ((out.float() - ref).norm() / ref.norm()).item() < (8e-3 if dtype == torch.bfloat16 else 2e-3)


# ---------------------------------------------------------------- o_proj's quantization fused

@pytest.mark.parametrize("hq,hkv", [(16, 8), (32, 8), (8, 8), (24, 4), (6, 2)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prefill_attention_quant_matches_plain_and_act_quant(hiplib, hq, hkv, dtype):
    """tvq_prefill_attention_quant: the same output as tvq_prefill_attention,
    int8 codes and scales bit-identical to tvq_act_quant of that output (and
    to the oracle), counters zero afterwards; two calls in a row, the second
    smaller."""
    import numpy as np

    import oracle
    from nanovllm.quantization import _hip
    d = 128
    for lens in ([1, 5, 64, 65, 100, 300, 1024, 17, 128, 129, 255], [3, 70]):
        print(f"CASE prefill_attention_quant hq={hq} hkv={hkv} dtype={dtype} lens={lens}", flush=True)
        t = sum(lens)
        g = torch.Generator(device="cuda").manual_seed(hq + hkv + t)
        q = torch.randn(t, hq, d, device="cuda", generator=g).to(dtype)
        k = torch.randn(t, hkv, d, device="cuda", generator=g).to(dtype)
        qkv = torch.randn(t, (hq + 2 * hkv) * d, device="cuda", generator=g).to(dtype)
        v = qkv[:, (hq + hkv) * d:].view(t, hkv, d)
        offs, o = [], 0
        for n in lens:
            offs.append((o, n))
            o += n
        blocks = _hip.prefill_blocks(offs).cuda()
        ref = _hip.prefill_attention(q, k, v, blocks, d ** -0.5)
        out, xq, xs = _hip.prefill_attention_quant(q, k, v, blocks, d ** -0.5)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
        rq, rs = _hip.act_quant(ref.view(t, -1))
        assert torch.equal(xq, rq) and torch.equal(xs.view(torch.int32), rs.view(torch.int32))
        oq, os_ = oracle.c_act_quant(ref.view(t, -1).cpu().view(torch.int16).numpy().view(np.uint16),
                                     is_bf16=dtype == torch.bfloat16)
        np.testing.assert_array_equal(xq.cpu().numpy(), oq)
        assert int(_hip.attn_counters(torch.device("cuda", 0)).abs().sum()) == 0


@pytest.mark.parametrize("hq,hkv", [(16, 8), (32, 8), (8, 8)])
def test_decode_attention_quant_matches_plain_and_act_quant(hiplib, hq, hkv):
    from nanovllm.quantization import _hip
    print(f"CASE decode_attention_quant hq={hq} hkv={hkv}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(hq + 7 * hkv)
    n_slots, max_len, d, dtype = 12, 1100, 128, torch.bfloat16
    kc0 = torch.randn(n_slots, hkv, max_len, d, device="cuda", generator=g).to(dtype)
    vc0 = torch.randn(n_slots, hkv, max_len, d, device="cuda", generator=g).to(dtype)
    lens_l = [1, 2, 17, 16, 33, 100, 1000, 1100, 257, 0]   # the last sequence is invalid
    slots_l = [3, 0, 11, 5, 7, 1, 2, 9, 10, 4]
    b = len(lens_l)
    qkv = torch.randn(b, (hq + 2 * hkv) * d, device="cuda", generator=g).to(dtype)
    q = qkv[:, : hq * d].view(b, hq, d)
    k = qkv[:, hq * d: (hq + hkv) * d].view(b, hkv, d)
    v = qkv[:, (hq + hkv) * d:].view(b, hkv, d)
    slots = torch.tensor(slots_l, dtype=torch.int32, device="cuda")
    lens = torch.tensor(lens_l, dtype=torch.int32, device="cuda")
    kc, vc = kc0.clone(), vc0.clone()
    ref = _hip.decode_attention(q, k, v, kc, vc, slots, lens, d ** -0.5)
    kc2, vc2 = kc0.clone(), vc0.clone()
    out, xq, xs = _hip.decode_attention_quant(q, k, v, kc2, vc2, slots, lens, d ** -0.5)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    assert torch.equal(kc, kc2) and torch.equal(vc, vc2)
    rq, rs = _hip.act_quant(ref.view(b, -1))
    assert torch.equal(xq, rq) and torch.equal(xs.view(torch.int32), rs.view(torch.int32))
    assert int(_hip.attn_counters(torch.device("cuda", 0)).abs().sum()) == 0


def test_decode_attention_quant_in_graph_replays(hiplib):
    """Captured with its counters allocated beforehand, the quantizing decode
    attention replays with new lengths exactly as eager calls do."""
    from nanovllm.quantization import _hip
    print("CASE decode_attention_quant graph", flush=True)
    hq, hkv, d, n_slots, max_len = 16, 8, 128, 4, 512
    g = torch.Generator(device="cuda").manual_seed(11)
    kc = torch.randn(n_slots, hkv, max_len, d, device="cuda", generator=g).to(torch.bfloat16)
    vc = torch.randn(n_slots, hkv, max_len, d, device="cuda", generator=g).to(torch.bfloat16)
    q = torch.randn(4, hq, d, device="cuda", generator=g).to(torch.bfloat16)
    k = torch.randn(4, hkv, d, device="cuda", generator=g).to(torch.bfloat16)
    v = torch.randn(4, hkv, d, device="cuda", generator=g).to(torch.bfloat16)
    slots = torch.tensor([0, 1, 2, 3], dtype=torch.int32, device="cuda")
    lens = torch.tensor([5, 9, 100, 1], dtype=torch.int32, device="cuda")
    _hip.attn_counters(torch.device("cuda", 0))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        _hip.decode_attention_quant(q, k, v, kc.clone(), vc.clone(), slots, lens, 0.088)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    kg, vg = kc.clone(), vc.clone()
    with torch.cuda.graph(graph):
        got = _hip.decode_attention_quant(q, k, v, kg, vg, slots, lens, 0.088)
    for new_lens in ([5, 9, 100, 1], [300, 2, 7, 512], [1, 1, 1, 1]):
        lens.copy_(torch.tensor(new_lens, dtype=torch.int32))
        graph.replay()
        torch.cuda.synchronize()
        ref = _hip.decode_attention_quant(q, k, v, kg.clone(), vg.clone(), slots, lens, 0.088)
        torch.cuda.synchronize()
        for a, b in zip(got, ref):
            assert torch.equal(a.view(torch.uint8) if a.dtype != torch.int8 else a,
                               b.view(torch.uint8) if b.dtype != torch.int8 else b)

