"""GPU parity of the fused per-head q/k RMSNorm + rotary kernel
(tvq_qk_norm_rope) against the reference's torch ops run on the CPU in fp32
(RMSNorm.rms_forward, layernorm.py:16-26, then apply_rotary_emb,
rotary_embedding.py:6-14): bit-exact on >= 99 % of elements. Elsewhere the
difference is one rounding flip of a normalised value (the device takes the
fp32 statistic in another order), carried through the rotation: within
2 ulps of the output plus one ulp of the head's largest value (a rotation can
cancel, so the flip is bounded by its input's scale, not the output's)."""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def _ref(qkv, pos, cos, sin, qw, kw, eps, hq, hkv, d):
    t = qkv.shape[0]
    q = qkv[:, : hq * d].reshape(t, hq, d)
    k = qkv[:, hq * d: (hq + hkv) * d].reshape(t, hkv, d)

    def norm(x, w):
        xf = x.float()
        y = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype)
        return y * w

    def rot(x):
        c, s = cos[pos].unsqueeze(1), sin[pos].unsqueeze(1)
        x1, x2 = x.float().chunk(2, -1)
        return torch.cat((x1 * c - x2 * s, x2 * c + x1 * s), -1).to(x.dtype)

    if qw is not None:
        q, k = norm(q, qw), norm(k, kw)
    return rot(q), rot(k)


@pytest.mark.parametrize("norm", [True, False])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("t,hq,hkv", [(1, 16, 8), (37, 16, 8), (300, 32, 8)])
def test_qk_norm_rope(hiplib, norm, dtype, t, hq, hkv):
    from nanovllm.quantization import _hip
    print(f"CASE qk_norm_rope t={t} hq={hq} hkv={hkv} dtype={dtype} norm={norm}", flush=True)
    d, max_pos = 128, 4096
    g = torch.Generator().manual_seed(t + hq)
    qkv = (torch.randn(t, (hq + 2 * hkv) * d + 8, generator=g) * 2).to(dtype)[:, : (hq + 2 * hkv) * d]
    pos = torch.randint(0, max_pos, (t,), generator=g)
    inv = 1.0 / (1e6 ** (torch.arange(0, d, 2, dtype=torch.float) / d))
    fr = torch.outer(torch.arange(max_pos, dtype=torch.float), inv)
    cos, sin = fr.cos(), fr.sin()
    qw = (torch.rand(d, generator=g) + 0.5).to(dtype) if norm else None
    kw = (torch.rand(d, generator=g) + 0.5).to(dtype) if norm else None
    rq, rk = _ref(qkv, pos, cos, sin, qw, kw, 1e-6, hq, hkv, d)
    buf = qkv.cuda()
    q, k = _hip.qk_norm_rope(buf, pos.cuda(), cos.cuda(), sin.cuda(), None if qw is None else qw.cuda(),
                             None if kw is None else kw.cuda(), 1e-6, hq, hkv, d)
    torch.cuda.synchronize()
    for got, ref in ((q.cpu(), rq), (k.cpu(), rk)):
        gf, rf = got.float(), ref.float()
        ulp = torch.where(rf == 0, torch.full_like(rf, 1e-30),
                          torch.exp2(torch.floor(torch.log2(rf.abs().clamp_min(1e-30))) - (7 if dtype == torch.bfloat16 else 10)))
        head_ulp = rf.abs().amax(-1, keepdim=True) * 2.0 ** (-7 if dtype == torch.bfloat16 else -10)
        assert torch.all((gf - rf).abs() <= 2.0001 * ulp + head_ulp + 1e-6)
        assert (gf == rf).float().mean() >= 0.99


def test_qk_norm_rope_stores_prompt_kv(hiplib):
    """With caches given, every token's rotated key and its value land at
    (slot, position); tokens with an out-of-range slot or position are not
    stored and nothing else in the caches changes."""
    from nanovllm.quantization import _hip
    t, hq, hkv, d, n_slots, max_len = 40, 16, 8, 128, 5, 64
    g = torch.Generator(device="cuda").manual_seed(7)
    qkv = torch.randn(t, (hq + 2 * hkv) * d, device="cuda", generator=g).bfloat16()
    pos = torch.cat([torch.arange(20), torch.arange(17), torch.tensor([63, 64, 5])]).cuda()
    slots = torch.tensor([3] * 20 + [0] * 17 + [4, 4, 9], dtype=torch.int64, device="cuda")
    inv = 1.0 / (1e6 ** (torch.arange(0, d, 2, dtype=torch.float) / d))
    fr = torch.outer(torch.arange(128, dtype=torch.float), inv)
    cos, sin = fr.cos().cuda(), fr.sin().cuda()
    w = torch.ones(d, device="cuda").bfloat16()
    kc = torch.randn(n_slots, hkv, max_len, d, device="cuda", generator=g).bfloat16()
    vc = torch.randn(n_slots, hkv, max_len, d, device="cuda", generator=g).bfloat16()
    kc0, vc0 = kc.clone(), vc.clone()
    q, k = _hip.qk_norm_rope(qkv, pos, cos, sin, w, w, 1e-6, hq, hkv, d, kc, vc, slots)
    q2, k2 = _hip.qk_norm_rope(qkv, pos, cos, sin, w, w, 1e-6, hq, hkv, d)
    torch.cuda.synchronize()
    assert torch.equal(q, q2) and torch.equal(k, k2)
    v = qkv[:, (hq + hkv) * d:].view(t, hkv, d)
    ek, ev = kc0.clone(), vc0.clone()
    for i in range(t):
        s, p = int(slots[i]), int(pos[i])
        if 0 <= s < n_slots and 0 <= p < max_len:
            ek[s, :, p] = k[i]
            ev[s, :, p] = v[i]
    assert torch.equal(kc, ek) and torch.equal(vc, ev)
