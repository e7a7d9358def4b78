"""A case of every kernel family on the CPU emulation, with parity checks,
run by tests/test_cpu_emu_kernels.py in child processes (test
infrastructure), because the emulation's modes are fixed per process:

  --asan   the AddressSanitizer build, with the ASan runtime preloaded. Every
           buffer is a CPU tensor of exactly its size, so a read or write past
           any input, output, workspace or dynamic LDS allocation aborts.
  --race   the race-checking build (tests/cpu_emu/racecheck.h), with
           EMU_DMA=late: an access that the GPU does not order against a
           conflicting one (a missing barrier between waves, a read of LDS
           before its DMA landed, two workgroups of a launch touching the same
           memory non-atomically) is reported on stderr and fails the run.
  (plain)  run with EMU_CONCURRENT=32 (workgroups interleaved),
           EMU_SHUFFLE=seed (random order, random stalls) and optionally
           EMU_DMA=late (each LDS DMA lands only at its wave's vmcnt wait): a
           missing DMA wait, a cross-wave race or an arrival-order assumption
           between workgroups shows as a parity failure.

Prints "all cases passed" at the end."""
from __future__ import annotations

import ctypes
import os
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path[:0] = [str(ROOT), str(ROOT / "tiny-vllm_amd"), str(HERE)]

import numpy as np  # noqa: E402
import torch  # noqa: E402

import emu  # noqa: E402
import oracle  # noqa: E402
from tests.helpers import bits16, make_activations, make_weights  # noqa: E402

CFG = dict(kI8_256x256=0, kI8_256x128=1, kI8_64x64=2, kI8_64x128=3, kI8_32x64=4, kH_128x256=5, kH_64x128=6,
           kH_64x64=7, kH_32x64=8, kH_64x128w8=9, kI8_256x256w4=10, kH_128x256w4=11, kH_16x128=12,
           kH_64x256=13, kH_32x256=14)


class _NoDevice:
    def __init__(self, *a, **k):
        pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        return False


def _w8a16_ok(y, x, q, s, bias=None) -> None:
    """Within the GPU tests' bound of the exact fp64 product."""
    y64 = oracle.c_w8a16_f64(bits16(x), q.numpy(), s.numpy(), None if bias is None else bias.float().numpy(),
                             is_bf16=x.dtype == torch.bfloat16)
    mag = (np.abs(x.float().numpy()).astype(np.float64) @ np.abs(q.numpy()).astype(np.float64).T) * s.numpy()[None]
    bound = np.abs(y64) * 2.0 ** -8 + mag * (x.shape[1] * 2.0 ** -23) + 1e-30
    assert np.all(np.abs(y.float().numpy().astype(np.float64) - y64) <= bound)


def _w8a8_ok(y, xq, a_s, q, s, bias=None) -> None:
    """Bit-exact against the restated reference epilogue."""
    xq, a_s = np.asarray(xq), np.asarray(a_s)
    yb, _ = oracle.c_w8a8_epilogue(oracle.c_gemm_i32(xq, q.numpy()), a_s, s.numpy(),
                                   None if bias is None else bias.float().numpy())
    assert np.array_equal(bits16(y), yb)


def _arg(flag: str) -> str | None:
    return sys.argv[sys.argv.index(flag) + 1] if flag in sys.argv else None


def main() -> None:
    lib_file = _arg("--lib")
    lib = emu.load_file(lib_file) if lib_file else emu.load(asan="--asan" in sys.argv, race="--race" in sys.argv)
    only = _arg("--only")
    only = only.split(",") if only else None
    from nanovllm.quantization import _hip
    n_ws = lib.tvq_gemm_workspace_bytes()
    raw = torch.zeros(n_ws + 256, dtype=torch.uint8)
    off = (-raw.data_ptr()) % 256
    ws = raw[off:off + n_ws]
    _hip.load_library = lambda: lib
    _hip._require_gpu = lambda *ts: torch.device("cpu")
    _hip._stream = lambda dev: None
    _hip.gemm_workspace = lambda dev: ws
    torch.cuda.device = _NoDevice
    force = ctypes.c_int.in_dll(lib, "tvq_test_force_dma_cfg")

    def case(name) -> bool:
        """Announce a case; False when --only leaves it out."""
        if only is not None and not any(name.startswith(o) for o in only):
            return False
        print("CASE", name, flush=True)
        return True

    # act-quant: vector (1, 2 and 4 waves per row) and scalar paths
    for m, k in [(3, 1024), (600, 64), (1030, 64), (5, 100), (2, 16384)]:
        if not case(f"act_quant {m}x{k}"):
            continue
        x = make_activations(m, k, seed=m)
        q, s = _hip.act_quant(x)
        rq, rs = oracle.c_act_quant(bits16(x))
        assert np.array_equal(q.numpy(), rq) and np.array_equal(s.numpy(), rs)

    # GEMMs through the default dispatch (GEMV, skinny, DMA, split-K, generic)
    for m, n, k in [(1, 64, 2048), (2, 72, 1024), (9, 96, 256), (40, 136, 512), (64, 128, 4096), (300, 130, 1024),
                    (7, 33, 40), (17, 16384, 128)]:
        if not case(f"gemm {m}x{n}x{k}"):
            continue
        x = make_activations(m, k, seed=n)
        q, s = make_weights(n, k, seed=k)
        bias = torch.randn(n).to(torch.bfloat16)
        _w8a16_ok(_hip.w8a16_gemm(x, q, s, bias), x, q, s, bias)
        _hip.w8a16_gemm_rounded(x, q, s, bias)
        y = _hip.w8a8_linear(x, q, s, bias)
        xq, a_s = oracle.c_act_quant(bits16(x))
        _w8a8_ok(y, xq, a_s, q, s, bias)
        acc = _hip.w8a8_gemm_i32(torch.from_numpy(xq), q)
        assert np.array_equal(acc.numpy(), oracle.c_gemm_i32(xq, q.numpy()))

    # every DMA tile configuration, ragged, one and several tiles per workgroup
    for name, c in CFG.items():
        bm = int(name.split("_")[1].split("x")[0])
        bn = int(name.split("x")[1].rstrip("w48"))
        for cus in ("256", "3"):
            m, n, k = bm + bm // 2 + 3, 2 * bn + 40, 384
            if not case(f"dma {name} cus={cus} {m}x{n}x{k}"):
                continue
            os.environ["EMU_CUS"] = cus
            force.value = c
            x = make_activations(m, k, seed=c)
            q, s = make_weights(n, k, seed=c + 1)
            bias = torch.randn(n).to(torch.bfloat16)
            if name.startswith("kI8"):
                xq, a_s = _hip.act_quant(x)
                y = _hip.w8a8_gemm(xq, a_s, q, s, bias, torch.bfloat16, split_k=False)
                _w8a8_ok(y, xq, a_s, q, s, bias)
                _hip.gemm_operand_floor(_hip.OP_W8A8, xq, q)
            else:
                _w8a16_ok(_hip.w8a16_gemm(x, q, s, bias, split_k=False), x, q, s, bias)
                _hip.gemm_operand_floor(_hip.OP_W8A16, x, q)
            force.value = -1
    os.environ["EMU_CUS"] = "256"

    # stream-K (opt-in)
    os.environ["TVQ_STREAMK"] = "1"
    os.environ["TVQ_STREAMK_MIN"] = "2"
    os.environ["EMU_CUS"] = "5"
    for m, n, k in [(1, 512, 1024), (16, 384, 2048), (33, 1280, 512)]:
        if not case(f"streamk {m}x{n}x{k}"):
            continue
        x = make_activations(m, k, seed=m)
        q, s = make_weights(n, k, seed=n)
        _w8a16_ok(_hip.w8a16_gemm(x, q, s), x, q, s)
        xq, a_s = oracle.c_act_quant(bits16(x))
        _w8a8_ok(_hip.w8a8_linear(x, q, s), xq, a_s, q, s)
    for v in ("TVQ_STREAMK", "TVQ_STREAMK_MIN"):
        del os.environ[v]
    os.environ["EMU_CUS"] = "256"

    # producers and the gate_up epilogue
    for m, k in [(7, 1024), (600, 256), (9, 1003)]:
        if not case(f"producers {m}x{k}"):
            continue
        x = make_activations(m, k, seed=k)
        res = make_activations(m, k, seed=k + 1)
        _hip.rmsnorm(x, torch.ones(k, dtype=torch.bfloat16), 1e-6, residual=res, out=True, quant=True)
        _hip.silu_mul(make_activations(m, 2 * k, seed=m), out=True, quant=True)
    if case("glu"):
        from nanovllm.quantization.utils import quantize_int8_per_channel
        qw, s = quantize_int8_per_channel(torch.randn(320, 384) * 0.02)
        xq, a_s = _hip.act_quant(make_activations(300, 384, seed=1))
        q2, s2 = _hip.glu_interleave(qw, s.float())
        yref, _ = _hip.silu_mul(_hip.w8a8_gemm(xq, a_s, qw, s.float(), out_dtype=torch.bfloat16, split_k=False))
        assert torch.equal(_hip.w8a8_gemm_glu(xq, a_s, q2, s2), yref)

    # no-alloc entry
    if case("noalloc"):
        x = make_activations(8, 1024, seed=3)
        q, s = make_weights(128, 1024, seed=4)
        y = torch.empty(8, 128, dtype=torch.bfloat16)
        assert lib.tvq_w8a8_linear_noalloc(x.data_ptr(), 1, q.data_ptr(), s.data_ptr(), None, y.data_ptr(), 8, 128,
                                           1024, None) == 0

    # attention and q/k-norm + rotary (exactly sized caches and tensors)
    d = 128
    for hq, hkv in [(4, 2), (8, 2), (2, 2), (6, 2)]:
        if not case(f"prefill_attention {hq}/{hkv}"):
            continue
        lens = [1, 65, 129]
        t = sum(lens)
        q = torch.randn(t, hq, d).to(torch.bfloat16)
        k = torch.randn(t, hkv, d).to(torch.bfloat16)
        v = torch.randn(t, hkv, d).to(torch.bfloat16)
        offs, o = [], 0
        for n in lens:
            offs.append((o, n))
            o += n
        blocks = _hip.prefill_blocks(offs)
        out = torch.empty_like(q)
        assert lib.tvq_prefill_attention(q.data_ptr(), k.data_ptr(), v.data_ptr(), v.stride(0), blocks.data_ptr(),
                                         blocks.shape[0], hq, hkv, d, 0.088, out.data_ptr(), 1, None) == 0
        case(f"prefill_attention_quant {hq}/{hkv}")
        out2 = torch.empty_like(q)
        xq = torch.empty(t, hq * d, dtype=torch.int8)
        xs = torch.empty(t)
        cnt = torch.zeros(blocks.shape[0], dtype=torch.int32)
        assert lib.tvq_prefill_attention_quant(q.data_ptr(), k.data_ptr(), v.data_ptr(), v.stride(0),
                                               blocks.data_ptr(), blocks.shape[0], hq, hkv, d, 0.088,
                                               out2.data_ptr(), 1, xq.data_ptr(), xs.data_ptr(), 1e-8,
                                               cnt.data_ptr(), cnt.numel(), None) == 0
        assert torch.equal(out2.view(torch.int16), out.view(torch.int16))
        rq, rs = oracle.c_act_quant(bits16(out.view(t, -1)))
        assert np.array_equal(xq.numpy(), rq) and np.array_equal(xs.numpy(), rs) and int(cnt.abs().sum()) == 0
    for hq, hkv in [(16, 8), (16, 4)]:
        if not case(f"decode_attention {hq}/{hkv}"):
            continue
        n_slots, max_len, b = 3, 40, 3
        kc = torch.randn(n_slots, hkv, max_len, d).to(torch.bfloat16)
        vc = torch.randn_like(kc)
        q = torch.randn(b, hq, d).to(torch.bfloat16)
        kn = torch.randn(b, hkv, d).to(torch.bfloat16)
        vn = torch.randn(b, hkv, d).to(torch.bfloat16)
        slots = torch.tensor([2, 0, 1], dtype=torch.int32)
        lens = torch.tensor([1, 40, 17], dtype=torch.int32)
        out = torch.empty(b, hq, d, dtype=torch.bfloat16)
        assert lib.tvq_decode_attention(q.data_ptr(), q.stride(0), kn.data_ptr(), kn.stride(0), vn.data_ptr(),
                                        vn.stride(0), kc.data_ptr(), vc.data_ptr(), slots.data_ptr(), lens.data_ptr(),
                                        b, hq, hkv, d, n_slots, max_len, 0.088, out.data_ptr(), 1, None) == 0
        case(f"decode_attention_quant {hq}/{hkv}")
        lens2 = torch.tensor([2, 40, 0], dtype=torch.int32)        # an invalid sequence too
        out2 = torch.empty(b, hq, d, dtype=torch.bfloat16)
        xq = torch.empty(b, hq * d, dtype=torch.int8)
        xs = torch.empty(b)
        cnt = torch.zeros(b, dtype=torch.int32)
        assert lib.tvq_decode_attention_quant(q.data_ptr(), q.stride(0), kn.data_ptr(), kn.stride(0), vn.data_ptr(),
                                              vn.stride(0), kc.data_ptr(), vc.data_ptr(), slots.data_ptr(),
                                              lens2.data_ptr(), b, hq, hkv, d, n_slots, max_len, 0.088,
                                              out2.data_ptr(), 1, xq.data_ptr(), xs.data_ptr(), 1e-8,
                                              cnt.data_ptr(), cnt.numel(), None) == 0
        rq, rs = oracle.c_act_quant(bits16(out2.view(b, -1)))
        assert np.array_equal(xq.numpy(), rq) and np.array_equal(xs.numpy(), rs) and int(cnt.abs().sum()) == 0
    if case("qk_norm_rope"):
        t, hq, hkv, max_pos = 5, 4, 2, 64
        qkv = torch.randn(t, (hq + 2 * hkv) * d).to(torch.bfloat16)
        pos = torch.tensor([0, 3, 63, 7, 9], dtype=torch.int64)
        cos = torch.rand(max_pos, d // 2)
        sin = torch.rand(max_pos, d // 2)
        kc = torch.zeros(2, hkv, max_pos, d, dtype=torch.bfloat16)
        vc = torch.zeros_like(kc)
        slots = torch.tensor([0, 1, 1, 0, 1], dtype=torch.int64)
        qo = torch.empty(t, hq, d, dtype=torch.bfloat16)
        ko = torch.empty(t, hkv, d, dtype=torch.bfloat16)
        w = torch.ones(d, dtype=torch.bfloat16)
        assert lib.tvq_qk_norm_rope(qkv.data_ptr(), qkv.stride(0), pos.data_ptr(), cos.data_ptr(), sin.data_ptr(),
                                    w.data_ptr(), w.data_ptr(), 1e-6, t, hq, hkv, d, max_pos, qo.data_ptr(),
                                    ko.data_ptr(), kc.data_ptr(), vc.data_ptr(), slots.data_ptr(), 2, max_pos, 1,
                                    None) == 0
    if "--race" in sys.argv:
        n = lib.tvq_emu_race_reports()
        assert n == 0, f"{n} race report(s)"
    print("all cases passed", flush=True)


if __name__ == "__main__":
    main()
