"""GPU parity of the stream-K DMA GEMM (TVQ_STREAMK=1) at decode-size M.

Bar: W8A8 int32 accumulators and bf16/fp16 outputs bit-identical to the
unsplit kernel (int32 sums are exact in any order) and to the oracle on
sampled rows; W8A16 outputs equal to the unsplit kernel up to fp32 summation
order, and within the oracle tolerance and fp64 bound.
"""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import bits16, make_activations, make_weights
from tests.test_gpu_parity import _same_up_to_order, _w8a16_check

# Stream-K is opt-in and has not yet run on a GPU: these tests run only when
# asked for (TVQ_RUN_UNVERIFIED=1) until they have passed there once.
pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(os.environ.get("TVQ_RUN_UNVERIFIED") != "1",
                                 reason="stream-K has not yet run on a GPU (opt-in, TVQ_STREAMK=1)")]

# Decode shapes: 8B gate_up / qkv / o / down at M = 64 and 48, Qwen3-0.6B
# shapes (config 1 among them), ragged M and N, and K with few stages.
STREAMK_SHAPES = [(64, 24576, 4096), (64, 6144, 4096), (48, 4096, 4096), (64, 4096, 12288), (64, 6144, 1024),
                  (40, 1000, 2048), (33, 136, 2048), (24, 3072, 1024), (17, 4096, 1024), (64, 2048, 128),
                  (16, 24576, 4096), (8, 4096, 12288), (3, 6144, 4096), (13, 1000, 2048)]


def _log_case(**kw):
    print("CASE", " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


@pytest.fixture
def streamk(monkeypatch):
    monkeypatch.setenv("TVQ_STREAMK", "1")


# Short K with fewer stages per workgroup (TVQ_STREAMK_MIN): tiles of 8 or
# 16 stages are shared by two to eight workgroups.
SHORT_K_CASES = [((64, 6144, 1024), 2), ((24, 3072, 1024), 1), ((17, 4096, 1024), 3), ((64, 1024, 2048), 1)]


@pytest.mark.parametrize("case", SHORT_K_CASES, ids=lambda c: "x".join(map(str, c[0])) + f"-min{c[1]}")
def test_streamk_short_k(hiplib, streamk, monkeypatch, case):
    shape, min_stages = case
    monkeypatch.setenv("TVQ_STREAMK_MIN", str(min_stages))
    test_streamk_matches_unsplit_and_oracle(hiplib, None, shape)


@pytest.mark.parametrize("shape", STREAMK_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_streamk_matches_unsplit_and_oracle(hiplib, streamk, shape):
    from nanovllm.quantization import _hip
    m, n, k = shape
    for op in (_hip.OP_W8A8, _hip.OP_W8A16):
        path = _hip.select_path(op, m, n, k)
        _log_case(test="streamk", m=m, n=n, k=k, path=path)
        assert path.endswith("_streamk"), path
    d = torch.device("cuda", 0)
    x = make_activations(m, k, seed=m + n + k)
    xq, a_s = oracle.c_act_quant(bits16(x))
    q, w_s = make_weights(n, k, seed=m + 7 * n + k)
    xq_d, a_d = torch.from_numpy(xq).to(d), torch.from_numpy(a_s).to(d)
    q_d, w_d = q.to(d), w_s.to(d)
    acc_s = _hip.w8a8_gemm_i32(xq_d, q_d)
    acc_u = _hip.w8a8_gemm_i32(xq_d, q_d, split_k=False)   # no workspace: the same tiles, unsplit
    assert torch.equal(acc_s, acc_u)
    rows = np.unique(np.linspace(0, m - 1, 8).astype(np.int64))
    np.testing.assert_array_equal(acc_s.cpu().numpy()[rows], oracle.c_gemm_i32(xq[rows], q.numpy()))
    for dt in (torch.bfloat16, torch.float16):
        y_s = _hip.w8a8_gemm(xq_d, a_d, q_d, w_d, None, dt)
        y_u = _hip.w8a8_gemm(xq_d, a_d, q_d, w_d, None, dt, split_k=False)
        assert torch.equal(y_s.view(torch.int16), y_u.view(torch.int16))
    ref, _ = oracle.c_w8a8_epilogue(oracle.c_gemm_i32(xq[rows], q.numpy()), a_s[rows], w_s.numpy())
    y_b = _hip.w8a8_gemm(xq_d, a_d, q_d, w_d, None, torch.bfloat16).cpu()
    np.testing.assert_array_equal(bits16(y_b)[rows], ref)
    xh = make_activations(m, k, seed=3 * m + n, outlier_frac=0.0).to(d)
    h_s = _hip.w8a16_gemm(xh, q_d, w_d)
    h_u = _hip.w8a16_gemm(xh, q_d, w_d, split_k=False)
    _same_up_to_order(h_s, h_u, xh, q.numpy(), w_s.numpy())
    t_rows = torch.from_numpy(rows)
    _w8a16_check(h_s.cpu()[t_rows], xh.cpu()[t_rows], q, w_s)


def test_streamk_deterministic_and_counters(hiplib, streamk):
    """Repeated calls give identical bits whatever order the workgroups finish
    in, bias included, and every tile counter is back at zero afterwards."""
    from nanovllm.quantization import _hip
    d = torch.device("cuda", 0)
    qa, sa = (t.to(d) for t in make_weights(24576, 4096, seed=41))
    qb, sb = (t.to(d) for t in make_weights(1000, 2048, seed=42))
    bias = (torch.randn(24576, generator=torch.Generator().manual_seed(43)) * 0.1).to(torch.bfloat16).to(d)
    xa = make_activations(64, 4096, seed=44, outlier_frac=0.0).to(d)
    xb = make_activations(40, 2048, seed=45, outlier_frac=0.0).to(d)
    _log_case(test="streamk_det", path=_hip.select_path(_hip.OP_W8A16, 64, 24576, 4096))
    first_a = _hip.w8a16_gemm(xa, qa, sa, bias)
    first_a8 = _hip.w8a8_linear(xa, qa, sa, bias)
    first_b = _hip.w8a16_gemm(xb, qb, sb)
    for i in range(5):
        assert torch.equal(_hip.w8a16_gemm(xa, qa, sa, bias).view(torch.int16), first_a.view(torch.int16)), i
        assert torch.equal(_hip.w8a8_linear(xa, qa, sa, bias).view(torch.int16), first_a8.view(torch.int16)), i
        assert torch.equal(_hip.w8a16_gemm(xb, qb, sb).view(torch.int16), first_b.view(torch.int16)), i
    assert torch.equal(first_a8.view(torch.int16), _hip.w8a8_linear(xa, qa, sa, bias, split_k=False).view(torch.int16))
    ws = _hip.gemm_workspace(d)
    torch.cuda.synchronize()
    assert int(ws[: 64 * 1024].view(torch.int32).abs().sum()) == 0


def test_streamk_graph_replay(hiplib, streamk):
    """Stream-K launches captured in a HIP graph replay correctly, with eager
    stream-K calls of another shape between the replays."""
    from nanovllm.quantization import _hip
    d = torch.device("cuda", 0)
    q, s = (t.to(d) for t in make_weights(6144, 4096, seed=51))
    x = make_activations(48, 4096, seed=52).to(d)
    _log_case(test="streamk_graph", path=_hip.select_path(_hip.OP_W8A16, 48, 6144, 4096))
    ref16 = _hip.w8a16_gemm(x, q, s)
    ref8 = _hip.w8a8_linear(x, q, s)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        _hip.w8a16_gemm(x, q, s)
        _hip.w8a8_linear(x, q, s)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y16 = _hip.w8a16_gemm(x, q, s)
        y8 = _hip.w8a8_linear(x, q, s)
    for i in range(4):
        y16.zero_()
        y8.zero_()
        other = _hip.w8a16_gemm(x[:20], q, s)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y16.view(torch.int16), ref16.view(torch.int16)), f"replay {i}"
        assert torch.equal(y8.view(torch.int16), ref8.view(torch.int16)), f"replay {i}"
        assert torch.equal(other.view(torch.int16), _hip.w8a16_gemm(x[:20], q, s).view(torch.int16))
