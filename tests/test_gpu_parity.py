"""GPU parity tests: the HIP kernels (through the C ABI) against the oracle.

Bar:
  * act-quant int8 values and fp32 scales: bit-exact;
  * W8A8 int32 accumulators: bit-exact;
  * W8A8 bf16/fp16 outputs: bit-exact against the oracle's restatement of the
    reference kernel's epilogue, and within rel-L2 <= 1e-2,
    max-abs <= 2e-2*max|ref| of the reference's torch path;
  * W8A16 outputs: within the same tolerance of the torch path and within a
    bf16-rounding bound of the exact fp64 product.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import bits16, f32, make_activations, make_weights

pytestmark = pytest.mark.gpu


def _dev():
    return torch.device("cuda", 0)


def _log_case(**kw):
    print("CASE", " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


# ---------------------------------------------------------------- act quant

# M picks the threads per row (four waves below 512 rows, two below 1024, then one)
ACT_SHAPES = [(1, 1024), (3, 1024), (64, 1024), (257, 3072), (33, 4096), (5, 12288), (2, 8), (7, 24), (9, 100),
              (1, 1), (1, 12288), (64, 12288), (511, 2048), (600, 2048), (1023, 3072), (1030, 1024), (2000, 12288),
              (513, 16384), (3, 24)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", ACT_SHAPES)
def test_act_quant_bit_exact(hiplib, shape, dtype):
    from nanovllm.quantization import _hip
    m, k = shape
    _log_case(test="act_quant", m=m, k=k, dtype=dtype)
    x = make_activations(m, k, seed=m * 131 + k, dtype=dtype)
    if m >= 3:
        x[1].zero_()                       # all-zero row -> s = eps, q = 0
        x[2] = x[2] * 1e-30 if dtype == torch.bfloat16 else x[2] * 1e-6  # tiny/subnormal row
    q_ref, s_ref = oracle.c_act_quant(bits16(x), is_bf16=dtype == torch.bfloat16)
    xq, s = _hip.act_quant(x.to(_dev()))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    np.testing.assert_array_equal(xq.cpu().numpy(), q_ref)
    # and against the reference's own torch expression on the CPU
    q_t, s_t = oracle.quantize_rows_torch(x)
    np.testing.assert_array_equal(xq.cpu().numpy(), q_t.numpy())


def test_act_quant_ties_half_even(hiplib):
    """x/s lands exactly on k+0.5: must round to even (torch.round semantics)."""
    from nanovllm.quantization import _hip
    # amax = 127 -> s = 1.0 exactly, so q = rint(x): ties at .5 go to even.
    row = torch.tensor([127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, 100.5, -126.5, 0.0, 7.0, 8.5, -8.5, 9.5, 1.0],
                       dtype=torch.float32)
    x = row.repeat(4, 1).to(torch.bfloat16)
    expect = np.array([127, 0, 2, 2, 0, -2, -2, 4, 100, -126, 0, 7, 8, -8, 10, 1], np.int8)
    xq, s = _hip.act_quant(x.to(_dev()))
    assert np.all(s.cpu().numpy() == 1.0)
    np.testing.assert_array_equal(xq.cpu().numpy()[0], expect)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_act_quant_near_ties_bit_exact(hiplib, dtype):
    """Rows built so that x/s lands on, or within a few ulps of, half-integers
    for non-power-of-two scales: the kernels' multiply-by-1/s fast path must
    hand exactly these to the IEEE divide (bit-exact vs the oracle), in
    act-quant and in the fused producers' quantization."""
    from nanovllm.quantization import _hip
    rng = np.random.default_rng(5)
    rows = []
    for _ in range(512):
        amax = np.float32(rng.uniform(0.5, 40.0))
        s = max(np.float32(amax / np.float32(127.0)), np.float32(1e-8))
        k = rng.integers(-126, 126, 255).astype(np.float32)
        t = (k + np.float32(0.5)) * s * (1 + rng.integers(-4, 5, 255) * np.float32(2.0 ** -23))
        rows.append(np.concatenate([[amax], t]).astype(np.float32))
    x = torch.from_numpy(np.stack(rows)).to(dtype)   # rounding to 16 bits keeps many exact/near ties
    q_ref, s_ref = oracle.c_act_quant(bits16(x), is_bf16=dtype == torch.bfloat16)
    xq, sc = _hip.act_quant(x.to(_dev()))
    np.testing.assert_array_equal(sc.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    np.testing.assert_array_equal(xq.cpu().numpy(), q_ref)
    # fused SiLU-and-mul quantization on rows whose SiLU output is x (u = x / silu(g) is awkward;
    # use the RMSNorm producer with unit weight on rows of constant RMS instead: its y is x * r)
    y, q = _hip.rmsnorm(x.to(_dev()), torch.ones(256, dtype=dtype, device=_dev()), 1e-6, out=True, quant=True)
    rq, rs = oracle.c_act_quant(bits16(y.cpu()), is_bf16=dtype == torch.bfloat16)
    np.testing.assert_array_equal(q[0].cpu().numpy(), rq)
    np.testing.assert_array_equal(q[1].cpu().numpy().view(np.uint32), rs.view(np.uint32))


# ---------------------------------------------------------------- W8A8

# (M, N, K) covering skinny (M <= 64), tiled, ragged edges and the generic path.
GEMM_SHAPES = [
    (1, 4096, 1024), (16, 4096, 1024), (17, 1000, 1024), (48, 6144, 1024), (64, 1024, 3072),
    (1, 1024, 12288), (33, 4096, 4096), (7, 200, 2048), (5, 96, 1040), (24, 16384, 512), (64, 16448, 256),
    (9, 20000, 768), (16, 16384, 1024), (40, 16384, 1024), (64, 24576, 256), (12, 6144, 4096), (16, 4096, 12288), (48, 16384, 1024),
    (65, 4096, 1024), (256, 4096, 1024), (512, 1024, 3072), (300, 1030, 2048), (129, 136, 80),
    (7, 33, 40), (3, 5, 1024), (2, 4104, 3072), (4, 24576, 4096), (1, 6144, 9216),
]


def _w8a8_inputs(m, n, k, seed):
    x = make_activations(m, k, seed=seed)
    xq, a_s = oracle.c_act_quant(bits16(x))
    q, w_s = make_weights(n, k, seed=seed + 1)
    return xq, a_s, q.numpy(), w_s.numpy()


@pytest.mark.parametrize("shape", GEMM_SHAPES)
def test_w8a8_accumulator_bit_exact(hiplib, shape):
    from nanovllm.quantization import _hip
    m, n, k = shape
    _log_case(test="w8a8_i32", m=m, n=n, k=k, path=_hip.select_path(_hip.OP_W8A8, m, n, k))
    xq, a_s, q, w_s = _w8a8_inputs(m, n, k, seed=m + n + k)
    acc = _hip.w8a8_gemm_i32(torch.from_numpy(xq).to(_dev()), torch.from_numpy(q).to(_dev()))
    np.testing.assert_array_equal(acc.cpu().numpy(), oracle.c_gemm_i32(xq, q))


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", GEMM_SHAPES)
def test_w8a8_output(hiplib, shape, out_dtype):
    from nanovllm.quantization import _hip
    m, n, k = shape
    _log_case(test="w8a8_out", m=m, n=n, k=k, dtype=out_dtype)
    xq, a_s, q, w_s = _w8a8_inputs(m, n, k, seed=3 * m + n + k)
    d = _dev()
    y = _hip.w8a8_gemm(torch.from_numpy(xq).to(d), torch.from_numpy(a_s).to(d), torch.from_numpy(q).to(d),
                       torch.from_numpy(w_s).to(d), None, out_dtype)
    acc = oracle.c_gemm_i32(xq, q)
    yb_ref, yf_ref = oracle.c_w8a8_epilogue(acc, a_s, w_s)
    if out_dtype == torch.bfloat16:
        np.testing.assert_array_equal(bits16(y), yb_ref)
    else:
        np.testing.assert_array_equal(bits16(y), yf_ref.astype(np.float16).view(np.uint16))
    ref = oracle.w8a8_torch_path(torch.from_numpy(xq), torch.from_numpy(a_s), torch.from_numpy(q),
                                 torch.from_numpy(w_s), None, out_dtype)
    assert oracle.rel_l2(f32(y), f32(ref)) <= oracle.REL_L2_TOL
    assert oracle.max_abs_ratio(f32(y), f32(ref)) <= oracle.MAX_ABS_TOL


def test_w8a8_bias(hiplib):
    from nanovllm.quantization import _hip
    m, n, k = 80, 264, 1024
    xq, a_s, q, w_s = _w8a8_inputs(m, n, k, seed=11)
    bias = torch.randn(n, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    d = _dev()
    for mm in (m, 8, 2, 1):  # DMA, skinny and GEMV paths
        y = _hip.w8a8_gemm(torch.from_numpy(xq[:mm]).to(d), torch.from_numpy(a_s[:mm]).to(d),
                           torch.from_numpy(q).to(d), torch.from_numpy(w_s).to(d), bias.to(d), torch.bfloat16)
        yb_ref, _ = oracle.c_w8a8_epilogue(oracle.c_gemm_i32(xq[:mm], q), a_s[:mm], w_s, f32(bias))
        np.testing.assert_array_equal(bits16(y), yb_ref)


def test_w8a8_fused_linear_matches_two_step(hiplib):
    from nanovllm.quantization import _hip
    d = _dev()
    for m in (1, 64, 256, 1000):
        x = make_activations(m, 1024, seed=m).to(d)
        q, w_s = make_weights(4096, 1024, seed=9)
        q, w_s = q.to(d), w_s.to(d)
        y1 = _hip.w8a8_linear(x, q, w_s)
        xq, a_s = _hip.act_quant(x)
        y2 = _hip.w8a8_gemm(xq, a_s, q, w_s, None, torch.bfloat16)
        assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))


@pytest.mark.parametrize("shape", [(256, 4096, 1024), (17, 1000, 1024), (100, 4096, 2048), (64, 6144, 1024), (96, 2048, 512),
                                   (257, 520, 1024), (33, 24576, 1024), (40, 1024, 2048), (8, 4096, 1024)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_w8a8_linear_buffers_and_output(hiplib, shape, dtype):
    """tvq_w8a8_linear fills the caller's xq / a_scales buffers exactly as
    tvq_act_quant does and its output equals act-quant + tvq_w8a8_gemm bit
    for bit (skinny, DMA and split-K GEMM paths)."""
    from nanovllm.quantization import _hip
    m, n, k = shape
    _log_case(test="w8a8_linear_buffers", m=m, n=n, k=k, dtype=dtype)
    d = _dev()
    x = make_activations(m, k, seed=m + n + k, dtype=dtype).to(d)
    q, w_s = (t.to(d) for t in make_weights(n, k, seed=n + 1))
    y = torch.empty((m, n), dtype=dtype, device=d)
    xq = torch.full((m, k), 99, dtype=torch.int8, device=d)
    a_s = torch.full((m,), -1.0, dtype=torch.float32, device=d)
    ws = _hip.gemm_workspace(d)
    rc = hiplib.tvq_w8a8_linear(x.data_ptr(), _hip._TORCH_TO_TVQ[dtype], q.data_ptr(), w_s.data_ptr(), None,
                                y.data_ptr(), m, n, k, xq.data_ptr(), a_s.data_ptr(), ws.data_ptr(), ws.numel(),
                                torch.cuda.current_stream().cuda_stream)
    assert rc == 0, hiplib.tvq_last_error()
    xq_ref, as_ref = _hip.act_quant(x)
    assert torch.equal(xq, xq_ref)
    assert torch.equal(a_s.view(torch.int32), as_ref.view(torch.int32))
    y_ref = _hip.w8a8_gemm(xq_ref, as_ref, q, w_s, None, dtype)
    assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16))


# ---------------------------------------------------------------- W8A16

def _w8a16_check(y, x, q, s, bias=None):
    """Tolerance vs the reference torch path, and a bf16-rounding bound vs fp64."""
    ref = oracle.w8a16_torch_path(x, q, s, bias)
    assert oracle.rel_l2(f32(y), f32(ref)) <= oracle.REL_L2_TOL
    assert oracle.max_abs_ratio(f32(y), f32(ref)) <= oracle.MAX_ABS_TOL
    y64 = oracle.c_w8a16_f64(bits16(x), q.numpy(), s.numpy(), None if bias is None else f32(bias),
                             is_bf16=x.dtype == torch.bfloat16)
    mag = (np.abs(f32(x)).astype(np.float64) @ np.abs(q.numpy()).astype(np.float64).T) * s.numpy()[None, :]
    k = x.shape[1]
    half_ulp = 2.0 ** -8 if x.dtype == torch.bfloat16 else 2.0 ** -11
    bound = np.abs(y64) * half_ulp + mag * (k * 2.0 ** -23) + 1e-30
    err = np.abs(f32(y).astype(np.float64) - y64)
    assert np.all(err <= bound), f"max excess {np.max(err - bound)}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", GEMM_SHAPES)
def test_w8a16_output(hiplib, shape, dtype):
    from nanovllm.quantization import _hip
    m, n, k = shape
    _log_case(test="w8a16", m=m, n=n, k=k, dtype=dtype, path=_hip.select_path(_hip.OP_W8A16, m, n, k))
    x = make_activations(m, k, seed=m * 7 + n + k, dtype=dtype, outlier_frac=0.0)
    q, s = make_weights(n, k, seed=m + 2 * n + k)
    d = _dev()
    y = _hip.w8a16_gemm(x.to(d), q.to(d), s.to(d))
    _w8a16_check(y, x, q, s)


def test_w8a16_bias(hiplib):
    from nanovllm.quantization import _hip
    d = _dev()
    q, s = make_weights(520, 1024, seed=3)
    bias = torch.randn(520, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    for m in (1, 2, 5, 130):  # GEMV, skinny and DMA paths
        x = make_activations(m, 1024, seed=m, outlier_frac=0.0)
        y = _hip.w8a16_gemm(x.to(d), q.to(d), s.to(d), bias.to(d))
        _w8a16_check(y, x, q, s, bias)


def test_unaligned_views_take_generic_path(hiplib):
    """A storage offset that breaks 16-byte alignment must still be correct."""
    from nanovllm.quantization import _hip
    d = _dev()
    m, n, k = 20, 64, 1024
    xb = make_activations(m * k + 1, 1, seed=1).view(-1)
    x = xb[1:].view(m, k)  # 2-byte offset
    q, s = make_weights(n, k, seed=2)
    y = _hip.w8a16_gemm(xb.to(d)[1:].view(m, k), q.to(d), s.to(d))
    _w8a16_check(y, x, q, s)


# ---------------------------------------------------------------- full-size properties

@pytest.mark.parametrize("mode", ["w8a8", "w8a16"])
@pytest.mark.parametrize("nk", [(1024, 3072), (1024, 2048), (6144, 1024)])
def test_prefill_full_size_sampled_rows(hiplib, mode, nk):
    """M=8192 prefill shapes (config 3): 48 sampled token rows checked exactly /
    within the bound; the full output checked for finiteness and row-scaling
    consistency."""
    from nanovllm.quantization import _hip
    n, k = nk
    m = 8192
    _log_case(test="prefill_full", mode=mode, m=m, n=n, k=k)
    d = _dev()
    x = make_activations(m, k, seed=n + k, outlier_frac=0.01 if mode == "w8a8" else 0.0)
    x[-100:].zero_()  # padded tail rows
    q, s = make_weights(n, k, seed=k)
    rows = np.sort(np.random.default_rng(0).choice(m, 48, replace=False))
    rows[-1] = m - 1
    if mode == "w8a8":
        y = _hip.w8a8_linear(x.to(d), q.to(d), s.to(d))
        xq, a_s = oracle.c_act_quant(bits16(x[torch.from_numpy(rows)]))
        yb_ref, _ = oracle.c_w8a8_epilogue(oracle.c_gemm_i32(xq, q.numpy()), a_s, s.numpy())
        np.testing.assert_array_equal(bits16(y)[rows], yb_ref)
    else:
        y = _hip.w8a16_gemm(x.to(d), q.to(d), s.to(d))
        _w8a16_check(y.cpu()[torch.from_numpy(rows)], x[torch.from_numpy(rows)], q, s)
    assert torch.isfinite(y.float()).all()
    assert (y[-100:].float() == 0).all()


# (M, N, K) hitting every DMA tile configuration with ragged M and N edges.
DMA_RAGGED = [("w8a8", 4100, 8200, 1024), ("w8a8", 4000, 1700, 1024), ("w8a8", 700, 1000, 1152),
              ("w8a8", 200, 3000, 1024), ("w8a16", 3000, 3300, 1024), ("w8a16", 700, 1000, 1152),
              ("w8a16", 100, 2050, 2048)]


@pytest.mark.parametrize("case", DMA_RAGGED, ids=lambda c: "-".join(map(str, c)))
def test_dma_ragged_sampled_rows(hiplib, case):
    """Every DMA tile configuration with M and N not multiples of the tile:
    sampled rows (always including the last) checked exactly (W8A8) or within
    the bound (W8A16), plus the last output column of every row."""
    from nanovllm.quantization import _hip
    mode, m, n, k = case
    op = _hip.OP_W8A8 if mode == "w8a8" else _hip.OP_W8A16
    _log_case(test="dma_ragged", mode=mode, m=m, n=n, k=k, path=_hip.select_path(op, m, n, k))
    assert _hip.select_path(op, m, n, k).startswith("dma_")
    d = _dev()
    x = make_activations(m, k, seed=m + n, outlier_frac=0.01 if mode == "w8a8" else 0.0)
    q, s = make_weights(n, k, seed=n + k)
    rows = np.unique(np.concatenate([np.random.default_rng(m).choice(m, 24, replace=False), [0, m - 1]]))
    xr = x[torch.from_numpy(rows)]
    if mode == "w8a8":
        y = _hip.w8a8_linear(x.to(d), q.to(d), s.to(d))
        xq, a_s = oracle.c_act_quant(bits16(xr))
        yb_ref, _ = oracle.c_w8a8_epilogue(oracle.c_gemm_i32(xq, q.numpy()), a_s, s.numpy())
        np.testing.assert_array_equal(bits16(y)[rows], yb_ref)
        xq_all, a_all = oracle.c_act_quant(bits16(x))
        col, _ = oracle.c_w8a8_epilogue(oracle.c_gemm_i32(xq_all, q.numpy()[-1:]), a_all, s.numpy()[-1:])
        np.testing.assert_array_equal(bits16(y)[:, -1:], col)
    else:
        y = _hip.w8a16_gemm(x.to(d), q.to(d), s.to(d))
        _w8a16_check(y.cpu()[torch.from_numpy(rows)], xr, q, s)
        _w8a16_check(y.cpu()[:, -1:], x, q[-1:], s[-1:])


# ---------------------------------------------------------------- graph capture

def test_hip_graph_capture_replay(hiplib):
    """The ABI never allocates or syncs, so both GEMMs can be captured and replayed."""
    from nanovllm.quantization import _hip
    d = _dev()
    q, s = make_weights(4096, 1024, seed=1)
    q, s = q.to(d), s.to(d)
    x = make_activations(16, 1024, seed=2).to(d)
    ref16 = _hip.w8a16_gemm(x, q, s)
    ref8 = _hip.w8a8_linear(x, q, s)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        _hip.w8a16_gemm(x, q, s)  # warm the allocator pools on this stream
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
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y16.view(torch.int16), ref16.view(torch.int16)), f"replay {i}"
        assert torch.equal(y8.view(torch.int16), ref8.view(torch.int16)), f"replay {i}"


# ---------------------------------------------------------------- split-K

# Decode-size shapes whose output tiles do not fill the GPU: K is split over
# several workgroups and reduced in-kernel through the GEMM workspace.
SPLIT_SHAPES = [(17, 1000, 2048), (24, 4096, 4096), (40, 6144, 4096), (64, 4096, 12288), (64, 1024, 3072),
                (33, 136, 2048)]


def _same_up_to_order(a, b, x, q, s):
    """W8A16 outputs that differ only in the fp32 summation order: within one
    bf16 rounding flip plus the fp32 reassociation bound K*2^-23*sum|terms|
    (checked on a sample of rows)."""
    rows = np.unique(np.linspace(0, x.shape[0] - 1, 6).astype(np.int64))
    fa, fb = f32(a)[rows].astype(np.float64), f32(b)[rows].astype(np.float64)
    mag = (np.abs(f32(x)[rows]).astype(np.float64) @ np.abs(q).astype(np.float64).T) * np.asarray(s)[None, :]
    bound = np.abs(fb) * 2.0 ** -7 + mag * (x.shape[1] * 2.0 ** -23) + 1e-30
    assert np.all(np.abs(fa - fb) <= bound), f"max excess {np.max(np.abs(fa - fb) - bound)}"


@pytest.mark.parametrize("shape", SPLIT_SHAPES)
def test_split_k_matches_unsplit(hiplib, shape):
    """Split-K gives the unsplit kernel's exact int32 accumulators and W8A8
    outputs, and W8A16 outputs equal up to fp32 summation order."""
    from nanovllm.quantization import _hip
    m, n, k = shape
    for op in (_hip.OP_W8A8, _hip.OP_W8A16):
        path = _hip.select_path(op, m, n, k)
        _log_case(test="split_k", m=m, n=n, k=k, path=path)
        assert path.endswith("_splitk"), path
    d = _dev()
    xq, a_s, q, w_s = _w8a8_inputs(m, n, k, seed=m * 5 + n + k)
    xq_d, a_d, q_d, w_d = (torch.from_numpy(t).to(d) for t in (xq, a_s, q, w_s))
    acc_s = _hip.w8a8_gemm_i32(xq_d, q_d)
    acc_u = _hip.w8a8_gemm_i32(xq_d, q_d, split_k=False)
    assert torch.equal(acc_s, acc_u)
    rows = np.unique(np.linspace(0, m - 1, 8).astype(np.int64))
    np.testing.assert_array_equal(acc_s.cpu().numpy()[rows], oracle.c_gemm_i32(xq[rows], q))
    y_s = _hip.w8a8_gemm(xq_d, a_d, q_d, w_d, None, torch.bfloat16)
    y_u = _hip.w8a8_gemm(xq_d, a_d, q_d, w_d, None, torch.bfloat16, split_k=False)
    assert torch.equal(y_s.view(torch.int16), y_u.view(torch.int16))
    x = make_activations(m, k, seed=m + 3 * n, outlier_frac=0.0).to(d)
    h_s = _hip.w8a16_gemm(x, q_d, w_d)
    h_u = _hip.w8a16_gemm(x, q_d, w_d, split_k=False)
    _same_up_to_order(h_s, h_u, x, q, w_s)
    _w8a16_check(h_s.cpu()[torch.from_numpy(rows)], x.cpu()[torch.from_numpy(rows)], torch.from_numpy(q),
                 torch.from_numpy(w_s))


def test_split_k_deterministic_and_workspace_reuse(hiplib):
    """Repeated split calls give identical bits whatever order their work units
    finish in, and a call leaves the workspace counters ready for the next
    call of another shape."""
    from nanovllm.quantization import _hip
    d = _dev()
    qa, sa = (t.to(d) for t in make_weights(4096, 4096, seed=21))
    qb, sb = (t.to(d) for t in make_weights(1000, 3072, seed=22))
    xa = make_activations(64, 4096, seed=23, outlier_frac=0.0).to(d)
    xb = make_activations(40, 3072, seed=24, outlier_frac=0.0).to(d)
    first_a = _hip.w8a16_gemm(xa, qa, sa)
    first_b8 = _hip.w8a8_linear(xb, qb, sb)
    for i in range(6):
        ya = _hip.w8a16_gemm(xa, qa, sa)
        yb8 = _hip.w8a8_linear(xb, qb, sb)
        yb = _hip.w8a16_gemm(xb, qb, sb)
        assert torch.equal(ya.view(torch.int16), first_a.view(torch.int16)), f"iteration {i}"
        assert torch.equal(yb8.view(torch.int16), first_b8.view(torch.int16)), f"iteration {i}"
        _same_up_to_order(yb, _hip.w8a16_gemm(xb, qb, sb, split_k=False), xb, qb.cpu().numpy(), sb.cpu().numpy())
    ws = _hip.gemm_workspace(d)
    torch.cuda.synchronize()
    assert int(ws[: 64 * 1024].view(torch.int32).abs().sum()) == 0   # every tile counter back at zero


def test_split_k_graph_replay(hiplib):
    """Split-K launches captured in a HIP graph replay correctly every time."""
    from nanovllm.quantization import _hip
    d = _dev()
    q, s = (t.to(d) for t in make_weights(4096, 4096, seed=31))
    x = make_activations(48, 4096, seed=32).to(d)
    assert _hip.select_path(_hip.OP_W8A16, 48, 4096, 4096).endswith("_splitk")
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
        other = _hip.w8a16_gemm(x[:20], q, s)   # eager split call between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y16.view(torch.int16), ref16.view(torch.int16)), f"replay {i}"
        assert torch.equal(y8.view(torch.int16), ref8.view(torch.int16)), f"replay {i}"
        assert torch.equal(other.view(torch.int16), _hip.w8a16_gemm(x[:20], q, s).view(torch.int16))


# ---------------------------------------------------------------- kernel families

# (M, N, K) and the families forced on it with TVQ_GEMM_PATH (each valid for
# the shape by its own rule): W8A8 outputs must agree bit for bit.
FAMILY_CASES = [((16, 4096, 1024), ("skinny", "dma", "stream")), ((64, 16384, 1024), ("skinny", "dma", "stream")),
                ((40, 6144, 2048), ("skinny", "dma")), ((2, 4096, 2048), ("gemv", "skinny"))]


@pytest.mark.parametrize("case", FAMILY_CASES, ids=lambda c: "x".join(map(str, c[0])))
def test_forced_kernel_families_agree(hiplib, monkeypatch, case):
    from nanovllm.quantization import _hip
    (m, n, k), fams = case
    d = _dev()
    xq, a_s, q, w_s = _w8a8_inputs(m, n, k, seed=m * n + k)
    args = [torch.from_numpy(t).to(d) for t in (xq, a_s, q, w_s)]
    ref, _ = oracle.c_w8a8_epilogue(oracle.c_gemm_i32(xq, q), a_s, w_s)
    for fam in fams:
        _log_case(test="family", fam=fam, m=m, n=n, k=k)
        monkeypatch.setenv("TVQ_GEMM_PATH", fam)
        y = _hip.w8a8_gemm(*args[:2], *args[2:], None, torch.bfloat16)
        np.testing.assert_array_equal(bits16(y), ref)
