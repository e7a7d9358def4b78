"""tvq_w8a8_linear_noalloc (static-scratch variant) against tvq_w8a8_linear."""
from __future__ import annotations

import pytest
import torch

from tests.helpers import make_activations, make_weights

pytestmark = pytest.mark.gpu


def _linear(hiplib, fn, x, q, w_s, noalloc: bool):
    from nanovllm.quantization import _hip
    m, k = x.shape
    n = q.shape[0]
    y = torch.empty((m, n), dtype=x.dtype, device=x.device)
    stream = torch.cuda.current_stream().cuda_stream
    dt = _hip._TORCH_TO_TVQ[x.dtype]
    if noalloc:
        rc = hiplib.tvq_w8a8_linear_noalloc(x.data_ptr(), dt, q.data_ptr(), w_s.data_ptr(), None, y.data_ptr(),
                                            m, n, k, stream)
    else:
        xq = torch.empty((m, k), dtype=torch.int8, device=x.device)
        a_s = torch.empty((m,), dtype=torch.float32, device=x.device)
        ws = _hip.gemm_workspace(x.device)
        rc = hiplib.tvq_w8a8_linear(x.data_ptr(), dt, q.data_ptr(), w_s.data_ptr(), None, y.data_ptr(), m, n, k,
                                    xq.data_ptr(), a_s.data_ptr(), ws.data_ptr(), ws.numel(), stream)
    assert rc == 0, hiplib.tvq_last_error()
    return y


# (first call, second smaller call): split-K shapes (M <= 64, K >= 2048),
# DMA tiles and the skinny / GEMV paths
PAIRS = [((64, 4096, 4096), (16, 1024, 2048)), ((256, 4096, 1024), (1, 4096, 1024)),
         ((2048, 1024, 4096), (40, 2048, 4096))]


@pytest.mark.parametrize("pair", PAIRS, ids=lambda p: f"{p[0]}-{p[1]}")
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_noalloc_matches_linear_two_calls(hiplib, gpu, pair, dtype):
    for i, (m, n, k) in enumerate(pair):
        print(f"CASE noalloc call={i} m={m} n={n} k={k} dtype={dtype}", flush=True)
        x = make_activations(m, k, seed=m + k + i, dtype=dtype).to(gpu)
        q, w_s = (t.to(gpu) for t in make_weights(n, k, seed=n + i))
        y0 = _linear(hiplib, None, x, q, w_s, noalloc=True)
        y1 = _linear(hiplib, None, x, q, w_s, noalloc=False)
        torch.cuda.synchronize()
        assert torch.equal(y0.view(torch.int16), y1.view(torch.int16))


def test_noalloc_at_the_scratch_limit(hiplib, gpu):
    """M*K exactly TVQ_NOALLOC_MAX_XQ_BYTES."""
    m, n, k = 8192, 1024, 1024
    print(f"CASE noalloc limit m={m} n={n} k={k}", flush=True)
    x = make_activations(m, k, seed=5).to(gpu)
    q, w_s = (t.to(gpu) for t in make_weights(n, k, seed=6))
    y0 = _linear(hiplib, None, x, q, w_s, noalloc=True)
    y1 = _linear(hiplib, None, x, q, w_s, noalloc=False)
    torch.cuda.synchronize()
    assert torch.equal(y0.view(torch.int16), y1.view(torch.int16))
