"""Run the GPU test files (tests/test_gpu_*.py, -m gpu) on the CPU emulation
of the kernels: test infrastructure, enabled by TVQ_GPU_TESTS_ON_EMU=1
through tests/conftest.py, e.g.

    TVQ_GPU_TESTS_ON_EMU=1 python -m pytest tests -m gpu -k parity

The emulated library (tests/cpu_emu/build.py) takes host pointers, so CPU
tensors stand in for device tensors:
  * a TorchFunctionMode maps every device="cuda" argument (factories,
    Tensor.to, Tensor.cuda) to the CPU, an upload to a copy, and pin_memory
    to a no-op;
  * every tensor reports is_cuda, so the package takes its device path;
  * torch.cuda's synchronisation, streams, device and memory queries become
    host no-ops (a 4 GiB device, which bounds the engine's KV cache);
  * nanovllm.quantization._hip loads the emulated library, with a 256-byte
    aligned workspace;
  * HIP graphs: capture runs its code eagerly and records, in order, every
    top-level torch call and every library call; replay runs them again,
    copying each out-of-place torch result into the tensor the capture
    produced (so the later calls, which hold its address, see the new
    values), as a replayed graph rewrites its buffers in place. This checks
    what a graph's users must get right (static inputs filled before
    replay, outputs read after it, nothing allocated while capturing); it
    does not model the GPU's graph nodes themselves.
The tests' own checks then run unchanged against the kernels' emulation.
Random data differ from a GPU run (CPU generators), and nothing is timed.
"""
from __future__ import annotations

import contextlib
import types

import torch
from torch.overrides import TorchFunctionMode


_CAPTURE = None  # the graph being captured


def _record(kind, fn, args, kwargs=None, out=None) -> None:
    if _CAPTURE is not None:
        _CAPTURE.ops.append((kind, fn, args, kwargs or {}, out))


_NO_REPLAY = {torch.empty, torch.empty_like, torch.Tensor.new_empty}


def _is_cuda(d) -> bool:
    if isinstance(d, torch.device):
        return d.type == "cuda"
    return isinstance(d, str) and d.startswith("cuda")


class _CudaAsCpu(TorchFunctionMode):
    def __torch_function__(self, func, types_, args=(), kwargs=None):
        kwargs = dict(kwargs or {})
        if func is torch.Tensor.pin_memory:
            return args[0]
        if func is torch.Tensor.cuda:
            return args[0].clone()  # an upload is a copy (callers may update the host tensor afterwards)
        upload = _is_cuda(kwargs.get("device"))
        if upload:
            kwargs["device"] = "cpu"
        if kwargs.get("pin_memory"):
            kwargs["pin_memory"] = False
        if func is torch.Tensor.to:
            upload = upload or any(_is_cuda(a) for a in args)
            args = tuple("cpu" if _is_cuda(a) else a for a in args)
            out = func(*args, **kwargs)
            out = out.clone() if upload and out is args[0] else out
        else:
            out = func(*args, **kwargs)
        if _CAPTURE is not None:
            if func in _NO_REPLAY:
                _CAPTURE.keep.append(out)  # the graph's pool owns what its capture allocates
            elif out is None or isinstance(out, torch.Tensor) or (
                    isinstance(out, tuple) and out and all(isinstance(o, torch.Tensor) for o in out)):
                _record("torch", func, args, kwargs, out)
        return out


class _Stream:
    cuda_stream = 0

    def __init__(self, *a, **k):
        pass

    def wait_stream(self, *a):
        pass

    def synchronize(self):
        pass

    def record_event(self, *a, **k):
        return None


class _Graph:
    """torch.cuda.CUDAGraph on the emulation (see the module docstring)."""

    def __init__(self, *a, **k):
        self.ops = []
        self.keep = []  # tensors allocated during capture (held like the graph's memory pool)

    def replay(self) -> None:
        global _CAPTURE
        assert _CAPTURE is None, "replay while capturing"
        for kind, fn, args, kwargs, out in self.ops:
            new = fn(*args, **kwargs)
            if kind == "torch":
                outs, news = (out, new) if isinstance(out, tuple) else ((out,), (new,))
                for o, n in zip(outs, news):
                    if isinstance(o, torch.Tensor) and n is not o:
                        o.copy_(n)

    def pool(self):
        return None

    def reset(self) -> None:
        self.ops, self.keep = [], []


@contextlib.contextmanager
def _graph(g, pool=None, stream=None, **kw):
    global _CAPTURE
    assert _CAPTURE is None, "nested capture"
    _CAPTURE = g
    try:
        yield g
    finally:
        _CAPTURE = None


class _Event:
    """torch.cuda.Event on the host clock (emulated kernels run synchronously)."""

    def __init__(self, *a, **k):
        self.t = None

    def record(self, *a):
        import time
        self.t = time.perf_counter()

    def synchronize(self):
        pass

    def elapsed_time(self, end) -> float:
        return (end.t - self.t) * 1e3


class _Lib:
    """The emulated library, each call also recorded while a graph captures."""

    def __init__(self, lib):
        self._lib = lib

    def __getattr__(self, name):
        fn = getattr(self._lib, name)
        if not callable(fn):
            return fn

        def call(*args):
            r = fn(*args)
            _record("lib", fn, args)
            return r
        return call


_GENERATOR = torch.Generator
_installed = False


def install(lib) -> None:
    """Make this process's torch treat the CPU as the GPU and point the
    package at the emulated library `lib`."""
    global _installed
    if _installed:
        return
    _installed = True
    _CudaAsCpu().__enter__()
    torch.Tensor.is_cuda = property(lambda self: True)

    def generator(device="cpu"):
        return _GENERATOR(device="cpu" if _is_cuda(device) else device)

    torch.Generator = generator
    c = torch.cuda
    c.is_available = lambda: True
    c.device_count = lambda: 1
    c.current_device = lambda: 0
    c.set_device = lambda *a: None
    c.synchronize = lambda *a, **k: None
    c.device = lambda *a, **k: contextlib.nullcontext()
    c.current_stream = lambda *a, **k: _Stream()
    c.default_stream = lambda *a, **k: _Stream()
    c.Stream = _Stream
    c.stream = lambda *a, **k: contextlib.nullcontext()
    c.is_current_stream_capturing = lambda: _CAPTURE is not None
    c.CUDAGraph = _Graph
    c.graph = _graph
    c.graph_pool_handle = lambda: None
    c.Event = _Event
    c.empty_cache = lambda: None
    # a 4 GiB "device", so that the engine sizes its KV cache within host memory
    c.mem_get_info = lambda *a: (4 << 30, 4 << 30)
    c.memory_stats = lambda *a: {"allocated_bytes.all.current": 0}
    c.reset_peak_memory_stats = lambda *a: None
    c.max_memory_allocated = lambda *a: 0
    c.manual_seed = lambda *a: None
    c.manual_seed_all = lambda *a: None
    c.get_device_properties = lambda *a: types.SimpleNamespace(name="CPU emulation of gfx950",
                                                               multi_processor_count=256,
                                                               total_memory=288 << 30)

    from nanovllm.quantization import _hip
    n = lib.tvq_gemm_workspace_bytes()
    raw = torch.zeros(n + 256, dtype=torch.uint8)
    off = (-raw.data_ptr()) % 256
    ws = raw[off:off + n]
    proxy = _Lib(lib)
    _hip.load_library = lambda: proxy
    _hip._stream = lambda dev: None
    _hip.gemm_workspace = lambda dev: ws
    _hip._emu_keep = raw
