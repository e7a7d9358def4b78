"""MI355X-native drop-in for tiny-vLLM's quantized-linear path.

`nanovllm.quantization` keeps the reference's plugin API; its GPU work runs on
the gfx950 HIP kernels of libtinyvllm_quant.so. `LLM` / `SamplingParams` are
the engine counterpart used for end-to-end runs; they are imported lazily so
that the quantization package stays importable on its own.
"""


def __getattr__(name):
    if name == "LLM":
        from nanovllm.llm import LLM
        return LLM
    if name == "SamplingParams":
        from nanovllm.sampling_params import SamplingParams
        return SamplingParams
    raise AttributeError(name)
