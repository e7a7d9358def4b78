"""MI355X-native drop-in for tiny-vLLM's quantized-linear path.

`nanovllm.quantization` keeps the reference's plugin API; its GPU work runs on
the gfx950 HIP kernels of libtinyvllm_quant.so.
"""
