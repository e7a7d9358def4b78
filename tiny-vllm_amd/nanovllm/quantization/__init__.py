from nanovllm.quantization.int8 import Int8WeightOnlyQuantMethod
from nanovllm.quantization.w8a8 import W8A8QuantMethod

__all__ = ["Int8WeightOnlyQuantMethod", "W8A8QuantMethod"]
