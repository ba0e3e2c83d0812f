from .int8_linear import FFN_LINEAR_SUFFIXES, INT8Linear, dequantized_weight, quantize_ffn_modules

__all__ = ["FFN_LINEAR_SUFFIXES", "INT8Linear", "dequantized_weight", "quantize_ffn_modules"]
