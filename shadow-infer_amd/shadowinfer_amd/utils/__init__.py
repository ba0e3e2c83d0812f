from .quantization import Quantizer

__all__ = ["Quantizer"]
