"""NF4 weight state and quantizer."""

from .nf4 import QuantState, quantize_nf4, nf4_code, dynamic_map, NF4_CODE

__all__ = ["QuantState", "quantize_nf4", "nf4_code", "dynamic_map", "NF4_CODE"]
