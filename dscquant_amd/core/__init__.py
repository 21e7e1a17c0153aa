"""Reference-named Python API (core/quantization.py, core/linear.py)."""
from .linear import QuantLinear  # noqa: F401
from .quantization import (activation_codes, pack_int4, quantize_activation,  # noqa: F401
                           quantize_weight, ste_round, unpack_int4, weight_codes)
