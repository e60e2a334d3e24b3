"""W8A8 int8 linear layers for LLM inference on AMD Instinct MI355X (gfx950).

Drop-in for the int8_linear package of AshrithaG/int8-linear: the same names, backed by
hand-written HIP kernels behind a C ABI (include/int8_linear_amd.h).
"""

from int8_linear.kernel import Config, NotSupported, default_config, tuned_config, w8a8_mm

__all__ = ["Config", "NotSupported", "default_config", "tuned_config", "w8a8_mm"]
