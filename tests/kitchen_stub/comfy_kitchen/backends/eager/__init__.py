from .quantization import int8_linear  # noqa: F401  (the exported callable)
