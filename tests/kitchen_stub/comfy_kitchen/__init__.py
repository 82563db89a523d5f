"""Test double of the comfy_kitchen 0.2.40 surface that the MOSS INT8 backend
touches (the package is not installed here). Only the interface is mirrored:
the registry lookup, the eager backend's exported int8_linear, the module
level _int8_matmul_accumulate hook and the helper functions. The arithmetic of
the helpers is this test suite's stand-in (the benchmark's per-token absmax/127
round-half-even quantizer, a normalised Sylvester Hadamard rotation, an
additive residual); Kitchen's own implementations are not available, so parity
with them is unpinned."""
