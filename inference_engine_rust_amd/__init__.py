"""inference_engine_rust_amd — MI355X-native greedy token loop for GGUF K-quant decoders.

The package holds the HIP/C++ engine (``csrc/`` -> ``libiek.so``, C ABI in ``include/iek.h``),
its Python mirror of the reference engine API (``engine``), the synthetic GGUF generator
(``synth``) and the build recipe (``build``). Import ``engine`` to use the device path; it
raises if the HIP library is not built.
"""

__all__ = ["engine", "synth", "build"]
