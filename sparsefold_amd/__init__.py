"""MI355X-native gated pair-biased attention for SparseFold.

Hand-written HIP kernels for gfx950 (``csrc/``) behind a C ABI (``include/sparsefold_hip.h``),
called from a Python mirror of SparseFold's attention-backend interface:
``runtime.config.configure_runtime(backend="hip", sdpa_implementation="hip")``,
``backends.init() / prepare()``, ``backends.hip.attention.dot_product_attention`` and the
module replacements in ``backends.hip.modules``.
"""
__version__ = "0.1.0"
