"""MI355X-native MoE block of c0ven's qwen4exp model: HIP kernels for gfx950 behind a C ABI (include/c0ven_moe.h).

The compute lives in libc0ven_moe.so (c0ven_amd/csrc); this package is its ctypes binding. Importing it without the
built library raises ImportError: there is no CPU fallback.
"""
from ._lib import (BLOCK, CODEBOOK_TYPES, EXPORTS, MOE_BAD_ARGUMENT, MOE_FLAG_EXACT_ROUTER, MOE_FLAG_HC_FIXED_ORDER, MOE_OK, MoeConfig, Q8_FAMILY, QGRID_BYTES, QGRID_IQ2S, QGRID_IQ3S,  # noqa: F401
                   QGRID_IQ3XXS, QGRID_KVALUES, QT_IQ2_S, QT_IQ3_S, QT_IQ3_XXS, QT_IQ4_NL, QT_Q2_0, QT_Q4_K, QT_Q8_0,
                   QT_Q8_K, QT_Q5_K, QT_Q6_K, QT_IQ4_XS, TYPE_IDS, TYPE_NAMES, GgufFile, MoeBlock, MoeError, abi_layout, gguf_architecture, synth_set_codebooks, lib, quantize, row_bytes, synth_matrix, synth_normal, zipf_bias)
