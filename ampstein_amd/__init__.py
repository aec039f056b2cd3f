"""MI355X-native EXL3 quantized-linear hot path (trellis decode, Hadamard rotations,
decode GEMV, prefill GEMM, mixed-K MoE) behind the C ABI of include/exl3_amd.h.

ops        -- the reference's operator interface over torch tensors
              (reconstruct, reconstruct_had_slice, had_r_128, exl3_gemm, exl3_gemm_recon)
linear     -- LinearEXL3, the caller-side routing of the reference's models.uc
synth      -- seeded synthetic EXL3 layers (benchmarks and tests)
"""
from . import _lib  # noqa: F401

__all__ = ["ops", "linear", "synth"]
