"""MI355X-native ZTCP fused cold-page codec (gfx950 HIP kernels behind a C ABI).

Modules:
  native_hip_codec  drop-in for the reference's native module functions
                    (research/baseline_codec/csrc/fused_cold_page_cpu.cpp:2540-2683)
  codec             session-bound codec class, drop-in for NativeCppFusedColdPageCodec
                    (research/baseline_codec/native_fused_codec.py:68-606)
  keyring           session key ring, drop-in for EphemeralSessionKeyRing
                    (research/baseline_codec/fused_quant_crypto.py:99-659), native state
  pages             descriptor-based batch API for paged, multi-layer KV pools
  serving           PoisonShield hit bitmap from per-page verdicts, pinned host ring
                    for the egress wire step
  spec              wire constants, AAD record and payload sizing (cold_page_spec.py mirror)
  workloads         synthetic page generators for the benchmark configurations
"""
from . import spec  # noqa: F401

__all__ = ["spec", "native_hip_codec", "codec", "keyring", "pages", "serving", "workloads", "load_native"]


def load_native():
    """Load the C-ABI library; raises if it has not been built."""
    from . import _native

    return _native.lib()
