"""MI355X-native MXFP8 FMHA forward (head dim 128): the reference's ``fmha_fwd_hd128_mxfp8_auto`` path.

``amdgpu_rustdsl_amd.ops.fmha_fwd_mxfp8`` mirrors the reference's Python op (python/amdgpu_jit/ops.py:88);
``amdgpu_rustdsl_amd.lib`` is the ctypes binding of the C ABI (include/fmha_mxfp8.h) it calls.
"""
from . import lib  # noqa: F401  (fails loudly when the native library is missing)

__all__ = ["lib", "ops"]
