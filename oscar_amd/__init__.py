"""oscar_amd: MI355X (gfx950) implementation of OSCAR's INT2 rotated KV-cache attention path.

Host side mirrors the reference's vLLM plugin surface (plugin.py / backend.py);
the arithmetic runs in hand-written HIP kernels reached through the C ABI in
include/oscar_amd.h (liboscar_amd.so, built by ``python -m oscar_amd.build``).
"""

__all__ = ["backend", "config", "format", "integration", "mtp_shadow", "ops", "plugin", "rotation", "torch_ops"]
__version__ = "0.1.0"
