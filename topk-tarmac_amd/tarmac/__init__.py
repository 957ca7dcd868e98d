"""tarmac -- MI355X-native TarMAC attention core.

Hand-written HIP kernels for gfx950 behind a C ABI (``include/tarmac.h``,
``libtarmac.so``), with PyTorch-ROCm used for device memory and streams.
Public surface mirrors the reference's ``src/kernels`` launch functions and
``src/agents`` ``AttentionComm``.
"""

from ._lib import LIB_PATH, TarmacError, abi_version
from . import kernels
from .agents import AttentionComm, MAPPOConfig

__all__ = ["LIB_PATH", "TarmacError", "abi_version", "kernels", "AttentionComm", "MAPPOConfig"]
