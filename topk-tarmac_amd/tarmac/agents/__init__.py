"""The communication module boundary (``src/agents`` of the reference)."""

from .mappo import AttentionComm, MAPPOConfig

__all__ = ["AttentionComm", "MAPPOConfig"]
