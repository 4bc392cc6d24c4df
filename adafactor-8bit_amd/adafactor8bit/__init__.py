"""adafactor8bit for AMD Instinct MI355X (gfx950).

Drop-in for the reference package's public API (adafactor8bit/__init__.py:4-8):
``Adafactor8Bit`` runs its step through the hand-written HIP library
``libadafactor8bit_amd.so``; ``build_param_groups`` builds the reference's
model-aware parameter groups.
"""
from .optimizer import Adafactor8Bit
from .routing import build_param_groups

__all__ = ["Adafactor8Bit", "build_param_groups"]
__version__ = "0.4.6"
