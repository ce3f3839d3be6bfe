"""anima_hip -- MI355X (gfx950) attention path of the Anima 2B DiT.

Torch-free host interface over libanima_hip.so:
  * `rt`: anima_rt drop-in functions, `AnimaRT` (NumpyRT mirror) and `AnimaVK`
    (NumpyVK mirror);
  * `dit`: the whole DiT on the device, `AnimaDiT` (NumpyDiT drop-in);
  * `rope`: the host-built 3D RoPE table.
"""
from . import _lib
from ._lib import AnimaHipError, LIB_PATH, last_error, load
from . import dit, rope, rt
from .rope import generate_rope_freqs
from .dit import AnimaDiT, DiTConfig
from .rt import AnimaRT, AnimaVK

__all__ = ["AnimaDiT", "AnimaHipError", "AnimaRT", "AnimaVK", "DiTConfig", "LIB_PATH", "dit",
           "generate_rope_freqs", "last_error", "load", "rope", "rt"]
