"""anima_hip -- MI355X (gfx950) attention path of the Anima 2B DiT.

Torch-free host interface over libanima_hip.so:
  * `rt`: anima_rt drop-in functions and the `AnimaRT` class (NumpyRT mirror);
  * `rope`: the host-built 3D RoPE table;
  * `workloads`: seeded synthetic inputs of the benchmark configurations.
"""
from . import _lib
from ._lib import AnimaHipError, LIB_PATH, last_error, load
from . import rope, rt
from .rope import generate_rope_freqs
from .rt import AnimaRT

__all__ = ["AnimaHipError", "AnimaRT", "LIB_PATH", "generate_rope_freqs", "last_error", "load",
           "rope", "rt"]
