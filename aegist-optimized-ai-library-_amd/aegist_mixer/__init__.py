"""MI355X (gfx950) token-mixer path of the Aegist hybrid engine: gated DeltaNet and gated
GQA attention as hand-written HIP kernels behind the C ABI of include/aegist_mixer.h.

``ops`` holds the torch-tensor host API; ``_lib`` the ctypes binding of the shared library.
"""
from ._lib import AegistError, LIB_PATH, lib  # noqa: F401
from . import ops  # noqa: F401

__all__ = ["AegistError", "LIB_PATH", "lib", "ops"]
