"""MI355X (gfx950) backend for furkanhaney/axis's training hot path.

``axis_amd.hip`` binds the C ABI of libaxis_hip.so (include/axis_hip.h); ``axis_amd.build``
compiles it ahead of time.  The named-axis tensor / autograd / optimizer host layer lives in
the C++ extension ``axis_amd._axis`` (imported on demand by ``axis_amd.host()``).
"""
import importlib
import os

__all__ = ["hip", "host", "library_path"]

from . import hip  # noqa: E402


def library_path() -> str:
    return hip.LIB_PATH


def host():
    """The C++ host layer (named-axis Tensor, tape, modules, optimizers, Trainer)."""
    here = os.path.dirname(os.path.abspath(__file__))
    if not any(f.startswith("_axis") and f.endswith(".so") for f in os.listdir(here)):
        raise ImportError("axis_amd._axis is not built: run `python -m axis_amd.build`")
    hip.load()  # the HIP library must be loadable first
    return importlib.import_module("axis_amd._axis")
