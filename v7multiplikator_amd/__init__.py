"""MI355X (gfx950) fused per-layer kernels of the v7 inference engine.

The product is the HIP library libv7g.so (C ABI: include/v7g_lib.h); this
package builds it (``v7multiplikator_amd.build``), binds it (``_lib``) and
exposes a torch-facing host API (``v7multiplikator_amd.ops``) that mirrors
the reference's kernel entry points.  ``ops`` imports torch, so it is loaded
on first use.
"""
import importlib

from . import _lib  # noqa: F401

__all__ = ["ops", "build", "_lib"]


def __getattr__(name):
    if name in ("ops", "build"):
        return importlib.import_module(f"{__name__}.{name}")
    raise AttributeError(name)
