"""MI355X-native (gfx950) temporal-attention aggregation for FAST.

Importing this package loads the in-tree ``fastAgg`` extension (built by
``fast_amd.build`` / ``__graft_entry__.build()``) and registers it as the top-level module
``fastAgg``, so code written against the reference binding (``import fastAgg``) resolves
to it. There is no CPU fallback: without the built extension the import fails.
"""
from __future__ import annotations

import importlib.util
import os
import sys

_PKG = os.path.dirname(os.path.abspath(__file__))


def _load_extension():
    import sysconfig

    import torch  # noqa: F401  (loads libc10/libtorch before the extension)

    path = os.path.join(_PKG, "fastAgg" + sysconfig.get_config_var("EXT_SUFFIX"))
    if not os.path.exists(path):
        raise ImportError(
            f"fast_amd: native extension not built ({path} missing); run "
            "`python -c 'import __graft_entry__ as g; g.build()'` or `python fast_amd/build.py`")
    spec = importlib.util.spec_from_file_location("fastAgg", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    sys.modules["fastAgg"] = mod
    return mod


fastAgg = sys.modules.get("fastAgg") or _load_extension()

__all__ = ["fastAgg", "lib_path"]


def lib_path() -> str:
    """Path of the C-ABI kernel library (libfastagg_hip.so)."""
    return os.path.join(_PKG, "lib", "libfastagg_hip.so")
