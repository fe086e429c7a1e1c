"""Loader of the in-tree PyTorch-ROCm extension (built by ``build.py``).

There is no fallback: when the extension is missing or fails to load, every decode entry
point raises. The extension needs an MI355X (gfx950, 256 CUs); constructing a decoder on any
other device raises from ``qtts_workspace_init``.
"""
from __future__ import annotations

import atexit
import importlib.util
import sys
from pathlib import Path

_PKG = Path(__file__).resolve().parent
_MOD = None


def extension_path() -> Path:
    import sysconfig
    return _PKG / ("_qwentts_amd_C" + sysconfig.get_config_var("EXT_SUFFIX"))


def library_path() -> Path:
    return _PKG / "lib" / "libqwentts_amd.so"


def load():
    """Import and return the compiled extension module; raise ImportError if it is not built."""
    global _MOD
    if _MOD is not None:
        return _MOD
    import torch  # noqa: F401  (loads libtorch / libc10_hip before the extension)
    path = extension_path()
    if not path.exists() or not library_path().exists():
        raise ImportError(
            f"qwentts-turbo_amd HIP extension is not built ({path.name} / lib/libqwentts_amd.so missing); "
            "run `python qwentts-turbo_amd/build.py` (or __graft_entry__.build())")
    spec = importlib.util.spec_from_file_location("_qwentts_amd_C", str(path))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    sys.modules["_qwentts_amd_C"] = mod
    _MOD = mod
    # library-owned device memory is freed while the HIP runtime is still up (Python's atexit
    # handlers run before the C runtime's exit handlers tear the runtime down)
    atexit.register(_shutdown)
    return mod


def _shutdown():
    if _MOD is not None:
        try:
            _MOD.shutdown()
        except RuntimeError:
            pass
