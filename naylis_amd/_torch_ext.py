"""Loader for the torch extension of the fused layer node
(``naylis_amd/_lib/ext/naylis_torch.so``, built from csrc/torch_layer.cpp by
naylis_amd/build.py).  The extension makes the library's C-ABI calls itself,
so libnaylis_mom.so is loaded first (with global visibility, _lib.load) and
the extension binds to that instance."""
from __future__ import annotations

import importlib.util
import os
import threading

from . import _lib

EXT_PATH = os.path.join(_lib.LIB_DIR, "ext", "naylis_torch.so")

_mod = None
_lock = threading.Lock()


def load():
    """Load (once) and return the extension module; raises if it is not built."""
    global _mod
    if _mod is not None:
        return _mod
    with _lock:
        if _mod is not None:
            return _mod
        import torch  # noqa: F401  (the extension links libtorch)
        _lib.load()
        if not os.path.exists(EXT_PATH):
            raise RuntimeError(
                f"naylis_amd: torch extension not built ({EXT_PATH} missing). "
                "Run `python -c 'import __graft_entry__ as g; g.build()'` or `python -m naylis_amd.build` first.")
        spec = importlib.util.spec_from_file_location("naylis_torch", EXT_PATH)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        _mod = mod
        return mod
