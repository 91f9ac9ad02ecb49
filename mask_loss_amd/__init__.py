"""MI355X (gfx950) implementation of mask_loss's pairwise mask cost ->
assignment -> matched-loss path.

Importing this package loads the in-tree extension module and registers it as
the top-level module ``mask_loss`` (the name the reference's ``functions/``
import), so both ``import mask_loss`` and ``mask_loss_amd.functions`` work.
The extension is HIP-only: if it has not been built this import fails.
"""
import importlib.util
import os
import sys

import torch  # noqa: F401  (loads the HIP runtime the extension links against)

_HERE = os.path.dirname(os.path.abspath(__file__))


def _load_ext():
    if "mask_loss" in sys.modules and getattr(sys.modules["mask_loss"], "__backend__", None):
        return sys.modules["mask_loss"]
    import sysconfig
    path = os.path.join(_HERE, "mask_loss" + (sysconfig.get_config_var("EXT_SUFFIX") or ".so"))
    if not os.path.exists(path):
        raise ImportError(
            f"mask_loss HIP extension not built ({path} missing); run "
            "`python -m mask_loss_amd._build` or __graft_entry__.build()")
    spec = importlib.util.spec_from_file_location("mask_loss", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    sys.modules["mask_loss"] = mod
    return mod


mask_loss = _load_ext()
HIP_LIBRARY = os.path.join(_HERE, "libmask_loss_hip.so")

__all__ = ["mask_loss", "HIP_LIBRARY"]
