"""Loader for the MI355X FlashAttention forward libraries.

Importing this package loads lib/libfa_mi355x_torch.so, which registers the
torch.ops.fa_mi355x operators (HIP kernels for gfx950 behind the C ABI in
lib/libfa_mi355x.so). There is no fallback: if the libraries are missing the
import fails, and calling an operator without a GPU raises.
"""
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(_HERE, "lib")
CORE_LIB = os.path.join(LIB_DIR, "libfa_mi355x.so")
TORCH_LIB = os.path.join(LIB_DIR, "libfa_mi355x_torch.so")

if not os.path.exists(TORCH_LIB):
    raise ImportError(
        f"fa_mi355x: {TORCH_LIB} is not built; run `python build.py` in {os.path.dirname(_HERE)}")

torch.ops.load_library(TORCH_LIB)
ops = torch.ops.fa_mi355x

from . import _fake  # noqa: E402,F401  (meta implementations for torch.compile)

__all__ = ["ops", "CORE_LIB", "TORCH_LIB", "LIB_DIR"]
