"""Locate and load the native operator library.

Mirrors the reference loader (sgl-glm53-ascend-ops/src/sgl_glm53_ascend_ops/
_load.py:13-48): search the package directory for
``sgl_glm53_ascend_ops_lib*.so`` and hand it to ``torch.ops.load_library``.
A missing library is an error, never a silent fallback: there is no
CPU/eager implementation of these operators.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch

_LOADED = False
_LIB_NAME = "sgl_glm53_ascend_ops_lib"
_ABI_NAME = "libkda_amd.so"


def package_dir() -> Path:
    return Path(__file__).resolve().parent


def _find_library() -> Path:
    here = package_dir()
    found = sorted(here.glob(f"{_LIB_NAME}*.so"))
    if not found:
        raise RuntimeError(
            f"Cannot find {_LIB_NAME}*.so in {here}. Build it with "
            "'python 01-glm53-ascend_amd/kda_build.py' (hipcc, gfx950)."
        )
    return found[0]


def abi_library_path() -> Path:
    """Path of the C-ABI library (``include/kda_abi.h``), for ctypes users."""
    p = package_dir() / _ABI_NAME
    if not p.exists():
        raise RuntimeError(f"Cannot find {_ABI_NAME} in {package_dir()}; build it first.")
    return p


def load_library() -> None:
    global _LOADED
    if _LOADED:
        return
    torch.ops.load_library(str(_find_library()))
    _LOADED = True


_ABI = None


def abi() -> ctypes.CDLL:
    """The C-ABI library (``include/kda_abi.h``) through ctypes, loaded once."""
    global _ABI
    if _ABI is None:
        lib = ctypes.CDLL(str(abi_library_path()))
        lib.kda_chunk_workspace_bytes.restype = ctypes.c_size_t
        lib.kda_chunk_workspace_bytes.argtypes = [ctypes.c_int32] * 4
        _ABI = lib
    return _ABI


def chunk_workspace_bytes(num_tokens: int, num_seqs: int, num_heads: int,
                          head_dim: int = 128) -> int:
    """Device scratch the chunked prefill takes for these sizes
    (``kda_chunk_workspace_bytes``)."""
    return int(abi().kda_chunk_workspace_bytes(num_tokens, num_seqs, num_heads, head_dim))
