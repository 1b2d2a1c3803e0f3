"""The C-ABI library loads without a GPU and exports every symbol kda_abi.h declares.

No compute call is made here: only the argument checks that return before any
HIP call (a null argument block, an unsupported head dimension).
"""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "kda_abi.h")
LIB = os.path.join(ROOT, "01-glm53-ascend_amd", "sgl_glm53_ascend_ops", "libkda_amd.so")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(kda_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


@pytest.fixture(scope="module")
def lib():
    assert os.path.exists(LIB), f"{LIB} missing: run python 01-glm53-ascend_amd/kda_build.py"
    return ctypes.CDLL(LIB)


def test_header_declares_the_entry_points():
    names = _declared_functions()
    for expected in ("kda_recurrent_launch", "kda_chunk_launch", "kda_chunk_workspace_bytes",
                     "kda_status_string", "kda_abi_version"):
        assert expected in names


def test_every_declared_symbol_is_exported(lib):
    missing = [n for n in _declared_functions() if not hasattr(lib, n)]
    assert not missing, f"declared in kda_abi.h but not exported: {missing}"


def test_version_and_status_text(lib):
    lib.kda_abi_version.restype = ctypes.c_int
    assert lib.kda_abi_version() == 1
    lib.kda_status_string.restype = ctypes.c_char_p
    lib.kda_status_string.argtypes = [ctypes.c_int]
    assert lib.kda_status_string(0) == b"ok"
    assert b"unsupported" in lib.kda_status_string(2)


def test_argument_checks_return_before_any_device_call(lib):
    lib.kda_recurrent_launch.restype = ctypes.c_int
    lib.kda_recurrent_launch.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    assert lib.kda_recurrent_launch(None, None) == 1  # KDA_ERR_INVALID_ARGUMENT
    lib.kda_chunk_launch.restype = ctypes.c_int
    lib.kda_chunk_launch.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                     ctypes.c_void_p]
    assert lib.kda_chunk_launch(None, None, 0, None) != 0
