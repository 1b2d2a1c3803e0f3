"""The package builds from pip: ``pip install ./01-glm53-ascend_amd`` compiles
both native libraries (hipcc for gfx950, g++ against torch) and installs them
with the Python sources, and the installed copy loads and registers the
operators. Offline, pip needs ``--no-build-isolation`` (the build uses the
installed setuptools, torch and ROCm). No GPU is used."""

import ctypes
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_SRC = os.path.join(ROOT, "01-glm53-ascend_amd")


def test_pip_install_builds_both_libraries(tmp_path):
    target = tmp_path / "site"
    r = subprocess.run([sys.executable, "-m", "pip", "install", "--no-build-isolation", "--no-deps",
                        "--target", str(target), PKG_SRC],
                       capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    pkg = target / "sgl_glm53_ascend_ops"
    for lib in ("libkda_amd.so", "sgl_glm53_ascend_ops_lib.so"):
        assert (pkg / lib).exists(), f"{lib} not installed"
    abi = ctypes.CDLL(str(pkg / "libkda_amd.so"))
    for sym in ("kda_recurrent_launch", "kda_chunk_launch", "kda_chunk_launch_noalloc",
                "kda_chunk_workspace_bytes", "kda_status_string", "kda_abi_version"):
        assert hasattr(abi, sym), sym
    # the installed copy (not the source tree) registers the operators
    code = ("import sys; sys.path.insert(0, sys.argv[1]); import torch, sgl_glm53_ascend_ops as m; "
            "assert m.__file__.startswith(sys.argv[1]), m.__file__; "
            "ops = torch.ops.sgl_glm53_ascend; "
            "[getattr(ops, n) for n in ('kda_varlen_recurrent', 'kda_varlen_chunk', "
            "'prepared_recurrent', 'kda_prepared_varlen_chunk')]; print('OK')")
    r = subprocess.run([sys.executable, "-c", code, str(target)], capture_output=True, text=True,
                       timeout=300, cwd=str(tmp_path))
    assert r.returncode == 0 and "OK" in r.stdout, r.stdout[-2000:] + r.stderr[-2000:]
