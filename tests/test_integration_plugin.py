"""sglang integration pieces on the CPU: the plugin hook and the op-then-fallback
dispatcher (reference: src/sgl_glm53_ascend_ops/plugin.py:1-35,
tests/integration/kda_ascendc_dispatch.py:52-96).

sglang is not installed, so its ``HookRegistry`` is replaced by a recording
stand-in module; no kernel runs here.
"""

import enum
import importlib
import sys
import types

import pytest

from tests.integration import kda_amd_dispatch as D


def _fake_sglang(monkeypatch):
    calls = []

    class HookType(enum.Enum):
        REPLACE = "replace"
        BEFORE = "before"

    class HookRegistry:
        @staticmethod
        def register(target, fn, kind):
            calls.append((target, fn, kind))

    mods = {}
    for name in ("sglang", "sglang.srt", "sglang.srt.plugins", "sglang.srt.plugins.hook_registry"):
        mods[name] = types.ModuleType(name)
    mods["sglang.srt.plugins.hook_registry"].HookRegistry = HookRegistry
    mods["sglang.srt.plugins.hook_registry"].HookType = HookType
    for name, mod in mods.items():
        monkeypatch.setitem(sys.modules, name, mod)
    monkeypatch.delitem(sys.modules, "sgl_glm53_ascend_ops.plugin", raising=False)
    return calls, HookType


def test_plugin_registers_a_replace_hook_that_forwards(monkeypatch):
    calls, HookType = _fake_sglang(monkeypatch)
    plugin = importlib.import_module("sgl_glm53_ascend_ops.plugin")
    plugin.register()
    assert len(calls) == 1
    target, fn, kind = calls[0]
    assert target == plugin.TARGET == "SGLANG_TARGET_PATH"
    assert kind is HookType.REPLACE

    import sgl_glm53_ascend_ops.ops.kda as kda

    seen = []
    monkeypatch.setattr(kda, "prepared_recurrent", lambda *args: seen.append(args) or "ran")
    args = tuple(f"arg{i}" for i in range(9))
    assert fn(*args) == "ran"
    assert seen[-1] == args + (None, None, False, 0)
    assert fn(*args, track_indices="ti", track_lens="tl", track_state=True, head_offset=4) == "ran"
    assert seen[-1] == args + ("ti", "tl", True, 4)


def test_plugin_import_needs_sglang(monkeypatch):
    monkeypatch.setitem(sys.modules, "sglang", None)
    monkeypatch.delitem(sys.modules, "sgl_glm53_ascend_ops.plugin", raising=False)
    with pytest.raises(ImportError):
        importlib.import_module("sgl_glm53_ascend_ops.plugin")


@pytest.mark.parametrize("marker", D.REJECTIONS)
def test_dispatcher_falls_back_on_each_rejection(marker):
    def op(**kw):
        raise RuntimeError(f"kda_varlen_recurrent {marker} this regime\ndetails")

    fallback_calls = []
    disp = D.Dispatcher(fallback=lambda **kw: fallback_calls.append(kw) or "fallback", op=op)
    assert disp(x=1) == "fallback"
    assert fallback_calls == [{"x": 1}]
    rep = disp.report()
    assert rep["native_calls"] == 0 and rep["fallback_calls"] == 1
    assert list(rep["fallback_reasons"]) == [f"kda_varlen_recurrent {marker} this regime"]


def test_dispatcher_propagates_other_errors():
    def op(**kw):
        raise RuntimeError("HIP error: invalid device pointer")

    disp = D.Dispatcher(fallback=lambda **kw: pytest.fail("must not fall back"), op=op)
    with pytest.raises(RuntimeError, match="invalid device pointer"):
        disp(x=1)
    with pytest.raises(ValueError):
        D.Dispatcher(fallback=lambda **kw: None, op=lambda **kw: (_ for _ in ()).throw(ValueError("x")))()


def test_dispatcher_counts_native_calls_and_patch_rebinds():
    module = types.SimpleNamespace(glm_kda_varlen_recurrent_npu=lambda **kw: "triton")
    disp = D.patch(module)
    assert module.glm_kda_varlen_recurrent_npu is disp
    assert disp.fallback(q=None) == "triton"
    disp.op = lambda **kw: "native"
    assert module.glm_kda_varlen_recurrent_npu(q=1) == "native"
    assert disp.report() == {"native_calls": 1, "fallback_calls": 0, "fallback_reasons": {}}
