"""Op-then-fallback dispatch of sglang's KDA recurrence (integration helper).

Same behaviour as the reference's dispatcher (tests/integration/
kda_ascendc_dispatch.py:1-101): call the native op where it applies, fall back
to the caller's implementation only on the op's deliberate rejections (the
same message markers), let every other error propagate, and count both paths
so a run that silently fell back everywhere cannot look like a pass.

sglang (and its Triton recurrence, the reference's fallback) is not installed
here, so the fallback is passed in; ``patch`` rebinds sglang's module attribute
when sglang is present, as the reference's ``patch`` does.
"""

from __future__ import annotations

from collections import Counter
from typing import Callable

# The op's deliberate TORCH_CHECK rejections (kda_ascendc_dispatch.py:52-58).
REJECTIONS = (
    "not implemented yet",
    "does not support",
    "supports H=",
    "expects one",
    "must be K-contiguous",
)


def native_recurrent(*, scale=None, **kwargs):
    """sglang's ``glm_kda_varlen_recurrent_npu`` keywords onto the native op.

    sglang lets ``scale`` default to ``K ** -0.5``; the op takes it explicitly.
    """
    from sgl_glm53_ascend_ops.ops.kda import kda_varlen_recurrent

    if scale is None:
        scale = kwargs["k"].shape[-1] ** -0.5
    return kda_varlen_recurrent(scale=scale, **kwargs)


class Dispatcher:
    """The native op where it applies, ``fallback`` where the op rejects the regime."""

    def __init__(self, fallback: Callable, op: Callable = native_recurrent):
        self.op = op
        self.fallback = fallback
        self.counts: Counter = Counter()
        self.fallbacks: Counter = Counter()

    def __call__(self, **kwargs):
        try:
            result = self.op(**kwargs)
        except RuntimeError as exc:
            message = str(exc)
            if not any(marker in message for marker in REJECTIONS):
                raise
            self.fallbacks[message.splitlines()[0].strip()] += 1
            return self.fallback(**kwargs)
        self.counts["native"] += 1
        return result

    def report(self) -> dict:
        return {
            "native_calls": self.counts["native"],
            "fallback_calls": sum(self.fallbacks.values()),
            "fallback_reasons": dict(self.fallbacks),
        }


def patch(module, attr: str = "glm_kda_varlen_recurrent_npu") -> Dispatcher:
    """Point ``module.attr`` (sglang's recurrence) at a dispatcher over the native
    op that falls back to the original function."""
    dispatcher = Dispatcher(fallback=getattr(module, attr))
    setattr(module, attr, dispatcher)
    return dispatcher
