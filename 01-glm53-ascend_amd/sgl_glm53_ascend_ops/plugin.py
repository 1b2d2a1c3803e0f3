"""sglang plugin hook: route sglang's prepared KDA recurrence to this package.

Same contract as the reference plugin (sgl-glm53-ascend-ops/src/
sgl_glm53_ascend_ops/plugin.py:1-36): sglang's ``HookRegistry`` is imported at
module scope, so importing this module without sglang raises ImportError, and
``register()`` installs a REPLACE hook whose callable forwards every argument,
in order, to ``ops.kda.prepared_recurrent``. The target name is the
reference's own placeholder (``"SGLANG_TARGET_PATH"``, plugin.py:33); the
deployment that enables the plugin sets the real sglang path.
"""

from typing import Optional

import torch
from sglang.srt.plugins.hook_registry import HookRegistry, HookType

TARGET = "SGLANG_TARGET_PATH"


def _prepared_recurrent(
    qn: torch.Tensor,
    kn: torch.Tensor,
    v: torch.Tensor,
    gdecay: torch.Tensor,
    beta: torch.Tensor,
    out: torch.Tensor,
    state: torch.Tensor,
    indices: torch.Tensor,
    starts: torch.Tensor,
    track_indices: Optional[torch.Tensor] = None,
    track_lens: Optional[torch.Tensor] = None,
    track_state: bool = False,
    head_offset: int = 0,
):
    from .ops.kda import prepared_recurrent

    return prepared_recurrent(qn, kn, v, gdecay, beta, out, state, indices, starts,
                              track_indices, track_lens, track_state, head_offset)


def register() -> None:
    """Replace sglang's target with the native prepared recurrence."""
    HookRegistry.register(TARGET, _prepared_recurrent, HookType.REPLACE)
