"""KDA operators for SGLang's GLM-5.3 backend on AMD Instinct MI355X (gfx950).

Drop-in for the reference package of the same name: importing it loads the
native operator library, which registers ``torch.ops.sgl_glm53_ascend.*``
(reference: sgl-glm53-ascend-ops/src/sgl_glm53_ascend_ops/__init__.py:1-5).
"""

from ._load import abi, chunk_workspace_bytes, load_library

load_library()
