"""The op-then-fallback dispatcher with the native op on the GPU (the
reference's tests/integration/kda_ascendc_dispatch.py:64-87).

A K-contiguous pool takes the native path and matches the oracle; a plain
[slots, H, K, V]-contiguous pool is one of the op's deliberate rejections
("must be K-contiguous") and goes to the fallback, counted in the report.
"""

import pytest
import torch

from oracle import kda_ref as R
from tests import kda_cases as C
from tests.integration import kda_amd_dispatch as D

pytestmark = pytest.mark.gpu

DEV = "cuda"


def test_dispatch_native_then_fallback(gpu_ops):
    case = C.raw_case(4, (1,) * 5, slots=8, seed=70)
    fallback_calls = []
    disp = D.Dispatcher(fallback=lambda **kw: fallback_calls.append(kw) or "fallback")

    pool = C.to_dev(case.pool, DEV)
    kw = case.kwargs(DEV, pool=pool)
    kw.pop("scale")  # sglang's default: K ** -0.5, the case's own scale
    out = disp(**kw, prefill=False)
    torch.cuda.synchronize()
    ref_pool = C.clone_pool(case.pool)
    qn, kn, g, beta = R.kda_prepare(case.A_log, case.a, case.dt_bias, case.q, case.k, case.b,
                                    case.lower_bound, case.scale)
    ref = R.kda_recurrent(qn, kn, case.v, g, beta, state_pool=ref_pool, state_indices=case.indices,
                          cu_seqlens=case.cu_seqlens, out_dtype=torch.float32)
    C.assert_out(out.cpu(), ref, C.OUT_TOL, "native output")
    C.assert_rel(pool.cpu(), ref_pool, C.STATE_TOL, "native pool")

    plain = case.pool.contiguous().to(DEV)  # [slots, H, K, V] with V contiguous
    assert plain.stride(2) != 1
    kw = case.kwargs(DEV, pool=plain)
    assert disp(**kw, prefill=False) == "fallback"
    assert len(fallback_calls) == 1
    rep = disp.report()
    assert rep["native_calls"] == 1 and rep["fallback_calls"] == 1
    assert any("must be K-contiguous" in r for r in rep["fallback_reasons"])
