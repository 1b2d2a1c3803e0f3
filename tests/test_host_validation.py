"""Host-side validation of the torch operators, on the CPU.

The operators are also registered for host tensors so that their checks can
run here: every rule raises the reference's message text (callers match the
substrings, tests/integration/kda_ascendc_dispatch.py:52-58), and a request
that passes every rule still fails -- on the device check -- because there is
no CPU implementation. Mirrors the rejection tests of tests/ops/test_kda.py:149-229
for the rules this build keeps.
"""

import pytest
import torch

import sgl_glm53_ascend_ops  # noqa: F401
from sgl_glm53_ascend_ops.ops import (
    kda_prepared_varlen_chunk,
    kda_prepared_varlen_recurrent,
    kda_varlen_chunk,
    kda_varlen_recurrent,
    prepared_recurrent,
)

D = 128


def _case(heads=4, lengths=(1, 1, 1), prefill=False, D=D):
    T = sum(lengths)
    N = len(lengths)
    t = {n: torch.zeros(1, T, heads, D, dtype=torch.bfloat16) for n in ("q", "k", "v", "a")}
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    return dict(
        **t,
        b=torch.zeros(1, T, heads, dtype=torch.bfloat16),
        A_log=torch.zeros(heads),
        dt_bias=torch.zeros(heads * D),
        initial_state_source=torch.zeros(N + 1, heads, D, D).transpose(-1, -2),
        initial_state_indices=torch.arange(1, N + 1, dtype=torch.int32),
        cu_seqlens=torch.tensor(cu, dtype=torch.int32),
        lower_bound=-5.0,
        scale=D ** -0.5,
        prefill=prefill,
    )


def _mid(rows, steps, heads):
    return torch.zeros(rows, steps, heads, D, D).transpose(-1, -2)


@pytest.mark.parametrize("prefill", [False, True])
def test_valid_host_call_fails_on_device_check(prefill):
    with pytest.raises(RuntimeError, match="must be a CUDA"):
        kda_varlen_recurrent(**_case(prefill=prefill))


def test_rejects_transposed_state():
    case = _case()
    case["initial_state_source"] = case["initial_state_source"].transpose(-1, -2)
    with pytest.raises(RuntimeError, match="K-contiguous"):
        kda_varlen_recurrent(**case)


def test_rejects_transposed_intermediate_state():
    case = _case(16, (4,) * 3)
    case["intermediate_state"] = _mid(3, 4, 16).transpose(-1, -2)
    with pytest.raises(RuntimeError, match="K-contiguous"):
        kda_varlen_recurrent(**case)


def test_rejects_prefill_intermediate_state():
    case = _case(8, (128,), prefill=True)
    case["intermediate_state"] = _mid(1, 128, 8)
    with pytest.raises(RuntimeError, match="does not support intermediate_state"):
        kda_varlen_recurrent(**case)


def test_accepts_decode_intermediate_state_up_to_device():
    case = _case(16, (4,) * 3)
    case["intermediate_state"] = _mid(3, 4, 16)
    with pytest.raises(RuntimeError, match="must be a CUDA"):
        kda_varlen_recurrent(**case)


def test_rejects_fewer_tokens_than_requests():
    with pytest.raises(RuntimeError, match="one token per request"):
        kda_varlen_recurrent(**_case(16, (1, 1, 0)))


def test_rejects_decode_tracking():
    case = _case(16, (1, 1))
    case["track_state_indices"] = torch.tensor([1, 2], dtype=torch.int32)
    case["track_state_lens"] = torch.tensor([1, 1], dtype=torch.int32)
    with pytest.raises(RuntimeError, match="tracking is prefill-only"):
        kda_varlen_recurrent(**case)


def test_accepts_what_ascend_kernels_rejected_up_to_device():
    """H outside {4,8}/{16,32,64} and several prefill sequences are supported here."""
    for case in (_case(2, (128,), prefill=True), _case(8, (128, 128), prefill=True),
                 _case(12, (1, 1), prefill=False)):
        with pytest.raises(RuntimeError, match="must be a CUDA"):
            kda_varlen_recurrent(**case)


@pytest.mark.parametrize("name", ["q", "k", "v", "a", "b"])
def test_rejects_non_bf16(name):
    case = _case()
    case[name] = case[name].float()
    with pytest.raises(RuntimeError, match=f"{name} must be bf16"):
        kda_varlen_recurrent(**case)


def test_rejects_float_indices():
    case = _case()
    case["initial_state_indices"] = case["initial_state_indices"].float()
    with pytest.raises(RuntimeError, match="must be int32 or int64"):
        kda_varlen_recurrent(**case)


def test_rejects_head_mismatch():
    case = _case()
    case["v"] = torch.zeros(1, 3, 2, D, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="requires H == HV"):
        kda_varlen_recurrent(**case)


def test_rejects_unsupported_head_dim():
    case = _case(D=96)
    with pytest.raises(RuntimeError, match="requires K == V"):
        kda_varlen_recurrent(**case)


def test_rejects_bad_gate_params():
    case = _case()
    case["A_log"] = torch.zeros(3)
    with pytest.raises(RuntimeError, match="A_log must be fp32 with HV elements"):
        kda_varlen_recurrent(**case)
    case = _case()
    case["dt_bias"] = torch.zeros(5)
    with pytest.raises(RuntimeError, match="dt_bias must be fp32 with HV\\*K elements"):
        kda_varlen_recurrent(**case)


def test_chunk_accepts_unaligned_lengths_up_to_device():
    """The reference rejects length 100 ("multiple of 64"); ragged tails run here."""
    case = _case(1, (100,), prefill=True)
    with pytest.raises(RuntimeError, match="must be a CUDA"):
        kda_varlen_chunk(**case)


def test_chunk_rejects_head_dim_64():
    case = _case(2, (64,), prefill=True, D=64)
    with pytest.raises(RuntimeError, match="K == V == 128"):
        kda_varlen_chunk(**case)


def test_chunk_requires_track_lens():
    case = _case(2, (64,), prefill=True)
    case["track_state_indices"] = torch.tensor([1], dtype=torch.int32)
    with pytest.raises(RuntimeError, match="requires track_state_lens"):
        kda_varlen_chunk(**case)


def test_prepared_forms_validate():
    T, H = 4, 2
    q = torch.zeros(1, T, H, D, dtype=torch.bfloat16)
    g = torch.zeros(1, T, H, D)
    beta = torch.zeros(1, T, H)
    pool = torch.zeros(3, H, D, D).transpose(-1, -2)
    idx = torch.tensor([1, 2], dtype=torch.int32)
    cu = torch.tensor([0, 2, 4], dtype=torch.int32)
    for fn in (kda_prepared_varlen_recurrent, kda_prepared_varlen_chunk):
        with pytest.raises(RuntimeError, match="must be a CUDA"):
            fn(q, q, q, g, beta, initial_state_source=pool, initial_state_indices=idx,
               cu_seqlens=cu, scale=0.1)
        with pytest.raises(RuntimeError, match="g must be fp32"):
            fn(q, q, q, g.bfloat16(), beta, initial_state_source=pool,
               initial_state_indices=idx, cu_seqlens=cu, scale=0.1)
        with pytest.raises(RuntimeError, match="numReq\\+1"):
            fn(q, q, q, g, beta, initial_state_source=pool, initial_state_indices=idx,
               cu_seqlens=cu[:2], scale=0.1)


def test_prepared_recurrent_validates():
    H, T = 8, 4
    qn = torch.zeros(T * H, D)
    v = torch.zeros(T * H, D, dtype=torch.bfloat16)
    out = torch.zeros_like(v)
    state = torch.zeros(2, H, D, D)
    idx = torch.tensor([1], dtype=torch.int32)
    starts = torch.tensor([0, T], dtype=torch.int32)
    with pytest.raises(RuntimeError, match="must be a CUDA"):
        prepared_recurrent(qn, qn, v, qn, torch.zeros(T * H), out, state, idx, starts)
    with pytest.raises(RuntimeError, match="head_offset"):
        prepared_recurrent(qn, qn, v, qn, torch.zeros(T * H), out, state, idx, starts,
                           head_offset=2)
    with pytest.raises(RuntimeError, match="track_indices is required"):
        prepared_recurrent(qn, qn, v, qn, torch.zeros(T * H), out, state, idx, starts,
                           track_state=True)


@pytest.mark.parametrize("op", [kda_varlen_recurrent, kda_varlen_chunk])
def test_rejects_batched_tokens(op):
    case = _case(lengths=(1, 1), prefill=op is kda_varlen_chunk)
    for n in ("q", "k", "v", "a"):
        case[n] = torch.cat([case[n], case[n]])  # [2, T, H, D]
    case["b"] = torch.cat([case["b"], case["b"]])
    with pytest.raises(RuntimeError, match="expects one packed token batch"):
        op(**case)


def test_rejects_strided_gate_params():
    case = _case()
    case["dt_bias"] = torch.zeros(2 * 4 * D)[::2]
    with pytest.raises(RuntimeError, match="A_log and dt_bias must be contiguous"):
        kda_varlen_recurrent(**case)
