"""The tolerance metric itself: exact rounding passes, a real error does not."""

import torch

from tests import kda_cases as C


def test_correctly_rounded_bf16_has_zero_excess():
    ref = torch.randn(4096, generator=C.gen(1), dtype=torch.float64) * 1e-3
    x = ref.to(torch.bfloat16)
    assert C.out_err(x, ref) == 0.0
    # the plain metric on the same tensors can exceed the 2e-3 budget
    assert C.max_rel_err(x, ref) <= 2.0 ** -8


def test_planted_error_is_caught():
    ref = torch.randn(4096, generator=C.gen(2), dtype=torch.float64)
    bad = ref.clone()
    i = int(ref.abs().argmax())
    bad[i] *= 1.01  # a 1% error on the largest element
    assert C.out_err(bad.to(torch.bfloat16), ref) > 5e-3
    assert C.out_err(bad.float(), ref) > 5e-3


def test_fp32_outputs_use_the_plain_metric():
    ref = torch.randn(100, generator=C.gen(3), dtype=torch.float64)
    x = ref.float()
    assert C.out_err(x, ref) == C.max_rel_err(x, ref) < 1e-6


def test_empty_batches_compare_equal_and_shapes_must_match():
    empty = torch.zeros(1, 0, 4, 128)
    assert C.max_rel_err(empty, empty.double()) == 0.0
    assert C.out_err(empty.bfloat16(), empty.double()) == 0.0
    try:
        C.max_rel_err(torch.zeros(3), torch.zeros(4))
    except AssertionError:
        pass
    else:
        raise AssertionError("a shape mismatch must not pass")
