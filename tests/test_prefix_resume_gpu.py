"""Prefix tracking leaves the run unchanged, and a tracked state resumes it.

The reference's prefix suite (tests/integration/test_glm53_kda_prefix_ascendc.py:
97-182) asserts, for a prefill with ``track_state_indices/lens``:

* the output and every source slot are bit-identical to the same call
  without tracking (:125-126), and every slot neither read nor tracked is
  untouched (:127-129);
* the checkpoint equals the state a prefill of the prefix alone leaves
  (:143-160);
* the checkpoint fed back as the initial state of the suffix reproduces the
  full run's suffix output and final state (:161-167).

Here the same three checks run for both operators: ``kda_varlen_recurrent``
(``prefill=True``: the token loop for short requests, the chunked kernels from
128 tokens per request) and ``kda_varlen_chunk``, including a checkpoint
inside a ragged last chunk and a single long sequence on few heads, which
runs in the affine form (segments scanned in parallel and combined) or as
pipelined scan segments (the tracked prefix then ends in a later segment). Suffix outputs and final states are checked against the fp32 oracle
of the full run at the tolerance contract, and final states also against the
full GPU run.
"""

import dataclasses

import pytest
import torch

from oracle import kda_ref as R
from tests import kda_cases as C

pytestmark = pytest.mark.gpu

DEV = "cuda"
SLOTS = 12


def _call(ops, op, case, pool):
    kw = case.kwargs(DEV, pool=pool)
    if op == "recurrent":
        out = ops.kda_varlen_recurrent(prefill=True, **kw)
    else:
        out = ops.kda_varlen_chunk(prefill=True, **kw)
    torch.cuda.synchronize()
    return out


def _sub(case, t0, t1, index):
    """The tokens [t0, t1) of ``case`` as one request on slot ``index``."""
    cut = lambda t: t[:, t0:t1].contiguous()  # noqa: E731
    return dataclasses.replace(
        case, q=cut(case.q), k=cut(case.k), v=cut(case.v), a=cut(case.a), b=cut(case.b),
        indices=torch.tensor([index], dtype=torch.int32),
        cu_seqlens=torch.tensor([0, t1 - t0], dtype=torch.int32),
        track_indices=None, track_lens=None)


def _oracle(case, pool_cpu):
    qn, kn, g, beta = R.kda_prepare(case.A_log, case.a, case.dt_bias, case.q, case.k, case.b,
                                    case.lower_bound, case.scale)
    return R.kda_recurrent(qn, kn, case.v, g, beta, state_pool=pool_cpu,
                           state_indices=case.indices, cu_seqlens=case.cu_seqlens,
                           out_dtype=torch.float32)


# (label, heads, lengths, cuts, source slots, destination slots, raw lower bound)
CASES = [
    # the reference's own layout: three short requests, one of them untracked
    ("short varlen", 4, (100, 37, 63), (50, 37, 0), (3, 1, 5), (9, 7, 0), -5.0),
    # cuts inside ragged last chunks, one request on the padding slot 0;
    # 400 tokens over 2 requests take the chunked route in the recurrent op
    ("ragged tails", 4, (300, 100), (290, 64), (2, 0), (6, 8), -5.0),
    # a chunk boundary and a cut one token past it, 3 requests of 130-260
    ("chunk boundaries", 2, (260, 130, 200), (128, 65, 200), (1, 4, 10), (11, 2, 3), -5.0),
    # one long sequence on one head: the affine form (eight segments of 32
    # chunks), the checkpoint in the fifth
    ("two segments", 1, (16384,), (9000,), (1,), (3,), -5.0),
    # the same with weak decay (raw lower bound -2e-4): the checkpoint and the
    # resumed suffix depend on the combined segment transitions
    ("weak decay segments", 1, (16384,), (9000,), (1,), (3,), -2e-4),
    # 16 heads: the pipelined scan segments (four of 64 chunks)
    ("pipelined segments", 16, (16384,), (5000,), (1,), (3,), -5.0),
    # 8 heads: the affine form with two segments of 64 chunks, the checkpoint
    # in the second
    ("two affine segments", 8, (8192,), (5000,), (1,), (3,), -2e-4),
]


@pytest.mark.parametrize("op", ["recurrent", "chunk"])
@pytest.mark.parametrize("label,heads,lengths,cuts,slots,dests,lower_bound", CASES,
                         ids=[c[0].replace(" ", "-") for c in CASES])
def test_tracking_is_invisible_and_resumes(gpu_ops, op, label, heads, lengths, cuts, slots,
                                           dests, lower_bound):
    tracked_case = C.raw_case(heads, lengths, indices=list(slots), slots=SLOTS,
                              seed=194195 + sum(lengths), track=(list(dests), list(cuts)),
                              lower_bound=lower_bound)
    plain_case = dataclasses.replace(tracked_case, track_indices=None, track_lens=None)

    # 1. tracking changes nothing but the destination slots
    pool_plain = C.to_dev(tracked_case.pool, DEV)
    out_plain = _call(gpu_ops, op, plain_case, pool_plain)
    pool_tr = C.to_dev(tracked_case.pool, DEV)
    out_tr = _call(gpu_ops, op, tracked_case, pool_tr)
    assert torch.equal(out_tr, out_plain), f"{label}: tracking changed the output"
    src = [s for s in slots if s > 0]
    assert torch.equal(pool_tr[src], pool_plain[src]), f"{label}: tracking changed a source slot"
    untouched = sorted(set(range(SLOTS)) - set(slots) - set(dests) | {0})
    assert torch.equal(pool_tr.cpu()[untouched], tracked_case.pool[untouched]), (
        f"{label}: a slot neither read nor tracked changed")

    ref_pool = C.clone_pool(tracked_case.pool)
    ref_out = _oracle(plain_case, ref_pool)
    begin = 0
    for row, (length, cut, slot, dest) in enumerate(zip(lengths, cuts, slots, dests)):
        if dest == 0:
            begin += length
            continue
        checkpoint = pool_tr[dest].clone()
        # 2. the checkpoint is the state the prefix alone leaves
        prefix_pool = C.to_dev(tracked_case.pool, DEV)
        if cut > 0:
            _call(gpu_ops, op, _sub(tracked_case, begin, begin + cut, slot), prefix_pool)
        if slot > 0:
            prefix_state = prefix_pool[slot]
        elif cut == 0:
            prefix_state = torch.zeros_like(checkpoint)
        else:  # slot 0 is never written: take the prefix run's state from the oracle
            p = torch.zeros(2, heads, 128, 128).transpose(-1, -2)
            _oracle(_sub(tracked_case, begin, begin + cut, 1), p)
            prefix_state = p[1].to(DEV)
        C.assert_rel(checkpoint.cpu(), prefix_state.cpu(), C.STATE_TOL,
                     f"{label} request {row}: checkpoint vs prefix run")
        # 3. resumed from the checkpoint, the suffix reproduces the full run
        if cut < length:
            resume_slot = SLOTS - 1 if slot == 0 else slot
            pool_r = C.to_dev(tracked_case.pool, DEV)
            pool_r[resume_slot] = checkpoint
            suffix = _call(gpu_ops, op, _sub(tracked_case, begin + cut, begin + length,
                                             resume_slot), pool_r)
            C.assert_out(suffix.cpu(), ref_out[:, begin + cut:begin + length], C.OUT_TOL,
                         f"{label} request {row}: resumed suffix output vs oracle")
            if slot > 0:
                C.assert_rel(pool_r[resume_slot].cpu(), ref_pool[slot], C.STATE_TOL,
                             f"{label} request {row}: resumed final state vs oracle")
                C.assert_rel(pool_r[resume_slot].cpu(), pool_plain[slot].cpu(), C.STATE_TOL,
                             f"{label} request {row}: resumed final state vs full run")
        begin += length


def test_token_loop_checkpoint_is_bitwise_the_prefix_run(gpu_ops):
    """In the token loop (short requests) the tracked state after step ``cut``
    is computed exactly as a prefill of the first ``cut`` tokens computes its
    final state, so the two are bit-identical."""
    case = C.raw_case(8, (90, 41), indices=[2, 5], slots=SLOTS, seed=808,
                      track=([7, 9], [33, 41]))
    pool = C.to_dev(case.pool, DEV)
    _call(gpu_ops, "recurrent", case, pool)
    begin = 0
    for length, cut, slot, dest in zip((90, 41), (33, 41), (2, 5), (7, 9)):
        prefix_pool = C.to_dev(case.pool, DEV)
        _call(gpu_ops, "recurrent", _sub(case, begin, begin + cut, slot), prefix_pool)
        assert torch.equal(pool[dest], prefix_pool[slot]), f"checkpoint of slot {slot}"
        begin += length
