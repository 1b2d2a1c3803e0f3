"""Seeded random varlen cases for both ops against the CPU oracle.

Each case draws a head count on either side of the chunk scan's 16/32-column
switch (more than 32 (sequence, head) chains run 32-column scan groups on a
256-CU part), 1-6 sequences whose lengths favour chunk boundaries (1, 63, 64,
65, 127, 128, 129 tokens, or any length up to 300; in the prefill forms some
sequences are empty; one chunk set draws 9-80 sequences, enough chains for the
persistent scan), state slots with the
padding slot 0 mixed in, and, for most cases, a tracked prefix per sequence
into its own distinct slot (sometimes none, i.e. track slot 0). The chunk op is
checked against ``oracle.kda_ref.kda_chunk`` and the recurrent op against
``oracle.kda_ref.kda_recurrent`` (half of its cases in the prefill mode with
tracking, half in the decode mode, some of those with per-step checkpoints),
at the tolerance contract; slots that no sequence reads, writes or tracks must
come back byte-identical.
"""

import random

import pytest
import torch

from oracle import kda_ref as R
from tests import kda_cases as C

pytestmark = pytest.mark.gpu

DEV = "cuda"
HEADS = (1, 2, 3, 5, 8, 17, 33, 40)
LENGTHS = (1, 2, 63, 64, 65, 127, 128, 129)


def _draw(seed, max_len=300, track_prob=0.6, empty_prob=0.0, many=False):
    rng = random.Random(seed)
    heads = rng.choice(HEADS)
    if many:
        # 9-80 sequences with more (sequence, head) chains than the 64 scan
        # teams of a 256-CU part: the persistent scan's item streams (at most
        # about 20k token-heads, so the oracle stays quick)
        n = rng.randint(max(9, 65 // heads + 1), max(9, min(80, 20000 // (heads * 128))))
    else:
        n = rng.randint(1, 6)
    lengths = [rng.choice(LENGTHS) if rng.random() < 0.6 else rng.randint(1, max_len)
               for _ in range(n)]
    lengths = [0 if rng.random() < empty_prob else min(x, max_len) for x in lengths]
    slots = 2 * n + 2
    state_slots = rng.sample(range(1, slots), n)
    indices = [0 if rng.random() < 0.2 else s for s in state_slots]
    track = None
    if rng.random() < track_prob:
        free = [s for s in range(1, slots) if s not in state_slots]
        tidx = [s if rng.random() < 0.75 else 0 for s in rng.sample(free, n)]
        tlens = [rng.randint(0, length) for length in lengths]
        track = (tidx, tlens)
    return heads, lengths, slots, indices, track


def _untouched(case, indices, track, slots):
    used = set(s for s in indices if s > 0)
    if track is not None:
        used |= set(s for s in track[0] if s > 0)
    return [s for s in range(slots) if s not in used]


def _prepared(case):
    return R.kda_prepare(case.A_log, case.a, case.dt_bias, case.q, case.k, case.b,
                         case.lower_bound, case.scale)


def _check_chunk(gpu_ops, draw, case_seed, label):
    heads, lengths, slots, indices, track = draw
    label = f"{label}: H={heads} lengths={lengths} indices={indices} track={track}"
    print(label, flush=True)
    case = C.raw_case(heads, lengths, indices=indices, slots=slots, seed=case_seed, track=track)
    pool = C.to_dev(case.pool, DEV)
    out = gpu_ops.kda_varlen_chunk(prefill=True, **case.kwargs(DEV, pool=pool))
    torch.cuda.synchronize()
    ref_pool = C.clone_pool(case.pool)
    qn, kn, g, beta = _prepared(case)
    ref = R.kda_chunk(qn, kn, case.v, g, beta, state_pool=ref_pool, state_indices=case.indices,
                      cu_seqlens=case.cu_seqlens, track_state_indices=case.track_indices,
                      track_state_lens=case.track_lens, out_dtype=torch.float32)
    C.assert_out(out.cpu(), ref, C.OUT_TOL, f"{label} output")
    C.assert_rel(pool.cpu(), ref_pool, C.STATE_TOL, f"{label} pool")
    other = _untouched(case, indices, track, slots)
    assert torch.equal(pool.cpu()[other], case.pool[other]), f"{label}: an unused slot was written"


@pytest.mark.parametrize("seed", range(16))
def test_random_chunk_matches_oracle(gpu_ops, seed):
    _check_chunk(gpu_ops, _draw(1000 + seed, empty_prob=0.1), 7000 + seed, f"seed {seed}")


@pytest.mark.parametrize("seed", range(10))
def test_random_chunk_many_sequences(gpu_ops, seed):
    _check_chunk(gpu_ops, _draw(3000 + seed, max_len=400, empty_prob=0.05, many=True), 10000 + seed,
                 f"many-sequence seed {seed}")


@pytest.mark.parametrize("seed", range(12))
def test_random_recurrent_matches_oracle(gpu_ops, seed):
    # the op's regime rules (as the reference's): tracking is prefill-only,
    # checkpoints are decode-only
    prefill = seed % 2 == 0
    checkpoints = seed % 4 == 3
    heads, lengths, slots, indices, track = _draw(2000 + seed, max_len=8 if checkpoints else 300,
                                                  track_prob=0.6 if prefill else 0.0,
                                                  empty_prob=0.1 if prefill else 0.0)
    label = (f"seed {seed}: H={heads} lengths={lengths} indices={indices} track={track} "
             f"prefill={prefill} checkpoints={checkpoints}")
    print(label, flush=True)
    case = C.raw_case(heads, lengths, indices=indices, slots=slots, seed=8000 + seed, track=track)
    pool = C.to_dev(case.pool, DEV)
    mid_dev = mid_ref = noise = None
    if checkpoints:
        steps = max(lengths)
        noise = (torch.randn(len(lengths), steps, heads, 128, 128, generator=C.gen(9000 + seed))
                 * 0.1).transpose(-1, -2)
        mid_dev = noise.transpose(-1, -2).contiguous().to(DEV).transpose(-1, -2)
        mid_ref = noise.clone()
    out = gpu_ops.kda_varlen_recurrent(intermediate_state=mid_dev, prefill=prefill,
                                       **case.kwargs(DEV, pool=pool))
    torch.cuda.synchronize()
    ref_pool = C.clone_pool(case.pool)
    qn, kn, g, beta = _prepared(case)
    ref = R.kda_recurrent(qn, kn, case.v, g, beta, state_pool=ref_pool,
                          state_indices=case.indices, cu_seqlens=case.cu_seqlens,
                          intermediate_state=mid_ref, track_state_indices=case.track_indices,
                          track_state_lens=case.track_lens, out_dtype=torch.float32)
    C.assert_out(out.cpu(), ref, C.OUT_TOL, f"{label} output")
    if checkpoints:
        got = mid_dev.cpu()
        for n, length in enumerate(lengths):
            if indices[n] > 0:
                C.assert_rel(got[n, :length], mid_ref[n, :length], C.STATE_TOL,
                             f"{label} checkpoints of request {n}")
            else:
                assert torch.equal(got[n], noise[n]), f"{label}: slot-0 request {n} checkpointed"
        assert torch.equal(pool.cpu(), case.pool), f"{label}: checkpointing must not write back"
        return
    C.assert_rel(pool.cpu(), ref_pool, C.STATE_TOL, f"{label} pool")
    other = _untouched(case, indices, track, slots)
    assert torch.equal(pool.cpu()[other], case.pool[other]), f"{label}: an unused slot was written"
