"""GPU parity of the chunked prefill (bf16 MFMA, fp32 state) against the oracle.

Small cases follow the reference's own chunk suite (tests/ops/test_kda_chunk.py:
202-249): one and several chunks, several sequences, the zero slot, every
position of the tracked checkpoint, untouched slots; plus what this build adds:
sequence lengths that are not a multiple of 64 (the reference rejects them,
:245-249). They are checked against the CPU oracle's chunked form
(``oracle.kda_ref.kda_chunk``, the restatement of kda_python.py:41-188).

BASELINE configs 3, 4 and 5 run at full size. At those sizes the CPU oracle
would take minutes, so the reference there is this build's recurrent kernel
run in fp32 (bf16 inputs widened exactly; that kernel is itself pinned to the
oracle at <= 1e-5 by test_recurrent_gpu.py) -- the chunk == recurrent identity
the reference cross-checks its own anchors with (kda_python.py:312-344).
"""

import pytest
import torch

from oracle import kda_ref as R
from tests import kda_cases as C

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _oracle_chunk(case, pool_cpu):
    qn, kn, g, beta = R.kda_prepare(case.A_log, case.a, case.dt_bias, case.q, case.k, case.b,
                                    case.lower_bound, case.scale)
    return R.kda_chunk(qn, kn, case.v, g, beta, state_pool=pool_cpu, state_indices=case.indices,
                       cu_seqlens=case.cu_seqlens, track_state_indices=case.track_indices,
                       track_state_lens=case.track_lens, out_dtype=torch.float32)


def _run_chunk(ops, case, index_dtype=torch.int32):
    pool = C.to_dev(case.pool, DEV)
    out = ops.kda_varlen_chunk(prefill=True, **case.kwargs(DEV, pool=pool, index_dtype=index_dtype))
    torch.cuda.synchronize()
    return out, pool


# (label, heads, cu_seqlens lengths, slots, track) -- test_kda_chunk.py:203-214
REF_CASES = [
    ("one chunk", 1, (64,), [1], None),
    ("two chunks", 1, (128,), [1], None),
    ("four chunks", 2, (256,), [1], None),
    ("two sequences", 2, (128, 128), [1, 2], None),
    ("ragged varlen", 1, (64, 128, 64), [1, 2, 3], None),
    ("zero slot", 1, (128,), [0], None),
    ("track at 0", 2, (128,), [1], ([4], [0])),
    ("track mid-chunk", 2, (128,), [1], ([4], [32])),
    ("track on boundary", 2, (128,), [1], ([4], [64])),
    ("track at end", 1, (192,), [1], ([4], [192])),
    # beyond the reference: lengths that are not a multiple of 64
    ("unaligned 100", 1, (100,), [1], None),
    ("unaligned varlen", 3, (1, 37, 100, 64, 130), [1, 2, 3, 0, 5], None),
    ("track in ragged tail", 2, (100, 37), [1, 2], ([6, 0], [90, 3])),
    ("track end of ragged", 2, (100,), [1], ([6], [100])),
    # more than 32 (sequence, head) chains: the scan runs 32-column groups
    ("wide groups varlen", 40, (130, 64, 37), [1, 2, 3], ([4, 0, 5], [100, 0, 20])),
    ("wide groups zero slot", 33, (70,), [0], None),
]


@pytest.mark.parametrize("label,heads,lengths,slots,track", REF_CASES,
                         ids=[c[0].replace(" ", "-") for c in REF_CASES])
def test_chunk_matches_oracle(gpu_ops, label, heads, lengths, slots, track):
    case = C.raw_case(heads, lengths, indices=slots, slots=8, seed=20261103 + len(label),
                      track=track)
    out, pool = _run_chunk(gpu_ops, case)
    ref_pool = C.clone_pool(case.pool)
    ref = _oracle_chunk(case, ref_pool)
    C.assert_out(out.cpu(), ref, C.OUT_TOL, f"{label} output")
    C.assert_rel(pool.cpu(), ref_pool, C.STATE_TOL, f"{label} pool")
    touched = set(s for s in slots if s > 0)
    if track is not None:
        touched |= set(s for s in track[0] if s > 0)
    other = [s for s in range(8) if s not in touched]
    assert torch.equal(pool.cpu()[other], case.pool[other]), "an unindexed slot was written"


def test_chunk_leaves_other_slots_untouched(gpu_ops):
    case = C.raw_case(2, (128,), indices=[3], slots=8, seed=3)
    _, pool = _run_chunk(gpu_ops, case)
    got = pool.cpu()
    other = [s for s in range(8) if s != 3]
    assert torch.equal(got[other], case.pool[other])
    assert not torch.equal(got[3], case.pool[3])


def test_chunk_index_dtypes_bit_identical(gpu_ops):
    case = C.raw_case(4, (257, 64), indices=[3, 1], slots=6, seed=5, track=([5, 0], [64, 0]))
    base_out, base_pool = _run_chunk(gpu_ops, case)
    out, pool = _run_chunk(gpu_ops, case, index_dtype=torch.int64)
    assert out.float().abs().sum().item() > 0
    assert torch.equal(out, base_out)
    assert torch.equal(pool.cpu(), base_pool.cpu())


@pytest.mark.parametrize("heads", [2, 40])
def test_chunk_tokens_outside_sequences_are_zero(gpu_ops, heads):
    case = C.raw_case(heads, (70, 30), slots=4, seed=8)
    T = case.q.shape[1]
    case.cu_seqlens = torch.tensor([0, 70, T - 5], dtype=torch.int32)
    out, _ = _run_chunk(gpu_ops, case)
    out = out.cpu()
    assert torch.equal(out[0, T - 5:], torch.zeros_like(out[0, T - 5:]))
    ref_pool = C.clone_pool(case.pool)
    C.assert_out(out, _oracle_chunk(case, ref_pool), C.OUT_TOL, "output")


def test_chunk_sequences_are_independent(gpu_ops):
    case = C.raw_case(2, (70, 90, 40), slots=5, seed=9)
    out1, _ = _run_chunk(gpu_ops, case)
    case.v = case.v.clone()
    case.v[0, 160:] += 1.0
    out2, _ = _run_chunk(gpu_ops, case)
    assert torch.equal(out1[0, :160], out2[0, :160])
    assert not torch.equal(out1[0, 160:], out2[0, 160:])


# --- prepared gates, BASELINE configs -----------------------------------------


def _prepared_dev(case):
    return {n: getattr(case, n).to(DEV) for n in ("q", "k", "v", "g", "beta")}


def _chunk_prepared(ops, case, pool, dev):
    out = ops.kda_prepared_varlen_chunk(
        dev["q"], dev["k"], dev["v"], dev["g"], dev["beta"], initial_state_source=pool,
        initial_state_indices=case.indices.to(DEV), cu_seqlens=case.cu_seqlens.to(DEV),
        scale=case.scale)
    torch.cuda.synchronize()
    return out


def _recurrent_fp32(ops, case, pool, dev):
    """This build's recurrent kernel with fp32 I/O (exact widening of bf16)."""
    out = ops.kda_prepared_varlen_recurrent(
        dev["q"].float(), dev["k"].float(), dev["v"].float(), dev["g"], dev["beta"],
        initial_state_source=pool, initial_state_indices=case.indices.to(DEV),
        cu_seqlens=case.cu_seqlens.to(DEV), scale=case.scale)
    torch.cuda.synchronize()
    return out


def test_prepared_chunk_matches_oracle_small(gpu_ops):
    case = C.prepared_case(4, (300, 64, 1, 129), slots=6, indices=[1, 0, 3, 5], seed=31)
    dev = _prepared_dev(case)
    pool = C.to_dev(case.pool, DEV)
    out = _chunk_prepared(gpu_ops, case, pool, dev)
    ref_pool = C.clone_pool(case.pool)
    ref = R.kda_chunk(case.q.float() * case.scale, case.k, case.v, case.g, case.beta,
                      state_pool=ref_pool, state_indices=case.indices,
                      cu_seqlens=case.cu_seqlens, out_dtype=torch.float32)
    C.assert_out(out.cpu(), ref, C.OUT_TOL, "output")
    C.assert_rel(pool.cpu(), ref_pool, C.STATE_TOL, "pool")


@pytest.mark.parametrize("q_mul,v_mul,pool_mul", [
    (1e7, 1.0, 1.0),    # outputs near 1e6: q e^G far beyond fp16's range unscaled
    (1.0, 1e6, 1e6),    # states near 1e5, values 1e6
    (1.0, 1e-6, 1e-6),  # states near 1e-8: below fp16's normal range unscaled
    (1.0, 1.0, 1e4),    # the carried state dominates every output
    (1.0, 1e4, 0.0),    # zero initial state, large values
])
def test_prepared_chunk_extreme_magnitudes(gpu_ops, q_mul, v_mul, pool_mul):
    """The scan's fp16 operands (w, q e^G, the exchanged S slices) carry
    power-of-two scales; magnitudes far outside fp16's range must leave the
    error (relative to the largest output / state) inside the contract."""
    import dataclasses

    case = C.prepared_case(2, (200, 64, 1), slots=4, indices=[1, 3, 2], seed=41)
    case = dataclasses.replace(case, q=(case.q.float() * q_mul).to(case.q.dtype),
                               v=(case.v.float() * v_mul).to(case.v.dtype),
                               pool=C.clone_pool(case.pool * pool_mul))
    dev = _prepared_dev(case)
    pool = C.to_dev(case.pool, DEV)
    out = _chunk_prepared(gpu_ops, case, pool, dev)
    ref_pool = C.clone_pool(case.pool).double()
    ref = R.kda_chunk(case.q.double() * case.scale, case.k.double(), case.v.double(),
                      case.g.double(), case.beta.double(), state_pool=ref_pool,
                      state_indices=case.indices, cu_seqlens=case.cu_seqlens,
                      dtype=torch.float64, out_dtype=torch.float64)
    assert torch.isfinite(out).all() and torch.isfinite(pool).all()
    C.assert_out(out.cpu(), ref, C.OUT_TOL, "output")
    C.assert_rel(pool.cpu(), ref_pool, C.STATE_TOL, "pool")


@pytest.mark.parametrize("label,gfun", [
    ("constant -7", lambda shape, gen: torch.full(shape, -7.0)),
    ("constant -10", lambda shape, gen: torch.full(shape, -10.0)),
    ("logsigmoid(randn-7)",
     lambda shape, gen: torch.nn.functional.logsigmoid(torch.randn(shape, generator=gen) - 7.0)),
    ("mixed per channel",
     lambda shape, gen: torch.where(torch.rand(shape, generator=gen) < 0.5,
                                    torch.full(shape, -9.5),
                                    torch.nn.functional.logsigmoid(torch.randn(shape, generator=gen)))),
])
def test_prepared_chunk_strong_decay(gpu_ops, label, gfun):
    """Planted strong per-token decays: the factored Akk / Aqk exponentials
    are anchored at each 16-row block's midpoint, so within a diagonal block a
    factor spans at most 8 tokens of decay (80 nat at g = -10). Outputs and
    states stay finite and match the fp64 oracle, which evaluates
    exp(G_i - G_j) directly."""
    import dataclasses

    case = C.prepared_case(2, (200, 64, 37), slots=5, indices=[1, 3, 2], seed=43)
    case = dataclasses.replace(case, g=gfun(tuple(case.g.shape), C.gen(44)).float())
    dev = _prepared_dev(case)
    pool = C.to_dev(case.pool, DEV)
    out = _chunk_prepared(gpu_ops, case, pool, dev)
    ref_pool = C.clone_pool(case.pool).double()
    ref = R.kda_chunk(case.q.double() * case.scale, case.k.double(), case.v.double(),
                      case.g.double(), case.beta.double(), state_pool=ref_pool,
                      state_indices=case.indices, cu_seqlens=case.cu_seqlens,
                      dtype=torch.float64, out_dtype=torch.float64)
    assert torch.isfinite(out).all() and torch.isfinite(pool).all(), label
    C.assert_out(out.cpu(), ref, C.OUT_TOL, f"{label} output")
    C.assert_rel(pool.cpu(), ref_pool, C.STATE_TOL, f"{label} pool")


@pytest.mark.parametrize("heads,T", [(4, 4096), (2, 8192)])
def test_prepared_chunk_weak_decay(gpu_ops, heads, T):
    """Weak decay, g = logsigmoid(randn + 9) ~ -1.2e-4 per token: the state
    remembers the whole sequence, so every chunk's rounding (in T, the record
    operands and the published states) reaches the final state. Against the
    fp64 oracle at the tolerance contract."""
    case = C.prepared_case(heads, (T,), slots=3, indices=[1], seed=47, gate_shift=9.0)
    dev = _prepared_dev(case)
    pool = C.to_dev(case.pool, DEV)
    out = _chunk_prepared(gpu_ops, case, pool, dev)
    ref_pool = C.clone_pool(case.pool).double()
    ref = R.kda_chunk(case.q.double() * case.scale, case.k.double(), case.v.double(),
                      case.g.double(), case.beta.double(), state_pool=ref_pool,
                      state_indices=case.indices, cu_seqlens=case.cu_seqlens,
                      dtype=torch.float64, out_dtype=torch.float64)
    e_o = C.assert_out(out.cpu(), ref, C.OUT_TOL, "weak decay output")
    e_s = C.assert_rel(pool.cpu(), ref_pool, C.STATE_TOL, "weak decay pool")
    print(f"weak decay H{heads} T{T}: output err {e_o:.2e}, state err {e_s:.2e}")


@pytest.mark.parametrize("form", ["all chunks", "bursts"])
def test_prepared_chunk_beyond_envelope_exact(gpu_ops, form):
    """Decays steeper than the anchored factors hold (8 tokens spanning more
    than 2^125): such a chunk takes the exact form (per-element
    e^(G_i - G_j)) and matches the fp64 oracle like any other. "all chunks":
    g = -20 on every token (8 tokens span 160 nat). "bursts": ordinary gates
    with g = -25 on 16 channels of tokens 70-89 and -40 on every channel of
    tokens 200-203, so two chunks of the first sequence take the exact form
    and the rest the anchored one, in one call."""
    import dataclasses

    case = C.prepared_case(2, (300, 100), slots=4, indices=[1, 3], seed=45)
    g = case.g.clone()
    if form == "all chunks":
        g.fill_(-20.0)
    else:
        g[:, 70:90, :, 0:16] = -25.0
        g[:, 200:204] = -40.0
    case = dataclasses.replace(case, g=g)
    dev = _prepared_dev(case)
    pool = C.to_dev(case.pool, DEV)
    out = _chunk_prepared(gpu_ops, case, pool, dev)
    assert torch.isfinite(out).all() and torch.isfinite(pool).all()
    ref_pool = C.clone_pool(case.pool).double()
    ref = R.kda_chunk(case.q.double() * case.scale, case.k.double(), case.v.double(),
                      case.g.double(), case.beta.double(), state_pool=ref_pool,
                      state_indices=case.indices, cu_seqlens=case.cu_seqlens,
                      dtype=torch.float64, out_dtype=torch.float64)
    C.assert_out(out.cpu(), ref, C.OUT_TOL, f"{form} output")
    C.assert_rel(pool.cpu(), ref_pool, C.STATE_TOL, f"{form} pool")


def test_raw_chunk_beyond_envelope_exact_with_tracking(gpu_ops):
    """The raw-gate chunk op below the router's bound (lower_bound = -15 with
    the gate saturated, g ~ -14.7 per token: every chunk takes the exact
    form), with prefixes tracked inside a chunk and on a chunk boundary,
    against the oracle."""
    case = C.raw_case(4, (200, 130), indices=[1, 2], slots=6, seed=1213, lower_bound=-15.0,
                      track=([4, 5], [90, 64]))
    case.a = (case.a.float() + 4.0).bfloat16()
    out, pool = _run_chunk(gpu_ops, case)
    assert torch.isfinite(out).all() and torch.isfinite(pool).all()
    ref_pool = C.clone_pool(case.pool)
    ref = _oracle_chunk(case, ref_pool)
    C.assert_out(out.cpu(), ref, C.OUT_TOL, "output")
    C.assert_rel(pool.cpu(), ref_pool, C.STATE_TOL, "pool")


def test_prepared_chunk_many_sequences(gpu_ops):
    """More sequences than the chunk-index kernel has threads (1500 > 1024, so
    each thread sums several sequences' chunk counts): short ragged and empty
    sequences, some on the padding slot 0, against the oracle; unused slots
    byte-identical."""
    import random

    rng = random.Random(5)
    n = 1500
    lengths = [rng.choice([0, 1, 63, 64, 65]) if rng.random() < 0.3 else rng.randint(1, 70)
               for _ in range(n)]
    slots = n + 40
    indices = [0 if rng.random() < 0.05 else s for s in rng.sample(range(1, slots), n)]
    case = C.prepared_case(2, lengths, slots=slots, indices=indices, seed=77)
    dev = _prepared_dev(case)
    pool = C.to_dev(case.pool, DEV)
    out = _chunk_prepared(gpu_ops, case, pool, dev)
    ref_pool = C.clone_pool(case.pool)
    ref = R.kda_chunk(case.q.float() * case.scale, case.k, case.v, case.g, case.beta,
                      state_pool=ref_pool, state_indices=case.indices,
                      cu_seqlens=case.cu_seqlens, out_dtype=torch.float32)
    C.assert_out(out.cpu(), ref, C.OUT_TOL, "output")
    C.assert_rel(pool.cpu(), ref_pool, C.STATE_TOL, "pool")
    used = set(s for s in indices if s > 0)
    other = [s for s in range(slots) if s not in used]
    assert torch.equal(pool.cpu()[other], case.pool[other]), "an unused slot was written"


@pytest.mark.parametrize("n,heads", [(5000, 1), (2100, 8)])
def test_prepared_chunk_beyond_persistent_limits(gpu_ops, n, heads):
    """Batches the persistent scan does not take, so the chunk-index pass
    writes no schedule: more sequences than it sorts (5000 > 4096), and more
    (sequence, head) items than 256 per team of 64 (2100 x 8 = 16800 >
    16384). Short ragged and empty sequences against the oracle; unused slots
    byte-identical."""
    import random

    rng = random.Random(n + heads)
    lengths = [rng.choice([0, 1, 2, 64, 65]) if rng.random() < 0.2 else rng.randint(1, 40) for _ in range(n)]
    slots = n + 8
    indices = [0 if rng.random() < 0.03 else s for s in rng.sample(range(1, slots), n)]
    case = C.prepared_case(heads, lengths, slots=slots, indices=indices, seed=n + 7 * heads)
    dev = _prepared_dev(case)
    pool = C.to_dev(case.pool, DEV)
    out = _chunk_prepared(gpu_ops, case, pool, dev)
    ref_pool = C.clone_pool(case.pool)
    ref = R.kda_chunk(case.q.float() * case.scale, case.k, case.v, case.g, case.beta,
                      state_pool=ref_pool, state_indices=case.indices,
                      cu_seqlens=case.cu_seqlens, out_dtype=torch.float32)
    C.assert_out(out.cpu(), ref, C.OUT_TOL, "output")
    C.assert_rel(pool.cpu(), ref_pool, C.STATE_TOL, "pool")
    used = set(s for s in indices if s > 0)
    other = [s for s in range(slots) if s not in used]
    assert torch.equal(pool.cpu()[other], case.pool[other]), "an unused slot was written"


@pytest.mark.parametrize("heads", [1, 2, 4])
def test_chunk_persistent_scan_tracking_and_padding(gpu_ops, heads):
    """More (sequence, head) items than the scan has teams of workgroups (64 on
    a 256-CU device), so persistent workgroups take several items each,
    longest first, and stage an item's first chunks while the previous one
    finishes (167, 87 and 47 sequences: the schedule is sorted in LDS, and
    for 64 or fewer within one wave): ragged and empty sequences, the padding slot, tracked prefixes
    at 0, inside a chunk, on a chunk boundary and at the end (also of empty
    sequences), and tokens before the first and after the last sequence --
    against the oracle; unindexed slots byte-identical."""
    import random

    rng = random.Random(11 + heads)
    n = 160 // heads + 7
    lengths = [rng.choice([0, 1, 16, 17, 63, 64, 65, 128, 130, 200]) for _ in range(n)]
    indices = [0 if rng.random() < 0.08 else s for s in range(1, n + 1)]
    track_idx, track_lens = [], []
    for i, length in enumerate(lengths):
        if i % 4 == 1:
            track_idx.append(n + 1 + i)
            track_lens.append(rng.choice([0, length, rng.randint(0, length), length // 64 * 64]))
        else:
            track_idx.append(0)
            track_lens.append(0)
    slots = 2 * n + 2
    # two dummy sequences frame the real ones: their tokens lie outside every
    # sequence once they are dropped from cu_seqlens
    case = C.raw_case(heads, [3] + lengths + [5], indices=[0] + indices + [0], slots=slots,
                      seed=4000 + heads, track=([0] + track_idx + [0], [0] + track_lens + [0]))
    case.cu_seqlens = case.cu_seqlens[1:-1].clone()
    case.indices = case.indices[1:-1].clone()
    case.track_indices = case.track_indices[1:-1].clone()
    case.track_lens = case.track_lens[1:-1].clone()
    assert len(case.indices) * heads > 64
    out, pool = _run_chunk(gpu_ops, case)
    ref_pool = C.clone_pool(case.pool)
    ref = _oracle_chunk(case, ref_pool)
    out = out.cpu()
    T = case.q.shape[1]
    assert torch.equal(out[0, :3], torch.zeros_like(out[0, :3]))
    assert torch.equal(out[0, T - 5:], torch.zeros_like(out[0, T - 5:]))
    C.assert_out(out, ref, C.OUT_TOL, "output")
    C.assert_rel(pool.cpu(), ref_pool, C.STATE_TOL, "pool")
    touched = set(s for s in indices if s > 0) | set(s for s in track_idx if s > 0)
    other = [s for s in range(slots) if s not in touched]
    assert torch.equal(pool.cpu()[other], case.pool[other]), "an unindexed slot was written"


@pytest.mark.parametrize(
    "name,heads,lengths,slots,indices,gate",
    [
        # config 3: T=8192 single sequence, H=32, zero initial state
        ("config3", 32, (8192,), 2, [1], (1.0, 0.0)),
        # config 4: 16 sequences, lengths uniform in [1, 4096], 64-slot pool
        ("config4", 32, None, 64, None, (1.0, 0.0)),
        # config 5 (prefill half): T=65536, H=16, harsh decay
        ("config5", 16, (65536,), 2, [1], (2.0, -2.0)),
        # config 3's shape with weak decay, g = logsigmoid(randn + 9) ~ -1e-4:
        # the state keeps every chunk's rounding for the whole sequence
        ("config3 weak decay", 32, (8192,), 2, [1], (1.0, 9.0)),
    ],
)
def test_baseline_configs_chunk_vs_recurrent(gpu_ops, name, heads, lengths, slots, indices, gate):
    if lengths is None:
        g_ = C.gen(4)
        lengths = tuple(int(x) for x in torch.randint(1, 4097, (16,), generator=g_))
        indices = torch.randperm(64, generator=g_)[:16].tolist()
    case = C.prepared_case(heads, lengths, slots=slots, indices=indices, seed=len(name) + 3,
                           gate_scale=gate[0], gate_shift=gate[1],
                           zero_pool=not name.startswith("config4"))
    dev = _prepared_dev(case)
    pool_c = C.to_dev(case.pool, DEV)
    pool_r = C.to_dev(case.pool, DEV)
    out_c = _chunk_prepared(gpu_ops, case, pool_c, dev)
    out_r = _recurrent_fp32(gpu_ops, case, pool_r, dev)
    e_o = C.assert_out(out_c.cpu(), out_r.cpu(), C.OUT_TOL, f"{name} output")
    e_s = C.assert_rel(pool_c.cpu(), pool_r.cpu(), C.STATE_TOL, f"{name} final states")
    print(f"{name}: output err {e_o:.2e}, state err {e_s:.2e}")
    assert torch.isfinite(out_c.float()).all()


def test_chunk_no_tokens_tracks_initial_state(gpu_ops):
    """An empty batch (two requests, no tokens) still runs the requests: the
    prefix tracked at length 0 receives the request's initial state, the
    source slots are rewritten unchanged and nothing else moves
    (kda_python.py:168-179 semantics, as the oracle)."""
    case = C.raw_case(4, (0, 0), indices=[2, 0], slots=6, seed=91, track=([4, 5], [0, 0]))
    pool = C.to_dev(case.pool, DEV)
    out = gpu_ops.kda_varlen_chunk(prefill=True, **case.kwargs(DEV, pool=pool))
    torch.cuda.synchronize()
    assert out.shape == case.v.shape and out.numel() == 0
    got = pool.cpu()
    assert torch.equal(got[4], case.pool[2]), "tracked slot 4 must hold slot 2's state"
    assert torch.equal(got[5], torch.zeros_like(got[5])), "slot-0 request tracks a zero state"
    for s in (0, 1, 2, 3):
        assert torch.equal(got[s], case.pool[s]), f"slot {s} changed"


def test_chunk_c_abi_launch_direct(gpu_ops):
    """kda_chunk_launch through ctypes with a caller-owned workspace (no torch
    operator in between): against the oracle, bitwise equal to the torch op,
    and the same workspace reused by a second, smaller call."""
    import ctypes

    from sgl_glm53_ascend_ops._load import abi_library_path
    from tests.test_abi_exports import _ChunkArgs

    lib = ctypes.CDLL(str(abi_library_path()))
    lib.kda_chunk_workspace_bytes.restype = ctypes.c_size_t
    lib.kda_chunk_workspace_bytes.argtypes = [ctypes.c_int32] * 4
    lib.kda_chunk_launch.restype = ctypes.c_int
    lib.kda_chunk_launch.argtypes = [ctypes.POINTER(_ChunkArgs), ctypes.c_void_p,
                                     ctypes.c_size_t, ctypes.c_void_p]
    stream = torch.cuda.current_stream().cuda_stream
    big = C.prepared_case(3, (150, 64, 9), slots=5, indices=[4, 0, 2], seed=23)
    T_big = int(big.cu_seqlens[-1])
    nbytes = lib.kda_chunk_workspace_bytes(T_big, 3, 3, 128)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    for case in (big, C.prepared_case(3, (40, 70), slots=5, indices=[1, 3], seed=24)):
        dev = _prepared_dev(case)
        pool = C.to_dev(case.pool, DEV)
        idx = case.indices.to(DEV)
        cu = case.cu_seqlens.to(DEV)
        out = torch.empty_like(dev["v"])
        T, H, D = case.q.shape[1:]
        a = _ChunkArgs(q=dev["q"].data_ptr(), k=dev["k"].data_ptr(), v=dev["v"].data_ptr(),
                       gate=dev["g"].data_ptr(), beta=dev["beta"].data_ptr(),
                       state=pool.data_ptr(), state_stride_slot=pool.stride(0),
                       state_stride_head=pool.stride(1), num_slots=pool.shape[0],
                       state_indices=idx.data_ptr(), cu_seqlens=cu.data_ptr(),
                       out=out.data_ptr(), scale=case.scale, num_seqs=len(case.indices),
                       num_tokens=T, num_heads=H, head_dim=D, qk_dtype=0, v_dtype=0,
                       gate_mode=1, qk_l2norm=0)
        assert lib.kda_chunk_workspace_bytes(T, len(case.indices), H, D) <= nbytes
        assert lib.kda_chunk_launch(ctypes.byref(a), ctypes.c_void_p(ws.data_ptr()),
                                    ctypes.c_size_t(nbytes), ctypes.c_void_p(stream)) == 0
        torch.cuda.synchronize()
        ref_pool = C.clone_pool(case.pool)
        ref = R.kda_chunk(case.q.float() * case.scale, case.k, case.v, case.g, case.beta,
                          state_pool=ref_pool, state_indices=case.indices,
                          cu_seqlens=case.cu_seqlens, out_dtype=torch.float32)
        C.assert_out(out.cpu(), ref, C.OUT_TOL, "output")
        C.assert_rel(pool.cpu(), ref_pool, C.STATE_TOL, "pool")
        pool_op = C.to_dev(case.pool, DEV)
        out_op = _chunk_prepared(gpu_ops, case, pool_op, dev)
        assert torch.equal(out, out_op) and torch.equal(pool, pool_op)


# A single sequence of at least 16384 tokens on at most 16 heads runs in
# segments (two here: 120 and 136 of its 256 chunks), each segment's prepare
# kernel on a second stream under the previous segment's scan, the records in
# a ring of two segments' slots and the state between the segments in the
# workspace; segments past a shorter sequence's end do nothing.
_SEG = 120 * 64
_T_SPLIT = 16384


@pytest.mark.parametrize("label,bounds,slot,track", [
    ("whole", (0, _T_SPLIT), 1, None),
    ("zero slot", (0, _T_SPLIT), 0, None),
    ("offset and ragged", (37, _T_SPLIT - 42), 2, None),
    ("short sequence", (5, 100), 1, None),
    ("one segment exactly", (0, _SEG), 1, None),
    ("track at 0", (0, _T_SPLIT), 1, 0),
    ("track in first segment", (0, _T_SPLIT), 1, 1000),
    ("track at a segment end", (0, _T_SPLIT), 1, _SEG),
    ("track after a segment end", (0, _T_SPLIT), 1, _SEG + 1),
    ("track in a later segment", (0, _T_SPLIT), 0, 14000),
    ("track at end", (0, _T_SPLIT), 1, _T_SPLIT),
])
def test_chunk_two_segment_path(gpu_ops, label, bounds, slot, track):
    import dataclasses

    case = C.raw_case(1, (_T_SPLIT,), indices=[slot], slots=4, seed=777 + len(label),
                      track=None if track is None else ([3], [track]))
    case = dataclasses.replace(case, cu_seqlens=torch.tensor(bounds, dtype=torch.int32))
    out, pool = _run_chunk(gpu_ops, case)
    ref_pool = C.clone_pool(case.pool)
    ref = _oracle_chunk(case, ref_pool)
    C.assert_out(out.cpu(), ref, C.OUT_TOL, f"{label} output")
    C.assert_rel(pool.cpu(), ref_pool, C.STATE_TOL, f"{label} pool")
    assert torch.all(out.cpu()[:, :bounds[0]] == 0) and torch.all(out.cpu()[:, bounds[1]:] == 0)
    touched = {s for s in (slot, 3 if track is not None else 0) if s > 0}
    other = [s for s in range(4) if s not in touched]
    assert torch.equal(pool.cpu()[other], case.pool[other]), "an unindexed slot was written"
