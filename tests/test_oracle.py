"""Pins the CPU oracle (``oracle/kda_ref.py``) without trusting its own formulas.

Each check is chosen so a plausible slip in the oracle fails it:

* closed forms -- one token from a zero state gives ``o = (qn.kn) v``
  (catches a readout before the update, a dropped beta, a transposed state);
  ``beta = 0`` is pure per-channel decay (catches a decay on the wrong axis);
  the delta-rule fixed point ``kn^T S = v`` for ``beta = 1, g = 0``;
* a library routine -- the reference's forward substitution equals
  ``torch.linalg.solve_triangular`` in float64;
* brute force -- chunk == recurrent in float64 to ~1e-10 on ragged varlen
  inputs, including chunk sizes that leave short tail chunks (the reference's
  own cross-check, bench/kda_chunk/kda_python.py:312-344);
* invariants -- slot 0 reads zero and is never written, untouched slots are
  byte-identical, tracked prefixes equal the final state of the prefix run,
  checkpoints equal truncated runs, sequences are independent.
"""

import math

import numpy as np
import pytest
import torch

from oracle import kda_ref as R
from tests import kda_cases as C

F64 = torch.float64


def _gen(seed):
    g = torch.Generator().manual_seed(seed)
    return g


def _prepared_inputs(T, H, D, seed, gate_scale=1.0, gate_shift=0.0, dtype=F64):
    gen = _gen(seed)
    q = R.l2norm_last(torch.randn(1, T, H, D, generator=gen, dtype=dtype)) * D ** -0.5
    k = R.l2norm_last(torch.randn(1, T, H, D, generator=gen, dtype=dtype))
    v = torch.randn(1, T, H, D, generator=gen, dtype=dtype)
    g = torch.nn.functional.logsigmoid(
        torch.randn(1, T, H, D, generator=gen, dtype=dtype) * gate_scale + gate_shift
    )
    beta = torch.sigmoid(torch.randn(1, T, H, generator=gen, dtype=dtype))
    return q, k, v, g, beta


def _pool(slots, H, D, seed, dtype=F64):
    gen = _gen(seed)
    # K-contiguous, as the production pool: [slots, H, V, K] viewed [.., K, V].
    return (torch.randn(slots, H, D, D, generator=gen, dtype=dtype) * 0.1).transpose(-1, -2)


def _clone_pool(p):
    return p.transpose(-1, -2).clone().transpose(-1, -2)


# --- closed forms -----------------------------------------------------------


@pytest.mark.parametrize("form", ["recurrent", "chunk"])
def test_one_token_from_zero_state(form):
    H, D = 3, 16
    q, k, v, g, beta = _prepared_inputs(1, H, D, seed=1)
    g = torch.zeros_like(g)
    beta = torch.ones_like(beta)
    pool = torch.zeros(2, H, D, D, dtype=F64)
    fn = R.kda_recurrent if form == "recurrent" else R.kda_chunk
    o = fn(q, k, v, g, beta, state_pool=pool, state_indices=torch.tensor([1]),
           cu_seqlens=torch.tensor([0, 1]), dtype=F64)
    # S = k v^T (zero state, beta 1), o = S^T q = (q.k) v
    expect = (q[0, 0] * k[0, 0]).sum(-1, keepdim=True) * v[0, 0]
    torch.testing.assert_close(o[0, 0], expect, rtol=1e-12, atol=1e-14)
    torch.testing.assert_close(pool[1], k[0, 0][:, :, None] * v[0, 0][:, None, :],
                               rtol=1e-12, atol=1e-14)


@pytest.mark.parametrize("form", ["recurrent", "chunk"])
def test_beta_zero_is_pure_decay(form):
    T, H, D = 37, 2, 8
    q, k, v, g, beta = _prepared_inputs(T, H, D, seed=2)
    beta = torch.zeros_like(beta)
    pool = _pool(3, H, D, seed=3)
    S0 = pool[2].clone()
    fn = R.kda_recurrent if form == "recurrent" else R.kda_chunk
    kw = dict(chunk_size=8) if form == "chunk" else {}
    o = fn(q, k, v, g, beta, state_pool=pool, state_indices=torch.tensor([2]),
           cu_seqlens=torch.tensor([0, T]), dtype=F64, **kw)
    G = g[0].cumsum(0)  # [T, H, K]
    for t in (0, 5, T - 1):
        St = torch.exp(G[t])[:, :, None] * S0  # decay acts on the K axis
        torch.testing.assert_close(o[0, t], torch.einsum("hk,hkv->hv", q[0, t], St),
                                   rtol=1e-10, atol=1e-13)
    torch.testing.assert_close(pool[2], torch.exp(G[-1])[:, :, None] * S0,
                               rtol=1e-10, atol=1e-13)


def test_delta_rule_fixed_point():
    """With g=0, beta=1 and a unit key, the update makes k^T S equal v."""
    H, D = 2, 16
    q, k, v, g, beta = _prepared_inputs(1, H, D, seed=4)
    g = torch.zeros_like(g)
    beta = torch.ones_like(beta)
    k = k / k.norm(dim=-1, keepdim=True)  # exactly unit (l2norm_last keeps an eps)
    pool = _pool(2, H, D, seed=5)
    R.kda_recurrent(q, k, v, g, beta, state_pool=pool, state_indices=torch.tensor([1]),
                    cu_seqlens=torch.tensor([0, 1]), dtype=F64)
    kS = torch.einsum("hk,hkv->hv", k[0, 0], pool[1])
    torch.testing.assert_close(kS, v[0, 0], rtol=1e-10, atol=1e-12)


def test_prepare_elementwise():
    """kda_prepare against the formulas evaluated independently in numpy."""
    gen = _gen(6)
    T, H, D = 5, 3, 8
    q, k, a = (torch.randn(1, T, H, D, generator=gen) for _ in range(3))
    b = torch.randn(1, T, H, generator=gen)
    A_log = torch.randn(H, generator=gen) * 0.1
    dt = torch.randn(H * D, generator=gen) * 0.1
    lb, sc = -5.0, D ** -0.5
    qn, kn, g, beta = R.kda_prepare(A_log, a, dt, q, k, b, lb, sc, dtype=F64)
    qd, kd, ad, bd = (x.double().numpy() for x in (q, k, a, b))
    Ad, dtd = A_log.double().numpy(), dt.double().numpy().reshape(H, D)
    np.testing.assert_allclose(qn.numpy(), qd / np.sqrt((qd**2).sum(-1, keepdims=True) + 1e-6) * sc, rtol=1e-13)
    np.testing.assert_allclose(kn.numpy(), kd / np.sqrt((kd**2).sum(-1, keepdims=True) + 1e-6), rtol=1e-13)
    x = np.exp(Ad)[None, None, :, None] * (ad + dtd[None, None])
    np.testing.assert_allclose(g.numpy(), lb / (1.0 + np.exp(-x)), rtol=1e-13)
    np.testing.assert_allclose(beta.numpy(), 1.0 / (1.0 + np.exp(-bd)), rtol=1e-13)
    assert (g < 0).all()


# --- library routine ----------------------------------------------------------


@pytest.mark.parametrize("c", [1, 5, 16, 64])
def test_forward_substitution_matches_solve_triangular(c):
    gen = _gen(7 + c)
    N = torch.tril(torch.randn(3, c, c, generator=gen, dtype=F64) * 0.3, diagonal=-1)
    X = R.forward_substitution_inverse(N)
    eye = torch.eye(c, dtype=F64).expand(3, c, c)
    ref = torch.linalg.solve_triangular(eye - N, eye, upper=False, unitriangular=True)
    torch.testing.assert_close(X + eye, ref, rtol=1e-11, atol=1e-12)


def test_chunk_factors_ut_transform():
    """Tm = (I + diag(beta) tril(Akk,-1))^-1 diag(beta), with Akk from the definition."""
    c, H, D = 12, 2, 8
    q, k, v, g, beta = _prepared_inputs(c, H, D, seed=9)
    kc, qc = k[0].transpose(0, 1), q[0].transpose(0, 1)
    Gc = g[0].transpose(0, 1).cumsum(1)
    bc = beta[0].transpose(0, 1)
    Tm, Aqk = R.chunk_factors(kc, qc, Gc, bc)
    for h in range(H):
        Akk = torch.zeros(c, c, dtype=F64)
        Aq = torch.zeros(c, c, dtype=F64)
        for i in range(c):
            for j in range(i + 1):
                e = torch.exp(Gc[h, i] - Gc[h, j])
                Akk[i, j] = (kc[h, i] * kc[h, j] * e).sum()
                Aq[i, j] = (qc[h, i] * kc[h, j] * e).sum()
        L = torch.diag(bc[h]) @ torch.tril(Akk, -1)
        ref = torch.linalg.inv(torch.eye(c, dtype=F64) + L) @ torch.diag(bc[h])
        torch.testing.assert_close(Tm[h], ref, rtol=1e-11, atol=1e-12)
        torch.testing.assert_close(Aqk[h], Aq, rtol=1e-12, atol=1e-13)


# --- brute force: chunk == recurrent ------------------------------------------


@pytest.mark.parametrize(
    "cu,chunk,gate",
    [
        ([0, 37, 100], 64, (1.0, 0.0)),
        ([0, 64, 192, 256], 64, (1.0, 0.0)),
        ([0, 1, 2, 70, 71, 200], 64, (1.0, 0.0)),
        ([0, 29, 90], 8, (1.0, 0.0)),
        ([0, 150], 16, (2.0, -2.0)),  # harsh decay, as BASELINE config 5
    ],
)
def test_chunk_equals_recurrent_f64(cu, chunk, gate):
    T, H, D = cu[-1], 2, 16
    q, k, v, g, beta = _prepared_inputs(T, H, D, seed=11 + T, gate_scale=gate[0], gate_shift=gate[1])
    nseq = len(cu) - 1
    pool_r = _pool(nseq + 2, H, D, seed=12)
    pool_c = _clone_pool(pool_r)
    idx = torch.tensor([0] + list(range(2, nseq + 1)))  # first sequence uses slot 0
    cu_t = torch.tensor(cu)
    o_r = R.kda_recurrent(q, k, v, g, beta, state_pool=pool_r, state_indices=idx,
                          cu_seqlens=cu_t, dtype=F64)
    o_c = R.kda_chunk(q, k, v, g, beta, state_pool=pool_c, state_indices=idx,
                      cu_seqlens=cu_t, chunk_size=chunk, dtype=F64)
    torch.testing.assert_close(o_c, o_r, rtol=1e-9, atol=1e-11)
    torch.testing.assert_close(pool_c, pool_r, rtol=1e-9, atol=1e-11)


@pytest.mark.parametrize("track_len", [0, 1, 13, 16, 31, 32, 45])
@pytest.mark.parametrize("form", ["recurrent", "chunk"])
def test_tracking_equals_prefix_run(form, track_len):
    """The tracked slot holds the state after ``track_len`` tokens."""
    T, H, D = 45, 2, 8
    q, k, v, g, beta = _prepared_inputs(T, H, D, seed=13)
    pool = _pool(5, H, D, seed=14)
    pool_prefix = _clone_pool(pool)
    fn = R.kda_recurrent if form == "recurrent" else R.kda_chunk
    kw = dict(chunk_size=16) if form == "chunk" else {}
    fn(q, k, v, g, beta, state_pool=pool, state_indices=torch.tensor([2]),
       cu_seqlens=torch.tensor([0, T]), track_state_indices=torch.tensor([4]),
       track_state_lens=torch.tensor([track_len]), dtype=F64, **kw)
    # The prefix run, through the recurrence, from the same initial state.
    R.kda_recurrent(q[:, :track_len], k[:, :track_len], v[:, :track_len],
                    g[:, :track_len], beta[:, :track_len], state_pool=pool_prefix,
                    state_indices=torch.tensor([2]), cu_seqlens=torch.tensor([0, track_len]),
                    dtype=F64)
    torch.testing.assert_close(pool[4], pool_prefix[2], rtol=1e-10, atol=1e-12)


def test_intermediate_checkpoints_equal_truncated_runs():
    T, H, D = 6, 2, 8
    q, k, v, g, beta = _prepared_inputs(2 * T, H, D, seed=15)
    pool = _pool(4, H, D, seed=16)
    before = pool.clone()
    mid = torch.full((2, T, H, D, D), 7.0, dtype=F64)
    cu = torch.tensor([0, T, 2 * T])
    idx = torch.tensor([3, 0])  # second request is the padding slot
    R.kda_recurrent(q, k, v, g, beta, state_pool=pool, state_indices=idx, cu_seqlens=cu,
                    intermediate_state=mid, dtype=F64)
    assert torch.equal(pool, before), "checkpointing must skip the final write-back"
    assert torch.equal(mid[1], torch.full_like(mid[1], 7.0)), "slot 0 writes no checkpoint"
    for t in range(T):
        p = _clone_pool(before)
        R.kda_recurrent(q[:, : t + 1], k[:, : t + 1], v[:, : t + 1], g[:, : t + 1],
                        beta[:, : t + 1], state_pool=p, state_indices=torch.tensor([3]),
                        cu_seqlens=torch.tensor([0, t + 1]), dtype=F64)
        torch.testing.assert_close(mid[0, t], p[3], rtol=1e-12, atol=1e-14)


# --- invariants --------------------------------------------------------------


@pytest.mark.parametrize("form", ["recurrent", "chunk"])
def test_slots_and_independence(form):
    T, H, D = 50, 2, 8
    q, k, v, g, beta = _prepared_inputs(T, H, D, seed=17)
    cu = torch.tensor([0, 20, 20, 50])  # includes an empty sequence
    idx = torch.tensor([0, 3, 2])
    pool = _pool(5, H, D, seed=18)
    before = pool.clone()
    fn = R.kda_recurrent if form == "recurrent" else R.kda_chunk
    kw = dict(chunk_size=16) if form == "chunk" else {}
    o = fn(q, k, v, g, beta, state_pool=pool, state_indices=idx, cu_seqlens=cu, dtype=F64, **kw)
    # slot 0 untouched (padding), slots 1 and 4 untouched (not indexed),
    # slot 3 belongs to an empty sequence: rewritten with its own value.
    for s in (0, 1, 3, 4):
        assert torch.equal(pool[s], before[s])
    assert not torch.equal(pool[2], before[2])
    # Perturb the last sequence: the first one's output must not move.
    v2 = v.clone()
    v2[0, 30:] += 1.0
    o2 = fn(q, k, v2, g, beta, state_pool=before.clone(), state_indices=idx, cu_seqlens=cu,
            dtype=F64, **kw)
    assert torch.equal(o2[0, :20], o[0, :20])
    assert not torch.equal(o2[0, 20:], o[0, 20:])


def test_tokens_past_last_sequence_are_zero():
    T, H, D = 10, 1, 4
    q, k, v, g, beta = _prepared_inputs(T, H, D, seed=19)
    pool = torch.zeros(2, H, D, D, dtype=F64)
    o = R.kda_recurrent(q, k, v, g, beta, state_pool=pool, state_indices=torch.tensor([1]),
                        cu_seqlens=torch.tensor([0, 7]), dtype=F64)
    assert torch.equal(o[0, 7:], torch.zeros_like(o[0, 7:]))


def test_fp32_oracle_close_to_f64():
    """The fp32 anchor is itself within the tolerance contract of the f64 truth."""
    T, H, D = 130, 2, 64
    q, k, v, g, beta = _prepared_inputs(T, H, D, seed=21)
    cu = torch.tensor([0, 61, 130])
    idx = torch.tensor([1, 2])
    p64 = _pool(3, H, D, seed=22)
    p32 = _clone_pool(p64).float()
    o64 = R.kda_chunk(q, k, v, g, beta, state_pool=p64, state_indices=idx, cu_seqlens=cu, dtype=F64)
    o32 = R.kda_chunk(*(t.float() for t in (q, k, v, g, beta)), state_pool=p32,
                      state_indices=idx, cu_seqlens=cu, dtype=torch.float32)
    assert C.max_rel_err(o32, o64) < 1e-5
    assert C.max_rel_err(p32, p64) < 1e-5


def test_raw_wrappers_agree():
    """The sglang-signature wrappers route through the same recurrence."""
    gen = _gen(23)
    T, H, D = 40, 2, 16
    q, k, v, a = ((torch.randn(1, T, H, D, generator=gen) * 0.2) for _ in range(4))
    b = torch.randn(1, T, H, generator=gen)
    A_log = torch.randn(H, generator=gen) * 0.1
    dt = torch.randn(H * D, generator=gen) * 0.1
    pool_r = _pool(3, H, D, seed=24, dtype=F64)
    pool_c = _clone_pool(pool_r)
    kw = dict(A_log=A_log, a=a, dt_bias=dt, q=q, k=k, v=v, b=b,
              initial_state_indices=torch.tensor([1, 2]), cu_seqlens=torch.tensor([0, 17, 40]),
              lower_bound=-5.0, scale=D ** -0.5, dtype=F64)
    o_r = R.kda_varlen_recurrent_ref(initial_state_source=pool_r, **kw)
    o_c = R.kda_varlen_chunk_ref(initial_state_source=pool_c, chunk_size=8, **kw)
    torch.testing.assert_close(o_c.double(), o_r.double(), rtol=1e-9, atol=1e-11)
    torch.testing.assert_close(pool_c, pool_r, rtol=1e-9, atol=1e-11)


def test_planted_mistake_is_caught():
    """A readout taken before the update fails the one-token closed form.

    Planted in a copy of the recurrence here on the CPU, to show the closed
    form is not vacuous.
    """
    H, D = 2, 8
    q, k, v, g, beta = _prepared_inputs(1, H, D, seed=25)
    S = torch.zeros(H, D, D, dtype=F64)
    o_wrong = torch.einsum("hk,hkv->hv", q[0, 0], S)  # readout before update
    expect = (q[0, 0] * k[0, 0]).sum(-1, keepdim=True) * v[0, 0]
    assert not torch.allclose(o_wrong, expect)
    assert math.isfinite(float(expect.abs().sum()))


# --- prepared_recurrent_ref (the prepared_recurrent op's oracle) -------------


def _prepared_rec_inputs(T, H, D, seed):
    q, k, v, g, beta = _prepared_inputs(T, H, D, seed)
    flat = lambda x: x.reshape(T * H, D).clone()  # noqa: E731
    return flat(q), flat(k), flat(v), flat(g.exp()), beta.reshape(T * H).clone(), g


def test_prepared_recurrent_ref_equals_log_form():
    """Two launches (heads 0-3, then 4-7) with multiplicative decays equal the
    log-gate recurrence over all eight heads, outputs, pool and tracked slot,
    in float64 -- a wrong head offset, a decay taken as a log, or a head range
    that is not advanced would each break it."""
    T, H, D = 23, 8, 16
    qn, kn, v, dec, beta, g = _prepared_rec_inputs(T, H, D, seed=41)
    starts = torch.tensor([0, 9, 23])
    idx = torch.tensor([2, 0])  # the second request starts from the padding slot
    tr_i, tr_l = torch.tensor([4, 0]), torch.tensor([5, 0])
    pool = _pool(5, H, D, seed=42)
    ref_pool = _clone_pool(pool)
    out = torch.zeros(T * H, D, dtype=F64)
    for off in (0, 4):
        R.prepared_recurrent_ref(qn, kn, v, dec, beta, out, pool, idx, starts, tr_i, tr_l,
                                 True, off, dtype=F64)
    shp = (1, T, H, D)
    ref = R.kda_recurrent(qn.reshape(shp), kn.reshape(shp), v.reshape(shp), g,
                          beta.reshape(1, T, H), state_pool=ref_pool, state_indices=idx,
                          cu_seqlens=starts, track_state_indices=tr_i, track_state_lens=tr_l,
                          dtype=F64)
    torch.testing.assert_close(out.reshape(shp), ref, rtol=1e-12, atol=1e-14)
    torch.testing.assert_close(pool, ref_pool, rtol=1e-12, atol=1e-14)
    assert not torch.equal(pool[4], _pool(5, H, D, seed=42)[4]), "tracked slot not written"


def test_prepared_recurrent_ref_one_token_closed_form():
    """One token from a zero state, decay 1: o = beta (qn . kn) v on the
    launched heads only."""
    H, D = 8, 8
    qn, kn, v, _, beta, _ = _prepared_rec_inputs(1, H, D, seed=43)
    dec = torch.ones(H, D, dtype=F64)
    pool = torch.zeros(2, H, D, D, dtype=F64)
    out = torch.zeros(H, D, dtype=F64)
    R.prepared_recurrent_ref(qn, kn, v, dec, beta, out, pool, torch.tensor([1]),
                             torch.tensor([0, 1]), head_offset=4, dtype=F64)
    expect = beta[:, None] * (qn * kn).sum(-1, keepdim=True) * v
    torch.testing.assert_close(out[4:], expect[4:], rtol=1e-12, atol=1e-14)
    assert torch.equal(out[:4], torch.zeros(4, D, dtype=F64))


def test_prepared_recurrent_ref_writes_only_its_rows_and_heads():
    """Rows outside [starts[0], starts[N]) and heads outside the launch keep
    the caller's values in ``out`` and in the pool (prepared_recurrent.cpp
    writes rows [bos, eos) of its four heads only)."""
    T, H, D = 12, 8, 8
    qn, kn, v, dec, beta, _ = _prepared_rec_inputs(T, H, D, seed=44)
    pool = _pool(3, H, D, seed=45)
    before = _clone_pool(pool)
    out = torch.full((T * H, D), 7.0, dtype=F64)
    R.prepared_recurrent_ref(qn, kn, v, dec, beta, out, pool, torch.tensor([1]),
                             torch.tensor([3, T - 2]), head_offset=4, dtype=F64)
    o = out.reshape(T, H, D)
    assert torch.equal(o[:3], torch.full_like(o[:3], 7.0))
    assert torch.equal(o[T - 2:], torch.full_like(o[T - 2:], 7.0))
    assert torch.equal(o[:, :4], torch.full_like(o[:, :4], 7.0))
    assert not torch.equal(o[3:T - 2, 4:], torch.full_like(o[3:T - 2, 4:], 7.0))
    assert torch.equal(pool[:, :4], before[:, :4])
    assert torch.equal(pool[0], before[0]) and torch.equal(pool[2], before[2])
    assert not torch.equal(pool[1, 4:], before[1, 4:])
