"""CPU oracle for the KDA (Kimi Delta Attention) recurrent and chunked operators.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker or as the timed CPU baseline. The product path (the HIP kernels behind
``torch.ops.sgl_glm53_ascend.*``) never calls into it.

This is a torch restatement of the reference's own fp32 torch reference,
``bench/kda_chunk/kda_python.py``, written dtype-generic so the same code runs
in float32 (the parity anchor) and float64 (the pinning anchor). Every function
cites the reference lines it follows. Layout conventions:

* token tensors are ``[1, T, H, D]`` (packed varlen, ``cu_seqlens`` delimits
  sequences) exactly as the reference's sglang-facing ops take them;
* the state pool is indexed logically as ``[slots, H, K, V]`` whatever its
  strides, so a K-contiguous pool (the production layout) and a plain one give
  the same answer;
* slot 0 is the padding row: it reads as a zero state and is never written.

Two extensions beyond the reference, both required by the BASELINE configs:

* ``kda_chunk`` accepts sequence lengths that are not a multiple of the chunk
  size (the last chunk of a sequence is shorter). The chunk equations hold for
  any chunk length, so the ragged tail is the same algebra on a smaller block;
  it is pinned against the length-agnostic recurrence in the tests.
* both functions take prepared gates (``g`` log-decay, ``beta`` in (0,1)) as
  well as the raw gate form through ``kda_prepare``.

Pinning (see tests/test_oracle.py): closed forms for one token, the beta=0 pure
decay, the delta-rule fixed point; the forward substitution against
``torch.linalg.solve_triangular``; chunk == recurrent in float64 to ~1e-10 on
ragged varlen inputs; slot / tracking / checkpoint invariants.
"""

from __future__ import annotations

from typing import Optional

import torch

EPS = 1e-6


# ---------------------------------------------------------------------------
# preparation
# ---------------------------------------------------------------------------


def l2norm_last(x: torch.Tensor, eps: float = EPS) -> torch.Tensor:
    """``x / sqrt(sum(x*x) + eps)`` over the last axis, eps inside the sqrt.

    Follows ``kda_pre_torch`` (bench/kda_chunk/kda_python.py:28-29).
    """
    return x / torch.sqrt((x * x).sum(-1, keepdim=True) + eps)


def kda_prepare(
    A_log: torch.Tensor,
    a: torch.Tensor,
    dt_bias: torch.Tensor,
    q: torch.Tensor,
    k: torch.Tensor,
    b: torch.Tensor,
    lower_bound: float,
    scale: float,
    dtype: torch.dtype = torch.float32,
):
    """Raw gates -> (qn, kn, g, beta).

    Follows ``kda_pre_torch`` (bench/kda_chunk/kda_python.py:16-39):

    * ``qn = q / sqrt(sum q^2 + 1e-6) * scale`` (divide, then scale);
    * ``kn = k / sqrt(sum k^2 + 1e-6)``;
    * ``g = lower_bound * sigmoid(exp(A_log)[h] * (a + dt_bias[h, :]))``, the
      per-channel log decay, ``[1, T, H, K]``;
    * ``beta = sigmoid(b)``, ``[1, T, H]``.

    ``dt_bias`` may be ``[H*K]`` or ``[H, K]`` (the op accepts both).
    """
    H = q.shape[2]
    K = q.shape[3]
    q, k, a, b = (t.to(dtype) for t in (q, k, a, b))
    qn = l2norm_last(q) * scale
    kn = l2norm_last(k)
    dtb = dt_bias.to(dtype).reshape(H, K)
    gate = A_log.to(dtype).exp()[None, None, :, None] * (a + dtb[None, None])
    g = lower_bound * torch.sigmoid(gate)
    beta = torch.sigmoid(b)
    return qn, kn, g, beta


def _as_list(t: Optional[torch.Tensor]):
    return None if t is None else [int(x) for x in t.reshape(-1).tolist()]


# ---------------------------------------------------------------------------
# recurrent form
# ---------------------------------------------------------------------------


def kda_recurrent(
    qn: torch.Tensor,
    kn: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    beta: torch.Tensor,
    *,
    state_pool: torch.Tensor,
    state_indices: torch.Tensor,
    cu_seqlens: torch.Tensor,
    intermediate_state: Optional[torch.Tensor] = None,
    track_state_indices: Optional[torch.Tensor] = None,
    track_state_lens: Optional[torch.Tensor] = None,
    dtype: torch.dtype = torch.float32,
    out_dtype: Optional[torch.dtype] = None,
    decay: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Token-by-token delta rule on prepared inputs; updates pools in place.

    Follows ``kda_recur_torch`` (bench/kda_chunk/kda_python.py:190-309), per
    sequence ``n`` with ``S`` of shape ``[H, K, V]``:

    * ``S0 = pool[slot]`` if ``slot > 0`` else zeros (:259-262);
    * a tracked slot with ``track_len == 0`` receives ``S0`` (:264-269);
    * per token: ``S = exp(g_t)[:, None] * S``; ``d = beta_t (v_t - kn_t^T S)``;
      ``S = S + kn_t d^T``; checkpoint / track stores; ``o_t = qn_t^T S``
      (:271-303) -- the readout is AFTER the update;
    * ``intermediate_state[n, t] = S`` after every step when ``slot > 0``,
      indexed by the sequence's position ``n`` and its local step ``t``
      (:299-300);
    * token inputs are read at their packed positions ``bos + t``. The anchor
      itself indexes ``decay[:, t]``, ``kn[:, t]``, ``v[:, t]``, ``beta[:, t]``
      and ``qn[:, t]`` with the sequence-local ``t`` (:276-303) while it writes
      ``output[:, i]`` at the packed ``i``, which reads the first sequence's
      tokens for every later one; the reference kernel reads packed rows
      (kda_varlen_recurrent_decode_h32.cpp:393,595), and so does this
      restatement (pinned by chunk == recurrent on multi-sequence batches);
    * the final write-back ``pool[slot] = S`` happens only when ``slot > 0``
      and no ``intermediate_state`` is given (:305-307).

    ``qn`` must already carry the query scale. ``decay`` (``exp(g)``), when
    given, is used as is and ``g`` is ignored (the prepared form of
    ``prepared_recurrent``). Returns ``o`` as ``[1, T, H, V]``
    in ``out_dtype`` (default: ``v.dtype``); tokens outside every sequence stay
    zero (the reference allocates ``zeros_like(v)``, :251).
    """
    T, H, K = qn.shape[1:]
    V = v.shape[3]
    out_dtype = v.dtype if out_dtype is None else out_dtype
    qn, kn, v, beta = (t.to(dtype) for t in (qn, kn, v, beta))
    decay = g.to(dtype).exp() if decay is None else decay.to(dtype)
    out = torch.zeros(1, T, H, V, dtype=dtype)
    cu = _as_list(cu_seqlens)
    slots = _as_list(state_indices)
    tidx = _as_list(track_state_indices)
    tlen = _as_list(track_state_lens)

    for n in range(len(cu) - 1):
        bos, eos, slot = cu[n], cu[n + 1], slots[n]
        if slot > 0:
            S = state_pool[slot].to(dtype).clone()
        else:
            S = torch.zeros(H, K, V, dtype=dtype)
        ti = 0 if tidx is None else tidx[n]
        tl = None if (tidx is None or ti <= 0) else tlen[n]
        if tl == 0:
            state_pool[ti].copy_(S)
        for t in range(eos - bos):
            i = bos + t
            S = S * decay[0, i][:, :, None]
            pred = torch.einsum("hk,hkv->hv", kn[0, i], S)
            d = (v[0, i] - pred) * beta[0, i][:, None]
            S = S + kn[0, i][:, :, None] * d[:, None, :]
            if tl is not None and t + 1 == tl:
                state_pool[ti].copy_(S)
            if intermediate_state is not None and slot > 0:
                intermediate_state[n, t].copy_(S)
            out[0, i] = torch.einsum("hk,hkv->hv", qn[0, i], S)
        if intermediate_state is None and slot > 0:
            state_pool[slot].copy_(S)
    return out.to(out_dtype)


# ---------------------------------------------------------------------------
# chunked (WY / UT-transform) form
# ---------------------------------------------------------------------------


def forward_substitution_inverse(N: torch.Tensor) -> torch.Tensor:
    """``X = (I - N)^-1 - I`` for strictly lower-triangular ``N`` (``[..., c, c]``).

    The reference's row-by-row forward substitution
    (bench/kda_chunk/kda_python.py:140-141, restated per head at
    tests/ops/test_kda_chunk.py:154-156): row ``i`` of ``X`` is
    ``N[i, :i] + sum_j N[i, j] X[j, :i]``.
    """
    X = N.clone()
    c = N.shape[-1]
    for i in range(1, c):
        X[..., i, :i] = X[..., i, :i] + (X[..., i, :, None] * X[..., :, :i]).sum(-2)
    return X


def chunk_factors(kc: torch.Tensor, qc: torch.Tensor, Gc: torch.Tensor, bc: torch.Tensor):
    """Intra-chunk matrices of one chunk, all heads at once.

    ``kc, qc, Gc``: ``[H, c, K]`` (``Gc`` is the in-chunk inclusive cumsum of
    the log decay), ``bc``: ``[H, c]``. Returns ``(Tm, Aqk)``:

    * ``Akk[i, j] = sum_k k_i k_j exp(G_i - G_j)`` and ``Aqk`` likewise with
      ``q_i`` (bench/kda_chunk/kda_python.py:133-137, :158-163);
    * ``Tm = (I + diag(beta) tril(Akk, -1))^-1 diag(beta)``, the UT transform,
      computed as ``(X + I) diag(beta)`` with ``X`` from
      :func:`forward_substitution_inverse` of ``-diag(beta) tril(Akk, -1)``
      (:138-142);
    * ``Aqk`` keeps ``j <= i`` (:149, :163).
    """
    H, c, K = kc.shape
    diff = Gc[:, :, None, :] - Gc[:, None, :, :]  # [H, i, j, K] = G_i - G_j
    lower = torch.tril(torch.ones(c, c, dtype=torch.bool), diagonal=-1)
    lower_eq = torch.tril(torch.ones(c, c, dtype=torch.bool), diagonal=0)
    # exp of the positive (upper-triangle) differences may overflow; those
    # entries are masked out, so evaluate the exponent only where kept.
    e = torch.where(lower_eq[None, :, :, None], diff, torch.zeros((), dtype=diff.dtype)).exp()
    Akk = torch.einsum("hik,hjk,hijk->hij", kc, kc, e)
    Aqk = torch.einsum("hik,hjk,hijk->hij", qc, kc, e)
    N = -(Akk * bc[:, :, None]).masked_fill(~lower[None], 0)
    X = forward_substitution_inverse(N)
    eye = torch.eye(c, dtype=kc.dtype)
    Tm = (X + eye) * bc[:, None, :]
    Aqk = Aqk.masked_fill(~lower_eq[None], 0)
    return Tm, Aqk


def kda_chunk(
    qn: torch.Tensor,
    kn: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    beta: torch.Tensor,
    *,
    state_pool: torch.Tensor,
    state_indices: torch.Tensor,
    cu_seqlens: torch.Tensor,
    chunk_size: int = 64,
    track_state_indices: Optional[torch.Tensor] = None,
    track_state_lens: Optional[torch.Tensor] = None,
    dtype: torch.dtype = torch.float32,
    out_dtype: Optional[torch.dtype] = None,
) -> torch.Tensor:
    """Chunked delta rule on prepared inputs; updates the pool in place.

    Follows ``kda_chunk_torch`` (bench/kda_chunk/kda_python.py:41-188). Per
    sequence and chunk ``c`` (``G`` = in-chunk cumsum of ``g``):

    * ``w = Tm (exp(G) * k)``, ``u = Tm v`` (:145-146);
    * ``vnew = u - w S``; ``o = (q * exp(G)) S + Aqk vnew`` (:165-167);
    * ``S = exp(G_last)[:, None] * S + (exp(G_last - G) * k)^T vnew``
      (:181-182);
    * tracking inside a chunk reconstructs the state after ``r`` of its tokens
      as ``exp(G_{r-1}) S + (exp(G_{r-1} - G[:r]) * k[:r])^T vnew[:r]``, and
      ``track_len == 0`` stores the initial state (:110-120, :168-179);
    * ``pool[slot] = S`` at the end when ``slot > 0`` (:185-186).

    Unlike the reference (which asserts ``len % chunk_size == 0``, :102), a
    sequence's last chunk may be shorter; it is evaluated as a chunk of its
    own length.
    """
    T, H, K = qn.shape[1:]
    V = v.shape[3]
    out_dtype = v.dtype if out_dtype is None else out_dtype
    qn, kn, v, g, beta = (t.to(dtype) for t in (qn, kn, v, g, beta))
    out = torch.zeros(1, T, H, V, dtype=dtype)
    cu = _as_list(cu_seqlens)
    slots = _as_list(state_indices)
    tidx = _as_list(track_state_indices)
    tlen = _as_list(track_state_lens)

    for n in range(len(cu) - 1):
        bos, eos, slot = cu[n], cu[n + 1], slots[n]
        if slot > 0:
            S = state_pool[slot].to(dtype).clone()
        else:
            S = torch.zeros(H, K, V, dtype=dtype)
        ti = 0 if tidx is None else tidx[n]
        tl = None if (tidx is None or ti <= 0) else tlen[n]
        if tl == 0:
            state_pool[ti].copy_(S)
        for c0 in range(bos, eos, chunk_size):
            c1 = min(c0 + chunk_size, eos)
            kc = kn[0, c0:c1].transpose(0, 1)  # [H, c, K]
            qc = qn[0, c0:c1].transpose(0, 1)
            vc = v[0, c0:c1].transpose(0, 1)  # [H, c, V]
            Gc = g[0, c0:c1].transpose(0, 1).cumsum(1)  # [H, c, K]
            bc = beta[0, c0:c1].transpose(0, 1)  # [H, c]
            Tm, Aqk = chunk_factors(kc, qc, Gc, bc)
            w = Tm @ (Gc.exp() * kc)
            u = Tm @ vc
            vnew = u - w @ S
            out[0, c0:c1] = ((qc * Gc.exp()) @ S + Aqk @ vnew).transpose(0, 1)
            if tl is not None and c0 - bos < tl <= c1 - bos:
                r = tl - (c0 - bos)
                gr = Gc[:, r - 1 : r, :]  # [H, 1, K]
                Sr = S * gr.transpose(1, 2).exp()
                Sr = Sr + ((gr - Gc[:, :r]).exp() * kc[:, :r]).transpose(1, 2) @ vnew[:, :r]
                state_pool[ti].copy_(Sr)
            gl = Gc[:, -1:, :]  # [H, 1, K]
            S = S * gl.transpose(1, 2).exp()
            S = S + ((gl - Gc).exp() * kc).transpose(1, 2) @ vnew
        if slot > 0:
            state_pool[slot].copy_(S)
    return out.to(out_dtype)


# ---------------------------------------------------------------------------
# the sglang-facing (raw gate) forms
# ---------------------------------------------------------------------------


def kda_varlen_recurrent_ref(
    *,
    A_log, a, dt_bias, q, k, v, b,
    initial_state_source, initial_state_indices, cu_seqlens,
    lower_bound, scale, intermediate_state=None, prefill=False,
    track_state_indices=None, track_state_lens=None,
    dtype: torch.dtype = torch.float32,
):
    """``kda_recur_torch`` with the op's keyword signature (kda_python.py:190-309)."""
    qn, kn, g, beta = kda_prepare(A_log, a, dt_bias, q, k, b, lower_bound, scale, dtype)
    return kda_recurrent(
        qn, kn, v, g, beta,
        state_pool=initial_state_source, state_indices=initial_state_indices,
        cu_seqlens=cu_seqlens, intermediate_state=intermediate_state,
        track_state_indices=track_state_indices, track_state_lens=track_state_lens,
        dtype=dtype,
    )


def kda_varlen_chunk_ref(
    *,
    A_log, a, dt_bias, q, k, v, b,
    initial_state_source, initial_state_indices, cu_seqlens,
    lower_bound, scale, prefill=False,
    track_state_indices=None, track_state_lens=None,
    chunk_size: int = 64,
    dtype: torch.dtype = torch.float32,
):
    """``kda_chunk_torch`` with the op's keyword signature (kda_python.py:41-188)."""
    qn, kn, g, beta = kda_prepare(A_log, a, dt_bias, q, k, b, lower_bound, scale, dtype)
    return kda_chunk(
        qn, kn, v, g, beta,
        state_pool=initial_state_source, state_indices=initial_state_indices,
        cu_seqlens=cu_seqlens, chunk_size=chunk_size,
        track_state_indices=track_state_indices, track_state_lens=track_state_lens,
        dtype=dtype,
    )


def prepared_recurrent_ref(
    qn, kn, v, gdecay, beta, out, state, indices, starts,
    track_indices=None, track_lens=None, track_state=False, head_offset=0,
    dtype: torch.dtype = torch.float32,
):
    """The ``prepared_recurrent`` op's recurrence (multiplicative decay input).

    Follows the prepared-gate recurrence stated in
    bench/_prepared_recurrent/bench_prepared_recurrent.py:84-121 and the
    Ascend launcher (sgl-glm53-ascend-ops/csrc/kda/prepared_recurrent.cpp:
    620-707): ``qn``/``kn`` fp32 already normalized (``qn`` scaled),
    ``gdecay = exp(g)``; one launch covers the four heads
    ``[head_offset, head_offset + 4)`` (:629-634, program id 2 offset by
    ``HEAD_OFFSET`` at bench_prepared_recurrent.py:84); each request ``n``
    covers rows ``[starts[n], starts[n+1])`` and only those rows of those
    heads are written to ``out`` (:117-118); the final state is written back
    when ``slot > 0`` (:120-121). ``qn, kn, v, gdecay`` are ``[T*H, D]`` or
    ``[1, T, H, D]``; ``beta`` is ``[T*H]`` or ``[1, T, H]``. Writes ``out``
    and ``state`` in place.
    """
    H = state.shape[1]
    D = state.shape[2]
    T = qn.numel() // (H * D)
    shp = (1, T, H, D)
    heads = list(range(head_offset, min(head_offset + 4, H)))
    sub = lambda x: x.reshape(shp)[:, :, heads]  # noqa: E731
    pool = state[:, heads]
    o = kda_recurrent(
        sub(qn), sub(kn), sub(v), None, beta.reshape(1, T, H)[:, :, heads],
        state_pool=pool, state_indices=indices, cu_seqlens=starts,
        track_state_indices=track_indices if track_state else None,
        track_state_lens=track_lens if track_state else None,
        dtype=dtype, decay=sub(gdecay),
    )
    state[:, heads] = pool
    o4 = out.view(shp)
    cu = _as_list(starts)
    for n in range(len(cu) - 1):
        o4[:, cu[n]:cu[n + 1], heads] = o[:, cu[n]:cu[n + 1]].to(out.dtype)
    return None
