"""Keyword-only Python wrappers over ``torch.ops.sgl_glm53_ascend``.

Names, keywords and in-place behaviour are those of the reference wrappers
(sgl-glm53-ascend-ops/src/sgl_glm53_ascend_ops/ops/kda.py:6-236). Behind them
sit hand-written HIP kernels for gfx950 (``libkda_amd.so``); nothing here
computes anything itself.

Differences from the reference contract, all widening it:

* ``kda_varlen_recurrent`` runs any head count H and any number of prefill
  sequences (the reference's Ascend kernels exist for H in {4, 8} prefill and
  {16, 32, 64} decode only), and K == V in {64, 128};
* ``kda_varlen_chunk`` accepts sequence lengths that are not a multiple of 64
  (the last chunk of a sequence is simply shorter) and never synchronizes the
  host;
* the ``*_v2`` names are served by the same kernels (the reference's v2 ops
  are unfinished stubs awaiting cutover, ops/kda.py:46-52).

Added for the prepared-gate form the measured configurations use:
``kda_prepared_varlen_recurrent`` / ``kda_prepared_varlen_chunk`` (q, k, v;
fp32 log decay ``g``; fp32 ``beta``) and ``kda_varlen_chunk_with_state``,
which also returns the final states.
"""

from typing import Optional, Tuple

import torch

from .. import load_library

load_library()
_OPS = torch.ops.sgl_glm53_ascend


def prepared_recurrent(
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
    """Recurrence on prepared fp32 ``qn``/``kn``/``gdecay`` (= exp(g)), fp32 ``beta``.

    Writes ``out`` and ``state`` in place for heads
    ``[head_offset, head_offset + 4)`` (the reference's four heads per
    launch, prepared_recurrent.cpp:629-634). ``state`` may be K-contiguous
    (native) or [K,V]-contiguous (the reference's layout); either is read and
    updated in place, with no pool-sized working copy.
    """
    return _OPS.prepared_recurrent(
        qn, kn, v, gdecay, beta, out, state, indices, starts,
        track_indices, track_lens, track_state, head_offset,
    )


def kda_varlen_recurrent(
    *,
    A_log: torch.Tensor,
    a: torch.Tensor,
    dt_bias: torch.Tensor,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    b: torch.Tensor,
    initial_state_source: torch.Tensor,
    initial_state_indices: torch.Tensor,
    cu_seqlens: torch.Tensor,
    lower_bound: float,
    scale: float,
    intermediate_state: Optional[torch.Tensor] = None,
    prefill: bool = False,
    track_state_indices: Optional[torch.Tensor] = None,
    track_state_lens: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Fused KDA varlen recurrence; returns the output, updates state in place.

    Raw gates as sglang passes them: ``q, k, a`` bf16 ``[1, T, H, K]``, ``v``
    bf16 ``[1, T, H, V]``, ``b`` bf16 ``[1, T, H]``, ``A_log`` fp32 ``[H]``,
    ``dt_bias`` fp32 ``[H*K]``. ``initial_state_source`` is the fp32 pool
    ``[slots, H, K, V]`` with K contiguous (stride(2)==1, stride(3)==K);
    slot 0 is the padding row (zero state, never written).

    ``intermediate_state`` (decode only) receives the state after every step,
    indexed ``[request, step]``, and suppresses the final write-back.
    ``track_state_indices/lens`` (prefill only) store the state after
    ``lens[i]`` tokens of request ``i`` into slot ``indices[i]``.
    """
    return _OPS.kda_varlen_recurrent(
        A_log=A_log, a=a, dt_bias=dt_bias, q=q, k=k, v=v, b=b,
        initial_state_source=initial_state_source,
        initial_state_indices=initial_state_indices,
        cu_seqlens=cu_seqlens, lower_bound=lower_bound, scale=scale,
        intermediate_state=intermediate_state, prefill=prefill,
        track_state_indices=track_state_indices, track_state_lens=track_state_lens,
    )


def kda_varlen_recurrent_v2(**kwargs) -> torch.Tensor:
    """Interface identical to :func:`kda_varlen_recurrent` (same kernels)."""
    return _OPS.kda_varlen_recurrent_v2(**kwargs)


def kda_varlen_chunk(
    *,
    A_log: torch.Tensor,
    a: torch.Tensor,
    dt_bias: torch.Tensor,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    b: torch.Tensor,
    initial_state_source: torch.Tensor,
    initial_state_indices: torch.Tensor,
    cu_seqlens: torch.Tensor,
    lower_bound: float,
    scale: float,
    prefill: bool = False,
    track_state_indices: Optional[torch.Tensor] = None,
    track_state_lens: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Chunked KDA (64-token chunks); returns the output, updates state in place.

    The chunked form of :func:`kda_varlen_recurrent` with the same interface
    minus ``intermediate_state``. Requires H == HV and K == V == 128; any
    sequence lengths. The final state of request ``i`` is written to
    ``initial_state_source[initial_state_indices[i]]`` when that slot is > 0.
    """
    return _OPS.kda_varlen_chunk(
        A_log=A_log, a=a, dt_bias=dt_bias, q=q, k=k, v=v, b=b,
        initial_state_source=initial_state_source,
        initial_state_indices=initial_state_indices,
        cu_seqlens=cu_seqlens, lower_bound=lower_bound, scale=scale,
        prefill=prefill, track_state_indices=track_state_indices,
        track_state_lens=track_state_lens,
    )


def kda_varlen_chunk_v2(**kwargs) -> torch.Tensor:
    """Interface identical to :func:`kda_varlen_chunk` (same kernels)."""
    return _OPS.kda_varlen_chunk_v2(**kwargs)


def kda_prepared_varlen_recurrent(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    beta: torch.Tensor,
    *,
    initial_state_source: torch.Tensor,
    initial_state_indices: torch.Tensor,
    cu_seqlens: torch.Tensor,
    scale: float,
    use_qk_l2norm: bool = False,
    intermediate_state: Optional[torch.Tensor] = None,
    track_state_indices: Optional[torch.Tensor] = None,
    track_state_lens: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Recurrence on prepared gates: fp32 log decay ``g`` ``[1,T,H,K]``, fp32 ``beta`` ``[1,T,H]``.

    ``q, k, v`` share one dtype (bf16 or fp32); ``q`` is multiplied by
    ``scale`` (after an in-kernel L2 norm when ``use_qk_l2norm``). Pool and
    slot rules as :func:`kda_varlen_recurrent`. Returns ``o`` in ``v``'s dtype.
    """
    return _OPS.kda_prepared_varlen_recurrent(
        q, k, v, g, beta,
        initial_state_source=initial_state_source,
        initial_state_indices=initial_state_indices,
        cu_seqlens=cu_seqlens, scale=scale, use_qk_l2norm=use_qk_l2norm,
        intermediate_state=intermediate_state,
        track_state_indices=track_state_indices, track_state_lens=track_state_lens,
    )


def kda_prepared_varlen_chunk(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    beta: torch.Tensor,
    *,
    initial_state_source: torch.Tensor,
    initial_state_indices: torch.Tensor,
    cu_seqlens: torch.Tensor,
    scale: float,
    use_qk_l2norm: bool = False,
    track_state_indices: Optional[torch.Tensor] = None,
    track_state_lens: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Chunked prefill on prepared gates (bf16 ``q, k, v``; fp32 ``g``, ``beta``)."""
    return _OPS.kda_prepared_varlen_chunk(
        q, k, v, g, beta,
        initial_state_source=initial_state_source,
        initial_state_indices=initial_state_indices,
        cu_seqlens=cu_seqlens, scale=scale, use_qk_l2norm=use_qk_l2norm,
        track_state_indices=track_state_indices, track_state_lens=track_state_lens,
    )


def kda_varlen_chunk_with_state(**kwargs) -> Tuple[torch.Tensor, torch.Tensor]:
    """``(o, final_state)``: :func:`kda_varlen_chunk`, then the updated slots.

    ``final_state`` is ``initial_state_source[initial_state_indices]`` read
    after the call (fp32 ``[N, H, K, V]``), the way the reference bench reads
    the chunk op's result back out of the pool (bench_kda_chunk.py:467).
    Requests on slot 0 have no stored state; their rows read slot 0.
    """
    out = kda_varlen_chunk(**kwargs)
    pool = kwargs["initial_state_source"]
    idx = kwargs["initial_state_indices"].long()
    return out, pool[idx]
