"""Seeded input builders and the tolerance contract shared by the tests and bench.

Inputs are drawn on the CPU with ``torch.Generator().manual_seed(seed)`` so the
oracle, the CPU baseline and the GPU kernels see identical bytes; GPU tests
copy them to the device.

Tolerance contract (stated in the north star, metric defined here):

* ``max_rel_err(x, ref) = max|x - ref| / max|ref|`` per tensor;
* outputs: <= 2e-3 against the fp32 oracle's unrounded output. A bf16 output
  (the reference op's output dtype) carries its own rounding of up to half a
  bf16 ulp, i.e. up to 2**-8 of each element -- more than the budget itself --
  so for bf16 outputs the budget applies to the error beyond that rounding:
  ``max_i max(0, |x_i - ref_i| - ulp(x_i)/2) / max|ref|`` (``out_err``). fp32
  outputs use ``max_rel_err`` as is;
* states (fp32): <= 1e-3;
* slot selection, varlen boundaries, untouched slots: bit-exact.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional, Sequence

import torch

OUT_TOL = 2e-3
STATE_TOL = 1e-3


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def native_pool(slots: int, heads: int, D: int, seed: int, scale: float = 0.1) -> torch.Tensor:
    """fp32 pool ``[slots, H, K, V]`` with K contiguous (allocated [.., V, K])."""
    return (torch.randn(slots, heads, D, D, generator=gen(seed)) * scale).transpose(-1, -2)


def clone_pool(p: torch.Tensor) -> torch.Tensor:
    """Copy a pool keeping its [V, K] backing (a plain clone would change strides)."""
    return p.transpose(-1, -2).clone().transpose(-1, -2)


def to_dev(p: torch.Tensor, device) -> torch.Tensor:
    """Move a K-contiguous pool to ``device`` keeping its layout."""
    return p.transpose(-1, -2).contiguous().to(device).transpose(-1, -2)


def cu_from_lengths(lengths: Sequence[int]) -> torch.Tensor:
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    return torch.tensor(cu, dtype=torch.int32)


@dataclass
class RawCase:
    """Inputs of the sglang-facing (raw gate) ops, on the CPU."""

    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    a: torch.Tensor
    b: torch.Tensor
    A_log: torch.Tensor
    dt_bias: torch.Tensor
    pool: torch.Tensor
    indices: torch.Tensor
    cu_seqlens: torch.Tensor
    lower_bound: float
    scale: float
    track_indices: Optional[torch.Tensor] = None
    track_lens: Optional[torch.Tensor] = None

    def kwargs(self, device=None, pool=None, index_dtype=torch.int32):
        dev = (lambda t: t) if device is None else (lambda t: t.to(device))
        kw = dict(
            A_log=dev(self.A_log), a=dev(self.a), dt_bias=dev(self.dt_bias),
            q=dev(self.q), k=dev(self.k), v=dev(self.v), b=dev(self.b),
            initial_state_source=pool if pool is not None else self.pool,
            initial_state_indices=dev(self.indices.to(index_dtype)),
            cu_seqlens=dev(self.cu_seqlens.to(index_dtype)),
            lower_bound=self.lower_bound, scale=self.scale,
        )
        if self.track_indices is not None:
            kw["track_state_indices"] = dev(self.track_indices.to(index_dtype))
            kw["track_state_lens"] = dev(self.track_lens.to(index_dtype))
        return kw


def raw_case(heads: int, lengths: Sequence[int], *, D: int = 128, slots: Optional[int] = None,
             indices: Optional[Sequence[int]] = None, seed: int = 0, lower_bound: float = -5.0,
             track: Optional[tuple] = None) -> RawCase:
    """Distributions of the reference tests (test_kda_chunk.py:59-88): q,k,v,a
    ``randn*0.2`` bf16, ``b`` randn bf16, ``A_log, dt_bias`` ``randn*0.1``, pool
    ``randn*0.1`` K-contiguous."""
    g = gen(seed)
    T = int(sum(lengths))
    N = len(lengths)
    q, k, v, a = ((torch.randn(1, T, heads, D, generator=g) * 0.2).bfloat16() for _ in range(4))
    b = torch.randn(1, T, heads, generator=g).bfloat16()
    A_log = torch.randn(heads, generator=g) * 0.1
    dt_bias = torch.randn(heads * D, generator=g) * 0.1
    if indices is None:
        indices = list(range(1, N + 1))
    if slots is None:
        slots = max(list(indices) + [0]) + 2
    pool = native_pool(slots, heads, D, seed + 1000)
    case = RawCase(q, k, v, a, b, A_log, dt_bias, pool,
                   torch.tensor(indices, dtype=torch.int32), cu_from_lengths(lengths),
                   lower_bound, D ** -0.5)
    if track is not None:
        case.track_indices = torch.tensor(track[0], dtype=torch.int32)
        case.track_lens = torch.tensor(track[1], dtype=torch.int32)
    return case


@dataclass
class PreparedCase:
    """Inputs of the prepared-gate ops, on the CPU."""

    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    g: torch.Tensor
    beta: torch.Tensor
    pool: torch.Tensor
    indices: torch.Tensor
    cu_seqlens: torch.Tensor
    scale: float
    extra: dict = field(default_factory=dict)


def prepared_case(heads: int, lengths: Sequence[int], *, D: int = 128, dtype=torch.bfloat16,
                  slots: int = 0, indices: Optional[Sequence[int]] = None, seed: int = 0,
                  gate_scale: float = 1.0, gate_shift: float = 0.0, pool_scale: float = 0.05,
                  zero_pool: bool = False) -> PreparedCase:
    """BASELINE-config distributions: q, k L2-normalized (then cast), v randn,
    ``g = logsigmoid(randn*gate_scale + gate_shift)`` fp32 per channel,
    ``beta = sigmoid(randn)`` fp32, pool ``randn*pool_scale`` K-contiguous."""
    g_ = gen(seed)
    T = int(sum(lengths))
    N = len(lengths)

    def l2(x):
        return x / torch.sqrt((x * x).sum(-1, keepdim=True) + 1e-6)

    q = l2(torch.randn(1, T, heads, D, generator=g_)).to(dtype)
    k = l2(torch.randn(1, T, heads, D, generator=g_)).to(dtype)
    v = torch.randn(1, T, heads, D, generator=g_).to(dtype)
    g = torch.nn.functional.logsigmoid(
        torch.randn(1, T, heads, D, generator=g_) * gate_scale + gate_shift)
    beta = torch.sigmoid(torch.randn(1, T, heads, generator=g_))
    if indices is None:
        indices = list(range(1, N + 1))
    if slots <= 0:
        slots = max(list(indices) + [0]) + 1
    if zero_pool:
        pool = torch.zeros(slots, heads, D, D).transpose(-1, -2)
    else:
        pool = native_pool(slots, heads, D, seed + 1000, scale=pool_scale)
    return PreparedCase(q, k, v, g, beta, pool, torch.tensor(list(indices), dtype=torch.int32),
                        cu_from_lengths(lengths), D ** -0.5)


def max_rel_err(x: torch.Tensor, ref: torch.Tensor) -> float:
    x = x.detach().double().cpu()
    ref = ref.detach().double().cpu()
    assert x.shape == ref.shape, f"shape {tuple(x.shape)} != {tuple(ref.shape)}"
    if ref.numel() == 0:  # an empty batch (no tokens) has nothing to compare
        return 0.0
    den = ref.abs().max().item()
    num = (x - ref).abs().max().item()
    return num if den == 0.0 else num / den


def half_ulp_bf16(x: torch.Tensor) -> torch.Tensor:
    """Half a bf16 ulp at each element of ``x`` (a bf16-representable tensor)."""
    xd = x.detach().double().cpu().abs()
    _, e = torch.frexp(xd)  # |x| in [2**(e-1), 2**e)
    h = torch.ldexp(torch.ones_like(xd), e - 9)
    return torch.where(xd > 0, h, torch.full_like(xd, 2.0 ** -134))


def out_err(x: torch.Tensor, ref: torch.Tensor) -> float:
    """Output error of the tolerance contract (see the module docstring)."""
    if x.dtype != torch.bfloat16:
        return max_rel_err(x, ref)
    xd = x.detach().double().cpu()
    rd = ref.detach().double().cpu()
    assert xd.shape == rd.shape, f"shape {tuple(xd.shape)} != {tuple(rd.shape)}"
    if rd.numel() == 0:
        return 0.0
    den = rd.abs().max().item()
    beyond = ((xd - rd).abs() - half_ulp_bf16(x)).clamp_min(0).max().item()
    return beyond if den == 0.0 else beyond / den


def assert_rel(x: torch.Tensor, ref: torch.Tensor, tol: float, what: str) -> float:
    err = max_rel_err(x, ref)
    assert err <= tol, f"{what}: max|x-ref|/max|ref| = {err:.3e} > {tol:.1e}"
    return err


def assert_out(x: torch.Tensor, ref: torch.Tensor, tol: float, what: str) -> float:
    err = out_err(x, ref)
    raw = max_rel_err(x, ref)
    assert err <= tol, (f"{what}: error beyond output rounding {err:.3e} > {tol:.1e} "
                        f"(raw max|x-ref|/max|ref| {raw:.3e})")
    return err
