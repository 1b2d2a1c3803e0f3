"""GPU parity of the recurrent (decode / verify / prefill) kernel against the oracle.

Cases follow the reference's own suites:

* decode at H in {16, 32, 64} over the step-group lengths of
  tests/ops/test_kda_decode_numerics.py:42-53 (bit-exact against sglang's
  Triton there; against the fp32 oracle at the tolerance contract here, since
  that kernel is not available);
* per-step checkpoints (:152-167) and untouched slots (:170-180);
* int32 / int64 metadata invariance (tests/ops/test_kda_index_dtypes.py);
* prefix tracking at 0 / mid / boundary / end (tests/ops/test_kda_chunk.py:203-214);
* BASELINE config 1 (golden fixture) and config 2 (B=256 decode, 512-slot pool
  with a random slot permutation that may include the padding slot 0).

Outputs are bf16 and are compared with the oracle's unrounded fp32 output
through ``kda_cases.out_err`` (the error beyond the output's own bf16
rounding); states are compared fp32 to fp32.
"""

import ctypes
import os

import numpy as np
import pytest
import torch

from oracle import kda_ref as R
from tests import kda_cases as C

pytestmark = pytest.mark.gpu

DEV = "cuda"
HEADS = (16, 32, 64)
DECODE_CASES = [
    (1,), (4,), (5,), (8,), (9,), (16,), (1,) * 8, (4,) * 4, (1, 2, 3, 4, 5, 6, 7), (7, 1, 4, 9),
]


def _oracle_raw(case, pool_cpu, mid=None):
    qn, kn, g, beta = R.kda_prepare(case.A_log, case.a, case.dt_bias, case.q, case.k, case.b,
                                    case.lower_bound, case.scale)
    return R.kda_recurrent(qn, kn, case.v, g, beta, state_pool=pool_cpu,
                           state_indices=case.indices, cu_seqlens=case.cu_seqlens,
                           intermediate_state=mid, track_state_indices=case.track_indices,
                           track_state_lens=case.track_lens, out_dtype=torch.float32)


def _run_raw(ops, case, prefill, mid=None, index_dtype=torch.int32):
    pool = C.to_dev(case.pool, DEV)
    kw = case.kwargs(DEV, pool=pool, index_dtype=index_dtype)
    out = ops.kda_varlen_recurrent(intermediate_state=mid, prefill=prefill, **kw)
    torch.cuda.synchronize()
    return out, pool


@pytest.mark.parametrize("lengths", DECODE_CASES, ids=lambda l: "x".join(map(str, l)))
@pytest.mark.parametrize("heads", HEADS)
def test_decode_matches_oracle(gpu_ops, heads, lengths):
    case = C.raw_case(heads, lengths, slots=16, seed=31337 + 97 * sum(lengths) + len(lengths))
    out, pool = _run_raw(gpu_ops, case, prefill=False)
    ref_pool = C.clone_pool(case.pool)
    ref = _oracle_raw(case, ref_pool)
    C.assert_out(out.cpu(), ref, C.OUT_TOL, f"H={heads} {lengths} output")
    C.assert_rel(pool.cpu(), ref_pool, C.STATE_TOL, f"H={heads} {lengths} state")
    touched = set(case.indices.tolist())
    other = [s for s in range(case.pool.shape[0]) if s not in touched]
    assert torch.equal(pool.cpu()[other], case.pool[other]), "an unindexed slot was written"


@pytest.mark.parametrize("lengths", [(4,), (4,) * 4, (5,), (1, 2, 3, 4, 5, 6, 7)],
                         ids=lambda l: "x".join(map(str, l)))
@pytest.mark.parametrize("heads", HEADS)
def test_decode_checkpoints_match_oracle(gpu_ops, heads, lengths):
    """Verify regime: every step checkpointed, the source slot left alone."""
    case = C.raw_case(heads, lengths, slots=16, seed=5150 + sum(lengths))
    steps = max(lengths)
    noise = (torch.randn(len(lengths), steps, heads, 128, 128, generator=C.gen(5150)) * 0.1
             ).transpose(-1, -2)
    mid_dev = noise.transpose(-1, -2).contiguous().to(DEV).transpose(-1, -2)
    out, pool = _run_raw(gpu_ops, case, prefill=False, mid=mid_dev)
    ref_pool = C.clone_pool(case.pool)
    ref_mid = noise.clone()
    ref = _oracle_raw(case, ref_pool, mid=ref_mid)
    C.assert_out(out.cpu(), ref, C.OUT_TOL, "output")
    got_mid = mid_dev.cpu()
    for n, L in enumerate(lengths):
        C.assert_rel(got_mid[n, :L], ref_mid[n, :L], C.STATE_TOL, f"checkpoints of request {n}")
        assert torch.equal(got_mid[n, L:], noise[n, L:]), "a step past the request was written"
    assert torch.equal(pool.cpu(), case.pool), "checkpointing must skip the write-back"


def test_decode_padding_slot_and_untouched(gpu_ops):
    """Slot 0 reads as zero and is never written; other slots stay byte-identical."""
    case = C.raw_case(32, (3, 1, 2), indices=[0, 5, 2], slots=8, seed=11)
    out, pool = _run_raw(gpu_ops, case, prefill=False)
    ref_pool = C.clone_pool(case.pool)
    ref = _oracle_raw(case, ref_pool)
    C.assert_out(out.cpu(), ref, C.OUT_TOL, "output")
    got = pool.cpu()
    for s in (0, 1, 3, 4, 6, 7):
        assert torch.equal(got[s], case.pool[s]), f"slot {s} changed"
    C.assert_rel(got[[2, 5]], ref_pool[[2, 5]], C.STATE_TOL, "written slots")


@pytest.mark.parametrize("index_dtype,starts_dtype",
                         [(torch.int64, torch.int32), (torch.int32, torch.int64),
                          (torch.int64, torch.int64)])
def test_index_dtype_does_not_change_result(gpu_ops, index_dtype, starts_dtype):
    """int64 metadata is narrowed on the device, never misread (test_kda_index_dtypes.py)."""
    case = C.raw_case(4, (257,), indices=[3], slots=6, seed=5)
    base_out, base_pool = _run_raw(gpu_ops, case, prefill=True)
    pool = C.to_dev(case.pool, DEV)
    kw = case.kwargs(DEV, pool=pool)
    kw["initial_state_indices"] = kw["initial_state_indices"].to(index_dtype)
    kw["cu_seqlens"] = kw["cu_seqlens"].to(starts_dtype)
    out = gpu_ops.kda_varlen_recurrent(prefill=True, **kw)
    torch.cuda.synchronize()
    assert out.float().abs().sum().item() > 0, "op returned an unwritten output"
    assert torch.equal(out, base_out)
    assert torch.equal(pool.cpu(), base_pool.cpu())


@pytest.mark.parametrize("track_len", [0, 32, 64, 100, 192])
def test_prefill_tracking_matches_oracle(gpu_ops, track_len):
    case = C.raw_case(2, (192, 70), indices=[1, 2], slots=8, seed=40 + track_len,
                      track=([4, 0], [track_len, 5]))
    out, pool = _run_raw(gpu_ops, case, prefill=True)
    ref_pool = C.clone_pool(case.pool)
    ref = _oracle_raw(case, ref_pool)
    C.assert_out(out.cpu(), ref, C.OUT_TOL, "output")
    C.assert_rel(pool.cpu(), ref_pool, C.STATE_TOL, "pool incl. tracked slot 4")
    assert not torch.equal(pool.cpu()[4], case.pool[4]), "tracked slot unwritten"


@pytest.mark.parametrize("track_dtype", (torch.int32, torch.int64))
def test_track_dtype_does_not_change_checkpoint(gpu_ops, track_dtype):
    case = C.raw_case(4, (257,), indices=[3], slots=6, seed=5, track=([5], [64]))
    base_out, base_pool = _run_raw(gpu_ops, case, prefill=True)
    out, pool = _run_raw(gpu_ops, case, prefill=True, index_dtype=track_dtype)
    assert torch.equal(out, base_out)
    assert torch.equal(pool.cpu(), base_pool.cpu())
    assert pool.cpu()[5].abs().sum().item() > 0, "checkpoint slot unwritten"


def test_tokens_outside_sequences_are_zero(gpu_ops):
    case = C.raw_case(8, (10, 7, 3), slots=6, seed=21)
    T = case.q.shape[1]
    case.cu_seqlens = torch.tensor([0, 10, 17, T - 3], dtype=torch.int32)  # 3 tail tokens
    pool = C.to_dev(case.pool, DEV)
    kw = case.kwargs(DEV, pool=pool)
    # Poison the allocator so a skipped token would show as garbage.
    torch.full((1, T, 8, 128), float("nan"), device=DEV, dtype=torch.bfloat16)
    out = gpu_ops.kda_varlen_recurrent(prefill=True, **kw).cpu()
    ref_pool = C.clone_pool(case.pool)
    ref = _oracle_raw(case, ref_pool)
    assert torch.equal(out[0, T - 3:], torch.zeros_like(out[0, T - 3:]))
    C.assert_out(out, ref, C.OUT_TOL, "output")


def test_sequences_are_independent(gpu_ops):
    case = C.raw_case(16, (9, 4, 12), slots=6, seed=77)
    out1, _ = _run_raw(gpu_ops, case, prefill=True)
    case.v = case.v.clone()
    case.v[0, 13:] += 1.0  # perturb the last request only
    out2, _ = _run_raw(gpu_ops, case, prefill=True)
    assert torch.equal(out1[0, :13], out2[0, :13])
    assert not torch.equal(out1[0, 13:], out2[0, 13:])


@pytest.mark.parametrize("batch", [1, 3, 40])
@pytest.mark.parametrize("D", [64, 128])
def test_value_split_launches(gpu_ops, batch, D):
    """Small batches split the value rows over workgroups; same numbers."""
    case = C.raw_case(8, (2,) * batch, D=D, slots=batch + 2, seed=300 + batch + D)
    out, pool = _run_raw(gpu_ops, case, prefill=False)
    ref_pool = C.clone_pool(case.pool)
    ref = _oracle_raw(case, ref_pool)
    C.assert_out(out.cpu(), ref, C.OUT_TOL, "output")
    C.assert_rel(pool.cpu(), ref_pool, C.STATE_TOL, "state")


# --- prepared-gate forms ----------------------------------


def _oracle_prepared(case, pool_cpu, mid=None):
    return R.kda_recurrent(case.q.float() * case.scale, case.k, case.v, case.g, case.beta,
                           state_pool=pool_cpu, state_indices=case.indices,
                           cu_seqlens=case.cu_seqlens, intermediate_state=mid,
                           out_dtype=torch.float32)


def _run_prepared(ops, case, mid=None):
    pool = C.to_dev(case.pool, DEV)
    out = ops.kda_prepared_varlen_recurrent(
        case.q.to(DEV), case.k.to(DEV), case.v.to(DEV), case.g.to(DEV), case.beta.to(DEV),
        initial_state_source=pool, initial_state_indices=case.indices.to(DEV),
        cu_seqlens=case.cu_seqlens.to(DEV), scale=case.scale, intermediate_state=mid)
    torch.cuda.synchronize()
    return out, pool


def test_config1_golden_fixture(gpu_ops):
    """BASELINE config 1 (fp32, D=64, cu=[0,37,100]) against the committed fp64 truth."""
    path = os.path.join(os.path.dirname(__file__), "golden", "config1.npz")
    z = np.load(path)
    T, H, D = z["q"].shape
    f = lambda n: torch.from_numpy(z[n]).unsqueeze(0).to(DEV)  # noqa: E731
    pool = torch.zeros(3, H, D, D, device=DEV).transpose(-1, -2)
    out = gpu_ops.kda_prepared_varlen_recurrent(
        f("q"), f("k"), f("v"), f("g"), f("beta"), initial_state_source=pool,
        initial_state_indices=torch.from_numpy(z["state_indices"]).to(DEV),
        cu_seqlens=torch.from_numpy(z["cu_seqlens"]).to(DEV), scale=float(z["scale"]))
    torch.cuda.synchronize()
    o_ref = torch.from_numpy(z["o_f64"])
    s_ref = torch.from_numpy(z["state_f64"])
    assert C.max_rel_err(out[0].cpu(), o_ref) < 1e-5
    assert C.max_rel_err(pool[1:3].cpu(), s_ref) < 1e-5


def test_config2_decode_b256(gpu_ops):
    """256 sequences x 1 token, H=32, D=128, 512-slot pool.

    The seeded permutation (seed 2) happens to miss slot 0, so its first entry
    is replaced by the padding slot: one sequence then starts from a zero
    state and must not write back, and slot 0 stays byte-identical."""
    perm = torch.randperm(512, generator=C.gen(2))[:256].tolist()
    if 0 not in perm:
        perm[0] = 0
    case = C.prepared_case(32, (1,) * 256, slots=512, indices=perm, seed=2)
    out, pool = _run_prepared(gpu_ops, case)
    ref_pool = C.clone_pool(case.pool)
    ref = _oracle_prepared(case, ref_pool)
    C.assert_out(out.cpu(), ref, C.OUT_TOL, "output")
    got = pool.cpu()
    C.assert_rel(got, ref_pool, C.STATE_TOL, "pool")
    untouched = sorted(set(range(512)) - set(perm) | {0})
    assert torch.equal(got[untouched], case.pool[untouched]), "unindexed slot written"


def test_multistep_decode_harsh_gate(gpu_ops):
    """BASELINE config 5's decode half, scaled down: 4 tokens x 256 sequences,
    H=16, harsh decay logsigmoid(randn*2-2), 512-slot pool."""
    perm = torch.randperm(512, generator=C.gen(5))[:256].tolist()
    case = C.prepared_case(16, (4,) * 256, slots=512, indices=perm, seed=5,
                           gate_scale=2.0, gate_shift=-2.0)
    out, pool = _run_prepared(gpu_ops, case)
    ref_pool = C.clone_pool(case.pool)
    ref = _oracle_prepared(case, ref_pool)
    C.assert_out(out.cpu(), ref, C.OUT_TOL, "output")
    C.assert_rel(pool.cpu(), ref_pool, C.STATE_TOL, "pool")


def test_prepared_fp32_l2norm_in_kernel(gpu_ops):
    """use_qk_l2norm normalizes q and k on the device (fp32 I/O)."""
    case = C.prepared_case(4, (33, 20), D=64, dtype=torch.float32, seed=9)
    g_ = C.gen(10)
    case.q = torch.randn(case.q.shape, generator=g_)
    case.k = torch.randn(case.k.shape, generator=g_)
    pool = C.to_dev(case.pool, DEV)
    out = gpu_ops.kda_prepared_varlen_recurrent(
        case.q.to(DEV), case.k.to(DEV), case.v.to(DEV), case.g.to(DEV), case.beta.to(DEV),
        initial_state_source=pool, initial_state_indices=case.indices.to(DEV),
        cu_seqlens=case.cu_seqlens.to(DEV), scale=case.scale, use_qk_l2norm=True)
    torch.cuda.synchronize()
    ref_pool = C.clone_pool(case.pool)
    ref = R.kda_recurrent(R.l2norm_last(case.q) * case.scale, R.l2norm_last(case.k), case.v,
                          case.g, case.beta, state_pool=ref_pool, state_indices=case.indices,
                          cu_seqlens=case.cu_seqlens, out_dtype=torch.float32)
    assert C.max_rel_err(out.cpu(), ref) < 1e-5
    assert C.max_rel_err(pool.cpu(), ref_pool) < 1e-5


@pytest.mark.parametrize("k_contiguous", [True, False])
def test_prepared_recurrent_decay_form(gpu_ops, k_contiguous):
    """The reference's prepared_recurrent op: fp32 qn/kn/gdecay, two 4-head launches."""
    H, D, T = 8, 128, 12
    g_ = C.gen(13)
    qn = R.l2norm_last(torch.randn(T * H, D, generator=g_)) * D ** -0.5
    kn = R.l2norm_last(torch.randn(T * H, D, generator=g_))
    v = torch.randn(T * H, D, generator=g_).bfloat16()
    gdecay = torch.exp(torch.nn.functional.logsigmoid(torch.randn(T * H, D, generator=g_)))
    beta = torch.sigmoid(torch.randn(T * H, generator=g_))
    pool_k = C.native_pool(3, H, D, seed=14)
    pool = C.to_dev(pool_k, DEV) if k_contiguous else pool_k.contiguous().to(DEV)
    out = torch.zeros(T * H, D, dtype=torch.bfloat16, device=DEV)
    idx = torch.tensor([2], dtype=torch.int32, device=DEV)
    starts = torch.tensor([0, T], dtype=torch.int32, device=DEV)
    args = [qn.to(DEV), kn.to(DEV), v.to(DEV), gdecay.to(DEV), beta.to(DEV), out, pool, idx, starts]
    gpu_ops.prepared_recurrent(*args, None, None, False, 0)
    torch.cuda.synchronize()
    half = pool.cpu().clone()
    gpu_ops.prepared_recurrent(*args, None, None, False, 4)
    torch.cuda.synchronize()
    ref_pool = C.clone_pool(pool_k)
    ref_out = torch.zeros(T * H, D, dtype=torch.float32)
    for off in (0, 4):
        R.prepared_recurrent_ref(qn, kn, v, gdecay, beta, ref_out, ref_pool, torch.tensor([2]),
                                 torch.tensor([0, T]), head_offset=off)
    C.assert_out(out.cpu(), ref_out, C.OUT_TOL, "out")
    C.assert_rel(pool.cpu(), ref_pool, C.STATE_TOL, "state")
    # The first launch touched heads 0-3 only.
    assert torch.equal(half[2, 4:], pool_k[2, 4:])
    assert not torch.equal(half[2, :4], pool_k[2, :4])
    # Neither layout makes a pool-sized working copy: a pool of 256 slots
    # (128 MiB) costs the call no more than its small index conversions.
    big = (C.to_dev(C.native_pool(256, H, D, seed=15), DEV) if k_contiguous
           else C.native_pool(256, H, D, seed=15).contiguous().to(DEV))
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    base = torch.cuda.memory_allocated()
    args[6] = big
    gpu_ops.prepared_recurrent(*args, None, None, False, 0)
    torch.cuda.synchronize()
    assert torch.cuda.max_memory_allocated() - base < (1 << 20)


def test_prepared_recurrent_writes_only_covered_rows(gpu_ops):
    """A caller-owned ``out`` keeps every row its requests do not cover and
    every head outside the launch (the reference's prepared kernels write rows
    [bos, eos) of their four heads only): starts=[3, T-2], sentinel fill."""
    H, D, T = 8, 128, 14
    g_ = C.gen(15)
    qn = R.l2norm_last(torch.randn(T * H, D, generator=g_)) * D ** -0.5
    kn = R.l2norm_last(torch.randn(T * H, D, generator=g_))
    v = torch.randn(T * H, D, generator=g_).bfloat16()
    gdecay = torch.exp(torch.nn.functional.logsigmoid(torch.randn(T * H, D, generator=g_)))
    beta = torch.sigmoid(torch.randn(T * H, generator=g_))
    pool_k = C.native_pool(3, H, D, seed=16)
    pool = C.to_dev(pool_k, DEV)
    out = torch.full((T * H, D), 7.0, dtype=torch.bfloat16, device=DEV)
    starts = torch.tensor([3, T - 2], dtype=torch.int32)
    gpu_ops.prepared_recurrent(qn.to(DEV), kn.to(DEV), v.to(DEV), gdecay.to(DEV), beta.to(DEV),
                               out, pool, torch.tensor([1], dtype=torch.int32, device=DEV),
                               starts.to(DEV), None, None, False, 4)
    torch.cuda.synchronize()
    ref_pool = C.clone_pool(pool_k)
    ref_out = torch.full((T * H, D), 7.0, dtype=torch.float32)
    R.prepared_recurrent_ref(qn, kn, v, gdecay, beta, ref_out, ref_pool, torch.tensor([1]),
                             starts, head_offset=4)
    got = out.cpu().float().reshape(T, H, D)
    exp = ref_out.reshape(T, H, D)
    sentinel = torch.full_like(got[:3], 7.0)
    assert torch.equal(got[:3], sentinel), "rows before starts[0] were written"
    assert torch.equal(got[T - 2:], torch.full_like(got[T - 2:], 7.0)), "rows past starts[N] written"
    assert torch.equal(got[:, :4], torch.full_like(got[:, :4], 7.0)), "heads outside the launch written"
    C.assert_out(out.cpu().reshape(T, H, D)[3:T - 2, 4:], exp[3:T - 2, 4:], C.OUT_TOL, "covered rows")
    C.assert_rel(pool.cpu(), ref_pool, C.STATE_TOL, "state")
    assert torch.equal(pool.cpu()[:, :4], pool_k[:, :4])


# --- the C ABI on its own ------------------------------------------------------


class _Args(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("gate", ctypes.c_void_p), ("beta", ctypes.c_void_p),
        ("A_log", ctypes.c_void_p), ("dt_bias", ctypes.c_void_p),
        ("state", ctypes.c_void_p), ("state_stride_slot", ctypes.c_int64),
        ("state_stride_head", ctypes.c_int64), ("num_slots", ctypes.c_int64),
        ("state_indices", ctypes.c_void_p), ("cu_seqlens", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("intermediate", ctypes.c_void_p), ("mid_stride_req", ctypes.c_int64),
        ("mid_stride_step", ctypes.c_int64), ("mid_stride_head", ctypes.c_int64),
        ("mid_rows", ctypes.c_int64), ("mid_steps", ctypes.c_int64),
        ("track_indices", ctypes.c_void_p), ("track_lens", ctypes.c_void_p),
        ("scale", ctypes.c_float), ("lower_bound", ctypes.c_float),
        ("num_seqs", ctypes.c_int32), ("num_tokens", ctypes.c_int32),
        ("num_heads", ctypes.c_int32), ("head_begin", ctypes.c_int32),
        ("head_count", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("qk_dtype", ctypes.c_int32), ("v_dtype", ctypes.c_int32),
        ("gate_mode", ctypes.c_int32), ("qk_l2norm", ctypes.c_int32),
        ("state_v_contiguous", ctypes.c_int32),
    ]


def test_c_abi_launch_direct(gpu_ops):
    """kda_recurrent_launch through ctypes, no torch operator in between."""
    from sgl_glm53_ascend_ops._load import abi_library_path

    lib = ctypes.CDLL(str(abi_library_path()))
    lib.kda_recurrent_launch.argtypes = [ctypes.POINTER(_Args), ctypes.c_void_p]
    lib.kda_recurrent_launch.restype = ctypes.c_int
    case = C.prepared_case(4, (5, 3), D=128, seed=17)
    dev = {n: getattr(case, n).to(DEV) for n in ("q", "k", "v", "g", "beta")}
    pool = C.to_dev(case.pool, DEV)
    idx = case.indices.to(DEV)
    cu = case.cu_seqlens.to(DEV)
    out = torch.empty_like(dev["v"])
    T, H, D = case.q.shape[1:]
    a = _Args(q=dev["q"].data_ptr(), k=dev["k"].data_ptr(), v=dev["v"].data_ptr(),
              gate=dev["g"].data_ptr(), beta=dev["beta"].data_ptr(),
              state=pool.data_ptr(), state_stride_slot=pool.stride(0),
              state_stride_head=pool.stride(1), num_slots=pool.shape[0],
              state_indices=idx.data_ptr(), cu_seqlens=cu.data_ptr(), out=out.data_ptr(),
              scale=case.scale, num_seqs=2, num_tokens=T, num_heads=H, head_begin=0,
              head_count=H, head_dim=D, qk_dtype=0, v_dtype=0, gate_mode=1, qk_l2norm=0)
    stream = torch.cuda.current_stream().cuda_stream
    assert lib.kda_recurrent_launch(ctypes.byref(a), ctypes.c_void_p(stream)) == 0
    torch.cuda.synchronize()
    ref_pool = C.clone_pool(case.pool)
    ref = _oracle_prepared(case, ref_pool)
    C.assert_out(out.cpu(), ref, C.OUT_TOL, "output")
    C.assert_rel(pool.cpu(), ref_pool, C.STATE_TOL, "state")


def _shifted(x, shift):
    """``x`` on the device at a storage offset of ``shift`` elements (so a
    nonzero shift leaves it misaligned for vector access), plus the flat
    buffer that owns it."""
    flat = torch.zeros(x.numel() + shift, dtype=x.dtype, device=DEV)
    view = flat[shift:].view(x.shape)
    view.copy_(x.to(DEV))
    return view, flat


# (gate mode, q/k dtype, v dtype): the prepared forms the launcher accepts.
_FORMS = {
    "log-bf16": (1, torch.bfloat16, torch.bfloat16),
    "log-f32": (1, torch.float32, torch.float32),
    "decay-f32-bf16": (2, torch.float32, torch.bfloat16),
    "decay-f32": (2, torch.float32, torch.float32),
}
_KDA_DTYPE = {torch.bfloat16: 0, torch.float32: 1}


@pytest.mark.parametrize("shift", [0, 1], ids=["aligned", "misaligned"])
@pytest.mark.parametrize("form", sorted(_FORMS))
@pytest.mark.parametrize("lengths,heads", [((1,) * 128, 1), ((2,) * 8, 16), ((4,) * 8, 16),
                                           ((1, 7, 3, 5, 2, 6, 4, 8), 16), ((3,) * 64, 16)],
                         ids=["decode", "2tok", "4tok", "ragged", "3tok-1024pairs"])
def test_tile_shapes_and_io_forms(gpu_ops, lengths, heads, form, shift):
    """Every tile shape the launcher picks for D=128 with at least 128
    (sequence, head) pairs (one token: 32-lane rows, 16-row tiles; two
    tokens per sequence: 32-lane rows, 32-row tiles; more: 16-lane rows,
    64-row tiles, or 128-row tiles from 1024 pairs, whose v and o rows move
    as vectors), in every prepared input form, with v and out aligned or
    shifted by one element (the per-element path), through the C ABI,
    against the oracle."""
    from sgl_glm53_ascend_ops._load import abi_library_path

    mode, qk_dt, v_dt = _FORMS[form]
    case = C.prepared_case(heads, lengths, D=128, dtype=torch.float32,
                           seed=400 + sum(lengths) + mode)
    q, k = case.q.to(qk_dt), case.k.to(qk_dt)
    v = case.v.to(v_dt)
    gate = case.g if mode == 1 else torch.exp(case.g)
    dq, dk = q.to(DEV), k.to(DEV)
    dg, db = gate.to(DEV), case.beta.to(DEV)
    dv, _v_owner = _shifted(v, shift)
    out, _o_owner = _shifted(torch.zeros(v.shape, dtype=v_dt), shift)
    pool = C.to_dev(case.pool, DEV)
    idx = case.indices.to(DEV)
    cu = case.cu_seqlens.to(DEV)
    T, H, D = q.shape[1:]
    lib = ctypes.CDLL(str(abi_library_path()))
    lib.kda_recurrent_launch.argtypes = [ctypes.POINTER(_Args), ctypes.c_void_p]
    lib.kda_recurrent_launch.restype = ctypes.c_int
    a = _Args(q=dq.data_ptr(), k=dk.data_ptr(), v=dv.data_ptr(), gate=dg.data_ptr(),
              beta=db.data_ptr(), state=pool.data_ptr(), state_stride_slot=pool.stride(0),
              state_stride_head=pool.stride(1), num_slots=pool.shape[0],
              state_indices=idx.data_ptr(), cu_seqlens=cu.data_ptr(), out=out.data_ptr(),
              scale=case.scale, num_seqs=len(lengths), num_tokens=T, num_heads=H, head_begin=0,
              head_count=H, head_dim=D, qk_dtype=_KDA_DTYPE[qk_dt], v_dtype=_KDA_DTYPE[v_dt],
              gate_mode=mode, qk_l2norm=0)
    stream = torch.cuda.current_stream().cuda_stream
    assert lib.kda_recurrent_launch(ctypes.byref(a), ctypes.c_void_p(stream)) == 0
    torch.cuda.synchronize()
    ref_pool = C.clone_pool(case.pool)
    ref = R.kda_recurrent(q.float() * case.scale, k, v, case.g, case.beta, state_pool=ref_pool,
                          state_indices=case.indices, cu_seqlens=case.cu_seqlens,
                          out_dtype=torch.float32)
    if v_dt == torch.bfloat16:
        C.assert_out(out.cpu(), ref, C.OUT_TOL, f"{form} output")
    else:
        assert C.max_rel_err(out.cpu(), ref) < 1e-5, f"{form} output"
    C.assert_rel(pool.cpu(), ref_pool, C.STATE_TOL, f"{form} state")
    if shift:
        # the element before the shifted output is never written
        assert _o_owner[0].item() == 0


def test_config5_decode_full_size(gpu_ops):
    """BASELINE config 5's decode half at full size: 1024 sequences x 4 tokens,
    H=16, harsh decay, 2048-slot pool. Sequences are independent, so a seeded
    sample of 12 is checked against the oracle from their own initial slots;
    every slot no sequence indexes must come back bit-identical."""
    n, steps, heads, slots, D = 1024, 4, 16, 2048, 128
    dev = "cuda"
    gen = torch.Generator(device=dev).manual_seed(55)

    def rnd(*shape):
        return torch.randn(*shape, generator=gen, device=dev)

    def l2(x):
        return x / torch.sqrt((x * x).sum(-1, keepdim=True) + 1e-6)

    T = n * steps
    q = l2(rnd(1, T, heads, D)).bfloat16()
    k = l2(rnd(1, T, heads, D)).bfloat16()
    v = rnd(1, T, heads, D).bfloat16()
    g = torch.nn.functional.logsigmoid(rnd(1, T, heads, D) * 2.0 - 2.0)
    beta = torch.sigmoid(rnd(1, T, heads))
    pool = (rnd(slots, heads, D, D) * 0.05).transpose(-1, -2)
    perm = torch.randperm(slots, generator=C.gen(5))[:n]
    idx = perm.to(torch.int32).to(dev)
    cu = C.cu_from_lengths([steps] * n).to(dev)
    sample = torch.randperm(n, generator=C.gen(6))[:12].tolist()
    before = {s: pool[int(perm[s])].cpu().clone() for s in sample}
    untouched = torch.ones(slots, dtype=torch.bool)
    untouched[perm] = False
    untouched[0] = True  # the padding slot is read as zero and never written
    untouched_idx = untouched.nonzero().flatten().to(dev)
    untouched_before = pool.index_select(0, untouched_idx).clone()

    out = gpu_ops.kda_prepared_varlen_recurrent(q, k, v, g, beta, initial_state_source=pool,
                                                initial_state_indices=idx, cu_seqlens=cu,
                                                scale=D ** -0.5)
    torch.cuda.synchronize()
    assert torch.equal(pool.index_select(0, untouched_idx), untouched_before)
    e_o = e_s = 0.0
    for s in sample:
        rows = slice(s * steps, (s + 1) * steps)
        ref_pool = torch.zeros(2, heads, D, D)
        if int(perm[s]) > 0:
            ref_pool[1] = before[s]  # the sequence's own slot as slot 1
        ref = R.kda_recurrent(q[:, rows].float().cpu() * D ** -0.5, k[:, rows].float().cpu(),
                              v[:, rows].float().cpu(), g[:, rows].cpu(), beta[:, rows].cpu(),
                              state_pool=ref_pool,
                              state_indices=torch.tensor([1 if int(perm[s]) > 0 else 0],
                                                         dtype=torch.int32),
                              cu_seqlens=torch.tensor([0, steps], dtype=torch.int32),
                              out_dtype=torch.float32)
        e_o = max(e_o, C.assert_out(out[:, rows].cpu(), ref, C.OUT_TOL, f"sequence {s} output"))
        if int(perm[s]) > 0:
            e_s = max(e_s, C.assert_rel(pool[int(perm[s])].cpu(), ref_pool[1], C.STATE_TOL,
                                        f"sequence {s} state"))
    print(f"config5 decode: output err {e_o:.2e}, state err {e_s:.2e}")


def test_recurrent_no_tokens_tracks_initial_state(gpu_ops):
    """The recurrent op's empty batch: as the chunk op's (prefill mode)."""
    case = C.raw_case(4, (0, 0), indices=[2, 0], slots=6, seed=92, track=([4, 5], [0, 0]))
    out, pool = _run_raw(gpu_ops, case, prefill=True)
    assert out.shape == case.v.shape and out.numel() == 0
    got = pool.cpu()
    assert torch.equal(got[4], case.pool[2]), "tracked slot 4 must hold slot 2's state"
    assert torch.equal(got[5], torch.zeros_like(got[5])), "slot-0 request tracks a zero state"
    for s in (0, 1, 2, 3):
        assert torch.equal(got[s], case.pool[s]), f"slot {s} changed"


@pytest.mark.parametrize("lower_bound,chunk_route", [(-12.0, False), (-10.0, True)])
def test_prefill_route_respects_exponent_envelope(gpu_ops, lower_bound, chunk_route):
    """A long raw-gate prefill runs the chunked kernels only while 8 tokens
    of decay stay inside their exponent envelope (lower_bound >= -10.9); a
    harsher bound keeps the token loop. The gate input is shifted so that
    sigmoid saturates and g sits near 0.98 * lower_bound on every token
    (8 tokens: about 94 nat at -12, beyond the envelope; 78 at -10)."""
    case = C.raw_case(4, (200, 130), indices=[1, 2], slots=4, seed=1212,
                      lower_bound=lower_bound)
    case.a = (case.a.float() + 4.0).bfloat16()
    out, pool = _run_raw(gpu_ops, case, prefill=True)
    ref_pool = C.clone_pool(case.pool)
    ref = _oracle_raw(case, ref_pool)
    C.assert_out(out.cpu(), ref, C.OUT_TOL, f"lower_bound {lower_bound} output")
    C.assert_rel(pool.cpu(), ref_pool, C.STATE_TOL, f"lower_bound {lower_bound} state")
    pool_c = C.to_dev(case.pool, DEV)
    out_c = gpu_ops.kda_varlen_chunk(prefill=True, **case.kwargs(DEV, pool=pool_c))
    torch.cuda.synchronize()
    same = torch.equal(out, out_c) and torch.equal(pool, pool_c)
    assert same == chunk_route, "prefill took the wrong route"
