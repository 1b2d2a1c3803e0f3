"""The chunked prefill's affine form (a long single sequence on few heads).

When the scan of one sequence would leave most of the device idle (8 H
workgroups of 256 CUs), the launcher splits it into P segments: segment 0
is scanned from the pool as usual, every later segment twice from its
start (from zero with the real v, and from the identity with v = 0), then
a serial pass combines the segment transitions into the true states
S_{s+1} = Phi_s S_s + Z_s and a parallel pass adds O_t S_s to the later
outputs -- the linearity of the recurrence in (state, v), the same
mathematics that shards a long context across devices.

Checked against the CPU oracle (oracle.kda_ref.kda_chunk) at the tolerance
contract, with the reference chunk suite's invariants: untouched slots
byte-identical, the padding slot 0, zeros outside the sequence, and a
tracked prefix ending in segment 0, exactly on a segment boundary, inside a
later segment and at the sequence's end (tests/ops/test_kda_chunk.py:
203-214 for the positions; the suffix-resume check for these shapes is in
test_prefix_resume_gpu.py).
"""

import ctypes
import dataclasses

import pytest
import torch

from oracle import kda_ref as R
from tests import kda_cases as C

pytestmark = pytest.mark.gpu

DEV = "cuda"
SLOTS = 5

# (label, heads, token bounds in a buffer of T tokens, T, slot, track (slot,
# length), lower_bound). Segments on a 256-CU device: H=1 16384 tokens -> 8 x
# 32 chunks; H=2 8192 -> 4 x 32; H=4 6144 -> 3 x 32; H=5 6144 -> 3 x 32;
# H=6 6208 -> 3 x 33 chunks; H=7 and H=8 8192 -> 2 x 64 (two segments need
# at least 64 chunks each).
# At lower_bound -5 (the raw gates' decay is then about -2.5 per token) a
# segment's start barely reaches its outputs; at -2e-4 (about -1e-4 per
# token, 0.2 nat over a 2048-token segment) every later output and the final
# state depend on the combined transitions.
CASES = [
    ("H1 whole", 1, (0, 16384), 16384, 1, None, -5.0),
    ("H2 ragged, track in segment 2", 2, (37, 8192 - 5), 8192, 2, (3, 5000), -5.0),
    ("H4 track on the segment boundary", 4, (0, 6144), 6144, 1, (3, 2048), -5.0),
    ("H4 zero slot, track one past the boundary", 4, (0, 6144), 6144, 0, (3, 2049), -5.0),
    ("H6 partial last chunk, track at the end", 6, (0, 6208 - 20), 6208, 1, (3, 6188), -5.0),
    ("H2 track at 0", 2, (0, 8192), 8192, 4, (3, 0), -5.0),
    ("H1 short sequence in a long batch", 1, (100, 1500), 16384, 2, (3, 700), -5.0),
    ("weak decay H1 eight segments, track in segment 5", 1, (0, 16384), 16384, 1, (3, 11000), -2e-4),
    ("weak decay H4 ragged, track on the boundary", 4, (11, 6144 - 30), 6144, 2, (3, 2048), -2e-4),
    ("weak decay H2 zero slot, track inside segment 3", 2, (0, 8192), 8192, 0, (3, 7001), -2e-4),
    ("weak decay H5", 5, (0, 6144), 6144, 1, (3, 4100), -2e-4),
    ("H8 two segments, track in segment 1", 8, (0, 8192), 8192, 1, (3, 5000), -5.0),
    ("weak decay H8 two segments, track on the boundary", 8, (0, 8192), 8192, 2, (3, 4096), -2e-4),
    ("weak decay H7 ragged two segments", 7, (13, 8192 - 9), 8192, 1, (3, 100), -2e-4),
]


def _oracle(case, pool_cpu):
    qn, kn, g, beta = R.kda_prepare(case.A_log, case.a, case.dt_bias, case.q, case.k, case.b,
                                    case.lower_bound, case.scale)
    return R.kda_chunk(qn, kn, case.v, g, beta, state_pool=pool_cpu, state_indices=case.indices,
                       cu_seqlens=case.cu_seqlens, track_state_indices=case.track_indices,
                       track_state_lens=case.track_lens, out_dtype=torch.float32)


@pytest.mark.parametrize("label,heads,bounds,T,slot,track,lower_bound", CASES,
                         ids=[c[0].replace(" ", "-").replace(",", "") for c in CASES])
def test_affine_form_matches_oracle(gpu_ops, label, heads, bounds, T, slot, track, lower_bound):
    case = C.raw_case(heads, (T,), indices=[slot], slots=SLOTS, seed=6000 + len(label),
                      lower_bound=lower_bound,
                      track=None if track is None else ([track[0]], [track[1]]))
    case = dataclasses.replace(case, cu_seqlens=torch.tensor(bounds, dtype=torch.int32))
    pool = C.to_dev(case.pool, DEV)
    out = gpu_ops.kda_varlen_chunk(prefill=True, **case.kwargs(DEV, pool=pool))
    torch.cuda.synchronize()
    ref_pool = C.clone_pool(case.pool)
    ref = _oracle(case, ref_pool)
    e_o = C.assert_out(out.cpu(), ref, C.OUT_TOL, f"{label} output")
    e_s = C.assert_rel(pool.cpu(), ref_pool, C.STATE_TOL, f"{label} pool")
    print(f"{label}: output err {e_o:.2e}, state err {e_s:.2e}")
    got = out.cpu()
    assert torch.all(got[:, :bounds[0]] == 0) and torch.all(got[:, bounds[1]:] == 0)
    touched = {s for s in (slot, track[0] if track is not None else 0) if s > 0}
    other = [s for s in range(SLOTS) if s not in touched]
    assert torch.equal(pool.cpu()[other], case.pool[other]), "an unindexed slot was written"
    if track is not None:
        assert not torch.equal(pool.cpu()[track[0]], case.pool[track[0]]), "tracked slot unwritten"


def test_affine_form_is_taken_and_agrees_with_one_pass(gpu_ops):
    """The recommended workspace runs the affine form, a workspace of the
    one-pass size the classic scan: different arithmetic (so not bitwise
    equal), the same results within the contract."""
    from sgl_glm53_ascend_ops._load import abi_library_path
    from tests.test_abi_exports import _ChunkArgs

    lib = ctypes.CDLL(str(abi_library_path()))
    lib.kda_chunk_workspace_bytes.restype = ctypes.c_size_t
    lib.kda_chunk_workspace_bytes.argtypes = [ctypes.c_int32] * 4
    lib.kda_chunk_launch.restype = ctypes.c_int
    lib.kda_chunk_launch.argtypes = [ctypes.POINTER(_ChunkArgs), ctypes.c_void_p,
                                     ctypes.c_size_t, ctypes.c_void_p]
    case = C.prepared_case(4, (16384,), slots=3, indices=[1], seed=96)
    T, H, D = case.q.shape[1:]
    dev = {n: getattr(case, n).to(DEV) for n in ("q", "k", "v", "g", "beta")}
    idx = case.indices.to(DEV)
    cu = case.cu_seqlens.to(DEV)
    full = lib.kda_chunk_workspace_bytes(T, 1, H, D)
    one_pass = 256 + (56320 * ((T + 63) // 64 + 1) + 17152 + 65536) * H
    assert full > one_pass
    results = []
    for nbytes in (full, one_pass):
        pool = C.to_dev(case.pool, DEV)
        out = torch.empty_like(dev["v"])
        ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
        a = _ChunkArgs(q=dev["q"].data_ptr(), k=dev["k"].data_ptr(), v=dev["v"].data_ptr(),
                       gate=dev["g"].data_ptr(), beta=dev["beta"].data_ptr(),
                       state=pool.data_ptr(), state_stride_slot=pool.stride(0),
                       state_stride_head=pool.stride(1), num_slots=pool.shape[0],
                       state_indices=idx.data_ptr(), cu_seqlens=cu.data_ptr(), out=out.data_ptr(),
                       scale=case.scale, num_seqs=1, num_tokens=T, num_heads=H, head_dim=D,
                       qk_dtype=0, v_dtype=0, gate_mode=1, qk_l2norm=0)
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        assert lib.kda_chunk_launch(ctypes.byref(a), ctypes.c_void_p(ws.data_ptr()),
                                    ctypes.c_size_t(nbytes), stream) == 0
        torch.cuda.synchronize()
        results.append((out.cpu(), pool.cpu()))
    (o_aff, p_aff), (o_one, p_one) = results
    assert not torch.equal(o_aff, o_one), "the recommended workspace did not take the affine form"
    e_o = C.max_rel_err(o_aff, o_one.float())
    e_s = C.assert_rel(p_aff, p_one, C.STATE_TOL, "final state, affine vs one pass")
    assert e_o <= C.OUT_TOL + 2.0 ** -8, f"outputs, affine vs one pass: {e_o:.2e}"
    print(f"affine vs one pass: output {e_o:.2e}, state {e_s:.2e}")
