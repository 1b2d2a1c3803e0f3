"""kda_chunk_launch_noalloc against kda_chunk_launch, through the C ABI.

The no-allocation entry point runs the chunk kernels on the library's static
device scratch instead of a caller workspace. On the same arguments its
outputs and pool must equal kda_chunk_launch's bit for bit (same kernels), on
two calls in a row, the second smaller than the first (the scratch keeps the
first call's contents, which must not leak into the second). A single
sequence too long for the scratch runs in segments that fit it (the state
carried between them exactly, so still bit for bit); a batch of sequences too
large for it is refused before anything is written.
"""

import ctypes
import re

import pytest
import torch

from tests import kda_cases as C
from tests.test_abi_exports import HEADER, _ChunkArgs

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _lib():
    from sgl_glm53_ascend_ops._load import abi_library_path

    lib = ctypes.CDLL(str(abi_library_path()))
    lib.kda_chunk_workspace_bytes.restype = ctypes.c_size_t
    lib.kda_chunk_workspace_bytes.argtypes = [ctypes.c_int32] * 4
    lib.kda_chunk_launch.restype = ctypes.c_int
    lib.kda_chunk_launch.argtypes = [ctypes.POINTER(_ChunkArgs), ctypes.c_void_p,
                                     ctypes.c_size_t, ctypes.c_void_p]
    lib.kda_chunk_launch_noalloc.restype = ctypes.c_int
    lib.kda_chunk_launch_noalloc.argtypes = [ctypes.POINTER(_ChunkArgs), ctypes.c_void_p]
    return lib


def _prepare(case):
    """Device copies of a prepared case, a fresh pool, an output buffer and the
    argument block pointing at them."""
    dev = {n: getattr(case, n).to(DEV) for n in ("q", "k", "v", "g", "beta")}
    pool = C.to_dev(case.pool, DEV)
    idx = case.indices.to(DEV)
    cu = case.cu_seqlens.to(DEV)
    out = torch.full_like(dev["v"], 3.0)
    T, H, D = case.q.shape[1:]
    a = _ChunkArgs(q=dev["q"].data_ptr(), k=dev["k"].data_ptr(), v=dev["v"].data_ptr(),
                   gate=dev["g"].data_ptr(), beta=dev["beta"].data_ptr(), state=pool.data_ptr(),
                   state_stride_slot=pool.stride(0), state_stride_head=pool.stride(1),
                   num_slots=pool.shape[0], state_indices=idx.data_ptr(),
                   cu_seqlens=cu.data_ptr(), out=out.data_ptr(), scale=case.scale,
                   num_seqs=len(case.indices), num_tokens=T, num_heads=H, head_dim=D, qk_dtype=0,
                   v_dtype=0, gate_mode=1, qk_l2norm=0)
    keep = (dev, idx, cu)
    return a, out, pool, keep


def test_noalloc_matches_workspace_launch_twice():
    """Two calls in a row, the second with fewer tokens and heads: each equals
    the workspace launcher's result bit for bit."""
    lib = _lib()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    cases = [
        C.prepared_case(6, (300, 64, 129), slots=5, indices=[4, 0, 2], seed=71),
        C.prepared_case(3, (40, 70), slots=4, indices=[1, 3], seed=72),
    ]
    for i, case in enumerate(cases):
        T, H, D = case.q.shape[1:]
        nbytes = lib.kda_chunk_workspace_bytes(T, len(case.indices), H, D)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
        a_ref, out_ref, pool_ref, keep_ref = _prepare(case)
        a_na, out_na, pool_na, keep_na = _prepare(case)
        assert lib.kda_chunk_launch(ctypes.byref(a_ref), ctypes.c_void_p(ws.data_ptr()),
                                    ctypes.c_size_t(nbytes), stream) == 0
        assert lib.kda_chunk_launch_noalloc(ctypes.byref(a_na), stream) == 0
        torch.cuda.synchronize()
        assert torch.equal(out_na, out_ref), f"call {i}: outputs differ"
        assert torch.equal(pool_na, pool_ref), f"call {i}: pools differ"
        assert torch.isfinite(out_na.float()).all()


def test_noalloc_long_sequence_runs_in_segments():
    """One sequence whose records exceed the scratch (8192 tokens on 32 heads,
    ~370 MB in one pass) runs in segments of the scratch's size: outputs,
    the updated slot and a prefix tracked in the middle of a segment equal
    the one-pass workspace launch bit for bit."""
    lib = _lib()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    case = C.prepared_case(32, (8192,), slots=4, indices=[2], seed=74)
    T, H, D = case.q.shape[1:]
    nbytes = lib.kda_chunk_workspace_bytes(T, 1, H, D)
    assert nbytes > (64 << 20)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    a_ref, out_ref, pool_ref, keep_ref = _prepare(case)
    a_na, out_na, pool_na, keep_na = _prepare(case)
    tr = torch.tensor([3], dtype=torch.int32, device=DEV)
    tl = torch.tensor([4100], dtype=torch.int32, device=DEV)
    for a in (a_ref, a_na):
        a.track_indices = tr.data_ptr()
        a.track_lens = tl.data_ptr()
    assert lib.kda_chunk_launch(ctypes.byref(a_ref), ctypes.c_void_p(ws.data_ptr()),
                                ctypes.c_size_t(nbytes), stream) == 0
    assert lib.kda_chunk_launch_noalloc(ctypes.byref(a_na), stream) == 0
    torch.cuda.synchronize()
    assert torch.equal(out_na, out_ref), "outputs differ"
    assert torch.equal(pool_na, pool_ref), "pools differ"
    assert not torch.equal(pool_na[3], C.to_dev(case.pool, DEV)[3]), "the tracked slot was not written"


def test_noalloc_refuses_oversized_call_untouched():
    """A batch of sequences beyond the static scratch (only a single sequence
    can run in segments) returns KDA_ERR_TOO_LARGE and writes nothing."""
    lib = _lib()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    case = C.prepared_case(32, (2048, 2048), slots=3, indices=[1, 2], seed=73)
    T, H, D = case.q.shape[1:]
    limit = int(re.search(r"KDA_NOALLOC_SCRATCH_BYTES\s+\((\d+)u \* 1024u \* 1024u\)",
                          open(HEADER).read()).group(1)) << 20
    assert lib.kda_chunk_workspace_bytes(T, 2, H, D) > limit
    a, out, pool, keep = _prepare(case)
    before = pool.clone()
    assert lib.kda_chunk_launch_noalloc(ctypes.byref(a), stream) == 5
    torch.cuda.synchronize()
    assert torch.all(out == 3.0)
    assert torch.equal(pool, before)
