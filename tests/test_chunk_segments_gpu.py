"""The chunk launcher's segmented forms, through the C ABI.

A single sequence can run in segments whose records share a ring of slots:
pipelined (each segment's prepare kernel on the library's second stream
under the previous segment's scan; the default for a long sequence on few
heads) or one after another (any single sequence, when the caller's
workspace is smaller than kda_chunk_workspace_bytes). Segment boundaries only
move where the fp32 state is stored and reloaded, so every form must equal
the one-pass result bit for bit; the one-pass path itself is checked against
the oracle by the chunk parity tests.
"""

import ctypes

import pytest
import torch

from tests import kda_cases as C
from tests.test_zz_no_alloc import _lib, _prepare

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _rec_bytes(lib):
    """Bytes per (chunk, head) record: what one more chunk of a two-sequence
    batch adds to kda_chunk_workspace_bytes on one head."""
    return lib.kda_chunk_workspace_bytes(128, 2, 1, 128) - lib.kda_chunk_workspace_bytes(64, 2, 1, 128)


def _base_bytes(H):
    """A single sequence's workspace without its records: the chunk-start
    table, one tracking record and one carried state per head (the sizes
    test_abi_exports pins). A workspace of this plus W records per head runs
    windows of W chunks; with every chunk's record it runs in one pass (the
    affine form, when the shape takes it, needs more than either)."""
    return 256 + 17152 * H + 65536 * H


def _launch(lib, case, nbytes, track=None):
    a, out, pool, keep = _prepare(case)
    if track is not None:
        tr = torch.tensor([track[0]], dtype=torch.int32, device=DEV)
        tl = torch.tensor([track[1]], dtype=torch.int32, device=DEV)
        a.track_indices = tr.data_ptr()
        a.track_lens = tl.data_ptr()
        keep = keep + (tr, tl)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.kda_chunk_launch(ctypes.byref(a), ctypes.c_void_p(ws.data_ptr()),
                              ctypes.c_size_t(nbytes), stream)
    torch.cuda.synchronize()
    del keep
    return rc, out, pool


@pytest.mark.parametrize("label,heads,lens,bounds,window,track", [
    ("five-chunk segments", 8, (4096,), None, 5, None),
    ("ragged, track across", 8, (4096,), (37, 4096 - 42), 7, (3, 1500)),
    ("one-chunk segments", 8, (1024,), None, 1, (3, 640)),
    ("window of the whole", 8, (1024,), None, 16, None),
    # more than 32 heads: 32-column scan groups on a 256-CU part
    ("32-column groups", 40, (4096,), (1, 4096 - 5), 30, (3, 1101)),
    ("32-column groups, one chunk", 40, (64,), None, 1, None),
])
def test_small_workspace_runs_segments(label, heads, lens, bounds, window, track):
    """A workspace below kda_chunk_workspace_bytes but holding `window` records
    per head runs the sequence in segments of that many chunks, one after
    another, bit for bit equal to the one-pass launch."""
    import dataclasses

    lib = _lib()
    case = C.prepared_case(heads, lens, slots=4, indices=[2], seed=91 + len(label))
    if bounds is not None:
        case = dataclasses.replace(case, cu_seqlens=torch.tensor(bounds, dtype=torch.int32))
    T, H, D = case.q.shape[1:]
    REC = _rec_bytes(lib)
    base = _base_bytes(H)
    full = base + REC * ((T + 63) // 64 + 1) * H  # the one-pass form
    assert full <= lib.kda_chunk_workspace_bytes(T, 1, H, D)
    small = base + REC * window * H
    assert small < full
    rc_ref, out_ref, pool_ref = _launch(lib, case, full, track)
    rc_seg, out_seg, pool_seg = _launch(lib, case, small, track)
    assert rc_ref == 0 and rc_seg == 0
    assert torch.equal(out_seg, out_ref), f"{label}: outputs differ"
    assert torch.equal(pool_seg, pool_ref), f"{label}: pools differ"
    # one byte short of a single record per head cannot hold a segment
    rc, out, pool = _launch(lib, case, base + REC * H - 1)
    assert rc == 4  # KDA_ERR_WORKSPACE


def test_pipelined_segments_match_sequential_segments():
    """A 16384-token sequence on 4 heads takes the pipelined segments with a
    workspace of their ring (two segments, 120 and 136 chunks; less than the
    affine form's, which kda_chunk_workspace_bytes recommends for this
    shape); the same call with a workspace for 13-chunk segments run one
    after another gives the same bits."""
    lib = _lib()
    case = C.prepared_case(4, (16384,), slots=3, indices=[1], seed=95)
    T, H, D = case.q.shape[1:]
    REC = _rec_bytes(lib)
    base = _base_bytes(H)
    ring = base + REC * 2 * 136 * H
    assert ring < lib.kda_chunk_workspace_bytes(T, 1, H, D)
    rc_a, out_a, pool_a = _launch(lib, case, ring, (2, 9000))
    rc_b, out_b, pool_b = _launch(lib, case, base + REC * 13 * H, (2, 9000))
    assert rc_a == 0 and rc_b == 0
    assert torch.equal(out_a, out_b) and torch.equal(pool_a, pool_b)
    assert torch.isfinite(out_a.float()).all()
