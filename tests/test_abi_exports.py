"""The C-ABI library loads without a GPU and exports every symbol kda_abi.h declares.

No compute call is made here: only the argument checks that return before any
HIP call (a null argument block, an unsupported head dimension).
"""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "kda_abi.h")
LIB = os.path.join(ROOT, "01-glm53-ascend_amd", "sgl_glm53_ascend_ops", "libkda_amd.so")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(kda_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


@pytest.fixture(scope="module")
def lib():
    assert os.path.exists(LIB), f"{LIB} missing: run python 01-glm53-ascend_amd/kda_build.py"
    return ctypes.CDLL(LIB)


def test_header_declares_the_entry_points():
    names = _declared_functions()
    for expected in ("kda_recurrent_launch", "kda_chunk_launch", "kda_chunk_workspace_bytes",
                     "kda_chunk_launch_noalloc", "kda_status_string", "kda_abi_version"):
        assert expected in names


def test_every_declared_symbol_is_exported(lib):
    missing = [n for n in _declared_functions() if not hasattr(lib, n)]
    assert not missing, f"declared in kda_abi.h but not exported: {missing}"


def test_version_and_status_text(lib):
    lib.kda_abi_version.restype = ctypes.c_int
    assert lib.kda_abi_version() == 2
    lib.kda_status_string.restype = ctypes.c_char_p
    lib.kda_status_string.argtypes = [ctypes.c_int]
    assert lib.kda_status_string(0) == b"ok"
    assert b"unsupported" in lib.kda_status_string(2)


def test_argument_checks_return_before_any_device_call(lib):
    lib.kda_recurrent_launch.restype = ctypes.c_int
    lib.kda_recurrent_launch.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    assert lib.kda_recurrent_launch(None, None) == 1  # KDA_ERR_INVALID_ARGUMENT
    lib.kda_chunk_launch.restype = ctypes.c_int
    lib.kda_chunk_launch.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                     ctypes.c_void_p]
    assert lib.kda_chunk_launch(None, None, 0, None) != 0


class _RecArgs(ctypes.Structure):
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


def test_v_contiguous_pool_only_in_decay_mode(lib):
    """A [K,V]-contiguous pool is the prepared (DECAY) layout: with the RAW or
    LOG gate the launcher returns KDA_ERR_UNSUPPORTED before touching the
    device (the addresses are never dereferenced)."""
    lib.kda_recurrent_launch.restype = ctypes.c_int
    lib.kda_recurrent_launch.argtypes = [ctypes.POINTER(_RecArgs), ctypes.c_void_p]
    base = 1 << 20
    for gate in (0, 1):  # KDA_GATE_RAW, KDA_GATE_LOG
        a = _RecArgs(q=base, k=base, v=base, gate=base, beta=base, A_log=base, dt_bias=base,
                     state=base, state_stride_slot=32 * 128 * 128, state_stride_head=128 * 128,
                     num_slots=4, state_indices=base, cu_seqlens=base, out=base, scale=1.0,
                     num_seqs=1, num_tokens=1, num_heads=32, head_dim=128, gate_mode=gate,
                     state_v_contiguous=1)
        assert lib.kda_recurrent_launch(ctypes.byref(a), None) == 2, gate  # KDA_ERR_UNSUPPORTED


class _ChunkArgs(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("gate", ctypes.c_void_p), ("beta", ctypes.c_void_p),
        ("A_log", ctypes.c_void_p), ("dt_bias", ctypes.c_void_p),
        ("state", ctypes.c_void_p), ("state_stride_slot", ctypes.c_int64),
        ("state_stride_head", ctypes.c_int64), ("num_slots", ctypes.c_int64),
        ("state_indices", ctypes.c_void_p), ("cu_seqlens", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("track_indices", ctypes.c_void_p), ("track_lens", ctypes.c_void_p),
        ("scale", ctypes.c_float), ("lower_bound", ctypes.c_float),
        ("num_seqs", ctypes.c_int32), ("num_tokens", ctypes.c_int32),
        ("num_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("qk_dtype", ctypes.c_int32), ("v_dtype", ctypes.c_int32),
        ("gate_mode", ctypes.c_int32), ("qk_l2norm", ctypes.c_int32),
    ]


def test_chunk_launch_alignment_checks_need_no_device(lib):
    """The chunk launcher rejects misaligned pointers before touching the
    device (the addresses below are never dereferenced)."""
    lib.kda_chunk_launch.restype = ctypes.c_int
    lib.kda_chunk_launch.argtypes = [ctypes.POINTER(_ChunkArgs), ctypes.c_void_p,
                                     ctypes.c_size_t, ctypes.c_void_p]
    base = 1 << 20

    def args(**over):
        a = _ChunkArgs(q=base, k=base, v=base, gate=base, beta=base, state=base,
                       state_stride_slot=32 * 128 * 128, state_stride_head=128 * 128,
                       num_slots=4, state_indices=base, cu_seqlens=base, out=base, scale=1.0,
                       num_seqs=1, num_tokens=64, num_heads=32, head_dim=128, qk_dtype=0,
                       v_dtype=0, gate_mode=1)
        for k_, v_ in over.items():
            setattr(a, k_, v_)
        return a

    for field, bad in (("out", base + 2), ("v", base + 2), ("q", base + 4), ("gate", base + 8),
                       ("state", base + 8)):
        a = args(**{field: bad})
        assert lib.kda_chunk_launch(ctypes.byref(a), None, 0, None) == 1, field
    a = args(state_stride_head=128 * 128 + 2)
    assert lib.kda_chunk_launch(ctypes.byref(a), None, 0, None) == 1
    # aligned arguments pass these checks and stop at the missing workspace
    assert lib.kda_chunk_launch(ctypes.byref(args()), None, 0, None) == 4  # KDA_ERR_WORKSPACE


def test_chunk_workspace_size_formula(lib):
    """kda_chunk_workspace_bytes is a host-only function of (T, N, H, D): the
    chunk-start table (and for several sequences the schedule table that
    orders them for the persistent scan), 55 KiB records, one 16.75 KiB tracking record per
    (sequence, head) and, for a single sequence, one 64 KiB state per head
    carried between scan segments, each 256-byte aligned (the sizes the
    integration notes quote for sizing a reusable workspace). The records: one
    per possible (chunk, head), except for a single sequence of at least 16384
    tokens on at most 16 heads, which runs in S = max(2, ceil(chunks / 256))
    segments (two: 47% and 53% of the chunks; more: W = ceil(chunks / S)
    each) and needs a ring of two of the longest per head.

    A single sequence whose scan leaves most of a 256-CU device idle takes
    the affine form instead: P segments, the most for which its first pass's
    8 (2P - 1) H workgroups fit the CUs with segments of at least 32 chunks
    (of at least 64 when that is two), when the total stays within 1 GiB.
    It keeps one record per chunk and
    adds two fp32 outputs per token-head, and five sets of H 64 KiB states
    ((P - 1) each for the two scans' final states and the segment starts,
    one each for the two scans' tracked states)."""
    lib.kda_chunk_workspace_bytes.restype = ctypes.c_size_t
    lib.kda_chunk_workspace_bytes.argtypes = [ctypes.c_int32] * 4
    rec, track = 56320, 17152
    assert rec == 55 * 1024 and track == 16.75 * 1024
    cus = 256  # no device here: the library assumes MI355X's count

    def classic(T, N, H):
        header = ((N + 1) * 4 + 255) // 256 * 256
        if N > 1:  # the schedule table of several sequences: 2N + 1 int4
            header += ((2 * N + 1) * 16 + 255) // 256 * 256
        chunks = (T + 63) // 64
        slots = chunks + N
        if N == 1 and T >= 16384 and H <= 16:
            segs = max(2, (chunks + 255) // 256)
            first = (chunks * 47 + 50) // 100 if segs == 2 else (chunks + segs - 1) // segs
            slots = 2 * (chunks - first if segs == 2 else first)
        return header + rec * slots * H + track * N * H + (65536 * H if N == 1 else 0)

    def affine(T, H):
        chunks = (T + 63) // 64
        P = 0
        p = 2
        while 8 * H * (2 * p - 1) <= cus and (chunks + p - 1) // p >= 32:
            P = p
            p += 1
        if P < 2 or (P == 2 and (chunks + 1) // 2 < 64):
            return None
        outs = 2 * ((T * H * 512 + 255) // 256 * 256)
        one_pass = 256 + rec * (chunks + 1) * H + track * H + 65536 * H
        total = one_pass + outs + 65536 * H * (3 * (P - 1) + 2)
        return total if total <= 1 << 30 else None

    for T, N, H in [(8192, 1, 32), (33814, 16, 32), (65536, 1, 16), (65536, 1, 17), (16383, 1, 4),
                    (16384, 1, 4), (100000, 1, 8), (1, 1, 1), (0, 3, 2), (4096, 1, 8), (4095, 1, 8),
                    (16384, 1, 1), (400000, 1, 4), (6144, 1, 4), (5952, 1, 4), (6144, 1, 6), (6144, 1, 7),
                    (16384, 1, 8), (8192, 1, 8), (8191, 1, 8), (8065, 1, 7), (8064, 1, 7)]:
        expected = (affine(T, H) if N == 1 else None) or classic(T, N, H)
        assert lib.kda_chunk_workspace_bytes(T, N, H, 128) == expected, (T, N, H)
    # which shapes take the affine form
    assert affine(16384, 4) and affine(6144, 4) and affine(16384, 1) and affine(6144, 6)
    assert affine(16384, 8) and affine(8192, 8) and affine(8065, 7)  # two segments of >= 64 chunks
    assert not affine(65536, 16) and not affine(8192, 32) and not affine(8064, 7)
    assert not affine(4096, 4) and not affine(6144, 7) and not affine(5952, 4)
    assert not affine(400000, 4) and not affine(100000, 8)  # beyond 1 GiB


def test_noalloc_rejects_what_its_scratch_cannot_hold(lib):
    """kda_chunk_launch_noalloc checks the arguments, then the size against its
    static scratch, before any HIP call: a null block is invalid and a batch
    of sequences bigger than KDA_NOALLOC_SCRATCH_BYTES is refused with
    KDA_ERR_TOO_LARGE (the addresses are never dereferenced; a single
    sequence that large runs in segments instead, a GPU test)."""
    lib.kda_chunk_launch_noalloc.restype = ctypes.c_int
    lib.kda_chunk_launch_noalloc.argtypes = [ctypes.POINTER(_ChunkArgs), ctypes.c_void_p]
    lib.kda_chunk_workspace_bytes.restype = ctypes.c_size_t
    lib.kda_chunk_workspace_bytes.argtypes = [ctypes.c_int32] * 4
    lib.kda_status_string.restype = ctypes.c_char_p
    lib.kda_status_string.argtypes = [ctypes.c_int]
    limit = int(re.search(r"KDA_NOALLOC_SCRATCH_BYTES\s+\((\d+)u \* 1024u \* 1024u\)",
                          open(HEADER).read()).group(1)) << 20
    assert lib.kda_chunk_launch_noalloc(None, None) == 1
    base = 1 << 20
    T = 8192
    # two sequences (only a single one can run in segments of the scratch)
    assert lib.kda_chunk_workspace_bytes(T, 2, 32, 128) > limit
    a = _ChunkArgs(q=base, k=base, v=base, gate=base, beta=base, state=base,
                   state_stride_slot=32 * 128 * 128, state_stride_head=128 * 128, num_slots=4,
                   state_indices=base, cu_seqlens=base, out=base, scale=1.0, num_seqs=2,
                   num_tokens=T, num_heads=32, head_dim=128, qk_dtype=0, v_dtype=0, gate_mode=1)
    assert lib.kda_chunk_launch_noalloc(ctypes.byref(a), None) == 5  # KDA_ERR_TOO_LARGE
    assert b"noalloc" in lib.kda_status_string(5)
    a.head_dim = 64
    assert lib.kda_chunk_launch_noalloc(ctypes.byref(a), None) == 2  # unsupported, checked first
