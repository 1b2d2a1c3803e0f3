"""HIP-graph capture and replay with metadata mutated behind the captured pointers.

Mirrors the reference's graph check (tests/integration/
test_glm53_kda_prefix_ascendc.py:185-293): one op call is
captured, then replayed eight times. Before every replay the slot indices
(including the padding slot 0), the packed sequence boundaries and the
tracking slots/lengths are rewritten in place, the inputs get fresh values and
the pool is reset; the same call then runs eagerly on a second pool, and the
replay must match it bitwise -- output, pool, and per-step checkpoints.
Between replays the test does its own eager work and synchronizes, so a graph
node that only works on its first replay would show.
"""

import pytest
import torch

from tests import kda_cases as C

pytestmark = pytest.mark.gpu

DEV = "cuda"
H = 4
D = 128


def _capture(fn):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fn()
    torch.cuda.synchronize()
    return graph, out


class _Inputs:
    """Static device buffers for q, k, v, a, b (refreshed in place) and the gate constants."""

    def __init__(self, T, seed, heads=H):
        case = C.raw_case(heads, (T,), D=D, seed=seed)
        self.seed = seed
        self.const = dict(A_log=case.A_log.to(DEV), dt_bias=case.dt_bias.to(DEV),
                          lower_bound=case.lower_bound, scale=case.scale)
        self.t = {n: getattr(case, n).to(DEV) for n in ("q", "k", "v", "a", "b")}

    def refresh(self, replay):
        g = C.gen(self.seed * 100 + replay)
        for n, t in self.t.items():
            t.copy_((torch.randn(t.shape, generator=g) * 0.2).to(t.dtype))


def _offsets(lengths):
    return C.cu_from_lengths(lengths).to(DEV)


@pytest.mark.parametrize("steps", [1, 2])
def test_decode_graph_replay(gpu_ops, steps):
    batch = 6
    size = 2 * batch + 3
    initial = C.to_dev(C.native_pool(size, H, D, seed=40 + steps), DEV)
    work, reference = C.clone_pool(initial), C.clone_pool(initial)
    inp = _Inputs(batch * steps, seed=50 + steps)
    slots = torch.arange(1, batch + 1, dtype=torch.int32, device=DEV)
    starts = _offsets([steps] * batch)
    mid = eager_mid = None
    if steps > 1:
        mid = torch.empty(batch, steps, H, D, D, device=DEV).transpose(-1, -2)
        eager_mid = torch.empty(batch, steps, H, D, D, device=DEV).transpose(-1, -2)

    def run(pool, middle):
        return gpu_ops.kda_varlen_recurrent(
            **inp.const, **inp.t, initial_state_source=pool, initial_state_indices=slots,
            cu_seqlens=starts, intermediate_state=middle, prefill=False)

    graph, captured = _capture(lambda: run(work, mid))
    for replay in range(8):
        active = [(row + replay) % (batch + 1) for row in range(batch)]
        slots.copy_(torch.tensor(active, dtype=torch.int32))
        inp.refresh(replay)
        work.copy_(initial)
        reference.copy_(initial)
        if mid is not None:
            mid.fill_(17.0)
            eager_mid.fill_(17.0)
        expected = run(reference, eager_mid)
        torch.cuda.synchronize()
        expected, ref_pool = expected.cpu(), reference.cpu()
        ref_mid = eager_mid.cpu() if eager_mid is not None else None
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured.cpu(), expected), f"replay {replay}: output"
        assert torch.equal(work.cpu(), ref_pool), f"replay {replay}: pool"
        if mid is not None:
            assert torch.equal(mid.cpu(), ref_mid), f"replay {replay}: checkpoints"
            assert torch.equal(work.cpu(), initial.cpu()), "checkpointed decode wrote the pool"
        assert expected.float().abs().sum() > 0


@pytest.mark.parametrize("op", ["kda_varlen_recurrent", "kda_varlen_chunk"])
def test_prefill_tracking_graph_replay(gpu_ops, op):
    lengths = [129, 65, 63]
    batch = len(lengths)
    size = 2 * batch + 4
    initial = C.to_dev(C.native_pool(size, H, D, seed=60), DEV)
    work, reference = C.clone_pool(initial), C.clone_pool(initial)
    inp = _Inputs(sum(lengths), seed=61 if op == "kda_varlen_chunk" else 62)
    slots = torch.arange(1, batch + 1, dtype=torch.int32, device=DEV)
    dests = slots + batch + 1
    cuts = torch.tensor([min(n, 64) for n in lengths], dtype=torch.int32, device=DEV)
    starts = _offsets(lengths)
    fn = getattr(gpu_ops, op)

    def run(pool):
        return fn(**inp.const, **inp.t, initial_state_source=pool, initial_state_indices=slots,
                  cu_seqlens=starts, prefill=True, track_state_indices=dests,
                  track_state_lens=cuts)

    graph, captured = _capture(lambda: run(work))
    for replay in range(8):
        active = [(row + replay) % (batch + 1) for row in range(batch)]
        dest = [batch + 2 + ((row + replay) % batch) for row in range(batch)]
        if replay % 3 == 0:
            dest[-1] = 0
        lens = lengths if replay % 2 == 0 else [65, 129, 63]
        bounds = [0, 32, 63, 64, 100, 129]
        cut = [min(lens[row], bounds[(row + replay) % len(bounds)]) if dest[row] else -12345
               for row in range(batch)]
        slots.copy_(torch.tensor(active, dtype=torch.int32))
        dests.copy_(torch.tensor(dest, dtype=torch.int32))
        starts.copy_(C.cu_from_lengths(lens))
        cuts.copy_(torch.tensor(cut, dtype=torch.int32))
        inp.refresh(replay)
        work.copy_(initial)
        reference.copy_(initial)
        expected = run(reference)
        torch.cuda.synchronize()
        expected, ref_pool = expected.cpu(), reference.cpu()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured.cpu(), expected), f"replay {replay}: output"
        assert torch.equal(work.cpu(), ref_pool), f"replay {replay}: pool"
        assert expected.float().abs().sum() > 0


@pytest.mark.parametrize("heads", [4, 12], ids=["affine", "pipelined"])
def test_chunk_two_segment_graph_replay(gpu_ops, heads):
    """One long sequence on few heads: at 4 heads the chunk op's affine form
    (four segments scanned at once, then combined), at 12 its pipelined
    segments (a second stream forked and joined inside the op). Captured once
    after eager calls, replayed with the slot (padding slot 0 included), the
    sequence bounds and the tracked length moved across segment boundaries."""
    T = 16384
    initial = C.to_dev(C.native_pool(6, heads, D, seed=70), DEV)
    work, reference = C.clone_pool(initial), C.clone_pool(initial)
    inp = _Inputs(T, seed=71, heads=heads)
    slots = torch.tensor([1], dtype=torch.int32, device=DEV)
    dests = torch.tensor([4], dtype=torch.int32, device=DEV)
    cuts = torch.tensor([100], dtype=torch.int32, device=DEV)
    starts = _offsets([T])

    def run(pool):
        return gpu_ops.kda_varlen_chunk(**inp.const, **inp.t, initial_state_source=pool,
                                        initial_state_indices=slots, cu_seqlens=starts,
                                        prefill=True, track_state_indices=dests,
                                        track_state_lens=cuts)

    graph, captured = _capture(lambda: run(work))
    bounds = [(0, T), (37, T - 42), (0, T), (5, 4000)]
    for replay in range(8):
        lo, hi = bounds[replay % len(bounds)]
        slots.copy_(torch.tensor([replay % 3], dtype=torch.int32))
        cuts.copy_(torch.tensor([[0, 100, 7680, 7681, 12000, hi - lo, 64, 129][replay]],
                                dtype=torch.int32))
        starts.copy_(torch.tensor([lo, hi], dtype=torch.int32))
        inp.refresh(replay)
        work.copy_(initial)
        reference.copy_(initial)
        expected = run(reference)
        torch.cuda.synchronize()
        expected, ref_pool = expected.cpu(), reference.cpu()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured.cpu(), expected), f"replay {replay}: output"
        assert torch.equal(work.cpu(), ref_pool), f"replay {replay}: pool"
        assert expected.float().abs().sum() > 0


_CAPTURE_FIRST = r"""
import os, sys
sys.path[:0] = [os.getcwd(), os.path.join(os.getcwd(), "01-glm53-ascend_amd")]
import torch
import sgl_glm53_ascend_ops  # noqa: F401
from tests import kda_cases as C

ops = torch.ops.sgl_glm53_ascend
case = C.raw_case(1, (16384,), D=128, slots=3, indices=[1], seed=4242)
pool = C.to_dev(case.pool, "cuda")
init = pool.clone()
kw = case.kwargs("cuda", pool=pool)
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):  # the first long call of the process
    out = ops.kda_varlen_chunk(prefill=True, **kw)
torch.cuda.synchronize()
pool2 = C.to_dev(case.pool, "cuda")
ref = ops.kda_varlen_chunk(prefill=True, **case.kwargs("cuda", pool=pool2))
torch.cuda.synchronize()
for replay in range(3):
    pool.copy_(init)
    junk = torch.randn(1 << 20, device="cuda").sum()  # eager work between replays
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, ref), f"replay {replay}: output differs"
    assert torch.equal(pool, pool2), f"replay {replay}: pool differs"
print("CAPTURE-OK")
"""


def test_long_prefill_captured_before_any_eager_call(gpu_ops):
    """A single long sequence eligible for the pipelined segments, captured
    into a graph as the process's first such call: the library has no side
    stream yet and must not create one during a capture, so the captured call
    runs the same segments one after another on the capturing stream. Runs in
    a fresh interpreter (this process has made long calls already); every
    replay equals the eager result bitwise."""
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _CAPTURE_FIRST], cwd=root, capture_output=True,
                       text=True, timeout=240)
    assert r.returncode == 0 and "CAPTURE-OK" in r.stdout, r.stdout[-2000:] + r.stderr[-2000:]
