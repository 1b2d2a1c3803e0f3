"""Benchmark of the KDA hot path on one MI355X: decode tok/s + state HBM GB/s, prefill tok/s.

Workload (BASELINE.json ``configs[1]``, the configuration the metric is quoted
on): varlen recurrent decode, one token for each of 256 sequences, H=32,
K=V=128, bf16 q/k/v (q, k L2-normalized), fp32 per-channel log decay
``g = logsigmoid(randn)`` and ``beta = sigmoid(randn)``, fp32 state pool of 512
slots (``randn*0.05``, K-contiguous), ``state_indices`` a seeded random
permutation of 256 of the slots, updated in place. One *step* is one call of
the decode operator over the whole batch (every step advances all 256
sequences by one token in place). ``value`` = tokens/s = 256 / step time.

Also reported in the same JSON line:

* ``prefill`` -- the chunked prefill of ``configs[2]`` (T=8192, one sequence,
  H=32, K=V=128, chunk 64);
* ``roofline`` -- the decode kernel: algorithmic bytes / HIP-event time per
  call on the launch stream; ``traffic`` is the HBM bytes per launch from the
  committed rocprofv3 counter summary, used only while the kernel source it was
  measured on is unchanged (``source_sha256`` in the summary); ``copy_gbs`` is
  what a plain 512 MiB device-to-device copy reaches on the same GPU (bytes read
  plus written per time), a reference for the achievable streaming rate;
* ``more_configs`` -- configs 4 and 5 (prefill), a serving-shaped batch of 64
  prompts x 256 tokens on 32 heads (prefill), and config 5's 4-token decode;
* ``latency_rows`` -- the reference bench's deployed shapes
  (bench/kda_recurrent/bench_kda_varlen_recurrent.py:81-114,534-551): decode
  H16/32/64 x B1/32/128, the five checkpointed verify shapes, recurrent
  prefill H4/H8, each validated against the oracle and timed;
* ``cpu_baseline`` -- this repository's torch oracle of the reference CPU path
  on the host cores over a bounded sample; the same leg is the checker that
  validates every timed workload before it is timed (``validated``). A failed
  validation makes the run exit non-zero.

Every timed workload first runs a settle phase (batches of 10 calls until two
successive batch means agree within 1%, at least ``--settle`` calls) so the
figures are steady-state whatever ``--warmup`` the caller passes; the call
count is reported as ``settle_calls``.

Usage: ``python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-more]``.
Profiling aids: ``--summarize-trace CSV``, ``--summarize-counters CSV``,
``--copy-calibration MIB``.
"""

from __future__ import annotations

import argparse
import csv
import hashlib
import json
import os
import re
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "01-glm53-ascend_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import torch  # noqa: E402

HBM_PEAK_GBS = 8000.0  # MI355X published HBM3E bandwidth
BF16_PEAK_TFLOPS = 2500.0  # MI355X published dense bf16 MFMA
CSRC = os.path.join(ROOT, "01-glm53-ascend_amd", "csrc")
PROFILES = os.path.join(ROOT, "profiles")

# Config 2 (decode) shape.
DEC_N, DEC_H, DEC_D, DEC_SLOTS = 256, 32, 128, 512
# Algorithmic bytes per token-head: state read + write (2*D*D*4), q, k, v
# (3*D*2), g (D*4), beta (4), o (D*2).
BYTES_PER_TOKEN_HEAD = 2 * DEC_D * DEC_D * 4 + 3 * DEC_D * 2 + DEC_D * 4 + 4 + DEC_D * 2
# + cu_seqlens (257 x 4) + indices (256 x 4): 2052 B of metadata.
DEC_BYTES = DEC_N * DEC_H * BYTES_PER_TOKEN_HEAD + (DEC_N + 1) * 4 + DEC_N * 4

# Config 3 (prefill) shape.
PF_T, PF_H, PF_D, PF_BT = 8192, 32, 128, 64
# Dense-tile FLOPs per token-head: 2*(5*BT*D + 3*D*D).
FLOP_PER_TOKEN_HEAD = 2 * (5 * PF_BT * PF_D + 3 * PF_D * PF_D)
PF_FLOP = PF_T * PF_H * FLOP_PER_TOKEN_HEAD
# q,k,v bf16 in, g fp32, beta fp32, o bf16 out, per token row.
BYTES_PER_TOKEN_ROW = 3 * 128 * 2 + 128 * 4 + 4 + 128 * 2
# Algorithmic bytes: the token rows plus the final state written (zero initial state).
PF_BYTES = PF_T * PF_H * BYTES_PER_TOKEN_ROW + PF_H * PF_D * PF_D * 4

# Reference 910B4 latencies (ms) at the same shapes, for context only:
# bench/kda_recurrent/DISCARDED-cann-recurrent-kda.md:22-30 (decode, eager call)
# and kda_varlen_recurrent_decode_h32.cpp:760-765 (verify R2, kernel only).
REF_910B4_MS = {
    "decode H16 B1": 0.121, "decode H16 B32": 0.133, "decode H16 B128": 0.303,
    "decode H32 B1": 0.118, "decode H32 B32": 0.146, "decode H32 B128": 0.633,
    "decode H64 B1": 0.140, "decode H64 B32": 0.301, "decode H64 B128": 1.225,
    "verify 256K DP4TP2 R2": 0.03698,
    # bench/kda_chunk/README.md:37-39 (kda_varlen_chunk, H8 C64, one sequence)
    "chunk H8 T1k": 2.03, "chunk H8 T2k": 3.83, "chunk H8 T4k": 7.36,
}


def _log(msg):
    print(msg, file=sys.stderr, flush=True)


# ---------------------------------------------------------------------------
# timing
# ---------------------------------------------------------------------------


def _batch_us(step, n):
    """Mean HIP-event time per call over ``n`` back-to-back calls on the
    current stream (the stream the operators launch on)."""
    stream = torch.cuda.current_stream()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for _ in range(n):
        step()
    ev1.record(stream)
    ev1.synchronize()
    return ev0.elapsed_time(ev1) * 1e3 / n


def settle(step, min_calls, max_calls=2000, batch=10, rel=0.01):
    """Run ``step`` until two successive 10-call batch means agree within
    ``rel`` and at least ``min_calls`` calls ran (a fresh box's clocks and
    translation caches take a few hundred microseconds of work to settle).
    Returns the number of calls made."""
    calls = 0
    prev = None
    while calls < max_calls:
        cur = _batch_us(step, batch)
        calls += batch
        if prev is not None and calls >= min_calls and abs(cur - prev) <= rel * prev:
            break
        prev = cur
    return calls


def timed(step, steps, warmup, min_settle, before_timed=None):
    """Settle, ``warmup`` untimed calls, ``before_timed()`` (untimed), then
    ``steps`` timed calls bracketed by device synchronization. Returns wall ms
    per call, HIP-event µs per call on the launch stream, and the settle call
    count."""
    settle_calls = settle(step, min_settle)
    for _ in range(warmup):
        step()
    if before_timed is not None:
        before_timed()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(steps):
        step()
    ev1.record(stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    return dict(ms_per_step=(t1 - t0) * 1e3 / steps,
                event_us_per_call=ev0.elapsed_time(ev1) * 1e3 / steps,
                settle_calls=settle_calls)


def graph_us(step, calls, replays=10):
    """Per-call time of ``calls`` back-to-back calls captured in one HIP graph
    and replayed ``replays`` times (HIP events on the replaying stream): the
    device-side time of a call without the host's launch path, which sets
    eager per-call times at small batch."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(calls):
            step()
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for _ in range(replays):
        graph.replay()
    ev1.record(stream)
    ev1.synchronize()
    us = ev0.elapsed_time(ev1) * 1e3 / (replays * calls)
    del graph
    return us


# ---------------------------------------------------------------------------
# committed profile figures
# ---------------------------------------------------------------------------


DECODE_SOURCES = ("kda_recurrent.hip", "kda_device.h")
PREFILL_SOURCES = ("kda_chunk.hip", "kda_device.h")


def source_sha256(names):
    """sha256 over the given kernel sources, in order (the key the profile
    summaries record, so a figure measured on other kernels is never
    reported)."""
    h = hashlib.sha256()
    for n in names:
        with open(os.path.join(CSRC, n), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def profile_figures(name, key="bench-figures"):
    """The ``<key>: {...}`` JSON line of ``profiles/<name>`` or None."""
    path = os.path.join(PROFILES, name)
    try:
        with open(path) as f:
            for line in f:
                m = re.match(r"\s*" + re.escape(key) + r":\s*(\{.*\})\s*$", line)
                if m:
                    return json.loads(m.group(1))
    except OSError:
        return None
    return None


def traffic_from_profile(name, source, key="bench-figures"):
    """HBM bytes per launch from a counter summary: FETCH_SIZE and WRITE_SIZE
    KiB per dispatch, each scaled by what the same counter reads for a device
    copy of known size. None (and the reason) when the summary is missing or
    was measured on other kernel sources."""
    fig = profile_figures(name, key)
    if fig is None:
        return None, f"no {key} line in profiles/{name}"
    if fig.get("source_sha256") != source:
        return None, (f"profiles/{name} was measured on kernel sources "
                      f"{fig.get('source_sha256')}, these are {source}")
    fs = fig["copy_bytes_kib"] / fig["copy_fetch_kib"]
    ws = fig["copy_bytes_kib"] / fig["copy_write_kib"]
    return (fig["fetch_kib"] * fs + fig["write_kib"] * ws) * 1024, f"profiles/{name}"


# ---------------------------------------------------------------------------
# workloads
# ---------------------------------------------------------------------------


def decode_case():
    """BASELINE config 2 on the CPU (seeded), the permutation drawn with seed 2."""
    from tests import kda_cases as C

    perm = torch.randperm(DEC_SLOTS, generator=C.gen(2))[:DEC_N].tolist()
    return C.prepared_case(DEC_H, (1,) * DEC_N, D=DEC_D, slots=DEC_SLOTS, indices=perm, seed=2)


def prefill_case():
    """BASELINE config 3 on the CPU: T=8192, H=32, zero initial state in slot 1
    (slot 2 is spare: the validation call tracks a prefix into it)."""
    from tests import kda_cases as C

    return C.prepared_case(PF_H, (PF_T,), D=PF_D, slots=3, indices=[1], seed=3, zero_pool=True)


def _device_case(heads, lengths, *, slots, indices, seed, gate=(1.0, 0.0), zero_pool=False,
                 device="cuda"):
    """BASELINE-config distributions drawn on the device (the large configs would
    take seconds to draw on the host): q, k L2-normalized bf16, v bf16,
    ``g = logsigmoid(randn*gate[0] + gate[1])`` fp32, ``beta = sigmoid(randn)``
    fp32, pool ``randn*0.05`` (or zeros) K-contiguous."""
    gen = torch.Generator(device=device).manual_seed(seed)
    T = int(sum(lengths))
    D = 128

    def l2(x):
        return x / torch.sqrt((x * x).sum(-1, keepdim=True) + 1e-6)

    def rnd(*shape):
        return torch.randn(*shape, generator=gen, device=device)

    q = l2(rnd(1, T, heads, D)).bfloat16()
    k = l2(rnd(1, T, heads, D)).bfloat16()
    v = rnd(1, T, heads, D).bfloat16()
    g = torch.nn.functional.logsigmoid(rnd(1, T, heads, D) * gate[0] + gate[1])
    beta = torch.sigmoid(rnd(1, T, heads))
    if zero_pool:
        pool = torch.zeros(slots, heads, D, D, device=device).transpose(-1, -2)
    else:
        pool = (rnd(slots, heads, D, D) * 0.05).transpose(-1, -2)
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + int(n))
    return dict(q=q, k=k, v=v, g=g, beta=beta, pool=pool,
                idx=torch.tensor(list(indices), dtype=torch.int32, device=device),
                cu=torch.tensor(cu, dtype=torch.int32, device=device), scale=D ** -0.5)


def run_more(steps, warmup):
    """Configs 4 and 5 prefill, a batch of 64 short prompts, and config 5's
    4-token decode, on the device."""
    from tests import kda_cases as C

    ops = torch.ops.sgl_glm53_ascend
    out = {}

    def prefill(name, heads, lengths, slots, indices, seed, gate, zero_pool):
        c = _device_case(heads, lengths, slots=slots, indices=indices, seed=seed, gate=gate,
                         zero_pool=zero_pool)
        T = int(sum(lengths))
        N = len(lengths)

        def step():
            return ops.kda_prepared_varlen_chunk(
                c["q"], c["k"], c["v"], c["g"], c["beta"], initial_state_source=c["pool"],
                initial_state_indices=c["idx"], cu_seqlens=c["cu"], scale=c["scale"])

        r = timed(step, steps, warmup, 30)
        us = r["event_us_per_call"]
        flop = T * heads * FLOP_PER_TOKEN_HEAD
        state_bytes = N * heads * 128 * 128 * 4 * (1 if zero_pool else 2)
        nbytes = T * heads * BYTES_PER_TOKEN_ROW + state_bytes
        tf = flop / (us * 1e-6) / 1e12
        out[name] = dict(tokens=T, heads=heads, seqs=N, event_us_per_call=us,
                         settle_calls=r["settle_calls"], tok_per_s=T / (us * 1e-6),
                         tflops=tf, mfma_frac=tf / BF16_PEAK_TFLOPS,
                         attainable_frac=(tf * 1e12) / min(BF16_PEAK_TFLOPS * 1e12,
                                                           HBM_PEAK_GBS * 1e9 * flop / nbytes),
                         algorithmic_flop=flop, algorithmic_bytes=nbytes)
        _log(f"{name}: {us:.1f} us, {tf:.1f} TFLOP/s")
        del c

    g4 = C.gen(4)
    lengths4 = [int(x) for x in torch.randint(1, 4097, (16,), generator=g4)]
    idx4 = torch.randperm(64, generator=g4)[:16].tolist()
    prefill("config4_prefill", 32, lengths4, 64, idx4, 4, (1.0, 0.0), False)
    prefill("config5_prefill", 16, [65536], 2, [1], 5, (2.0, -2.0), True)
    # a serving-shaped batch: 64 prompts x 256 tokens (2048 (sequence, head)
    # items, which the scan runs on persistent workgroups)
    prefill("batch64x256_prefill", 32, [256] * 64, 65, list(range(1, 65)), 6, (1.0, 0.0), False)

    # config 5 decode: 1024 sequences x 4 tokens from a 2048-slot pool, harsh decay
    n5, steps5, h5, slots5 = 1024, 4, 16, 2048
    idx5 = torch.randperm(slots5, generator=C.gen(5))[:n5].tolist()
    c = _device_case(h5, [steps5] * n5, slots=slots5, indices=idx5, seed=55, gate=(2.0, -2.0))

    def dstep():
        return ops.kda_prepared_varlen_recurrent(
            c["q"], c["k"], c["v"], c["g"], c["beta"], initial_state_source=c["pool"],
            initial_state_indices=c["idx"], cu_seqlens=c["cu"], scale=c["scale"])

    r = timed(dstep, max(steps, 10), warmup, 60)
    us = r["event_us_per_call"]
    nbytes = (n5 * h5 * 2 * 128 * 128 * 4 + n5 * steps5 * h5 * BYTES_PER_TOKEN_ROW
              + (n5 + 1) * 4 + n5 * 4)
    gbs = nbytes / (us * 1e-6) / 1e9
    out["config5_decode"] = dict(seqs=n5, tokens_per_seq=steps5, heads=h5, pool_slots=slots5,
                                 event_us_per_call=us, settle_calls=r["settle_calls"],
                                 tok_per_s=n5 * steps5 / (us * 1e-6),
                                 hbm_gbs=gbs, hbm_frac=gbs / HBM_PEAK_GBS,
                                 algorithmic_bytes=nbytes)
    _log(f"config5_decode: {us:.1f} us, {gbs:.0f} GB/s")
    return out


# Raw-gate decode at config 2's shape: bytes per token-head (state in + out,
# q, k, v, a bf16, b bf16, o bf16), plus A_log, dt_bias and the metadata.
RAW_BYTES_PER_TOKEN_HEAD = 2 * DEC_D * DEC_D * 4 + 4 * DEC_D * 2 + 2 + DEC_D * 2
RAW_DEC_BYTES = (DEC_N * DEC_H * RAW_BYTES_PER_TOKEN_HEAD + DEC_H * 4 + DEC_H * DEC_D * 4
                 + (DEC_N + 1) * 4 + DEC_N * 4)


def run_raw_decode(steps, warmup, min_settle, check):
    """The sglang-facing ``kda_varlen_recurrent`` (raw gates: A_log, a,
    dt_bias, b, lower_bound; q and k normalized in the kernel) at config 2's
    shape: 256 sequences x 1 token, H=32, a 512-slot pool (randn*0.05, drawn on
    the device), the seed-2 slot permutation. Validated on its first 64
    sequences against the oracle, then timed."""
    from oracle import kda_ref as R
    from tests import kda_cases as C

    ops = torch.ops.sgl_glm53_ascend
    perm = torch.randperm(DEC_SLOTS, generator=C.gen(2))[:DEC_N].tolist()
    case = C.raw_case(DEC_H, (1,) * DEC_N, slots=2, indices=perm, seed=21)
    gen = torch.Generator(device="cuda").manual_seed(22)
    pool = (torch.randn(DEC_SLOTS, DEC_H, DEC_D, DEC_D, generator=gen, device="cuda") * 0.05
            ).transpose(-1, -2)
    kw = case.kwargs("cuda", pool=pool)
    validated = None
    if check:
        n = 64
        before = pool[perm[:n]].cpu()
        out = ops.kda_varlen_recurrent(prefill=False, **kw)
        torch.cuda.synchronize()
        ref_pool = torch.zeros(n + 1, DEC_H, DEC_D, DEC_D).transpose(-1, -2)
        idx = []
        for i, s_ in enumerate(perm[:n]):
            if s_ > 0:
                ref_pool[i + 1] = before[i]
            idx.append(i + 1 if s_ > 0 else 0)
        qn, kn, g, beta = R.kda_prepare(case.A_log, case.a[:, :n], case.dt_bias, case.q[:, :n],
                                        case.k[:, :n], case.b[:, :n], case.lower_bound,
                                        case.scale)
        ref = R.kda_recurrent(qn, kn, case.v[:, :n], g, beta, state_pool=ref_pool,
                              state_indices=torch.tensor(idx, dtype=torch.int32),
                              cu_seqlens=torch.arange(n + 1, dtype=torch.int32),
                              out_dtype=torch.float32)
        got = torch.stack([pool[s_].cpu() if s_ > 0 else torch.zeros_like(ref_pool[0])
                           for s_ in perm[:n]])
        want = torch.stack([ref_pool[i] for i in idx])
        validated = _errs(out[:, :n].cpu(), ref, got, want)
        validated["sample"] = f"first {n} of {DEC_N} sequences"
        validated["passed"] = _passed(validated)

    def step():
        return ops.kda_varlen_recurrent(prefill=False, **kw)

    r = timed(step, steps, warmup, min_settle)
    us = r["event_us_per_call"]
    gbs = RAW_DEC_BYTES / (us * 1e-6) / 1e9
    traffic, traffic_src = traffic_from_profile("decode_recurrent_b256_h32_hbm_traffic.md",
                                                source_sha256(DECODE_SOURCES), "bench-figures-raw")
    del pool
    return dict(
        workload=("kda_varlen_recurrent (raw gates, sglang schema) B=256 x 1 token, H=32, "
                  "K=V=128, bf16 q/k/v/a/b, fp32 512-slot K-contiguous pool updated in place"),
        tok_per_s=DEC_N / (r["ms_per_step"] / 1e3), ms_per_step=r["ms_per_step"],
        event_us_per_call=us, settle_calls=r["settle_calls"], validated=validated,
        roofline=dict(bound="hbm", achieved=gbs, peak=HBM_PEAK_GBS, unit="GB/s",
                      frac=gbs / HBM_PEAK_GBS, traffic=traffic, traffic_source=traffic_src,
                      algorithmic_bytes_per_launch=RAW_DEC_BYTES,
                      kernel="recurrent_kernel<128,32,2,strided rows,decode,bf16,bf16,RAW>"))


# ---------------------------------------------------------------------------
# the CPU baseline leg: the oracle timed on the host, and as the checker
# ---------------------------------------------------------------------------


def _median_time(fn, budget_s, max_runs):
    fn()  # warm-up
    times = []
    start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - start < budget_s and len(times) < max_runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def cpu_decode(case, sample_n=64, budget_s=10.0):
    """The oracle's recurrent decode (the reference CPU path's loop structure,
    bench/kda_chunk/kda_python.py:253-307) on the first ``sample_n`` of the
    config-2 sequences, on the host cores. Returns the baseline figures and the
    oracle's outputs and states (the checker's reference for those sequences):
    their slots are renumbered 1..sample_n in a compact pool (0 stays 0)."""
    from oracle import kda_ref as R

    torch.set_num_threads(os.cpu_count() or 1)
    perm = case.indices[:sample_n].tolist()
    D = case.q.shape[-1]
    pool0 = torch.zeros(sample_n + 1, DEC_H, D, D).transpose(-1, -2)
    idx = []
    for i, s in enumerate(perm):
        if s > 0:
            pool0[i + 1] = case.pool[s]
        idx.append(i + 1 if s > 0 else 0)
    idx = torch.tensor(idx, dtype=torch.int32)
    cu = torch.arange(sample_n + 1, dtype=torch.int32)
    qs = case.q[:, :sample_n].float() * case.scale
    k, v, g, beta = (t[:, :sample_n] for t in (case.k, case.v, case.g, case.beta))
    box = {}

    def once():
        pool = pool0.transpose(-1, -2).clone().transpose(-1, -2)
        box["out"] = R.kda_recurrent(qs, k, v, g, beta, state_pool=pool, state_indices=idx,
                                     cu_seqlens=cu, out_dtype=torch.float32)
        box["pool"] = pool

    med, runs = _median_time(once, budget_s, 50)
    base = dict(value=sample_n / med, unit="tok/s", cores=torch.get_num_threads(), kind="port",
                sample=(f"oracle kda_recurrent (torch fp32, CPU) on {sample_n} of the 256 "
                        f"config-2 sequences x 1 token, H={DEC_H}, K=V={DEC_D}; median of "
                        f"{runs} runs; os.cpu_count()={os.cpu_count()}"))
    return base, box["out"], box["pool"], idx


def cpu_prefill(case, sample_t=512, budget_s=12.0):
    """The oracle's chunked prefill (bench/kda_chunk/kda_python.py:41-188) on
    the first ``sample_t`` of the config-3 tokens, all heads, on the host
    cores. Returns the baseline figures, the oracle's output and its state
    after the sample (the checker's reference for the same prefix)."""
    from oracle import kda_ref as R

    torch.set_num_threads(os.cpu_count() or 1)
    qs = case.q[:, :sample_t].float() * case.scale
    k, v, g, beta = (t[:, :sample_t] for t in (case.k, case.v, case.g, case.beta))
    D = case.q.shape[-1]
    box = {}

    def once():
        pool = torch.zeros(2, PF_H, D, D).transpose(-1, -2)
        box["out"] = R.kda_chunk(qs, k, v, g, beta, state_pool=pool,
                                 state_indices=torch.tensor([1], dtype=torch.int32),
                                 cu_seqlens=torch.tensor([0, sample_t], dtype=torch.int32),
                                 out_dtype=torch.float32)
        box["state"] = pool[1].clone()

    med, runs = _median_time(once, budget_s, 20)
    base = dict(value=sample_t / med, unit="tok/s", cores=torch.get_num_threads(), kind="port",
                sample=(f"oracle kda_chunk (torch fp32, CPU, chunk 64) on the first {sample_t} "
                        f"of the 8192 config-3 tokens, H={PF_H}, K=V={PF_D}; median of {runs} "
                        f"runs; os.cpu_count()={os.cpu_count()}"))
    return base, box["out"], box["state"]


def _errs(out, ref_out, state, ref_state):
    from tests import kda_cases as C

    return dict(out_err=C.out_err(out, ref_out), state_err=C.max_rel_err(state, ref_state))


def _passed(v):
    from tests import kda_cases as C

    return v["out_err"] <= C.OUT_TOL and v["state_err"] <= C.STATE_TOL


# ---------------------------------------------------------------------------
# latency rows (the reference bench's deployed shapes)
# ---------------------------------------------------------------------------


def latency_regimes():
    """(label, heads, lengths, prefill, checkpoints, op), as the reference
    bench's ``regimes()`` (bench_kda_varlen_recurrent.py:534-551) with its
    constants (:77-114): decode H16/32/64 x B1/32/128; the verify shapes with
    4 draft tokens per request, checkpointed; recurrent prefill H4/H8 x
    T1k-16k; and the reference chunk bench's rows (bench/kda_chunk/
    bench_kda_chunk.py:420-467, README.md:37-39): ``kda_varlen_chunk`` at H8,
    one sequence of 1k / 2k / 4k tokens."""
    for heads in (16, 32, 64):
        for batch in (1, 32, 128):
            yield f"decode H{heads} B{batch}", heads, (1,) * batch, False, False, "recurrent"
    for label, heads, req in (("256K DP4TP2", 32, 2), ("256K DP2TP4", 16, 3),
                              ("256K DP8TP1", 64, 1), ("512K DP4TP2", 32, 1),
                              ("512K DP2TP4", 16, 1)):
        yield f"verify {label} R{req}", heads, (4,) * req, False, True, "recurrent"
    for heads in (4, 8):
        for tokens in (1024, 2048, 4096, 8192, 16384):
            yield f"prefill H{heads} T{tokens // 1024}k", heads, (tokens,), True, False, "recurrent"
    for tokens in (1024, 2048, 4096):
        yield f"chunk H8 T{tokens // 1024}k", 8, (tokens,), True, False, "chunk"


def run_latency_rows(steps, check):
    """Each regime through the sglang-facing op (raw gates, the reference
    bench's distributions), validated against the oracle when ``check`` (the
    CPU leg is on), then timed twice: eagerly (HIP events around ``steps``
    back-to-back calls, what a caller without graphs sees, host launch path
    included) and as replays of a HIP graph of the same calls (the device
    time per call)."""
    from oracle import kda_ref as R
    from tests import kda_cases as C

    ops = torch.ops.sgl_glm53_ascend
    rows = []
    for label, heads, lengths, prefill, ckpt, op in latency_regimes():
        case = C.raw_case(heads, lengths, seed=1000 + heads + len(lengths) + sum(lengths))
        N = len(lengths)
        D = 128
        mid = None
        if ckpt:
            mid = (torch.randn(N, max(lengths), heads, D, D) * 0.1).transpose(-1, -2)
        pool = C.to_dev(case.pool, "cuda")
        mid_d = None if mid is None else mid.transpose(-1, -2).contiguous().cuda().transpose(-1, -2)
        kw = case.kwargs("cuda", pool=pool)

        def step():
            if op == "chunk":
                return ops.kda_varlen_chunk(prefill=True, **kw)
            return ops.kda_varlen_recurrent(intermediate_state=mid_d, prefill=prefill, **kw)

        row = dict(label=label, op=f"kda_varlen_{op}", heads=heads, requests=N,
                   tokens=int(sum(lengths)))
        if check:
            out = step()
            torch.cuda.synchronize()
            ref_pool = C.clone_pool(case.pool)
            ref_mid = None if mid is None else mid.transpose(-1, -2).clone().transpose(-1, -2)
            qn, kn, g, beta = R.kda_prepare(case.A_log, case.a, case.dt_bias, case.q, case.k,
                                            case.b, case.lower_bound, case.scale)
            if op == "chunk":
                ref = R.kda_chunk(qn, kn, case.v, g, beta, state_pool=ref_pool,
                                  state_indices=case.indices, cu_seqlens=case.cu_seqlens,
                                  out_dtype=torch.float32)
            else:
                ref = R.kda_recurrent(qn, kn, case.v, g, beta, state_pool=ref_pool,
                                      state_indices=case.indices, cu_seqlens=case.cu_seqlens,
                                      intermediate_state=ref_mid, out_dtype=torch.float32)
            v = _errs(out.cpu(), ref, pool.cpu(), ref_pool)
            if ref_mid is not None:
                v["checkpoint_err"] = C.max_rel_err(mid_d.cpu(), ref_mid)
            v["passed"] = _passed(v) and v.get("checkpoint_err", 0.0) <= C.STATE_TOL
            row["validated"] = v
        r = timed(step, steps, 2, 30)
        us = r["event_us_per_call"]
        T = int(sum(lengths))
        # state in + out per (sequence, head) (the checkpoints are written
        # instead of the final state), plus the token rows (raw gates: q, k,
        # v, a bf16 in, b bf16, o bf16 out)
        state_bytes = N * heads * D * D * 4 * (1 + (max(lengths) if ckpt else 1))
        nbytes = state_bytes + T * heads * (5 * D * 2 + 2)
        row.update(event_us_per_call=us, settle_calls=r["settle_calls"],
                   hbm_gbs=nbytes / (us * 1e-6) / 1e9, algorithmic_bytes=nbytes,
                   ref_910b4_ms=REF_910B4_MS.get(label))
        try:
            gus = graph_us(step, 10 if not prefill else 2)
            row.update(graph_us_per_call=gus, graph_hbm_gbs=nbytes / (gus * 1e-6) / 1e9)
        except RuntimeError as e:  # reported, never fatal to the run
            row.update(graph_us_per_call=None, graph_error=str(e)[:200])
            gus = float("nan")
        rows.append(row)
        ok = row.get("validated", {}).get("passed", True)
        _log(f"{label}: {us:.1f} us eager, {gus:.1f} us graph, {row['hbm_gbs']:.0f} GB/s"
             f"{'' if ok else '  VALIDATION FAILED'}")
        del pool, mid_d
    return rows


# ---------------------------------------------------------------------------
# profile summaries
# ---------------------------------------------------------------------------


def copy_gbs(mib=512, calls=10):
    """Read + write bytes per second of a plain device-to-device copy of `mib`
    MiB (torch's copy kernel), best of `calls`, timed with HIP events."""
    n = mib * 2 ** 20 // 4
    src = torch.ones(n, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    best = float("inf")
    for _ in range(calls):
        e0.record()
        dst.copy_(src)
        e1.record()
        e1.synchronize()
        best = min(best, e0.elapsed_time(e1))
    del src, dst
    torch.cuda.empty_cache()
    return 2 * n * 4 / (best * 1e-3) / 1e9


def summarize_trace(path, last):
    """Per-kernel duration statistics from a rocprofv3 kernel-trace CSV, one
    row per (kernel, grid size) -- the grid tells the workloads of one kernel
    apart -- over each row's last ``last`` dispatches (0 = all)."""
    by = {}
    with open(path) as f:
        for row in csv.DictReader(f):
            us = (int(row["End_Timestamp"]) - int(row["Start_Timestamp"])) / 1e3
            key = (row["Kernel_Name"], int(row["Grid_Size_X"]))
            by.setdefault(key, []).append((int(row["Dispatch_Id"]), us))
    print("| kernel | grid | dispatches | used | mean µs | median µs | min µs | max µs |")
    print("|---|---|---|---|---|---|---|---|")
    for (name, grid), xs in sorted(by.items(), key=lambda kv: -sum(u for _, u in kv[1])):
        xs.sort()
        sel = [u for _, u in (xs[-last:] if last > 0 else xs)]
        short = re.sub(r"\(KdaRecurrentArgs\)|\(KdaChunkArgs[^)]*\)", "", name).replace("unsigned short", "u16")
        print(f"| `{short[:150]}` | {grid} | {len(xs)} | {len(sel)} | {statistics.mean(sel):.2f} | "
              f"{statistics.median(sel):.2f} | {min(sel):.2f} | {max(sel):.2f} |")


def summarize_counters(path):
    """Mean value per dispatch of every counter, per kernel, from a rocprofv3
    counter-collection CSV."""
    by = {}
    with open(path) as f:
        for row in csv.DictReader(f):
            key = (row["Kernel_Name"], row["Counter_Name"])
            by.setdefault(key, []).append(float(row["Counter_Value"]))
    print("| kernel | counter | dispatches | mean per dispatch |")
    print("|---|---|---|---|")
    for (name, ctr), xs in sorted(by.items()):
        short = re.sub(r"\(KdaRecurrentArgs\)|\(KdaChunkArgs[^)]*\)", "", name).replace("unsigned short", "u16")
        print(f"| `{short[:150]}` | {ctr} | {len(xs)} | {statistics.mean(xs):.1f} |")


# ---------------------------------------------------------------------------
# main
# ---------------------------------------------------------------------------


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--settle", type=int, default=150,
                    help="minimum settle calls before the warm-up (decode; prefill: 2/3)")
    ap.add_argument("--no-cpu", action="store_true",
                    help="skip the CPU leg (baseline timing and the validation it checks)")
    ap.add_argument("--no-prefill", action="store_true", help="skip the prefill workload")
    ap.add_argument("--no-decode", action="store_true", help="skip the decode workload")
    ap.add_argument("--no-more", action="store_true",
                    help="skip the config 4 / 5 lines and the latency rows")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run 5 plain device copies of MIB MiB (the known-size kernel "
                         "the FETCH_SIZE / WRITE_SIZE counters are scaled by), then exit")
    ap.add_argument("--summarize-trace", metavar="CSV",
                    help="print per-kernel durations from a rocprofv3 kernel-trace CSV, then exit")
    ap.add_argument("--summarize-counters", metavar="CSV",
                    help="print per-kernel counter means from a rocprofv3 counter CSV, then exit")
    ap.add_argument("--last", type=int, default=0,
                    help="with --summarize-trace: use each kernel's last N dispatches")
    args = ap.parse_args()
    if args.summarize_trace:
        summarize_trace(args.summarize_trace, args.last)
        return
    if args.summarize_counters:
        summarize_counters(args.summarize_counters)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported "
              "(the KDA path shards by head and sequence with no exchange inside the op; "
              "this build runs and measures a single GPU).", file=sys.stderr)
        sys.exit(2)
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.copy_calibration > 0:
        n = args.copy_calibration * 2 ** 20 // 4
        src = torch.ones(n, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        _log(f"copy calibration: 5 x {args.copy_calibration} MiB device copies")
        return
    import sgl_glm53_ascend_ops  # noqa: F401
    from tests import kda_cases as C

    ops = torch.ops.sgl_glm53_ascend
    check = not args.no_cpu
    dec_sha = source_sha256(DECODE_SOURCES)
    pf_sha = source_sha256(PREFILL_SOURCES)
    validated = {}
    failed = False

    dec = None
    cpu = None
    if not args.no_decode:
        _log("decode: config 2 (B=256, H=32, K=V=128)")
        case = decode_case()
        q, k, v, g, beta = (getattr(case, n).cuda() for n in ("q", "k", "v", "g", "beta"))
        idx = case.indices.cuda()
        cu = case.cu_seqlens.cuda()
        if check:
            pool = C.to_dev(case.pool, "cuda")
            out = ops.kda_prepared_varlen_recurrent(q, k, v, g, beta, initial_state_source=pool,
                                                    initial_state_indices=idx, cu_seqlens=cu,
                                                    scale=case.scale)
            torch.cuda.synchronize()
            _log("cpu baseline / checker: oracle decode on host cores")
            cpu, ref_out, ref_pool, sidx = cpu_decode(case)
            n = ref_out.shape[1]
            slots = case.indices[:n].tolist()
            got_state = torch.stack([pool[s].cpu() if s > 0 else torch.zeros_like(ref_pool[0])
                                     for s in slots])
            ref_state = torch.stack([ref_pool[int(i)] for i in sidx.tolist()])
            validated["decode"] = _errs(out[:, :n].cpu(), ref_out, got_state, ref_state)
            validated["decode"]["sample"] = f"first {n} of {DEC_N} sequences"
            ok = _passed(validated["decode"])
            failed |= not ok
            _log(f"decode validation: {validated['decode']}{'' if ok else '  FAILED'}")
            _log(f"cpu baseline: {cpu['value']:.1f} tok/s on {cpu['cores']} threads")
            del pool
        pool = C.to_dev(case.pool, "cuda")

        def step():
            return ops.kda_prepared_varlen_recurrent(
                q, k, v, g, beta, initial_state_source=pool, initial_state_indices=idx,
                cu_seqlens=cu, scale=case.scale)

        dec = timed(step, args.steps, args.warmup, args.settle)
        _log(f"decode: {dec['event_us_per_call']:.1f} us/call after {dec['settle_calls']} "
             "settle calls")
        del pool, case

    dec_raw = None
    if not args.no_decode:
        _log("decode, raw gates: config 2's shape through kda_varlen_recurrent")
        dec_raw = run_raw_decode(args.steps, args.warmup, args.settle, check)
        if dec_raw["validated"] is not None:
            validated["decode_raw"] = dec_raw["validated"]
            failed |= not dec_raw["validated"]["passed"]
        _log(f"decode raw: {dec_raw['event_us_per_call']:.1f} us/call, "
             f"{dec_raw['roofline']['frac'] * 100:.1f}% of HBM peak; {dec_raw['validated']}")

    prefill = None
    if not args.no_prefill:
        _log("prefill: config 3 (T=8192, H=32, K=V=128, chunk 64)")
        case = prefill_case()
        q, k, v, g, beta = (getattr(case, n).cuda() for n in ("q", "k", "v", "g", "beta"))
        pool = C.to_dev(case.pool, "cuda")
        idx = case.indices.cuda()
        cu = case.cu_seqlens.cuda()
        pf_cpu = None
        if check:
            sample_t = 512
            out = ops.kda_prepared_varlen_chunk(
                q, k, v, g, beta, initial_state_source=pool, initial_state_indices=idx,
                cu_seqlens=cu, scale=case.scale,
                track_state_indices=torch.tensor([2], dtype=torch.int32, device="cuda"),
                track_state_lens=torch.tensor([sample_t], dtype=torch.int32, device="cuda"))
            torch.cuda.synchronize()
            _log("cpu baseline / checker: oracle chunked prefill on host cores")
            pf_cpu, ref_out, ref_state = cpu_prefill(case, sample_t)
            validated["prefill"] = _errs(out[:, :sample_t].cpu(), ref_out, pool[2].cpu(),
                                         ref_state)
            validated["prefill"]["sample"] = (f"first {sample_t} of {PF_T} tokens; state "
                                              f"tracked at {sample_t}")
            ok = _passed(validated["prefill"])
            failed |= not ok
            _log(f"prefill validation: {validated['prefill']}{'' if ok else '  FAILED'}")

        if check:
            # the whole sequence: this call's output and final state (slot 1)
            # against the recurrent kernel run in fp32 (bf16 inputs widened
            # exactly), itself pinned to the oracle at 1e-5 by the tests
            rpool = torch.zeros(2, PF_H, PF_D, PF_D, device="cuda").transpose(-1, -2)
            rout = ops.kda_prepared_varlen_recurrent(
                q.float(), k.float(), v.float(), g, beta, initial_state_source=rpool,
                initial_state_indices=idx, cu_seqlens=cu, scale=case.scale)
            torch.cuda.synchronize()
            full = _errs(out.cpu(), rout.cpu(), pool[1].cpu(), rpool[1].cpu())
            full["reference"] = ("this build's recurrent kernel with fp32 I/O over all 8192 tokens "
                                 "(final state and every output row)")
            validated["prefill_full"] = full
            ok = _passed(full)
            failed |= not ok
            _log(f"prefill full-length check: {full}{'' if ok else '  FAILED'}")
            del rpool, rout

        # Every timed call starts from a zero state (config 3) and writes its
        # final state: each takes its own slot of a pool zeroed before the
        # timed calls, outside the timed region.
        n_pf = max(5, args.steps // 2)
        tpool = torch.zeros(n_pf + 1, PF_H, PF_D, PF_D, device="cuda").transpose(-1, -2)
        tidx = [torch.tensor([i + 1], dtype=torch.int32, device="cuda") for i in range(n_pf)]
        calls = [0]

        def pstep():
            i = calls[0] % n_pf
            calls[0] += 1
            return ops.kda_prepared_varlen_chunk(
                q, k, v, g, beta, initial_state_source=tpool, initial_state_indices=tidx[i],
                cu_seqlens=cu, scale=case.scale)

        def zero_slots():
            tpool.zero_()
            calls[0] = 0

        pf = timed(pstep, n_pf, args.warmup, (2 * args.settle) // 3, before_timed=zero_slots)
        us = pf["event_us_per_call"]
        tf = PF_FLOP / (us * 1e-6) / 1e12
        traffic, traffic_src = traffic_from_profile("prefill_chunk_t8192_h32_hbm_traffic.md", pf_sha)
        prefill = dict(
            workload="chunk prefill T=8192 H=32 K=V=128 BT=64 bf16 qkv, fp32 g/beta/state",
            tok_per_s=PF_T / (pf["ms_per_step"] / 1e3),
            ms_per_step=pf["ms_per_step"],
            event_us_per_call=us,
            settle_calls=pf["settle_calls"],
            tflops=tf,
            mfma_frac=tf / BF16_PEAK_TFLOPS,
            attainable_frac=(tf * 1e12) / min(BF16_PEAK_TFLOPS * 1e12,
                                              HBM_PEAK_GBS * 1e9 * PF_FLOP / PF_BYTES),
            hbm_gbs=PF_BYTES / (us * 1e-6) / 1e9,
            algorithmic_flop=PF_FLOP,
            algorithmic_bytes=PF_BYTES,
            traffic=traffic,
            traffic_source=traffic_src,
            source_sha256=pf_sha,
            workspace_bytes=int(sgl_glm53_ascend_ops.chunk_workspace_bytes(PF_T, 1, PF_H)),
            timed_calls=("each from a zero state in its own slot of a pool zeroed before the "
                         "timed calls (no fill inside the timed region)"),
            cpu_baseline=pf_cpu,
        )
        _log(f"prefill: {us:.1f} us/call, {tf:.1f} TFLOP/s after {pf['settle_calls']} settle calls")
        del pool, case, tpool

    more = None
    rows = None
    if not args.no_more:
        more = run_more(max(3, args.steps // 5), 2)
        rows = run_latency_rows(10, check)
        bad = [r["label"] for r in rows if not r.get("validated", {}).get("passed", True)]
        if bad:
            failed = True
            _log(f"latency rows failing validation: {bad}")
        validated["latency_rows"] = "all passed" if not bad else f"failed: {bad}"

    if dec is None:
        return
    tok_s = DEC_N / (dec["ms_per_step"] / 1e3)
    achieved = DEC_BYTES / (dec["event_us_per_call"] * 1e-6) / 1e9
    traffic, traffic_src = traffic_from_profile("decode_recurrent_b256_h32_hbm_traffic.md", dec_sha)
    copy_ref = copy_gbs()
    _log(f"reference: a 512 MiB device copy reaches {copy_ref:.0f} GB/s (read + write); "
         f"the decode {achieved:.0f} GB/s")
    line = dict(
        metric="KDA decode tok/s + state HBM GB/s (B=256); chunk prefill tok/s (T=8k)",
        value=tok_s,
        unit="tok/s",
        n_gpus=1,
        steps=args.steps,
        warmup=args.warmup,
        settle_calls=dec["settle_calls"],
        ms_per_step=dec["ms_per_step"],
        higher_is_better=True,
        scaling="weak",
        vs_baseline=None,
        dtype="fp32",
        data="synthetic",
        config=dict(
            workload=("varlen recurrent decode B=256 x 1 token, H=32, K=V=128, bf16 q/k/v, "
                      "fp32 log-decay g and beta, fp32 K-contiguous state pool of 512 slots "
                      "updated in place (BASELINE configs[1])"),
            batch=DEC_N, heads=DEC_H, head_dim=DEC_D, pool_slots=DEC_SLOTS,
        ),
        validated=validated if check else None,
        state_hbm_gbs=achieved,
        roofline=dict(
            bound="hbm", achieved=achieved, peak=HBM_PEAK_GBS, unit="GB/s",
            frac=achieved / HBM_PEAK_GBS, traffic=traffic, traffic_source=traffic_src,
            kernel="recurrent_kernel<128,32,2,strided rows,decode,bf16,bf16,LOG>",
            algorithmic_bytes_per_launch=DEC_BYTES,
            event_us_per_call=dec["event_us_per_call"],
            source_sha256=dec_sha,
            copy_gbs=copy_ref,
        ),
        decode_raw=dec_raw,
        prefill=prefill,
        more_configs=more,
        latency_rows=rows,
        cpu_baseline=cpu,
    )
    print(json.dumps(line), flush=True)
    if failed:
        _log("validation failed: the figures above are not valid")
        sys.exit(1)


if __name__ == "__main__":
    main()
