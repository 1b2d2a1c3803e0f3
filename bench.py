"""Benchmark of the KDA hot path on one MI355X: decode tok/s + state HBM GB/s, prefill tok/s.

Workload (BASELINE.json ``configs[1]``, the configuration the metric is quoted
on): varlen recurrent decode, one token for each of 256 sequences, H=32,
K=V=128, bf16 q/k/v (q, k L2-normalized), fp32 per-channel log decay
``g = logsigmoid(randn)`` and ``beta = sigmoid(randn)``, fp32 state pool of 512
slots (``randn*0.05``, K-contiguous), ``state_indices`` a seeded random
permutation of 256 of the slots, updated in place. One *step* is one call of
the decode operator over the whole batch (every step advances all 256
sequences by one token in place). ``value`` = tokens/s = 256 / step time.

Also reported (same JSON line): the chunked prefill of ``configs[2]`` (T=8192
single sequence, H=32, K=V=128, chunk 64) as ``prefill``, the decode kernel's
roofline (algorithmic bytes / kernel time, measured with HIP events on the
launch stream), ``more_configs`` (configs 4 and 5 prefill and config 5's
4-token decode, a few timed calls each, inputs drawn on the device) and the CPU
baseline (this repository's torch oracle of the reference CPU path, on the
host cores, over a bounded sample).

Usage: ``python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-more]``.
"""

from __future__ import annotations

import argparse
import json
import os
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

# Config 2 (decode) shape.
DEC_N, DEC_H, DEC_D, DEC_SLOTS = 256, 32, 128, 512
# Algorithmic bytes per token-head: state read + write (2*D*D*4), q, k, v
# (3*D*2), g (D*4), beta (4), o (D*2).
BYTES_PER_TOKEN_HEAD = 2 * DEC_D * DEC_D * 4 + 3 * DEC_D * 2 + DEC_D * 4 + 4 + DEC_D * 2
# + cu_seqlens (257 x 4) + indices (256 x 4) + ... as quoted: 2052 B of metadata.
DEC_BYTES = DEC_N * DEC_H * BYTES_PER_TOKEN_HEAD + (DEC_N + 1) * 4 + DEC_N * 4

# HBM bytes per decode launch, from two rocprofv3 --pmc passes over
# ``bench.py --no-cpu --no-prefill`` (FETCH_SIZE, then WRITE_SIZE, KiB per
# dispatch), each scaled by what the same counter reads for a 512 MiB device
# copy (``--copy-calibration 512``): FETCH_SIZE reads 262156.8 KiB for the
# copy's 524288 KiB of reads (scale 2.0), WRITE_SIZE reads 524288 KiB (1.0).
# The kernel-trace/PMC summaries are kept under profiles/.
FETCH_SCALE = 524288.0 / 262156.8
WRITE_SCALE = 524288.0 / 524288.0
DEC_FETCH_KIB, DEC_WRITE_KIB = 267449.1, 526336.1
DEC_TRAFFIC = (DEC_FETCH_KIB * FETCH_SCALE + DEC_WRITE_KIB * WRITE_SCALE) * 1024
# Same for config 5's 4-token verify launch (1024 sequences, H=16).
VF_TRAFFIC = (565882.7 * FETCH_SCALE + 1063961.9 * WRITE_SCALE) * 1024
# Same for the two prefill kernels (prepare K1, scan K2) on config 3.
PF_TRAFFIC = ((168225.2 + 223851.4) * FETCH_SCALE + (444972.4 + 124021.7) * WRITE_SCALE) * 1024
# MFMA counters of the same two kernels (profiles/prefill_chunk_t8192_h32_mfma.md): matrix work
# executed per call (SQ_INSTS_VALU_MFMA_MOPS_* x 512 FLOP; the hi/lo operand splits roughly
# double the algorithmic count) and the fraction of SIMD cycles each kernel keeps the MFMA busy.
PF_MFMA_EXECUTED_FLOP = (39845888 + 69206016 + 50331648 + 1048576) * 512
PF_MFMA_BUSY = {"prepare": 28311552 / (3707468 / 8 * 1024), "scan": 59768832 / (3466918 / 8 * 1024)}

# Config 3 (prefill) shape.
PF_T, PF_H, PF_D, PF_BT = 8192, 32, 128, 64
# Dense-tile FLOPs per token-head: 2*(5*BT*D + 3*D*D).
PF_FLOP = PF_T * PF_H * 2 * (5 * PF_BT * PF_D + 3 * PF_D * PF_D)
# Algorithmic bytes: q,k,v bf16 in, g fp32, beta fp32, o bf16 out, final state fp32 out.
PF_BYTES = PF_T * PF_H * (3 * PF_D * 2 + PF_D * 4 + 4 + PF_D * 2) + PF_H * PF_D * PF_D * 4


def _log(msg):
    print(msg, file=sys.stderr, flush=True)


def decode_inputs(device):
    from tests import kda_cases as C

    perm = torch.randperm(DEC_SLOTS, generator=C.gen(2))[:DEC_N].tolist()
    case = C.prepared_case(DEC_H, (1,) * DEC_N, D=DEC_D, slots=DEC_SLOTS, indices=perm, seed=2)
    return case


def run_decode(steps, warmup, device="cuda"):
    from tests import kda_cases as C

    ops = torch.ops.sgl_glm53_ascend
    case = decode_inputs(device)
    q, k, v, g, beta = (getattr(case, n).to(device) for n in ("q", "k", "v", "g", "beta"))
    pool = C.to_dev(case.pool, device)
    idx = case.indices.to(device)
    cu = case.cu_seqlens.to(device)

    def step():
        return ops.kda_prepared_varlen_recurrent(
            q, k, v, g, beta, initial_state_source=pool, initial_state_indices=idx,
            cu_seqlens=cu, scale=case.scale)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(steps):
        step()
    ev1.record(stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_step = (t1 - t0) * 1e3 / steps
    kernel_us = ev0.elapsed_time(ev1) * 1e3 / steps
    return dict(ms_per_step=ms_step, kernel_us=kernel_us)


def run_prefill(steps, warmup, device="cuda"):
    from tests import kda_cases as C

    ops = torch.ops.sgl_glm53_ascend
    case = C.prepared_case(PF_H, (PF_T,), D=PF_D, slots=2, indices=[1], seed=3, zero_pool=True)
    q, k, v, g, beta = (getattr(case, n).to(device) for n in ("q", "k", "v", "g", "beta"))
    pool = C.to_dev(case.pool, device)
    idx = case.indices.to(device)
    cu = case.cu_seqlens.to(device)

    def step():
        pool.zero_()  # zero initial state each step (config 3)
        return ops.kda_prepared_varlen_chunk(
            q, k, v, g, beta, initial_state_source=pool, initial_state_indices=idx,
            cu_seqlens=cu, scale=case.scale)

    try:
        step()
        torch.cuda.synchronize()
    except RuntimeError as e:
        _log(f"prefill unavailable: {str(e).splitlines()[0]}")
        return None
    for _ in range(warmup):
        step()
    stream = torch.cuda.current_stream()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(steps):
        step()
    ev1.record(stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_step = (t1 - t0) * 1e3 / steps
    gpu_us = ev0.elapsed_time(ev1) * 1e3 / steps
    return dict(ms_per_step=ms_step, gpu_us=gpu_us)


# Configs 4 and 5 (reported beside the headline, a few timed calls each).
BYTES_PER_TOKEN_ROW = 3 * 128 * 2 + 128 * 4 + 4 + 128 * 2  # q,k,v bf16, g fp32, beta, o bf16
FLOP_PER_TOKEN_HEAD = 2 * (5 * 64 * 128 + 3 * 128 * 128)


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


def _time(step, steps, warmup):
    for _ in range(warmup):
        step()
    stream = torch.cuda.current_stream()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    ev0.record(stream)
    for _ in range(steps):
        step()
    ev1.record(stream)
    torch.cuda.synchronize()
    return ev0.elapsed_time(ev1) * 1e3 / steps


def run_more(steps=5, warmup=1):
    """Configs 4 and 5 prefill, and config 5's 4-token decode, on the device."""
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

        us = _time(step, steps, warmup)
        flop = T * heads * FLOP_PER_TOKEN_HEAD
        state_bytes = N * heads * 128 * 128 * 4 * (1 if zero_pool else 2)
        nbytes = T * heads * BYTES_PER_TOKEN_ROW + state_bytes
        tf = flop / (us * 1e-6) / 1e12
        out[name] = dict(tokens=T, heads=heads, seqs=N, gpu_us=us, tok_per_s=T / (us * 1e-6),
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

    # config 5 decode: 1024 sequences x 4 tokens from a 2048-slot pool, harsh decay
    n5, steps5, h5, slots5 = 1024, 4, 16, 2048
    idx5 = torch.randperm(slots5, generator=C.gen(5))[:n5].tolist()
    c = _device_case(h5, [steps5] * n5, slots=slots5, indices=idx5, seed=55, gate=(2.0, -2.0))

    def dstep():
        return ops.kda_prepared_varlen_recurrent(
            c["q"], c["k"], c["v"], c["g"], c["beta"], initial_state_source=c["pool"],
            initial_state_indices=c["idx"], cu_seqlens=c["cu"], scale=c["scale"])

    us = _time(dstep, max(steps, 10), max(warmup, 2))
    nbytes = (n5 * h5 * 2 * 128 * 128 * 4 + n5 * steps5 * h5 * BYTES_PER_TOKEN_ROW
              + (n5 + 1) * 4 + n5 * 4)
    gbs = nbytes / (us * 1e-6) / 1e9
    out["config5_decode"] = dict(seqs=n5, tokens_per_seq=steps5, heads=h5, pool_slots=slots5,
                                 kernel_us=us, tok_per_s=n5 * steps5 / (us * 1e-6),
                                 hbm_gbs=gbs, hbm_frac=gbs / HBM_PEAK_GBS,
                                 algorithmic_bytes=nbytes, traffic=VF_TRAFFIC,
                                 kernel="recurrent_kernel<128,16,8,consecutive rows,multi-token>")
    _log(f"config5_decode: {us:.1f} us, {gbs:.0f} GB/s")
    return out


def cpu_baseline(budget_s=10.0):
    """The oracle's recurrent decode (the reference CPU path's loop structure,
    bench/kda_chunk/kda_python.py:253-307) on the host cores."""
    from oracle import kda_ref as R
    from tests import kda_cases as C

    torch.set_num_threads(os.cpu_count() or 1)
    sample_n = 64
    case = C.prepared_case(DEC_H, (1,) * sample_n, D=DEC_D, slots=sample_n + 1, seed=2)
    qs = case.q.float() * case.scale

    def once():
        pool = C.clone_pool(case.pool)
        t0 = time.perf_counter()
        R.kda_recurrent(qs, case.k, case.v, case.g, case.beta, state_pool=pool,
                        state_indices=case.indices, cu_seqlens=case.cu_seqlens)
        return time.perf_counter() - t0

    once()  # warm-up
    times = []
    start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - start < budget_s and len(times) < 50):
        times.append(once())
    med = statistics.median(times)
    return dict(
        value=sample_n / med,
        unit="tok/s",
        cores=torch.get_num_threads(),
        kind="port",
        sample=(f"oracle kda_recurrent (torch fp32, CPU) on {sample_n} of the 256 config-2 "
                f"sequences x 1 token, H={DEC_H}, K=V={DEC_D}; median of {len(times)} runs; "
                f"os.cpu_count()={os.cpu_count()}"),
    )


def cpu_baseline_prefill(budget_s=12.0):
    """The oracle's chunked prefill (the reference CPU path's structure,
    bench/kda_chunk/kda_python.py:41-188) on the host cores, over a bounded
    sample of config 3: the first 512 of its 8192 tokens, all 32 heads."""
    from oracle import kda_ref as R
    from tests import kda_cases as C

    torch.set_num_threads(os.cpu_count() or 1)
    sample_t = 512
    case = C.prepared_case(PF_H, (sample_t,), D=PF_D, slots=2, indices=[1], seed=3,
                           zero_pool=True)
    qs = case.q.float() * case.scale

    def once():
        pool = C.clone_pool(case.pool)
        t0 = time.perf_counter()
        R.kda_chunk(qs, case.k, case.v, case.g, case.beta, state_pool=pool,
                    state_indices=case.indices, cu_seqlens=case.cu_seqlens)
        return time.perf_counter() - t0

    once()  # warm-up
    times = []
    start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - start < budget_s and len(times) < 20):
        times.append(once())
    med = statistics.median(times)
    return dict(
        value=sample_t / med,
        unit="tok/s",
        cores=torch.get_num_threads(),
        kind="port",
        sample=(f"oracle kda_chunk (torch fp32, CPU, chunk 64) on the first {sample_t} of the "
                f"8192 config-3 tokens, H={PF_H}, K=V={PF_D}; median of {len(times)} runs; "
                f"os.cpu_count()={os.cpu_count()}"),
    )


def _prefill_steps(args):
    """(steps, warmup) for the config-3 prefill: half the decode step count and
    the decode's warm-up count. On a fresh box the decode settles after ~150
    calls (~25 ms: 188 -> 173 us per call) and the prefill after ~100 (~40 ms:
    449 -> 381 us), hence the default of 200 warm-up calls."""
    return max(3, args.steps // 2), max(1, args.warmup)


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-prefill", action="store_true", help="skip the prefill workload")
    ap.add_argument("--no-decode", action="store_true", help="skip the decode workload")
    ap.add_argument("--no-more", action="store_true",
                    help="skip the config 4 / 5 lines reported beside the headline")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run 5 plain device copies of MIB MiB (the known-size kernel "
                         "the FETCH_SIZE / WRITE_SIZE counters are scaled by), then exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported "
              "(the KDA path shards by head and sequence with no exchange inside the op).",
              file=sys.stderr)
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

    if args.no_decode:
        # profiling aid: the prefill workload alone (no JSON line)
        _log("prefill: config 3 (T=8192, H=32, K=V=128, chunk 64)")
        pf = run_prefill(*_prefill_steps(args))
        if pf is not None:
            _log(f"prefill: {pf['ms_per_step']*1e3:.1f} us/step")
        return
    _log("decode: config 2 (B=256, H=32, K=V=128)")
    dec = run_decode(args.steps, args.warmup)
    tok_s = DEC_N / (dec["ms_per_step"] / 1e3)
    achieved = DEC_BYTES / (dec["kernel_us"] * 1e-6) / 1e9
    _log(f"decode: {dec['ms_per_step']*1e3:.1f} us/step, kernel {dec['kernel_us']:.1f} us, "
         f"{achieved:.0f} GB/s")

    prefill = None
    if not args.no_prefill:
        _log("prefill: config 3 (T=8192, H=32, K=V=128, chunk 64)")
        pf = run_prefill(*_prefill_steps(args))
        if pf is not None:
            tf = PF_FLOP / (pf["gpu_us"] * 1e-6) / 1e12
            prefill = dict(
                workload="chunk prefill T=8192 H=32 K=V=128 BT=64 bf16 qkv, fp32 g/beta/state",
                tok_per_s=PF_T / (pf["ms_per_step"] / 1e3),
                ms_per_step=pf["ms_per_step"],
                gpu_us=pf["gpu_us"],
                tflops=tf,
                mfma_frac=tf / BF16_PEAK_TFLOPS,
                hbm_gbs=PF_BYTES / (pf["gpu_us"] * 1e-6) / 1e9,
                traffic=PF_TRAFFIC,
                mfma_executed_tflops=PF_MFMA_EXECUTED_FLOP / (pf["gpu_us"] * 1e-6) / 1e12,
                mfma_busy=PF_MFMA_BUSY,
                attainable_frac=(tf * 1e12) / min(BF16_PEAK_TFLOPS * 1e12,
                                                  HBM_PEAK_GBS * 1e9 * PF_FLOP / PF_BYTES),
            )
            _log(f"prefill: {pf['ms_per_step']*1e3:.1f} us/step, {tf:.1f} TFLOP/s")

    more = None
    if not args.no_more:
        more = run_more(max(3, args.steps // 5), max(1, args.warmup // 4))

    cpu = None
    if not args.no_cpu:
        _log("cpu baseline: oracle decode on host cores")
        cpu = cpu_baseline()
        _log(f"cpu baseline: {cpu['value']:.1f} tok/s on {cpu['cores']} threads")
        if prefill is not None:
            _log("cpu baseline: oracle chunked prefill on host cores")
            prefill["cpu_baseline"] = cpu_baseline_prefill()
            _log(f"cpu baseline (prefill): {prefill['cpu_baseline']['value']:.1f} tok/s")

    line = dict(
        metric="KDA decode tok/s + state HBM GB/s (B=256); chunk prefill tok/s (T=8k)",
        value=tok_s,
        unit="tok/s",
        n_gpus=1,
        steps=args.steps,
        warmup=args.warmup,
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
        state_hbm_gbs=achieved,
        roofline=dict(
            bound="hbm", achieved=achieved, peak=HBM_PEAK_GBS, unit="GB/s",
            frac=achieved / HBM_PEAK_GBS, traffic=DEC_TRAFFIC,
            kernel="recurrent_kernel<128,32,2,strided rows,decode,bf16,bf16,LOG>",
            algorithmic_bytes_per_launch=DEC_BYTES, kernel_us=dec["kernel_us"],
        ),
        prefill=prefill,
        more_configs=more,
        cpu_baseline=cpu,
    )
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
