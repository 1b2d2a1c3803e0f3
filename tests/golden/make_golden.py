"""Write the committed golden vectors for BASELINE config 1.

Config 1 (the reference's own CPU-runnable case): fused recurrent KDA on the
CPU torch reference, fp32; varlen ``cu_seqlens = [0, 37, 100]`` (two
sequences), H = 4, K = V = 64, ``scale = K**-0.5``; q, k ~ randn then
L2-normalized over K; v ~ randn; ``g = logsigmoid(randn)`` per channel
``[T, H, K]``; ``beta = sigmoid(randn)`` ``[T, H]``; zero initial state.
Outputs ``o`` ``[T, H, V]`` and final states ``[2, H, K, V]``.

The inputs are drawn on the CPU with a seeded ``torch.Generator`` (seed 1),
stored as fp32; the expected outputs are the oracle's float64 evaluation (the
truth the fp32 paths are measured against) together with its fp32 evaluation.
Sequences use pool slots 1 and 2 of a zero pool (slot 0 is the padding row).

Run from the repository root: ``python tests/golden/make_golden.py``.
"""

import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import kda_ref as R  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "config1.npz")


def config1_inputs():
    gen = torch.Generator().manual_seed(1)
    T, H, D = 100, 4, 64
    cu = [0, 37, 100]
    q = R.l2norm_last(torch.randn(1, T, H, D, generator=gen))
    k = R.l2norm_last(torch.randn(1, T, H, D, generator=gen))
    v = torch.randn(1, T, H, D, generator=gen)
    g = torch.nn.functional.logsigmoid(torch.randn(1, T, H, D, generator=gen))
    beta = torch.sigmoid(torch.randn(1, T, H, generator=gen))
    return dict(q=q, k=k, v=v, g=g, beta=beta, cu_seqlens=torch.tensor(cu, dtype=torch.int32),
                state_indices=torch.tensor([1, 2], dtype=torch.int32), scale=D ** -0.5)


def evaluate(inp, dtype):
    H, D = inp["q"].shape[2], inp["q"].shape[3]
    pool = torch.zeros(3, H, D, D, dtype=dtype)
    o = R.kda_recurrent(
        inp["q"] * inp["scale"], inp["k"], inp["v"], inp["g"], inp["beta"],
        state_pool=pool, state_indices=inp["state_indices"], cu_seqlens=inp["cu_seqlens"],
        dtype=dtype, out_dtype=dtype,
    )
    return o[0], pool[1:3]


def main():
    inp = config1_inputs()
    o64, s64 = evaluate(inp, torch.float64)
    o32, s32 = evaluate(inp, torch.float32)
    np.savez_compressed(
        OUT,
        q=inp["q"][0].numpy(), k=inp["k"][0].numpy(), v=inp["v"][0].numpy(),
        g=inp["g"][0].numpy(), beta=inp["beta"][0].numpy(),
        cu_seqlens=inp["cu_seqlens"].numpy(), state_indices=inp["state_indices"].numpy(),
        scale=np.float64(inp["scale"]),
        o_f64=o64.numpy(), state_f64=s64.numpy(),
        o_f32=o32.numpy(), state_f32=s32.numpy(),
    )
    print("wrote", OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
