"""Writes the golden fixtures in this directory (run from the repository root: python tests/golden/make_golden.py).

The reference ships no golden vectors for this path (its tests draw inputs at run time and compare against fp64
token loops), so these fixtures are this repository's own: seeded inputs of the reference's CPU-runnable
configuration (B=1, T=256, H=2, dk=dv=64, chunk 64; q, k L2-normalised, v ~ N(0, 1), beta = sigmoid(N(0, 1)),
g = -softplus(N(0, 1)), zero initial state) for KDA, smaller cases of the other three variants and of the decode
step, with the expected outputs and final states of the fp64 token recurrence of the oracle.  q, k and v are
stored bf16-rounded (as raw uint16) because that is what the bf16 kernels consume, except in `c1_kda_fp32`: the
reference's CPU-runnable configuration in its own dtype, fp32 q, k, v as drawn (not bf16-representable), with the
fp64 recurrence of those exact values.  Gate, beta, states and outputs are fp32.  The fixtures lock the oracle
against regressions and give the GPU tests inputs that do not depend on the input generator.

Usage: python tests/golden/make_golden.py [name ...]   (no names: write every fixture)
"""

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import importlib  # noqa: E402

workloads = importlib.import_module("gtar-kimik3-public_amd.workloads")
from oracle import gdr_oracle as oracle  # noqa: E402

# name: (variant, B, T, H, dk, dv, seed, state_std, q/k/v dtype)
CASES = {
    "c1_kda": ("kda", 1, 256, 2, 64, 64, 0, None, torch.bfloat16),
    "c1_kda_fp32": ("kda", 1, 256, 2, 64, 64, 0, None, torch.float32),
    "gdn_t96": ("gdn", 1, 96, 2, 64, 64, 1, 0.5, torch.bfloat16),
    "gla_t96": ("gla", 1, 96, 2, 64, 64, 2, 0.5, torch.bfloat16),
    "deltanet_t96": ("deltanet", 1, 96, 2, 64, 64, 3, 0.5, torch.bfloat16),
    "decode_kda": ("kda", 4, 1, 2, 64, 64, 4, 1.0, torch.bfloat16),
}


def bf16_bits(x):
    return x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def main(names):
    for name, (variant, B, T, H, K, V, seed, std, dtype) in CASES.items():
        if names and name not in names:
            continue
        inp = workloads.make_inputs(variant, B, T, H, K, V, seed=seed, state_std=std, dtype=dtype)
        out, state = oracle.recurrence(variant, inp.query, inp.key, inp.value, inp.gate, inp.beta, None,
                                       inp.initial_state, dtype=torch.float64)
        store = bf16_bits if dtype == torch.bfloat16 else (lambda x: x.numpy())
        arrays = {"variant": np.array(variant), "seed": np.array(seed),
                  "query": store(inp.query), "key": store(inp.key), "value": store(inp.value),
                  "out": out.float().numpy(), "final_state": state.float().numpy()}
        for field in ("gate", "beta", "initial_state"):
            x = getattr(inp, field)
            if x is not None:
                arrays[field] = x.float().numpy()
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **arrays)
        print(name, {k: v.shape for k, v in arrays.items()})


if __name__ == "__main__":
    main(sys.argv[1:])
