"""Shared test helpers: package import (the package directory name is not a Python identifier), the oracle,
and the tolerance checks stated for this op family."""

import importlib
import os
import sys

import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

gdr = importlib.import_module("gtar-kimik3-public_amd")
workloads = importlib.import_module("gtar-kimik3-public_amd.workloads")
lib = importlib.import_module("gtar-kimik3-public_amd._lib")
from oracle import gdr_oracle as oracle  # noqa: E402

# Tolerances for the bf16-in / fp32-state kernels against an fp32-or-better oracle on the same bf16-rounded
# inputs: output max-abs error <= 2e-2 * max|o_ref| and final-state relative Frobenius error <= 1e-2.
OUT_TOL = 2e-2
STATE_TOL = 1e-2

CHUNK_FNS = {
    "kda": gdr.chunk_kimi_delta_attention,
    "gdn": gdr.chunk_gated_deltanet,
    "gla": gdr.chunk_gated_linear_attention,
    "deltanet": gdr.chunk_deltanet,
}
RECURRENT_FNS = {
    "kda": gdr.recurrent_kimi_delta_attention,
    "gdn": gdr.recurrent_gated_deltanet,
    "gla": gdr.recurrent_gated_linear_attention,
    "deltanet": gdr.recurrent_deltanet,
}


def out_error(out, ref):
    """max|out - ref| / max|ref|."""
    ref = ref.double().cpu()
    return ((out.double().cpu() - ref).abs().max() / ref.abs().max().clamp_min(1e-30)).item()


def state_error(state, ref):
    """||state - ref||_F / ||ref||_F."""
    ref = ref.double().cpu()
    return ((state.double().cpu() - ref).norm() / ref.norm().clamp_min(1e-30)).item()


def oracle_args(inp):
    """(q, k, v, gate, beta, h0) of a workloads.Inputs on the CPU, for the oracle."""
    cpu = lambda x: None if x is None else x.detach().cpu()
    return [cpu(x) for x in (inp.query, inp.key, inp.value, inp.gate, inp.beta, inp.initial_state)]
