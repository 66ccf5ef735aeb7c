"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py): seeded inputs with the fp64
oracle's expected outputs and final states.  On the CPU they lock the oracle and the input recipe against
regressions and check the reference's CPU path restatement (`kda_reference`, fp32) against fp64; on the GPU the
chunk and recurrent kernels are held to the stated tolerance against them."""

import glob
import os

import numpy as np
import pytest
import torch

from _helpers import CHUNK_FNS, OUT_TOL, RECURRENT_FNS, ROOT, STATE_TOL, oracle, out_error, state_error, workloads

# the op fixtures (stack_reference.npz, the reference's hybrid blocks, is checked in test_oracle.py)
FIXTURES = sorted(p for p in glob.glob(os.path.join(ROOT, "tests", "golden", "*.npz"))
                  if not p.endswith("stack_reference.npz"))
NAMES = [os.path.basename(p)[:-4] for p in FIXTURES]


def _load(name):
    with np.load(os.path.join(ROOT, "tests", "golden", name + ".npz")) as f:
        data = {k: f[k] for k in f.files}
    fx = {"variant": str(data.pop("variant")), "seed": int(data.pop("seed"))}
    for k in ("query", "key", "value"):
        x = data.pop(k)
        fx[k] = torch.from_numpy(x.copy()) if x.dtype == np.float32 else \
            torch.from_numpy(x.view(np.int16).copy()).view(torch.bfloat16)
    for k, v in data.items():
        fx[k] = torch.from_numpy(v)
    return fx


def _args(fx, device="cpu"):
    move = lambda x: None if x is None else x.to(device)
    return [move(fx.get(k)) for k in ("query", "key", "value", "gate", "beta", "initial_state")]


def test_fixtures_present():
    assert {"c1_kda", "c1_kda_fp32", "gdn_t96", "gla_t96", "deltanet_t96", "decode_kda"} <= set(NAMES)


def _tolerances(fx):
    """fp32 q, k, v run every product in fp32 (the exact path): held to 1e-4; bf16 inputs to the stated bound."""
    return (1e-4, 1e-4) if fx["query"].dtype == torch.float32 else (OUT_TOL, STATE_TOL)


@pytest.mark.parametrize("name", NAMES)
def test_fixture_inputs_follow_the_recipe(name):
    """The stored inputs are exactly what the seeded generator draws (q, k, v bf16-rounded, or fp32 as drawn)."""
    fx = _load(name)
    B, H, T, K = fx["query"].shape
    inp = workloads.make_inputs(fx["variant"], B, T, H, K, fx["value"].shape[-1], seed=fx["seed"],
                                dtype=fx["query"].dtype)
    for k in ("query", "key", "value"):
        assert torch.equal(getattr(inp, k), fx[k]), k
    for k in ("gate", "beta"):
        if k in fx:
            assert torch.equal(getattr(inp, k), fx[k]), k


@pytest.mark.parametrize("name", NAMES)
def test_oracle_reproduces_fixture(name):
    fx = _load(name)
    q, k, v, g, b, h0 = _args(fx)
    for fn in (oracle.recurrence, oracle.chunkwise):
        out, state = fn(fx["variant"], q, k, v, g, b, None, h0)
        assert out_error(out.float(), fx["out"].double()) < 1e-6, fn.__name__
        assert state_error(state.float(), fx["final_state"].double()) < 1e-6, fn.__name__


@pytest.mark.parametrize("name", ["c1_kda", "c1_kda_fp32"])
def test_reference_cpu_path_on_config1(name):
    """The reference's fp32 CPU loop on the reference's CPU-runnable configuration agrees with fp64."""
    fx = _load(name)
    q, k, v, g, b, h0 = _args(fx)
    out, state = oracle.kda_reference(q.float(), k.float(), v.float(), g, b, None, h0)
    assert out.dtype == torch.float32 and state.dtype == torch.float32
    assert out_error(out, fx["out"].double()) < 1e-5 and state_error(state, fx["final_state"].double()) < 1e-5


def test_fp32_fixture_is_not_bf16_representable():
    """c1_kda_fp32 holds the fp32 values themselves: rounding them to bf16 changes them and moves the fp64 result
    by more than the fp32 path's tolerance, so a path that rounds fp32 input to bf16 fails its GPU check."""
    fx = _load("c1_kda_fp32")
    q, k, v, g, b, h0 = _args(fx)
    assert not torch.equal(q.bfloat16().float(), q)
    out16, _ = oracle.recurrence("kda", q.bfloat16(), k.bfloat16(), v.bfloat16(), g, b, None, h0)
    assert out_error(out16.float(), fx["out"].double()) > 1e-3


@pytest.mark.gpu
@pytest.mark.parametrize("name", NAMES)
def test_kernels_match_fixture(name):
    fx = _load(name)
    variant = fx["variant"]
    args = [x for x in _args(fx, "cuda")[:5] if x is not None]
    h0 = None if "initial_state" not in fx else fx["initial_state"].cuda()
    modes = [("recurrent", RECURRENT_FNS)] + ([] if name.startswith("decode") else [("chunk", CHUNK_FNS)])
    for mode, fns in modes:
        with torch.no_grad():
            out, state = fns[variant](*args, initial_state=h0, output_final_state=True)
        torch.cuda.synchronize()
        eo, es = out_error(out, fx["out"].double()), state_error(state, fx["final_state"].double())
        print(f"golden {name} {mode}: out err {eo:.2e} state err {es:.2e}", flush=True)
        out_tol, state_tol = _tolerances(fx)
        assert out.dtype == fx["value"].dtype and eo <= out_tol and es <= state_tol, (mode, eo, es)
