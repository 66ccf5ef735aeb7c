"""Parity of the recurrent (decode) HIP kernels against the oracle, through the reference op API and libgdr.so.

Tolerance: out max-abs error <= 2e-2 * max|o_ref| and final-state relative Frobenius error <= 1e-2 against the
fp64 token recurrence on the same bf16-rounded inputs (the recurrent kernels keep everything in fp32, so the
observed errors are far smaller; they are printed).
"""

import pytest
import torch

from _helpers import OUT_TOL, RECURRENT_FNS, STATE_TOL, lib, oracle, oracle_args, out_error, state_error, workloads

pytestmark = pytest.mark.gpu

SHAPES = [
    # (B, H, T, K, V)
    (2, 4, 1, 128, 128),
    (3, 2, 1, 64, 64),
    (1, 2, 37, 64, 128),
    (2, 3, 9, 128, 64),
    (1, 1, 4, 128, 256),
]


def _run(variant, inp, **kw):
    fn = RECURRENT_FNS[variant]
    with torch.no_grad():
        return fn(*inp.args(), initial_state=inp.initial_state, output_final_state=True, **kw)


@pytest.mark.parametrize("variant", oracle.VARIANTS)
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("layer_layout", [False, True])
def test_recurrent_matches_oracle(variant, shape, layer_layout):
    B, H, T, K, V = shape
    print(f"recurrent {variant} B={B} H={H} T={T} K={K} V={V} layer_layout={layer_layout}", flush=True)
    inp = workloads.make_inputs(variant, B, T, H, K, V, seed=1, state_std=0.5, device="cuda",
                                layer_layout=layer_layout)
    out, state = _run(variant, inp)
    q, k, v, g, beta, h0 = oracle_args(inp)
    ref_o, ref_s = oracle.recurrence(variant, q, k, v, g, beta, None, h0)
    assert out.dtype == inp.value.dtype and state.dtype == torch.float32
    eo, es = out_error(out, ref_o), state_error(state, ref_s)
    print(f"  out err {eo:.2e}  state err {es:.2e}")
    assert eo <= OUT_TOL and es <= STATE_TOL


@pytest.mark.parametrize("variant", oracle.VARIANTS)
def test_recurrent_fp32_query_key_bf16_value(variant):
    """In decode the layer's q, k come out of F.normalize in fp32 while v is bf16 (mixed dtypes)."""
    inp = workloads.make_inputs(variant, 2, 1, 4, 128, 128, seed=2, state_std=0.02, device="cuda")
    inp.query, inp.key = inp.query.float(), inp.key.float()
    out, state = _run(variant, inp)
    q, k, v, g, beta, h0 = oracle_args(inp)
    ref_o, ref_s = oracle.recurrence(variant, q, k, v, g, beta, None, h0)
    assert out.dtype == torch.bfloat16
    assert out_error(out, ref_o) <= OUT_TOL and state_error(state, ref_s) <= STATE_TOL


def test_recurrent_decode_config_full_size():
    """Benchmark decode shape: 256 sequences x 16 heads, 128 x 128 fp32 state ~ N(0, 0.02)."""
    print("recurrent kda decode B=256 H=16 K=V=128", flush=True)
    inp = workloads.decode_inputs("kda", 256, 16, 128, 128, seed=3, device="cuda")
    h0 = workloads.decode_state(256, 16, 128, 128, std=0.02, seed=4, device="cuda")
    with torch.no_grad():
        out, state = RECURRENT_FNS["kda"](*inp.args(), initial_state=h0, output_final_state=True)
    q, k, v, g, beta, _ = oracle_args(inp)
    ref_o, ref_s = oracle.recurrence("kda", q, k, v, g, beta, None, h0.cpu(), dtype=torch.float64)
    eo, es = out_error(out, ref_o), state_error(state, ref_s)
    print(f"  out err {eo:.2e}  state err {es:.2e}")
    assert eo <= OUT_TOL and es <= STATE_TOL


def test_recurrent_reference_semantics():
    """Inputs are not modified, the final state is a fresh tensor, the default state is zero, and without
    output_final_state only the output is returned."""
    inp = workloads.make_inputs("kda", 2, 3, 2, 64, 64, seed=5, state_std=1.0, device="cuda")
    before = [x.clone() for x in inp.args()] + [inp.initial_state.clone()]
    out, state = _run("kda", inp)
    after = inp.args() + [inp.initial_state]
    for a, b in zip(before, after):
        assert torch.equal(a, b)
    assert state.data_ptr() != inp.initial_state.data_ptr()
    with torch.no_grad():
        only = RECURRENT_FNS["kda"](*inp.args(), initial_state=inp.initial_state)
    assert isinstance(only, torch.Tensor) and torch.equal(only, out)
    with torch.no_grad():
        zero_a = RECURRENT_FNS["kda"](*inp.args())
        zero_b = RECURRENT_FNS["kda"](*inp.args(), initial_state=torch.zeros_like(inp.initial_state))
    assert torch.equal(zero_a, zero_b)


def test_recurrent_state_passing_matches_single_call():
    inp = workloads.make_inputs("kda", 1, 20, 2, 128, 128, seed=6, state_std=0.1, device="cuda")
    full_o, full_s = _run("kda", inp)
    o_parts = []
    state = inp.initial_state
    for t in range(20):
        sl = slice(t, t + 1)
        with torch.no_grad():
            o, state = RECURRENT_FNS["kda"](inp.query[:, :, sl], inp.key[:, :, sl], inp.value[:, :, sl],
                                            inp.gate[:, :, sl], inp.beta[:, :, sl], initial_state=state,
                                            output_final_state=True)
        o_parts.append(o)
    torch.testing.assert_close(torch.cat(o_parts, 2).float(), full_o.float(), rtol=0, atol=1e-2)
    torch.testing.assert_close(state, full_s, rtol=1e-5, atol=1e-5)


def test_library_rejects_bad_arguments():
    inp = workloads.make_inputs("kda", 1, 1, 1, 96, 64, seed=0, device="cuda")
    with pytest.raises(RuntimeError, match="key dim 96"):
        _run("kda", inp)
