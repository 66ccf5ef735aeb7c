"""The chunk op's input-dtype rule on the GPU, against the fp64 oracle on the same input values.

The reference's chunk kernels take their dot operands in the input dtype (`.to(k.dtype)`,
src/ops/kimi_delta_attention.py:99-100, :130, :135, :160, :169, :196) after casting q, k, v to the autocast dtype
when autocast is on (src/ops/utils.py:84-88).  Here:
  * f16 q, k, v run the chunk kernels on f16 MFMA operands (f16 records, f16 state operand); the check below also
    shows that the result is closer to the f16 inputs' exact answer than rounding those inputs to bf16 would allow;
  * fp32 q, k, v (the reference's CPU-runnable configuration is fp32) run the fp32 recurrence, every product and sum
    in fp32, held to 1e-4 against fp64, including packed sequences with an empty one;
  * mixed fp32 / bf16 q, k, v run on bf16 operands, bit for bit the bf16 op on bf16-cast inputs;
  * under torch.autocast(bfloat16) the layer's fp32 q, k and bf16 v are cast to bf16 first, exactly as the bf16 op.
(The backward of f16 and fp32 inputs, which runs on bf16 operands, is checked in test_chunk_bwd_gpu.py.)
"""

import pytest
import torch

from _helpers import CHUNK_FNS, OUT_TOL, STATE_TOL, oracle, oracle_args, out_error, state_error, workloads

pytestmark = pytest.mark.gpu

F32_TOL = 1e-4  # fp32 inputs: max-abs output error / max|o| and relative Frobenius state error against fp64


def _run(variant, inp, **kw):
    with torch.no_grad():
        return CHUNK_FNS[variant](*inp.args(), initial_state=inp.initial_state, output_final_state=True, **kw)


F16_CASES = [
    # (B, H, T, K, V, gate_scale, state_std)
    (2, 4, 256, 64, 64, 16.0, 1.0),
    (1, 2, 200, 128, 128, 1.0, 0.02),
    (2, 2, 130, 128, 192, 4.0, 0.5),
    (1, 16, 64, 128, 128, 0.1, 1.0),
]


@pytest.mark.parametrize("variant", oracle.VARIANTS)
@pytest.mark.parametrize("case", F16_CASES, ids=lambda c: "B{}H{}T{}K{}V{}g{}".format(*c[:6]))
def test_chunk_f16_inputs_run_on_f16_operands(variant, case):
    B, H, T, K, V, gate_scale, state_std = case
    inp = workloads.make_inputs(variant, B, T, H, K, V, seed=5, dtype=torch.float16, gate_scale=gate_scale,
                                state_std=state_std, device="cuda")
    out, state = _run(variant, inp)
    torch.cuda.synchronize()
    q, k, v, g, beta, h0 = oracle_args(inp)
    ref_o, ref_s = oracle.chunkwise(variant, q, k, v, g, beta, None, h0)
    eo, es = out_error(out, ref_o), state_error(state, ref_s)
    # the same inputs rounded to bf16: how far a path that rounds f16 to bf16 would start from the exact answer
    bo, bs = oracle.chunkwise(variant, q.bfloat16(), k.bfloat16(), v.bfloat16(), g, beta, None, h0)
    e16o, e16s = out_error(bo, ref_o), state_error(bs, ref_s)
    print(f"f16 {variant} {case}: out err {eo:.2e} state err {es:.2e} (bf16-rounded inputs alone: {e16o:.2e}, "
          f"{e16s:.2e})", flush=True)
    assert out.dtype == torch.float16 and state.dtype == torch.float32
    assert torch.isfinite(out.float()).all() and torch.isfinite(state).all()
    assert eo <= OUT_TOL and es <= STATE_TOL, (eo, es)
    assert es < 0.5 * e16s, (es, e16s)


@pytest.mark.parametrize("variant", oracle.VARIANTS)
@pytest.mark.parametrize("case", [(1, 2, 256, 64, 64, 1.0, None), (2, 3, 130, 128, 128, 16.0, 0.5),
                                  (1, 2, 1, 128, 64, 1.0, 1.0)],
                         ids=lambda c: "B{}H{}T{}K{}V{}".format(*c[:5]))
def test_chunk_fp32_inputs_run_in_fp32(variant, case):
    """The reference's CPU-runnable configuration's recipe (fp32 q, k, v, not bf16-representable)."""
    B, H, T, K, V, gate_scale, state_std = case
    inp = workloads.make_inputs(variant, B, T, H, K, V, seed=6, dtype=torch.float32, gate_scale=gate_scale,
                                state_std=state_std, device="cuda")
    out, state = _run(variant, inp)
    torch.cuda.synchronize()
    q, k, v, g, beta, h0 = oracle_args(inp)
    ref_o, ref_s = oracle.recurrence(variant, q, k, v, g, beta, None, h0)
    eo, es = out_error(out, ref_o), state_error(state, ref_s)
    print(f"fp32 {variant} {case}: out err {eo:.2e} state err {es:.2e}", flush=True)
    assert out.dtype == torch.float32
    assert eo <= F32_TOL and es <= F32_TOL, (eo, es)


def test_chunk_fp32_packed_sequences():
    lengths = [70, 0, 130, 1]
    inp, cu = workloads.make_varlen_inputs("kda", lengths, 2, 64, 64, seed=7, dtype=torch.float32, device="cuda")
    out, state = _run("kda", inp, cu_seqlens=cu)
    torch.cuda.synchronize()
    q, k, v, g, beta, h0 = oracle_args(inp)
    ref_o, ref_s = oracle.varlen(oracle.recurrence, "kda", q, k, v, g, beta, None, h0, cu.cpu())
    assert out_error(out, ref_o) <= F32_TOL and state_error(state, ref_s) <= F32_TOL
    assert torch.equal(state[1], inp.initial_state[1])  # the empty sequence keeps its state


def test_chunk_under_autocast_casts_to_bf16():
    """The KDA layer's call under autocast: q, k come out of F.normalize in fp32, v is bf16.  The op casts them to
    the autocast dtype first (utils.py:84-88), so the result equals the bf16 op on bf16-cast inputs bit for bit."""
    inp = workloads.make_inputs("kda", 2, 200, 4, 128, 128, seed=8, dtype=torch.float32, state_std=0.02,
                                device="cuda")
    value = inp.value.bfloat16()
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        out, state = CHUNK_FNS["kda"](inp.query, inp.key, value, inp.gate, inp.beta, initial_state=inp.initial_state,
                                      output_final_state=True)
    with torch.no_grad():
        out16, state16 = CHUNK_FNS["kda"](inp.query.bfloat16(), inp.key.bfloat16(), value, inp.gate, inp.beta,
                                          initial_state=inp.initial_state, output_final_state=True)
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16 and torch.equal(out, out16) and torch.equal(state, state16)
    q, k, _, g, beta, h0 = oracle_args(inp)
    ref_o, ref_s = oracle.chunkwise("kda", q.bfloat16(), k.bfloat16(), value.cpu(), g, beta, None, h0)
    assert out_error(out, ref_o) <= OUT_TOL and state_error(state, ref_s) <= STATE_TOL


def test_chunk_mixed_fp32_and_bf16_inputs_run_on_bf16():
    """Mixed dtypes without gradients (bf16 q, k with an fp32 value; fp32 q, k with a bf16 value) run the chunk
    kernels on the 16-bit dtype, bit for bit the bf16 op on bf16-cast inputs, with the output in the value's dtype."""
    inp = workloads.make_inputs("kda", 2, 200, 4, 128, 128, seed=9, state_std=0.02, device="cuda")
    ref_o, ref_s = _run("kda", inp)
    with torch.no_grad():
        o1, s1 = CHUNK_FNS["kda"](inp.query, inp.key, inp.value.float(), inp.gate, inp.beta,
                                  initial_state=inp.initial_state, output_final_state=True)
        o2, s2 = CHUNK_FNS["kda"](inp.query.float(), inp.key.float(), inp.value, inp.gate, inp.beta,
                                  initial_state=inp.initial_state, output_final_state=True)
    torch.cuda.synchronize()
    assert o1.dtype == torch.float32 and o2.dtype == torch.bfloat16
    assert torch.equal(o2, ref_o) and torch.equal(s2, ref_s) and torch.equal(s1, ref_s)
    assert torch.equal(o1.bfloat16(), ref_o)
