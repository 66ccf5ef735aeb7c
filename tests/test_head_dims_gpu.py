"""Key dims beyond the chunk kernels' 64 and 128, on the GPU, against the fp64 oracle.

The reference's recurrent kernel takes any power-of-two head dim (src/ops/kimi_delta_attention.py:46) and its chunk
kernels any multiple of 64 (:88, :126).  Here the recurrent kernel is built for key dims 32, 64, 128, 192 and 256
(192 and 256 on 32-column state slices, 32 on both slice widths), and the chunk op runs key dims 32, 192 and 256 on
its sequential path: the recurrent kernel over every token of each (packed) sequence, everything in fp32.  Inputs
are bf16 (read exactly) or fp32, so the results are held to 1e-4 of the fp64 recurrence on the same values (max-abs
output error over max |o| and relative Frobenius state error), plus the one rounding of a bf16 output (2^-8).  These key dims have no chunk backward: a call that
needs gradients says so.
"""

import pytest
import torch

from _helpers import CHUNK_FNS, RECURRENT_FNS, oracle, oracle_args, out_error, state_error, workloads

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _check(fn, variant, inp, label, **kw):
    with torch.no_grad():
        out, state = fn(*inp.args(), initial_state=inp.initial_state, output_final_state=True, **kw)
    torch.cuda.synchronize()
    q, k, v, g, beta, h0 = oracle_args(inp)
    if "cu_seqlens" in kw:
        ref_o, ref_s = oracle.varlen(oracle.recurrence, variant, q, k, v, g, beta, None, h0, kw["cu_seqlens"].cpu())
    else:
        ref_o, ref_s = oracle.recurrence(variant, q, k, v, g, beta, None, h0)
    eo, es = out_error(out, ref_o), state_error(state, ref_s)
    print(f"{label}: out err {eo:.2e} state err {es:.2e}", flush=True)
    assert out.dtype == inp.value.dtype and state.dtype == torch.float32
    out_tol = TOL if out.dtype == torch.float32 else TOL + 2.0 ** -8
    assert eo <= out_tol and es <= TOL, (eo, es)


@pytest.mark.parametrize("variant", oracle.VARIANTS)
@pytest.mark.parametrize("shape", [(2, 4, 1, 32, 64), (1, 2, 19, 32, 128), (64, 16, 1, 32, 128),
                                   (2, 2, 9, 192, 96), (3, 2, 1, 256, 128), (1, 2, 11, 256, 256)],
                         ids=lambda s: "B{}H{}T{}K{}V{}".format(*s))
def test_recurrent_key_dims(variant, shape):
    """B=64, H=16, V=128 at K=32 reaches the 128-column slices (1,024 or more of them)."""
    B, H, T, K, V = shape
    inp = workloads.make_inputs(variant, B, T, H, K, V, seed=3, state_std=0.5, device="cuda")
    _check(RECURRENT_FNS[variant], variant, inp, f"recurrent {variant} {shape}")


@pytest.mark.parametrize("variant", oracle.VARIANTS)
@pytest.mark.parametrize("K", [32, 192, 256])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
def test_chunk_key_dims_run_sequential_path(variant, K, dtype):
    inp = workloads.make_inputs(variant, 2, 150, 2, K, 64, seed=4, dtype=dtype, gate_scale=4.0, state_std=0.5,
                                device="cuda", layer_layout=True)
    _check(CHUNK_FNS[variant], variant, inp, f"chunk {variant} K={K} {dtype}")


@pytest.mark.parametrize("K", [64, 256])
def test_chunk_sequential_path_packed_sequences(K):
    """Packed sequences (an empty one included) on the sequential path, one launch for all of them: fp32 q, k, v
    at K=64, bf16 at K=256."""
    lengths = [70, 0, 130, 1, 65]
    dtype = torch.float32 if K == 64 else torch.bfloat16
    inp, cu = workloads.make_varlen_inputs("kda", lengths, 2, K, 64, seed=5, dtype=dtype, device="cuda")
    _check(CHUNK_FNS["kda"], "kda", inp, f"chunk kda packed K={K} {dtype}", cu_seqlens=cu)


def test_chunk_key_dim_without_backward_says_so():
    inp = workloads.make_inputs("kda", 1, 64, 2, 256, 64, seed=6, device="cuda")
    q = inp.query.detach().clone().requires_grad_()
    with pytest.raises(NotImplementedError, match="key dim 256"):
        CHUNK_FNS["kda"](q, inp.key, inp.value, inp.gate, inp.beta)
