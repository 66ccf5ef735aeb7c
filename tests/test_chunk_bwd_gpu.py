"""Parity of the chunkwise backward (gdr_chunk_bwd, reached through torch.autograd on the reference op API)
against autograd of the fp64 oracle on the same bf16-rounded inputs.

Mirrors the reference's gradient check (src tests/test_kimi_delta_attention.py:46-53: loss = sum(out * grad_out)
plus a final-state term, gradients for q, k, v, gate, beta and the initial state) over its grid of shapes and gate
strengths (:107-114), for all four variants, plus the layer's transposed layout, partial requires_grad, an absent
initial state, a longer sequence, fp32 values and f16 / fp32 inputs (run on bf16 operands), the reverse scan's
32- and 64-column slices, and the benchmark's training shapes (a few heads against the oracle at the full length).
The op's default training path (gdr_chunk_fwd_train keeping records, states and u; gdr_chunk_bwd_saved) is checked
bit for bit against the recompute path (set_chunk_backward_workspace(False): plain forward, gdr_chunk_bwd).

Tolerance: max|d - d_ref| <= 2e-2 * max|d_ref| for dq, dk, dv, dbeta and d(initial state); 3e-2 for the gate
gradient, a reverse cumulative sum over each chunk of terms that each carry bf16 operand rounding.
"""

import pytest
import torch

from _helpers import CHUNK_FNS, gdr, oracle, workloads

pytestmark = pytest.mark.gpu

GRAD_TOL = 2e-2
GATE_TOL = 3e-2
NAMES = ("dq", "dk", "dv", "dgate", "dbeta", "dh0")


def _leaves(inp, device, requires=None):
    xs = [inp.query, inp.key, inp.value, inp.gate, inp.beta, inp.initial_state]
    out = []
    for i, x in enumerate(xs):
        if x is None:
            out.append(None)
            continue
        x = x.detach().to(device).clone()
        if requires is None or i in requires:
            x.requires_grad_()
        out.append(x)
    return out


def _call(variant, leaves, fn):
    q, k, v, g, b, h0 = leaves
    args = [x for x in (q, k, v, g, b) if x is not None]
    return fn(variant, args, h0)


def _gpu(variant, args, h0):
    return CHUNK_FNS[variant](*args, initial_state=h0, output_final_state=True)


def _cpu(variant, args, h0):
    q, k, v = args[:3]
    rest = args[3:]
    g = rest[0] if oracle_has_gate(variant) else None
    b = rest[-1] if variant != "gla" else None
    return oracle.chunkwise(variant, q, k, v, g, b, None, h0, dtype=torch.float64)


def oracle_has_gate(variant):
    return variant != "deltanet"


def _check(variant, inp, label, requires=None, with_final=True, seed=7):
    gen = torch.Generator().manual_seed(seed)
    B, H, T, K = inp.query.shape
    V = inp.value.shape[-1]
    d_out = torch.randn(B, H, T, V, generator=gen)
    d_final = torch.randn(B, H, K, V, generator=gen) if with_final else None

    gl = _leaves(inp, "cuda", requires)
    out, fin = _call(variant, gl, _gpu)
    loss = (out.float() * d_out.cuda()).sum()
    if with_final:
        loss = loss + (fin * d_final.cuda()).sum()
    g_need = [x for x in gl if x is not None and x.requires_grad]
    g_grads = torch.autograd.grad(loss, g_need)

    # oracle: fp64 leaves from the same (bf16-rounded) values; dO rounded as the kernel receives it (out dtype)
    cl = [None if x is None else x.detach().cpu().double().requires_grad_(x.requires_grad) for x in gl]
    o_ref, s_ref = _call(variant, cl, _cpu)
    d_out_ref = d_out.to(out.dtype).double()
    loss_ref = (o_ref * d_out_ref).sum()
    if with_final:
        loss_ref = loss_ref + (s_ref * d_final.double()).sum()
    c_need = [x for x in cl if x is not None and x.requires_grad]
    c_grads = torch.autograd.grad(loss_ref, c_need)

    names = [n for n, x in zip(NAMES, gl) if x is not None and x.requires_grad]
    report = []
    for name, a, r, x in zip(names, g_grads, c_grads, g_need):
        assert a.dtype == x.dtype and a.shape == x.shape, name
        assert torch.isfinite(a.float()).all(), name
        err = ((a.double().cpu() - r).abs().max() / r.abs().max().clamp_min(1e-30)).item()
        report.append(f"{name} {err:.1e}")
        assert err <= (GATE_TOL if name == "dgate" else GRAD_TOL), (name, err)
    print(f"{label}: " + " ".join(report), flush=True)


CASES = [
    # (B, H, T, K, V, gate_scale, state_std)
    (1, 2, 64, 64, 64, 1.0, 1.0),
    (2, 2, 200, 64, 64, 16.0, 1.0),
    (1, 2, 130, 128, 128, 1.0, 1.0),
    (1, 1, 256, 128, 64, 4.0, 1.0),
    (2, 2, 256, 64, 64, 0.1, 1.0),
    (1, 2, 129, 128, 192, 1.0, 0.02),
]


@pytest.mark.parametrize("variant", oracle.VARIANTS)
@pytest.mark.parametrize("case", CASES, ids=lambda c: "B{}H{}T{}K{}V{}g{}".format(*c[:6]))
def test_chunk_backward_matches_oracle(variant, case):
    B, H, T, K, V, gate_scale, state_std = case
    inp = workloads.make_inputs(variant, B, T, H, K, V, seed=1, gate_scale=gate_scale, state_std=state_std)
    _check(variant, inp, f"{variant} {case}")


def test_chunk_backward_correlated_keys():
    inp = workloads.make_inputs("kda", 2, 256, 4, 128, 128, seed=2, gate_scale=16.0, state_std=1.0)
    gen = torch.Generator().manual_seed(3)
    base = torch.randn(2, 4, 1, 128, generator=gen)
    inp.key = torch.nn.functional.normalize(base + 0.2 * inp.key.float(), dim=-1).to(torch.bfloat16)
    _check("kda", inp, "kda correlated keys")


def test_chunk_backward_layer_layout_and_partial_grads():
    # [B, T, H, D] storage seen through transposed views, as the layer passes it; only some inputs need grad
    inp = workloads.make_inputs("kda", 2, 300, 4, 128, 128, seed=4, state_std=0.5, layer_layout=True)
    assert not inp.query.is_contiguous()
    _check("kda", inp, "kda layer layout")
    _check("kda", inp, "kda grads for v and gate only", requires={2, 3})


def test_chunk_backward_without_initial_or_final_state():
    inp = workloads.make_inputs("gdn", 1, 200, 4, 64, 128, seed=5)
    assert inp.initial_state is None
    _check("gdn", inp, "gdn no h0, no final-state gradient", with_final=False)


def test_chunk_backward_long_sequence():
    inp = workloads.make_inputs("kda", 1, 1024, 2, 128, 128, seed=6, gate_scale=4.0, state_std=1.0)
    _check("kda", inp, "kda T=1024")


def test_chunk_backward_fp32_value():
    """bf16 q, k with an fp32 value (the reference trains on such mixes, casting its dot operands to k.dtype): the
    op runs on bf16 operands and returns the value's gradient in fp32; the output is fp32."""
    inp = workloads.make_inputs("kda", 1, 1024, 2, 128, 128, seed=6, gate_scale=4.0, state_std=1.0)
    inp.value = inp.value.float()
    _check("kda", inp, "kda fp32 value T=1024")


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32], ids=["f16", "fp32"])
@pytest.mark.parametrize("variant", oracle.VARIANTS)
def test_chunk_backward_f16_and_fp32_inputs(variant, dtype):
    """f16 or fp32 q, k, v that need gradients run the chunk forward and backward on bf16 operands (the backward
    kernels are bf16); each gradient comes back in its input's dtype.  The oracle differentiates the inputs' own
    values in fp64, so the check includes the rounding of f16 / fp32 inputs to bf16."""
    inp = workloads.make_inputs(variant, 2, 200, 2, 128, 128, seed=8, dtype=dtype, gate_scale=4.0, state_std=0.5)
    _check(variant, inp, f"{variant} {dtype} inputs")


def _slice_width(pairs, value_dim=128, cus=256):
    """The value columns per reverse-scan workgroup that the library picks on a 256-CU MI355X (scan_slice)."""
    return next((sl for sl in (64, 32) if pairs * (value_dim // sl) >= cus), 16)


@pytest.mark.parametrize("variant", oracle.VARIANTS)
@pytest.mark.parametrize("batch", [4, 8])
def test_chunk_backward_wide_slices(variant, batch):
    """64 and 128 (batch, head) pairs at H=16, d=128: the reverse scan runs 32- and 64-column slices (16-column
    slices run in every smaller case above)."""
    inp = workloads.make_inputs(variant, batch, 150, 16, 128, 128, seed=14, gate_scale=4.0, state_std=0.5)
    _check(variant, inp, f"{variant} B{batch} H16: {_slice_width(batch * 16)}-column reverse-scan slices")


def _check_heads(variant, inp, picks, label, seed=15, gate_tol=GATE_TOL):
    """_check at a full benchmark shape: the GPU differentiates every head; the fp64 oracle differentiates only
    the (batch, head) pairs in `picks` (heads are independent, and the loss is a sum over heads, so those pairs'
    gradients are the same in both)."""
    gen = torch.Generator().manual_seed(seed)
    B, H, T, K = inp.query.shape
    V = inp.value.shape[-1]
    d_out = torch.randn(B, H, T, V, generator=gen).to(torch.bfloat16)
    d_final = torch.randn(B, H, K, V, generator=gen)
    gl = _leaves(inp, "cuda")
    out, fin = _call(variant, gl, _gpu)
    loss = (out.float() * d_out.cuda().float()).sum() + (fin * d_final.cuda()).sum()
    g_need = [x for x in gl if x is not None]
    g_grads = [g.cpu() for g in torch.autograd.grad(loss, g_need)]
    del out, fin, loss
    names = [n for n, x in zip(NAMES, gl) if x is not None]
    for b, h in picks:
        pick = lambda x: None if x is None else x.detach().cpu()[b:b + 1, h:h + 1].double().requires_grad_()
        cl = [pick(x) for x in gl]
        o_ref, s_ref = _call(variant, cl, _cpu)
        loss_ref = (o_ref * d_out[b:b + 1, h:h + 1].double()).sum() + (s_ref * d_final[b:b + 1, h:h + 1].double()).sum()
        c_grads = torch.autograd.grad(loss_ref, [x for x in cl if x is not None])
        report = []
        for name, a, r in zip(names, g_grads, c_grads):
            a = a[b:b + 1, h:h + 1].double()
            assert torch.isfinite(a).all(), name
            err = ((a - r).abs().max() / r.abs().max().clamp_min(1e-30)).item()
            report.append(f"{name} {err:.1e}")
            assert err <= (gate_tol if name == "dgate" else GRAD_TOL), (name, b, h, err)
        print(f"{label} (b={b}, h={h}): " + " ".join(report), flush=True)


def test_chunk_backward_prefill_config():
    """The prefill configuration the training leg of the benchmark times (B=4, T=4096, H=16, d=128, KDA, initial
    state ~ N(0, 0.02)): three (batch, head) pairs against the oracle at the full T, covering the 0.69 GB backward
    workspace's indexing, the 64-step reverse scan and the 32-column slices."""
    print("kda backward B=4 T=4096 H=16 K=V=128", flush=True)
    inp = workloads.make_inputs("kda", 4, 4096, 16, 128, 128, seed=16, state_std=0.02)
    _check_heads("kda", inp, [(0, 0), (1, 9), (3, 15)], "kda backward prefill config")


@pytest.mark.parametrize("variant", ["kda", "gdn"])
def test_chunk_backward_gate_gradient_long_sequence_large_state(variant):
    """The gate gradient's boundary term rowsum(S (x) dS') is formed from the bf16 states and state gradients the
    reverse scan stores (the reference's _chunk_gate_gradient uses fp32 ones, kimi_delta_attention.py:484-490).
    Over a long sequence (T=4096) with a large state (initial state ~ N(0, 1), slow decay), the gate gradient stays
    within 1e-2 of the fp64 oracle, a third of the 3e-2 bound the other cases use."""
    print(f"{variant} backward B=1 T=4096 H=2 K=V=128, state ~ N(0, 1)", flush=True)
    inp = workloads.make_inputs(variant, 1, 4096, 2, 128, 128, seed=18, gate_scale=16.0, state_std=1.0)
    _check_heads(variant, inp, [(0, 0), (0, 1)], f"{variant} long sequence, large state", gate_tol=1e-2)


@pytest.mark.parametrize("variant", ["gdn", "gla", "deltanet"])
def test_chunk_backward_variant_config(variant):
    """The variant sweep shape (B=2, T=8192, H=16, d=128, no initial state): one head against the oracle at the
    full T (128-step reverse scan, 16-column slices)."""
    print(f"{variant} backward B=2 T=8192 H=16 K=V=128", flush=True)
    inp = workloads.make_inputs(variant, 2, 8192, 16, 128, 128, seed=17)
    _check_heads(variant, inp, [(1, 6)], f"{variant} backward variant config")


def _grads(variant, inp, recompute, retain=False):
    gen = torch.Generator().manual_seed(11)
    d_out = torch.randn(inp.value.shape, generator=gen).to(inp.value.dtype).cuda()
    d_final = torch.randn(inp.initial_state.shape, generator=gen).cuda()
    gdr.set_chunk_backward_workspace(not recompute)
    try:
        gl = _leaves(inp, "cuda")
        out, fin = _call(variant, gl, _gpu)
        need = [x for x in gl if x is not None]
        grads = torch.autograd.grad([out, fin], need, [d_out, d_final], retain_graph=retain)
        again = torch.autograd.grad([out, fin], need, [d_out, d_final]) if retain else None
    finally:
        gdr.set_chunk_backward_workspace(None)
    torch.cuda.synchronize()
    return out.detach(), fin.detach(), grads, again


@pytest.mark.parametrize("variant", oracle.VARIANTS)
def test_saved_forward_state_matches_recompute(variant):
    """gdr_chunk_fwd_train + gdr_chunk_bwd_saved against the plain forward + gdr_chunk_bwd: outputs, final state and
    every gradient bit for bit (the same kernels compute them; only who writes the states differs)."""
    inp = workloads.make_inputs(variant, 2, 300, 4, 128, 128, seed=12, gate_scale=4.0, state_std=0.5)
    o1, f1, g1, _ = _grads(variant, inp, recompute=False)
    o2, f2, g2, _ = _grads(variant, inp, recompute=True)
    assert torch.equal(o1, o2) and torch.equal(f1, f2)
    with torch.no_grad():
        gl = _leaves(inp, "cuda", requires=set())
        o3, f3 = _call(variant, gl, _gpu)
    assert torch.equal(o1, o3) and torch.equal(f1, f3)  # the training forward's output is the plain forward's
    for a, b in zip(g1, g2):
        assert torch.equal(a, b)


def test_saved_forward_state_second_backward():
    """retain_graph: the saved workspace serves the first backward; the second recomputes, with equal results."""
    inp = workloads.make_inputs("kda", 1, 200, 2, 64, 128, seed=13, state_std=1.0)
    _, _, g1, g2 = _grads("kda", inp, recompute=False, retain=True)
    for a, b in zip(g1, g2):
        assert torch.equal(a, b)
