"""The rest of the fused layer prologue / epilogue on the GPU: the short convolutions of q, k, v inside the fused
preparation kernel (GDR_PRO_CONV) and the RMSNorm x SiLU output epilogue (gdr_norm_gate_fwd).

Convolution parity: against the oracle's `short_convolution` (pinned against nn.Conv1d) composed with its
`layer_prologue` and the fp64 chunkwise oracle, at the op's tolerance (out max-abs error <= 2e-2 * max|o|, state
relative Frobenius error <= 1e-2); the oracle sees the convolution outputs rounded to bf16, as the kernel (and the
reference's bf16 layer) rounds them.  The updated conv states are copies of inputs, so they are compared exactly, and
the fused call must equal, bit for bit, gdr_short_conv_fwd followed by the fused op without the convolution (both
accumulate the W taps in the same order and round once), for the layer's width 4 and the other widths 2 to 8.

Epilogue parity: against the layer's own expression evaluated by PyTorch on the same device
(`weight * (x.float() * rsqrt(mean(x^2) + eps)).to(x.dtype) * F.silu(gate)`), to one rounding of the output dtype,
and against the fp64 oracle (`rms_norm`, silu) to 1e-2 of max |out|.
"""

import math

import pytest
import torch
import torch.nn.functional as F

from _helpers import OUT_TOL, STATE_TOL, gdr, oracle, out_error, state_error

pytestmark = pytest.mark.gpu


def _inputs(B, T, H, K, V, R, seed, n_states, width=4):
    gen = torch.Generator().manual_seed(seed)
    xq = (torch.randn(B, T, H * K, generator=gen) * 2.0).bfloat16()
    xk = (torch.randn(B, T, H * K, generator=gen) * 2.0).bfloat16()
    xv = torch.randn(B, T, H * V, generator=gen).bfloat16()
    bound = 1 / math.sqrt(width)
    cw = [((torch.rand(c, 1, width, generator=gen) * 2 - 1) * bound).bfloat16() for c in (H * K, H * K, H * V)]
    cs = [torch.randn(n_states, c, width - 1, generator=gen).bfloat16() for c in (H * K, H * K, H * V)]
    z = torch.randn(B, T, R, generator=gen).bfloat16()
    w = (torch.randn(H * K, R, generator=gen) / math.sqrt(R)).bfloat16()
    dt = torch.exp(torch.empty(H * K).uniform_(math.log(1e-3), math.log(1e-1), generator=gen))
    bias = dt + torch.log(-torch.expm1(-dt))
    a_log = torch.log(torch.empty(H).uniform_(1, 16, generator=gen))
    logits = torch.randn(B, H, T, generator=gen)
    h0 = torch.randn(n_states, H, K, V, generator=gen) * 0.02
    return xq, xk, xv, cw, cs, z, w, bias, a_log, logits, h0


def _heads(x, H):  # [B, T, H*D] -> the op's [B, H, T, D] view
    B, T, C = x.shape
    return x.view(B, T, H, C // H).transpose(1, 2)


def _oracle(H, xq, xk, xv, cw, cs, z, w, bias, a_log, logits, h0, cu=None):
    conv = [oracle.short_convolution(x, wt, st, cu) for x, wt, st in zip((xq, xk, xv), cw, cs)]
    q, k, v = (_heads(c.to(torch.bfloat16), H) for c, _ in conv)
    qn, kn, gate, beta = oracle.layer_prologue(q, k, z, w, bias, a_log, logits)
    q, k = qn.to(torch.bfloat16), kn.to(torch.bfloat16)
    if cu is not None:
        o, s = oracle.varlen(oracle.chunkwise, "kda", q, k, v, gate, beta, None, h0, cu)
    else:
        o, s = oracle.chunkwise("kda", q, k, v, gate, beta, None, h0)
    return o, s, [st.to(torch.bfloat16) for _, st in conv]


def _run(H, xq, xk, xv, cw, cs, z, w, bias, a_log, logits, h0, cu=None, with_states=True):
    cuda = lambda t: t.cuda()
    states = [cuda(s) for s in cs] if with_states else None
    with torch.no_grad():
        out, fs = gdr.chunk_kimi_delta_attention_fused(
            _heads(cuda(xq), H), _heads(cuda(xk), H), _heads(cuda(xv), H), cuda(z), cuda(w), cuda(bias),
            cuda(a_log), cuda(logits), initial_state=cuda(h0), output_final_state=True,
            cu_seqlens=None if cu is None else cuda(cu), conv_weights=[cuda(x) for x in cw], conv_states=states)
    return out, fs, states


@pytest.mark.parametrize("width", [4, 2, 3, 8])
@pytest.mark.parametrize("shape", [(2, 200, 2, 128, 128, 128), (1, 130, 3, 64, 64, 32), (1, 3, 2, 128, 128, 64)])
def test_fused_conv_matches_oracle(shape, width):
    B, T, H, K, V, R = shape
    print(f"fused conv kda B={B} T={T} H={H} K={K} V={V} R={R} W={width}", flush=True)
    xq, xk, xv, cw, cs, z, w, bias, a_log, logits, h0 = _inputs(B, T, H, K, V, R, seed=1, n_states=B, width=width)
    out, fs, states = _run(H, xq, xk, xv, cw, cs, z, w, bias, a_log, logits, h0)
    ref_o, ref_s, ref_cs = _oracle(H, xq, xk, xv, cw, cs, z, w, bias, a_log, logits, h0)
    eo, es = out_error(out, ref_o), state_error(fs, ref_s)
    print(f"  out err {eo:.2e}  state err {es:.2e}")
    assert eo <= OUT_TOL and es <= STATE_TOL
    for got, want in zip(states, ref_cs):
        assert torch.equal(got.cpu(), want)


@pytest.mark.parametrize("width", [4, 2, 6, 8])
def test_fused_conv_packed_sequences(width):
    """cu_seqlens: every sequence starts its convolutions from its own state (lengths around the W - 1-row halo and
    the 64-row chunk edges, and sequences shorter than the state)."""
    lens = [1, 2, 3, 4, 5, 7, 63, 64, 65, 130]
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32)
    H, K, V, R = 2, 128, 128, 64
    xq, xk, xv, cw, cs, z, w, bias, a_log, logits, h0 = _inputs(1, int(cu[-1]), H, K, V, R, seed=3,
                                                                  n_states=len(lens), width=width)
    out, fs, states = _run(H, xq, xk, xv, cw, cs, z, w, bias, a_log, logits, h0, cu=cu)
    ref_o, ref_s, ref_cs = _oracle(H, xq, xk, xv, cw, cs, z, w, bias, a_log, logits, h0, cu=cu)
    eo, es = out_error(out, ref_o), state_error(fs, ref_s)
    print(f"packed: out err {eo:.2e}  state err {es:.2e}", flush=True)
    assert eo <= OUT_TOL and es <= STATE_TOL
    for got, want in zip(states, ref_cs):
        assert torch.equal(got.cpu(), want)


@pytest.mark.parametrize("width", [4, 3, 8])
def test_fused_conv_equals_separate_convolutions(width):
    """Bit-identical to gdr_short_conv_fwd on q, k, v followed by the fused op without the convolution, with and
    without conv states (zero history)."""
    B, T, H, K, V, R = 2, 300, 4, 128, 128, 128
    xq, xk, xv, cw, cs, z, w, bias, a_log, logits, h0 = _inputs(B, T, H, K, V, R, seed=4, n_states=B, width=width)
    for with_states in (True, False):
        out, fs, _ = _run(H, xq, xk, xv, cw, cs, z, w, bias, a_log, logits, h0, with_states=with_states)
        with torch.no_grad():
            conv = [gdr.short_convolution(x.cuda(), wt.cuda(), st.cuda() if with_states else None)
                    for x, wt, st in zip((xq, xk, xv), cw, cs)]
            ref, rs = gdr.chunk_kimi_delta_attention_fused(
                *(_heads(c, H) for c in conv), z.cuda(), w.cuda(), bias.cuda(), a_log.cuda(), logits.cuda(),
                initial_state=h0.cuda(), output_final_state=True)
        assert torch.equal(out, ref) and torch.equal(fs, rs), with_states


def _norm_gate_ref(x, gate, weight, eps):
    """The layer's expression in PyTorch (src/layers/kimi_delta_attention.py:58-59, src/layers/rmsnorm.py:11-16)."""
    xf = x.float()
    normed = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype)
    return weight * normed * F.silu(gate)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("weight_f32", [True, False])
@pytest.mark.parametrize("V", [64, 128, 192, 256])
def test_norm_gate_matches_layer_expression(dtype, weight_f32, V):
    B, H, T, eps = 2, 3, 77, 1e-6
    gen = torch.Generator().manual_seed(5)
    o = (torch.randn(B, H, T, V, generator=gen) * 0.3).to(dtype)  # the op's output layout
    gate = (torch.randn(B, T, H, V, generator=gen) * 2).to(dtype)
    weight = (1 + 0.1 * torch.randn(V, generator=gen)).to(torch.float32 if weight_f32 else dtype)
    oc, gc, wc = o.cuda(), gate.cuda(), weight.cuda()
    with torch.no_grad():
        got = gdr.output_norm_gate(oc.transpose(1, 2), gc, wc, eps)
        want = _norm_gate_ref(oc.transpose(1, 2), gc, wc, eps)
    assert got.dtype == want.dtype and got.shape == want.shape
    ulp = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11, torch.float32: 2.0 ** -22}[dtype]
    scale = want.float().abs().max().item()
    err = (got.float() - want.float()).abs().max().item()
    print(f"norm-gate {dtype} w32={weight_f32} V={V}: max err {err:.2e} (max |out| {scale:.2f})", flush=True)
    assert err <= 4 * ulp * scale
    exact = oracle.rms_norm(o.transpose(1, 2), weight, eps) * F.silu(gate.double())
    assert (got.cpu().double() - exact).abs().max().item() <= 1e-2 * exact.abs().max().item()
