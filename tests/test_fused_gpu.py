"""Chunkwise KDA / GLA prefill with the layer prologue fused into the kernel (gdr_chunk_fwd_fused) on the GPU.

The kernel takes q, k before normalisation, the gate's rank-R activations z with decay_proj[1]'s weight and bias and
A_log, and beta logits.  Parity is against the oracle's `layer_prologue` (the reference layer's preparation,
src/layers/kimi_delta_attention.py:45-49, pinned against torch.nn.functional) followed by the fp64 chunkwise
oracle, at the op's tolerance: out max-abs error <= 2e-2 * max|o|, state relative Frobenius error <= 1e-2.  The
oracle sees q, k normalised in fp64 and then rounded to bf16, as the reference's chunk path rounds its inputs
(autocast_inputs, src/ops/utils.py:84-88).
"""

import math

import pytest
import torch

from _helpers import OUT_TOL, STATE_TOL, gdr, oracle, out_error, state_error

pytestmark = pytest.mark.gpu


def _layer_inputs(B, T, H, K, V, R, seed, gate_boost=0.0, varlen=None):
    """Seeded tensors shaped like the KDA layer's pre-op activations (initialisation as in the layer: A_log = log
    U[1, 16], decay bias = softplus^-1(dt), dt log-uniform in [1e-3, 1e-1]); `gate_boost` is added to the bias to
    drive the decay into the exact-diagonal (hot channel) regime."""
    gen = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, H, T, K, generator=gen) * 3.0).bfloat16()
    k = (torch.randn(B, H, T, K, generator=gen) * 3.0).bfloat16()
    v = torch.randn(B, H, T, V, generator=gen).bfloat16()
    z = torch.randn(B, T, R, generator=gen).bfloat16()
    w = (torch.randn(H * K, R, generator=gen) / math.sqrt(R)).bfloat16()
    dt = torch.exp(torch.empty(H * K).uniform_(math.log(1e-3), math.log(1e-1), generator=gen))
    bias = dt + torch.log(-torch.expm1(-dt)) + gate_boost
    a_log = torch.log(torch.empty(H).uniform_(1, 16, generator=gen))
    logits = torch.randn(B, H, T, generator=gen)
    h0 = torch.randn((B if varlen is None else len(varlen) - 1), H, K, V, generator=gen) * 0.02
    return q, k, v, z, w, bias, a_log, logits, h0


def _oracle(variant, q, k, v, z, w, bias, a_log, logits, h0, normalize=True, cu=None):
    qn, kn, gate, beta = oracle.layer_prologue(q, k, z, w, bias, a_log, logits if variant == "kda" else None)
    if normalize:
        q, k = qn.to(torch.bfloat16), kn.to(torch.bfloat16)
    if cu is not None:
        return oracle.varlen(oracle.chunkwise, variant, q, k, v, gate, beta, None, h0, cu)
    return oracle.chunkwise(variant, q, k, v, gate, beta, None, h0)


def _cuda(*xs):
    return [None if x is None else x.cuda() for x in xs]


@pytest.mark.parametrize("shape", [(2, 200, 2, 128, 128, 128), (1, 130, 3, 64, 64, 32), (1, 64, 2, 128, 256, 256),
                                   (1, 130, 3, 64, 64, 192), (1, 100, 2, 128, 128, 96)])
def test_fused_kda_matches_oracle(shape):
    B, T, H, K, V, R = shape
    print(f"fused kda B={B} T={T} H={H} K={K} V={V} R={R}", flush=True)
    q, k, v, z, w, bias, a_log, logits, h0 = _layer_inputs(B, T, H, K, V, R, seed=1)
    with torch.no_grad():
        out, state = gdr.chunk_kimi_delta_attention_fused(*_cuda(q, k, v, z, w, bias, a_log, logits),
                                                          initial_state=h0.cuda(), output_final_state=True)
    ref_o, ref_s = _oracle("kda", q, k, v, z, w, bias, a_log, logits, h0)
    eo, es = out_error(out, ref_o), state_error(state, ref_s)
    print(f"  out err {eo:.2e}  state err {es:.2e}")
    assert out.dtype == torch.bfloat16 and eo <= OUT_TOL and es <= STATE_TOL


def test_fused_equals_unfused_op_on_prepared_inputs():
    """The fused call against the plain op fed the torch-prepared inputs (what the reference layer does)."""
    B, T, H, K, V, R = 2, 256, 4, 128, 128, 128
    q, k, v, z, w, bias, a_log, logits, h0 = _layer_inputs(B, T, H, K, V, R, seed=2)
    qc, kc, vc, zc, wc, bc, ac, lc, hc = _cuda(q, k, v, z, w, bias, a_log, logits, h0)
    with torch.no_grad():
        fused, fs = gdr.chunk_kimi_delta_attention_fused(qc, kc, vc, zc, wc, bc, ac, lc, initial_state=hc,
                                                         output_final_state=True)
        qn = torch.nn.functional.normalize(qc.float(), dim=-1).bfloat16()
        kn = torch.nn.functional.normalize(kc.float(), dim=-1).bfloat16()
        raw = (zc.float() @ wc.float().t() + bc).view(B, T, H, K)
        gate = (-ac.exp()[:, None] * torch.nn.functional.softplus(raw)).transpose(1, 2)
        plain, ps = gdr.chunk_kimi_delta_attention(qn, kn, vc, gate, torch.sigmoid(lc), initial_state=hc,
                                                   output_final_state=True)
    eo, es = out_error(fused, plain), state_error(fs, ps)
    print(f"fused vs unfused: out {eo:.2e} state {es:.2e}")
    assert eo <= 5e-3 and es <= 2e-3


def test_fused_hot_channels():
    """Decay strong enough that in-block spans exceed the exact-diagonal threshold: the fix-up path recomputes
    the normalised q, k and the low-rank gate instead of reading them from memory."""
    B, T, H, K, V, R = 1, 128, 2, 128, 128, 64
    q, k, v, z, w, bias, a_log, logits, h0 = _layer_inputs(B, T, H, K, V, R, seed=3, gate_boost=4.0)
    qn, kn, gate, beta = oracle.layer_prologue(q, k, z, w, bias, a_log, logits)
    spans = -gate.view(B, H, T // 16, 16, K).sum(3)
    assert (spans > 60).any(), "inputs do not reach the hot regime"
    with torch.no_grad():
        out, state = gdr.chunk_kimi_delta_attention_fused(*_cuda(q, k, v, z, w, bias, a_log, logits),
                                                          initial_state=h0.cuda(), output_final_state=True)
    ref_o, ref_s = _oracle("kda", q, k, v, z, w, bias, a_log, logits, h0)
    eo, es = out_error(out, ref_o), state_error(state, ref_s)
    print(f"hot: out err {eo:.2e}  state err {es:.2e}")
    assert eo <= OUT_TOL and es <= STATE_TOL


def test_fused_gla_and_prenormalised_inputs():
    B, T, H, K, V, R = 1, 192, 2, 64, 128, 64
    q, k, v, z, w, bias, a_log, _, h0 = _layer_inputs(B, T, H, K, V, R, seed=4)
    q = torch.nn.functional.normalize(q.float(), dim=-1).bfloat16()  # GLA callers normalise themselves
    k = torch.nn.functional.normalize(k.float(), dim=-1).bfloat16()
    with torch.no_grad():
        out, state = gdr.chunk_gated_linear_attention_fused(*_cuda(q, k, v, z, w, bias, a_log),
                                                            initial_state=h0.cuda(), output_final_state=True)
    ref_o, ref_s = _oracle("gla", q, k, v, z, w, bias, a_log, None, h0, normalize=False)
    eo, es = out_error(out, ref_o), state_error(state, ref_s)
    print(f"gla: out err {eo:.2e}  state err {es:.2e}")
    assert eo <= OUT_TOL and es <= STATE_TOL


def test_fused_varlen_and_layer_layout():
    """Packed sequences through cu_seqlens, with q, k, v, beta given as the layer's transposed [B, T, H, D] views."""
    lens = [70, 1, 129, 64]
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32)
    T, H, K, V, R = int(cu[-1]), 2, 128, 128, 128
    q, k, v, z, w, bias, a_log, logits, h0 = _layer_inputs(1, T, H, K, V, R, seed=5, varlen=cu)
    to_layer = lambda x: x.transpose(1, 2).contiguous().cuda().transpose(1, 2)
    with torch.no_grad():
        out, state = gdr.chunk_kimi_delta_attention_fused(
            to_layer(q), to_layer(k), to_layer(v), z.cuda(), w.cuda(), bias.cuda(), a_log.cuda(),
            logits.transpose(1, 2).contiguous().cuda().transpose(1, 2), initial_state=h0.cuda(),
            output_final_state=True, cu_seqlens=cu.cuda())
    ref_o, ref_s = _oracle("kda", q, k, v, z, w, bias, a_log, logits, h0, cu=cu)
    eo, es = out_error(out, ref_o), state_error(state, ref_s)
    print(f"varlen: out err {eo:.2e}  state err {es:.2e}")
    assert eo <= OUT_TOL and es <= STATE_TOL
