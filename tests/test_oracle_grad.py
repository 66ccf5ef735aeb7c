"""Pins the gradient oracle the chunkwise-backward parity tests use: autograd of the fp64 oracle.

* `oracle.recurrence` (the token-by-token definition of each variant) is differentiated by torch autograd; a
  central finite-difference check (torch.autograd.gradcheck) on tiny inputs pins those gradients for every
  input the reference backward returns (q, k, v, gate, beta, initial state; src/ops/kimi_delta_attention.py:614-622).
* `oracle.chunkwise` (what the GPU tests differentiate, because it is fast at test sizes) must give the same
  gradients as the recurrence: the chunkwise form is an identity of the recurrence, so its gradients are too,
  at every chunk size.
"""

import pytest
import torch

from _helpers import oracle

VARIANTS = oracle.VARIANTS


def _inputs(variant, B, H, T, K, V, seed=0):
    gen = torch.Generator().manual_seed(seed)
    rn = lambda *s: torch.randn(*s, generator=gen, dtype=torch.float64)
    q = torch.nn.functional.normalize(rn(B, H, T, K), dim=-1)
    k = torch.nn.functional.normalize(rn(B, H, T, K), dim=-1)
    v = rn(B, H, T, V)
    g = None
    if variant in ("kda", "gla"):
        g = torch.nn.functional.logsigmoid(rn(B, H, T, K))
    elif variant == "gdn":
        g = torch.nn.functional.logsigmoid(rn(B, H, T))
    beta = torch.sigmoid(rn(B, H, T)) if variant != "gla" else None
    h0 = rn(B, H, K, V)
    return [q, k, v, g, beta, h0]


def _loss_fn(variant, fn, d_out, d_final, **kw):
    def f(q, k, v, g, beta, h0):
        o, s = fn(variant, q, k, v, g, beta, None, h0, dtype=torch.float64, **kw)
        return (o * d_out).sum() + (s * d_final).sum()
    return f


@pytest.mark.parametrize("variant", VARIANTS)
def test_recurrence_gradients_match_finite_differences(variant):
    ins = _inputs(variant, 1, 1, 5, 3, 2)
    gen = torch.Generator().manual_seed(1)
    d_out = torch.randn(1, 1, 5, 2, generator=gen, dtype=torch.float64)
    d_final = torch.randn(1, 1, 3, 2, generator=gen, dtype=torch.float64)
    f = _loss_fn(variant, oracle.recurrence, d_out, d_final)
    present = [i for i, x in enumerate(ins) if x is not None]
    leaves = [ins[i].clone().requires_grad_() for i in present]

    def g(*xs):
        full = list(ins)
        for i, x in zip(present, xs):
            full[i] = x
        return f(*full)

    assert torch.autograd.gradcheck(g, leaves, eps=1e-6, atol=1e-7, rtol=1e-5)


@pytest.mark.parametrize("variant", VARIANTS)
@pytest.mark.parametrize("chunk", [8, 64])
def test_chunkwise_gradients_equal_recurrence_gradients(variant, chunk):
    ins = _inputs(variant, 1, 2, 37, 8, 6, seed=3)
    gen = torch.Generator().manual_seed(4)
    d_out = torch.randn(1, 2, 37, 6, generator=gen, dtype=torch.float64)
    d_final = torch.randn(1, 2, 8, 6, generator=gen, dtype=torch.float64)
    grads = []
    for fn, kw in ((oracle.recurrence, {}), (oracle.chunkwise, {"chunk_size": chunk})):
        leaves = [None if x is None else x.clone().requires_grad_() for x in ins]
        loss = _loss_fn(variant, fn, d_out, d_final, **kw)(*leaves)
        grads.append(torch.autograd.grad(loss, [x for x in leaves if x is not None]))
    for a, b in zip(*grads):
        assert ((a - b).abs().max() / b.abs().max()).item() < 1e-10
