"""Gradients of the causal grouped-query attention (gdr_attention_bwd through `flash_attention` under autograd), on
the GPU.

Parity follows the reference's own check (tests/test_flash_attention_2.py:36-53): dq, dk and dv of the kernel
against the exact result (here autograd of the fp64 oracle, `oracle.causal_attention`) must have a max abs error of
at most 2x that of PyTorch's SDPA run in the same half dtype, plus 1e-4.  The SDPA baseline runs on the CPU
(half-precision attention's math path is kept off this GPU), on the same inputs and output gradient.  Packed
sequences are held to the same exact result per sequence, and must equal each sequence run on its own bit for bit.
"""

import pytest
import torch
import torch.nn.functional as F

from _helpers import gdr, oracle

pytestmark = pytest.mark.gpu


def _inputs(B, H, Hkv, T, D, dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    shape_q, shape_kv = (B, H, T, D), (B, Hkv, T, D)
    q, k, v = (torch.randn(s, generator=gen).to(dtype) for s in (shape_q, shape_kv, shape_kv))
    d_out = torch.randn(shape_q, generator=gen).to(dtype)
    return q, k, v, d_out


def _grads(fn, q, k, v, d_out, **kw):
    leaves = [x.detach().clone().requires_grad_() for x in (q, k, v)]
    out = fn(*leaves, **kw)
    return [out.detach()] + list(torch.autograd.grad(out, leaves, d_out.to(out.dtype)))


def _exact(q, k, v, d_out, scale=None, cu=None):
    return _grads(lambda a, b, c: oracle.causal_attention(a, b, c, scale, cu), q.double(), k.double(), v.double(),
                  d_out.double())


def _kernel(q, k, v, d_out, **kw):
    got = _grads(lambda a, b, c: gdr.flash_attention(a, b, c, **kw), q.cuda(), k.cuda(), v.cuda(), d_out.cuda())
    return [x.cpu() for x in got]


def _errors(got, exact):
    return [(a.double() - b).abs().max().item() for a, b in zip(got, exact)]


NAMES = ("out", "dq", "dk", "dv")


@pytest.mark.parametrize("shape", [(1, 8, 8, 128, 64), (2, 8, 8, 512, 64), (2, 8, 2, 1000, 128), (3, 12, 4, 777, 64),
                                   (1, 32, 8, 256, 128), (1, 4, 1, 64, 64), (1, 2, 2, 1, 128), (1, 4, 2, 65, 128)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_attention_gradients_within_reference_bar(shape, dtype):
    B, H, Hkv, T, D = shape
    print(f"attention backward {shape} {dtype}", flush=True)
    q, k, v, d_out = _inputs(B, H, Hkv, T, D, dtype, seed=11)
    exact = _exact(q, k, v, d_out)
    got = _kernel(q, k, v, d_out)
    sdpa = _grads(lambda a, b, c: F.scaled_dot_product_attention(a, b, c, is_causal=True, enable_gqa=True), q, k, v,
                  d_out)
    err, base = _errors(got, exact), _errors(sdpa, exact)
    print("  " + " | ".join(f"{n} {e:.2e}/{b:.2e}" for n, e, b in zip(NAMES, err, base)))
    for i, name in enumerate(NAMES):
        assert got[i].dtype == dtype, name
        assert err[i] <= 2 * base[i] + 1e-4, (name, err[i], base[i])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_attention_gradients_sharp_rows(dtype):
    """Sharp softmax rows (scale 0.5 at D = 64) over keys whose norms rise 8x along the sequence: the forward's
    exponent base moves many times, and the backward's probabilities come from the row log-sum-exp it saved."""
    B, H, Hkv, T, D = 1, 4, 2, 700, 64
    q, k, v, d_out = _inputs(B, H, Hkv, T, D, torch.float32, seed=12)
    k = k * torch.linspace(0.25, 2.0, T).view(1, 1, T, 1)
    q, k, v, d_out = (x.to(dtype) for x in (q, k, v, d_out))
    exact = _exact(q, k, v, d_out, 0.5)
    got = _kernel(q, k, v, d_out, softmax_scale=0.5)
    sdpa = _grads(lambda a, b, c: F.scaled_dot_product_attention(a, b, c, is_causal=True, enable_gqa=True, scale=0.5),
                  q, k, v, d_out)
    err, base = _errors(got, exact), _errors(sdpa, exact)
    print("  " + " | ".join(f"{n} {e:.2e}/{b:.2e}" for n, e, b in zip(NAMES, err, base)))
    for i, name in enumerate(NAMES):
        assert torch.isfinite(got[i]).all() and err[i] <= 2 * base[i] + 1e-4, (name, err[i], base[i])


def test_attention_gradients_packed_sequences_and_layer_layout():
    """cu_seqlens (lengths around the 128-row query block and 64-row key block edges, a single token) with q, k, v
    as the layer's transposed [B, T, H, D] views: each sequence's gradients against its exact result, and the packed
    call equal to each sequence run alone, bit for bit."""
    lens = [1, 63, 64, 65, 127, 128, 129, 300]
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32)
    T, H, Hkv, D = int(cu[-1]), 4, 2, 128
    q, k, v, d_out = _inputs(1, H, Hkv, T, D, torch.bfloat16, seed=13)
    layer = lambda x: x.transpose(1, 2).contiguous().cuda().transpose(1, 2).requires_grad_()
    leaves = [layer(x) for x in (q, k, v)]
    out = gdr.flash_attention(*leaves, cu_seqlens=cu.cuda())
    got = [out.detach().cpu()] + [x.cpu() for x in torch.autograd.grad(out, leaves, d_out.cuda())]
    exact = _exact(q, k, v, d_out, None, cu)
    err = _errors(got, exact)
    scale = [x.abs().max().item() for x in exact]
    print("packed: " + " | ".join(f"{n} {e:.2e} (max {s:.2e})" for n, e, s in zip(NAMES, err, scale)), flush=True)
    for i, name in enumerate(NAMES):
        assert err[i] <= 2e-2 * scale[i], (name, err[i], scale[i])
    for s, e in zip(cu[:-1].tolist(), cu[1:].tolist()):
        alone = _kernel(q[:, :, s:e], k[:, :, s:e], v[:, :, s:e], d_out[:, :, s:e])
        for i, name in enumerate(NAMES):
            assert torch.equal(alone[i], got[i][:, :, s:e]), (name, s, e)


def test_attention_gradients_under_autocast():
    """The reference's autocast case (tests/test_flash_attention_2.py:59-68): fp32 q and k with bf16 v under bf16
    autocast; the output is bf16 and the gradients reach the fp32 leaves."""
    gen = torch.Generator().manual_seed(14)
    q = torch.randn(2, 8, 256, 64, generator=gen)
    k = torch.randn(2, 4, 256, 64, generator=gen)
    v = torch.randn(2, 4, 256, 64, generator=gen).bfloat16()
    d_out = torch.randn(2, 8, 256, 64, generator=gen).bfloat16()
    leaves = [x.cuda().requires_grad_() for x in (q, k, v)]
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out = gdr.flash_attention(*leaves)
    assert out.dtype == torch.bfloat16
    grads = torch.autograd.grad(out, leaves, d_out.cuda())
    assert [g.dtype for g in grads] == [torch.float32, torch.float32, torch.bfloat16]
    exact = _exact(q.bfloat16(), k.bfloat16(), v, d_out)
    for name, a, b in zip(NAMES, [out.detach()] + list(grads), exact):
        err = (a.cpu().double() - b).abs().max().item()
        assert err <= 2e-2 * b.abs().max().item(), (name, err)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_attention_gradients_partial_leaves_and_strided_output_gradient(dtype):
    """Only q and v require gradients, D = 64 packed sequences with four query heads per key-value head, and the
    output gradient arrives as a transposed (non-contiguous) view: the returned gradients equal those of the full
    contiguous call bit for bit."""
    lens = [5, 64, 200]
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32)
    T, H, Hkv, D = int(cu[-1]), 8, 2, 64
    q, k, v, d_out = _inputs(1, H, Hkv, T, D, dtype, seed=15)
    d_strided = d_out.transpose(1, 2).contiguous().cuda().transpose(1, 2)
    qg, vg = q.cuda().requires_grad_(), v.cuda().requires_grad_()
    out = gdr.flash_attention(qg, k.cuda(), vg, cu_seqlens=cu.cuda())
    dq, dv = torch.autograd.grad(out, [qg, vg], d_strided)
    full = _kernel(q, k, v, d_out, cu_seqlens=cu.cuda())
    assert torch.equal(dq.cpu(), full[1]) and torch.equal(dv.cpu(), full[3])
    exact = _exact(q, k, v, d_out, None, cu)
    for got, want, name in ((dq.cpu(), exact[1], "dq"), (dv.cpu(), exact[3], "dv")):
        err = (got.double() - want).abs().max().item()
        assert err <= 2e-2 * want.abs().max().item(), (name, err)
