"""Causal grouped-query attention (gdr_attention_fwd) and the segment-aware short convolution (gdr_short_conv_fwd)
of the hybrid stack, on the GPU, through the package's ops and libgdr.so.

Attention parity uses the reference's own bar (tests/test_flash_attention_2.py:42-53): the kernel's max abs error
against the exact (fp64) result must be at most 2x that of PyTorch's SDPA run in the same half dtype, plus 1e-4.
The SDPA baseline runs on the CPU (half-precision attention's math path is kept off this GPU), on the same inputs.
The short convolution is held to the fp64 oracle at 1e-2 relative to max |out| (one half-precision rounding of
the output, fp32 accumulation inside).
"""

import importlib

import pytest
import torch
import torch.nn.functional as F

from _helpers import gdr, oracle

pytestmark = pytest.mark.gpu


def _qkv(B, H, Hkv, T, D, dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    shape_q, shape_kv = (B, H, T, D), (B, Hkv, T, D)
    return [torch.randn(s, generator=gen).to(dtype) for s in (shape_q, shape_kv, shape_kv)]


@pytest.mark.parametrize("shape", [(1, 8, 8, 128, 64), (2, 8, 8, 512, 64), (2, 8, 2, 1000, 128), (3, 12, 4, 777, 64),
                                   (1, 32, 8, 256, 128), (1, 4, 1, 64, 64), (1, 2, 2, 1, 128)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_attention_matches_exact_within_reference_bar(shape, dtype):
    B, H, Hkv, T, D = shape
    print(f"attention {shape} {dtype}", flush=True)
    q, k, v = _qkv(B, H, Hkv, T, D, dtype, seed=1)
    exact = oracle.causal_attention(q, k, v)
    with torch.no_grad():
        out = gdr.flash_attention(q.cuda(), k.cuda(), v.cuda())
    sdpa = F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True)  # CPU, same dtype
    err = (out.cpu().double() - exact).abs().max().item()
    base = (sdpa.double() - exact).abs().max().item()
    print(f"  kernel {err:.2e}  sdpa {base:.2e}")
    assert out.dtype == dtype and err <= 2 * base + 1e-4


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("order", ["rising", "falling"])
def test_attention_moving_row_maxima(dtype, order):
    """Sharp softmax rows (scale 0.5 at D = 64) over keys whose norms rise (or fall) 8x along the sequence: with
    rising norms each row's max keeps growing, so the exponent base moves many times, by small and large steps;
    with falling norms it is set early and later probabilities are tiny.  Same bar as above."""
    B, H, Hkv, T, D = 1, 4, 2, 700, 64
    q, k, v = _qkv(B, H, Hkv, T, D, torch.float32, seed=8)
    ramp = torch.linspace(0.25, 2.0, T).view(1, 1, T, 1)
    k = k * (ramp if order == "rising" else ramp.flip(2))
    q, k, v = q.to(dtype), k.to(dtype), v.to(dtype)
    exact = oracle.causal_attention(q, k, v, 0.5)
    with torch.no_grad():
        out = gdr.flash_attention(q.cuda(), k.cuda(), v.cuda(), softmax_scale=0.5)
    sdpa = F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True, scale=0.5)
    err = (out.cpu().double() - exact).abs().max().item()
    base = (sdpa.double() - exact).abs().max().item()
    print(f"  {order} {dtype}: kernel {err:.2e}  sdpa {base:.2e}")
    assert torch.isfinite(out).all() and err <= 2 * base + 1e-4


def test_attention_packed_sequences_and_layer_layout():
    """cu_seqlens confines attention to each packed sequence (lengths around the 128-row block and 64-key tile
    edges, and a single token); q, k, v are the layer's transposed [B, T, H, D] views."""
    lens = [1, 63, 64, 65, 127, 128, 129, 300]
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32)
    T, H, Hkv, D = int(cu[-1]), 4, 2, 128
    q, k, v = _qkv(1, H, Hkv, T, D, torch.bfloat16, seed=2)
    exact = oracle.causal_attention(q, k, v, None, cu)
    layer = lambda x: x.transpose(1, 2).contiguous().cuda().transpose(1, 2)
    with torch.no_grad():
        out = gdr.flash_attention(layer(q), layer(k), layer(v), cu_seqlens=cu.cuda())
    err = (out.cpu().double() - exact).abs().max().item()
    print(f"packed: err {err:.2e}")
    assert err <= 2e-2
    # every sequence alone gives the same numbers (no leakage across sequence boundaries)
    with torch.no_grad():
        for s, e in zip(cu[:-1].tolist(), cu[1:].tolist()):
            alone = gdr.flash_attention(q[:, :, s:e].cuda(), k[:, :, s:e].cuda(), v[:, :, s:e].cuda())
            assert torch.equal(alone, out[:, :, s:e].contiguous()), (s, e)


def test_attention_full_packed_shape_equals_each_sequence_alone():
    """The stack's packed configuration at its stated shape (32 sequences with lengths ~U[256, 4096], 16 query /
    8 key-value heads, head dim 128, bf16): the packed call equals each sequence run on its own bit for bit (the
    tiles start at each sequence's first token either way), a property that holds at any size, so no fp64 oracle
    has to run the full shape; the oracle bar is checked on the shortest sequence (every head) and on the longest
    one (two query heads of different key-value heads)."""
    workloads = importlib.import_module("gtar-kimik3-public_amd.workloads")
    lengths = workloads.varlen_lengths(32, 256, 4096, seed=0)
    cu = torch.tensor([0] + torch.tensor(lengths).cumsum(0).tolist(), dtype=torch.int32)
    T, H, Hkv, D = int(cu[-1]), 16, 8, 128
    print(f"attention full packed shape: {len(lengths)} seqs, {T} tokens", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(9)
    q = torch.randn(1, H, T, D, device="cuda", generator=gen).bfloat16()
    k, v = (torch.randn(1, Hkv, T, D, device="cuda", generator=gen).bfloat16() for _ in range(2))
    with torch.no_grad():
        out = gdr.flash_attention(q, k, v, cu_seqlens=cu.cuda())
        for s, e in zip(cu[:-1].tolist(), cu[1:].tolist()):
            alone = gdr.flash_attention(q[:, :, s:e].contiguous(), k[:, :, s:e].contiguous(), v[:, :, s:e].contiguous())
            assert torch.equal(alone, out[:, :, s:e].contiguous()), (s, e)
    i = min(range(len(lengths)), key=lambda j: lengths[j])  # the shortest sequence, so the CPU check stays quick
    s, e = int(cu[i]), int(cu[i + 1])
    qs, ks, vs = (x[:, :, s:e].cpu() for x in (q, k, v))
    exact = oracle.causal_attention(qs, ks, vs)
    sdpa = F.scaled_dot_product_attention(qs, ks, vs, is_causal=True, enable_gqa=True)
    err = (out[:, :, s:e].cpu().double() - exact).abs().max().item()
    base = (sdpa.double() - exact).abs().max().item()
    print(f"  sequence {i} ({e - s} tokens): kernel {err:.2e}  sdpa {base:.2e}")
    assert err <= 2 * base + 1e-4
    i = max(range(len(lengths)), key=lambda j: lengths[j])
    s, e = int(cu[i]), int(cu[i + 1])
    for h in (0, 11):  # query head h reads key-value head h // 2
        qs = q[:, h:h + 1, s:e].cpu()
        ks, vs = (x[:, h // 2:h // 2 + 1, s:e].cpu() for x in (k, v))
        exact = oracle.causal_attention(qs, ks, vs)
        sdpa = F.scaled_dot_product_attention(qs, ks, vs, is_causal=True)
        err = (out[:, h:h + 1, s:e].cpu().double() - exact).abs().max().item()
        base = (sdpa.double() - exact).abs().max().item()
        print(f"  sequence {i} ({e - s} tokens), head {h}: kernel {err:.2e}  sdpa {base:.2e}")
        assert err <= 2 * base + 1e-4


def test_attention_scale_and_autocast():
    q, k, v = _qkv(1, 4, 4, 200, 64, torch.float32, seed=3)
    exact = oracle.causal_attention(q.bfloat16(), k.bfloat16(), v.bfloat16(), 0.05)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        out = gdr.flash_attention(q.cuda(), k.cuda(), v.cuda(), softmax_scale=0.05)
    assert out.dtype == torch.bfloat16
    assert (out.cpu().double() - exact).abs().max().item() <= 1e-2


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("width", [2, 4, 8])
def test_short_convolution_packed_with_state(dtype, width):
    lens = [1, 2, 5, 64, 100]
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32)
    T, C = int(cu[-1]), 64
    gen = torch.Generator().manual_seed(4)
    x = torch.randn(1, T, C, generator=gen).to(dtype)
    w = (torch.randn(C, 1, width, generator=gen) * 0.5).to(dtype)
    state = torch.randn(len(lens), C, width - 1, generator=gen).to(dtype)
    ref, ref_state = oracle.short_convolution(x, w, state, cu)
    st = state.cuda()
    with torch.no_grad():
        out = gdr.short_convolution(x.cuda(), w.cuda(), st, cu_seqlens=cu.cuda())
    err = ((out.cpu().double() - ref).abs().max() / ref.abs().max()).item()
    print(f"conv {dtype} W={width}: err {err:.2e}")
    assert out.dtype == dtype and err <= 1e-2
    assert torch.equal(st.cpu(), ref_state.to(dtype))  # the new state is a copy of inputs: exact


def test_short_convolution_batched_matches_reference_module():
    """Batched (no cu_seqlens), no state: nn.Conv1d with left padding then SiLU, the reference module's path."""
    B, T, C, W = 2, 50, 128, 4
    gen = torch.Generator().manual_seed(5)
    x = torch.randn(B, T, C, generator=gen).bfloat16()
    w = (torch.randn(C, 1, W, generator=gen) * 0.5).bfloat16()
    ref, _ = oracle.short_convolution(x, w)
    with torch.no_grad():
        out = gdr.short_convolution(x.cuda(), w.cuda())
        plain = gdr.short_convolution(x.cuda(), w.cuda(), activation=False)
    assert ((out.cpu().double() - ref).abs().max() / ref.abs().max()).item() <= 1e-2
    lin, _ = oracle.short_convolution(x, w, activation=False)
    assert ((plain.cpu().double() - lin).abs().max() / lin.abs().max()).item() <= 1e-2


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_short_convolution_empty_sequences_keep_their_state(dtype):
    """Packed sequences of length 0 (first, inner and last) keep their conv state, as in the oracle (the reference
    leaves its cache untouched when no token arrives)."""
    lens, C, W = [0, 3, 0, 70, 1, 0], 32, 4
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32)
    T = int(cu[-1])
    gen = torch.Generator().manual_seed(6)
    x = torch.randn(1, T, C, generator=gen).to(dtype)
    w = (torch.randn(C, 1, W, generator=gen) * 0.5).to(dtype)
    state = torch.randn(len(lens), C, W - 1, generator=gen).to(dtype)
    ref, ref_state = oracle.short_convolution(x, w, state, cu)
    st = state.cuda()
    with torch.no_grad():
        out = gdr.short_convolution(x.cuda(), w.cuda(), st, cu_seqlens=cu.cuda())
    assert ((out.cpu().double() - ref).abs().max() / ref.abs().max()).item() <= 1e-2
    assert torch.equal(st.cpu(), ref_state.to(dtype))
    for n, length in enumerate(lens):
        if length == 0:
            assert torch.equal(st[n].cpu(), state[n])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("width", [2, 3, 4, 5, 6, 7, 8])
def test_short_convolution_tile_paths_agree(dtype, width):
    """Sequence lengths around the kernel's 8-token tiles.  A tile inside one sequence takes the register path, a
    tile at a sequence's start or end the token-by-token path; packed, a sequence's tokens sit at other tile offsets
    than when it runs alone, so the packed call equal to each sequence run alone (with its own state) bit for bit
    holds the two paths to the same arithmetic.  Both meet the oracle, and the new states are exact copies."""
    lens = [7, 8, 9, 1, 15, 16, 17, 3, 40, 2]
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32)
    T, C = int(cu[-1]), 48
    gen = torch.Generator().manual_seed(8)
    x = torch.randn(1, T, C, generator=gen).to(dtype)
    w = (torch.randn(C, 1, width, generator=gen) * 0.5).to(dtype)
    state = torch.randn(len(lens), C, width - 1, generator=gen).to(dtype)
    ref, ref_state = oracle.short_convolution(x, w, state, cu)
    st = state.cuda()
    with torch.no_grad():
        out = gdr.short_convolution(x.cuda(), w.cuda(), st, cu_seqlens=cu.cuda()).cpu()
        for n, (s, e) in enumerate(zip(cu[:-1].tolist(), cu[1:].tolist())):
            st_n = state[n:n + 1].cuda()
            alone = gdr.short_convolution(x[:, s:e].cuda(), w.cuda(), st_n).cpu()
            assert torch.equal(alone, out[:, s:e]), (n, s, e)
            assert torch.equal(st_n[0].cpu(), st[n].cpu()), n
    assert ((out.double() - ref).abs().max() / ref.abs().max()).item() <= 1e-2
    assert torch.equal(st.cpu(), ref_state.to(dtype))


def test_short_convolution_zero_tokens_keeps_the_state():
    """T == 0 launches nothing; the state passed in comes back unchanged."""
    gen = torch.Generator().manual_seed(7)
    x = torch.zeros(2, 0, 64).bfloat16()
    w = torch.randn(64, 1, 4, generator=gen).bfloat16()
    state = torch.randn(2, 64, 3, generator=gen).bfloat16()
    st = state.cuda()
    with torch.no_grad():
        out = gdr.short_convolution(x.cuda(), w.cuda(), st)
    torch.cuda.synchronize()
    assert out.shape == (2, 0, 64) and torch.equal(st.cpu(), state)
