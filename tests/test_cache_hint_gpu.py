"""The prefill's cache-hinted path against the plain path, on the GPU.

A call whose records total 256 MiB to 1 GiB loads its single-use input rows, and stores its output (and, in the
training forward, the saved states and u), with the non-temporal hint (`use_nt_hint`, csrc/chunk_split.hip); smaller
and larger calls do not.  The hint only places lines in the memory-side cache, and every (sequence, head) is
computed on its own, so a hinted call must equal the same work done as smaller, unhinted calls bit for bit:

* the forward at the c2 shape (B = 4, T = 4096, H = 16, 291 MB of records, hinted) against its two halves along
  the sequence (145 MB each, unhinted) chained through the fp32 state, which keeps the scan's slice width;
* the forward at the c2 and c4 shapes against each batch element run alone (unhinted, narrower scan slices);
* the training forward and backward at the c2 shape against each batch element's own training step;
* the fused-prologue call at the c2 shape (with and without the in-kernel convolutions) against each batch
  element's own call.
"""

import ctypes
import importlib

import pytest
import torch

from _helpers import CHUNK_FNS, gdr, oracle, workloads

pytestmark = pytest.mark.gpu

RECORD_BYTES = 71168  # bytes per (chunk, head) record at dk = dv = 128


def _records(batch, seq_len, heads):
    return batch * (-(-seq_len // 64)) * heads * RECORD_BYTES


def _fwd(variant, inp, **kw):
    with torch.no_grad():
        return CHUNK_FNS[variant](*inp.args(), initial_state=inp.initial_state, output_final_state=True, **kw)


def _part(inp, b=slice(None), t=slice(None)):
    """The inputs of batch elements b and tokens t (copies, contiguous, as the op's [B, H, T, ...] layout)."""
    cut = lambda x: None if x is None else x[b, :, t].contiguous()
    out = workloads.Inputs(cut(inp.query), cut(inp.key), cut(inp.value), cut(inp.gate), cut(inp.beta),
                           None if inp.initial_state is None else inp.initial_state[b].contiguous())
    return out


def test_hinted_forward_equals_its_halves_along_the_sequence():
    B, T, H = 4, 4096, 16
    assert _records(B, T, H) >= 256 << 20 > _records(B, T // 2, H)
    print(f"kda B{B} T{T} H{H}: one call against two halves", flush=True)
    inp = workloads.make_inputs("kda", B, T, H, 128, 128, seed=21, state_std=0.02, device="cuda")
    out, state = _fwd("kda", inp)
    first = _part(inp, t=slice(0, T // 2))
    o1, s1 = _fwd("kda", first)
    second = _part(inp, t=slice(T // 2, T))
    second.initial_state = s1
    o2, s2 = _fwd("kda", second)
    torch.cuda.synchronize()
    assert torch.equal(out, torch.cat([o1, o2], dim=2)) and torch.equal(state, s2)


def _record_bytes(K, V):
    """Bytes of one (chunk, head) record, as gdr_chunk_workspace_bytes reports them for a one-chunk, one-head call."""
    lib = importlib.import_module("gtar-kimik3-public_amd._lib")
    x = lambda d: torch.empty(1, 1, 64, d, dtype=torch.bfloat16)
    args = lib.make_args(lib.KDA, x(K), x(K), x(V), torch.empty(1, 1, 64, K), torch.empty(1, 1, 64), x(V), 1.0,
                         None, None)
    return lib.load_library().gdr_chunk_workspace_bytes(ctypes.byref(args))


@pytest.mark.parametrize("variant,batch,seq_len,K,V", [("kda", 4, 4096, 128, 128), ("kda", 4, 4096, 128, 256),
                                                       ("kda", 16, 4096, 64, 64)] +
                         [(v, 2, 8192, 128, 128) for v in oracle.VARIANTS])
def test_hinted_forward_equals_each_batch_element_alone(variant, batch, seq_len, K, V):
    H = 16
    rec = _record_bytes(K, V)
    assert batch * (seq_len // 64) * H * rec >= 256 << 20 > (seq_len // 64) * H * rec
    print(f"{variant} B{batch} T{seq_len} H{H} K{K} V{V}: one call against each element alone", flush=True)
    inp = workloads.make_inputs(variant, batch, seq_len, H, K, V, seed=22, state_std=0.02, device="cuda")
    out, state = _fwd(variant, inp)
    for b in range(batch):
        ob, sb = _fwd(variant, _part(inp, b=slice(b, b + 1)))
        torch.cuda.synchronize()
        assert torch.equal(out[b:b + 1], ob) and torch.equal(state[b:b + 1], sb), (variant, b)


def _train(variant, inp, d_out, d_final):
    leaves = [None if x is None else x.detach().clone().requires_grad_() for x in inp.args()]
    h0 = inp.initial_state.detach().clone().requires_grad_()
    out, fin = CHUNK_FNS[variant](*leaves, initial_state=h0, output_final_state=True)
    torch.autograd.backward([out, fin], [d_out, d_final])
    return [out.detach(), fin.detach()] + [x.grad for x in leaves if x is not None] + [h0.grad]


def test_hinted_training_step_equals_each_batch_element_alone():
    B, T, H = 4, 4096, 16
    print(f"kda training step B{B} T{T} H{H}: one call against each element alone", flush=True)
    inp = workloads.make_inputs("kda", B, T, H, 128, 128, seed=23, state_std=0.02, device="cuda")
    gen = torch.Generator(device="cuda").manual_seed(24)
    d_out = torch.randn(inp.value.shape, device="cuda", generator=gen).to(inp.value.dtype)
    d_final = torch.randn(inp.initial_state.shape, device="cuda", generator=gen)
    full = _train("kda", inp, d_out, d_final)
    names = ["out", "final state", "dq", "dk", "dv", "dgate", "dbeta", "dh0"]
    for b in range(B):
        part = _train("kda", _part(inp, b=slice(b, b + 1)), d_out[b:b + 1].contiguous(), d_final[b:b + 1].contiguous())
        torch.cuda.synchronize()
        for name, x, y in zip(names, full, part):
            assert torch.equal(x[b:b + 1], y), (name, b)


@pytest.mark.parametrize("conv", [False, True])
def test_hinted_fused_call_equals_each_batch_element_alone(conv):
    """The fused-prologue call (low-rank gate, optionally the short convolutions) at the c2 shape, whose scan stores
    its output with the hint, against each batch element's own call."""
    B, T, H, K, V, R = 4, 4096, 16, 128, 128, 128
    print(f"fused kda B{B} T{T} H{H} (convolutions: {conv}): one call against each element alone", flush=True)
    gen = torch.Generator().manual_seed(25)
    q = (torch.randn(B, H, T, K, generator=gen) * 3.0).bfloat16().cuda()
    k = (torch.randn(B, H, T, K, generator=gen) * 3.0).bfloat16().cuda()
    v = torch.randn(B, H, T, V, generator=gen).bfloat16().cuda()
    z = torch.randn(B, T, R, generator=gen).bfloat16().cuda()
    w = (torch.randn(H * K, R, generator=gen) / R ** 0.5).bfloat16().cuda()
    bias = torch.full((H * K,), -4.0).cuda()
    a_log = torch.log(torch.empty(H).uniform_(1, 16, generator=gen)).cuda()
    logits = torch.randn(B, H, T, generator=gen).cuda()
    h0 = (torch.randn(B, H, K, V, generator=gen) * 0.02).cuda()
    kw = {}
    if conv:  # q, k, v are then the convolutions' inputs, read as [B, T, C] rows
        C = H * K
        flat = lambda x: x.transpose(1, 2).contiguous().view(B, T, C)
        q, k, v = (flat(x).view(B, T, H, -1).transpose(1, 2) for x in (q, k, v))
        kw["conv_weights"] = [((torch.rand(C, 1, 4, generator=gen) * 2 - 1) * 0.5).bfloat16().cuda() for _ in range(3)]

    def call(b):
        with torch.no_grad():
            return gdr.chunk_kimi_delta_attention_fused(q[b], k[b], v[b], z[b], w, bias, a_log, logits[b],
                                                        initial_state=h0[b], output_final_state=True, **kw)

    out, state = call(slice(None))
    for b in range(B):
        ob, sb = call(slice(b, b + 1))
        torch.cuda.synchronize()
        assert torch.equal(out[b:b + 1], ob) and torch.equal(state[b:b + 1], sb), b
