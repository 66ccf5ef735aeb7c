"""Host-side glue shared by the four op modules: argument resolution, validation and the libgdr launch.

Mirrors the reference's per-op host code (src/ops/kimi_delta_attention.py:625-692 and the identical helpers in
gated_deltanet.py:472-520, gated_linear_attention.py:437-483, deltanet.py:399-445):
  * scale = `scale or head_dim ** -0.5` (so 0.0 also selects the default, as in the reference),
  * the chunk path casts q, k, v to the autocast dtype when autocast is enabled (utils.py:84-88), and takes its
    matrix-product operands in k's dtype as the reference's kernels do (.to(k.dtype)): bf16 and f16 q, k, v run the
    chunk kernels on bf16 / f16 MFMA operands; fp32 q, k, v run the recurrent kernel over the whole sequence, all in
    fp32, when no gradient is needed; mixed fp32 / 16-bit q, k, v run on the 16-bit dtype; and a call that needs
    gradients runs on bf16 operands whatever the input dtypes (the backward kernels are bf16),
  * a missing initial state is a zero fp32 state, a given one is used as `initial_state.float().contiguous()`,
  * the final state is always a fresh fp32 tensor and inputs are never modified,
  * the output has the value's dtype; `(out, final_state)` is returned only when `output_final_state`.
The chunk ops are differentiable like the reference's torch.autograd.Function classes
(kimi_delta_attention.py:534-622 and its twins): when an input requires grad, the forward runs through
`_ChunkFunction`, returning gradients for q, k, v, gate, beta and the initial state (none for `scale`).  Its
forward is gdr_chunk_fwd_train, which also keeps the forward records, the per-chunk states and u in the backward
workspace, and its backward is gdr_chunk_bwd_saved on that workspace.  The reference's backward recomputes the
states instead (:566-571); `set_chunk_backward_workspace(False)` (or GDR_CHUNK_BWD_RECOMPUTE=1 in the environment)
makes this module do the same (plain forward, gdr_chunk_bwd), holding less memory between forward and backward.
Differences, all deliberate: CPU tensors raise (the reference's CPU token loop is this repository's test oracle,
not a product path); gradients through the recurrent ops raise (the reference's recurrent ops have none either)
and so do gradients of packed varlen calls; packed variable-length input is accepted through `cu_seqlens` (the
reference has none).
"""

from __future__ import annotations

import os

import torch

from . import _lib

_VARIANT_NAMES = {_lib.KDA: "kimi delta attention", _lib.GDN: "gated deltanet", _lib.GLA: "gated linear attention",
                  _lib.DELTANET: "deltanet"}


_KEEP_WORKSPACE = None  # None: decided per call by the GDR_CHUNK_BWD_RECOMPUTE environment variable


def set_chunk_backward_workspace(keep: bool | None) -> None:
    """Choose what the chunk ops' training forward keeps for the backward.

    keep=True: the forward (gdr_chunk_fwd_train) fills the backward workspace -- the per-chunk records, the bf16
    state entering every chunk, the bf16 u, and room for the backward's state gradients -- and keeps it until the
    backward runs, which then skips recomputing them.  That is gdr_chunk_bwd_workspace_bytes per call, 0.69 GB at
    B=4, T=4096, H=16, K=V=128, held per layer from forward to backward.
    keep=False: the forward keeps only its inputs and the backward recomputes the records and states (a prep launch
    and a state scan, about 0.29 ms at that shape), as the reference's backward does
    (src/ops/kimi_delta_attention.py:566-571).  keep=None (the default) reads GDR_CHUNK_BWD_RECOMPUTE on each call:
    "1" recomputes, anything else keeps.
    """
    global _KEEP_WORKSPACE
    _KEEP_WORKSPACE = keep


def _keep_workspace() -> bool:
    if _KEEP_WORKSPACE is not None:
        return _KEEP_WORKSPACE
    return os.environ.get("GDR_CHUNK_BWD_RECOMPUTE", "0") != "1"


def _autocast(*tensors):
    if torch.is_autocast_enabled("cuda"):
        dtype = torch.get_autocast_dtype("cuda")
        return [x.to(dtype) for x in tensors]
    return list(tensors)


def _wants_grad(*tensors) -> bool:
    return torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in tensors)


def _aligned(x: torch.Tensor) -> bool:
    es = x.element_size()
    return x.data_ptr() % 16 == 0 and all((s * es) % 16 == 0 for s in x.stride()[:3])


def _as_row_aligned(x: torch.Tensor) -> torch.Tensor:
    if x.stride(-1) != 1:
        x = x.contiguous()
    return x if _aligned(x) else x.contiguous()


def run(variant: int, chunk: bool, query, key, value, gate, beta, scale, initial_state, output_final_state,
        cu_seqlens=None):
    name = _VARIANT_NAMES[variant]
    grad = _wants_grad(query, key, value, gate, beta, initial_state)
    if grad and not chunk:
        raise NotImplementedError(f"{name}: the recurrent op has no backward (as in the reference); use the chunk op "
                                  "for training or run under torch.no_grad()")
    if grad and cu_seqlens is not None:
        raise NotImplementedError(f"{name}: the chunk backward does not take packed varlen input (cu_seqlens)")
    tensors = [t for t in (query, key, value, gate, beta, initial_state, cu_seqlens) if t is not None]
    if not all(t.is_cuda for t in tensors):
        raise ValueError(f"{name}: all tensors must be on the GPU (this implementation has no CPU path)")
    device = query.device
    if any(t.device != device for t in tensors):
        raise ValueError(f"{name}: all tensors must be on one device")
    if query.dim() != 4 or key.shape != query.shape or value.dim() != 4 or value.shape[:3] != query.shape[:3]:
        raise ValueError(f"{name}: expected q, k [B,H,T,K] and v [B,H,T,V], got {tuple(query.shape)}, "
                         f"{tuple(key.shape)}, {tuple(value.shape)}")
    batch, heads, seq_len, key_dim = query.shape
    value_dim = value.shape[-1]

    scale = scale or key_dim ** -0.5
    if chunk:
        query, key, value = _autocast(query, key, value)
    out_dtype = value.dtype

    if gate is not None:
        expect = (batch, heads, seq_len) if variant == _lib.GDN else (batch, heads, seq_len, key_dim)
        if tuple(gate.shape) != expect:
            raise ValueError(f"{name}: gate must have shape {expect}, got {tuple(gate.shape)}")
        gate = gate.float()
    if beta is not None:
        if tuple(beta.shape) != (batch, heads, seq_len):
            raise ValueError(f"{name}: beta must have shape {(batch, heads, seq_len)}, got {tuple(beta.shape)}")
        beta = beta.float()

    n_states = batch
    if cu_seqlens is not None:
        if not chunk:
            raise ValueError(f"{name}: cu_seqlens is only supported by the chunk op")
        if batch != 1:
            raise ValueError(f"{name}: cu_seqlens requires batch size 1 (packed sequences), got {batch}")
        cu_seqlens = cu_seqlens.to(torch.int32).contiguous()
        n_states = cu_seqlens.numel() - 1
        if n_states < 1:
            raise ValueError(f"{name}: cu_seqlens needs at least two offsets")

    state_shape = (n_states, heads, key_dim, value_dim)
    if initial_state is not None:
        if tuple(initial_state.shape) != state_shape:
            raise ValueError(f"{name}: initial_state must have shape {state_shape}, got {tuple(initial_state.shape)}")
        initial_state = initial_state.float().contiguous()

    # The sequential path of the chunk op (libgdr's gdr_chunk_fwd runs the recurrent kernel over every token, the
    # state, every product and every sum in fp32): fp32 q, k, v when no gradient is needed -- the reference's chunk
    # kernels take their dot operands in the input dtype (.to(k.dtype), kimi_delta_attention.py:99-100, :130, :135),
    # so fp32 inputs get fp32 products, and the chunk kernels multiply 16-bit operands -- and key dims the chunk
    # kernels are not built for (they take 64 and 128; the reference's take any multiple of 64).
    sequential = chunk and (key_dim not in (64, 128) or
                            (not grad and all(x.dtype == torch.float32 for x in (query, key, value))))
    if sequential and grad:
        raise NotImplementedError(f"{name}: key dim {key_dim} runs the recurrent kernel, which has no backward (the "
                                  "chunk backward takes key dims 64 and 128)")
    if (sequential or not chunk) and not (query.dtype == key.dtype == value.dtype == torch.bfloat16):
        # The recurrent kernel reads q, k, v as one element type: all bf16, or else all fp32 (an exact widening).
        query, key, value = (x if x.dtype == torch.float32 else x.float() for x in (query, key, value))
    if chunk and not sequential:
        # The chunk kernels take their MFMA operands in one 16-bit type and read q, k, v with 16-byte rows.  As the
        # reference casts its dot operands to k.dtype, that is k's dtype when k is bf16 or f16, else the 16-bit
        # dtype among v and q (mixed fp32 / 16-bit inputs).  The backward kernels take bf16 operands, so a call
        # that needs gradients runs on bf16 whatever the input dtypes; the casts are differentiable, so each
        # input's gradient comes back in its own dtype.
        operand = next((x.dtype for x in (key, value, query) if x.dtype in _OPERAND_DTYPES), torch.bfloat16)
        if grad:
            operand = torch.bfloat16
        query, key, value = (x.to(operand) for x in (query, key, value))
        query, key, value = (_as_row_aligned(x) for x in (query, key, value))
        if gate is not None and variant != _lib.GDN:
            gate = _as_row_aligned(gate)

    if grad:
        out, final_state = _ChunkFunction.apply(variant, query, key, value, gate, beta, scale, initial_state,
                                                out_dtype)
        return (out, final_state) if output_final_state else out

    out = torch.empty(batch, heads, seq_len, value_dim, device=device, dtype=out_dtype)
    final_state = torch.empty(state_shape, device=device, dtype=torch.float32) if output_final_state else None
    args = _lib.make_args(variant, query, key, value, gate, beta, out, scale, initial_state, final_state, cu_seqlens)
    workspace = _lib.chunk_workspace(args, device) if chunk and not sequential else None  # noqa: F841 (alive until enqueued)
    _lib.launch("gdr_chunk_fwd" if chunk else "gdr_recurrent_fwd", args, device)
    return (out, final_state) if output_final_state else out


_OPERAND_DTYPES = (torch.bfloat16, torch.float16)


class _ChunkFunction(torch.autograd.Function):
    """Chunk forward + backward.  Inputs arrive resolved by `run`: bf16 q, k, v with 16-byte rows, fp32 gate / beta,
    fp32 contiguous initial state (or None).  The forward keeps the backward workspace it filled (records, states,
    u) unless GDR_CHUNK_BWD_RECOMPUTE=1, in which case the backward recomputes them from the saved inputs as the
    reference's does (kimi_delta_attention.py:555, :566-571)."""

    @staticmethod
    def forward(ctx, variant, query, key, value, gate, beta, scale, initial_state, out_dtype):
        batch, heads, seq_len, key_dim = query.shape
        value_dim = value.shape[-1]
        device = query.device
        # the training forward writes bf16 or fp32 output; an f16 output is written in fp32 and rounded once
        written = out_dtype if out_dtype in (torch.bfloat16, torch.float32) else torch.float32
        out = torch.empty(batch, heads, seq_len, value_dim, device=device, dtype=written)
        final_state = torch.empty(batch, heads, key_dim, value_dim, device=device, dtype=torch.float32)
        args = _lib.make_args(variant, query, key, value, gate, beta, out, scale, initial_state, final_state)
        if not _keep_workspace():
            ctx.saved_ws = None
            workspace = _lib.chunk_workspace(args, device)  # noqa: F841 (alive until enqueued)
            _lib.launch("gdr_chunk_fwd", args, device)
        else:
            ctx.saved_ws = _lib.bwd_workspace(args, device)
            _lib.chunk_forward_train(args, ctx.saved_ws, device)
        ctx.save_for_backward(query, key, value, gate, beta, initial_state)
        ctx.variant, ctx.scale = variant, scale
        return out.to(out_dtype), final_state

    @staticmethod
    def backward(ctx, d_out, d_final):
        query, key, value, gate, beta, initial_state = ctx.saved_tensors
        device = query.device
        if d_out is None:
            d_out = torch.zeros(value.shape, device=device, dtype=torch.bfloat16)
        d_out = _as_row_aligned(d_out.to(torch.bfloat16))
        if d_final is not None:
            d_final = d_final.float().contiguous()
        dq, dk, dv = torch.empty_like(query), torch.empty_like(key), torch.empty_like(value)
        dg = torch.empty_like(gate) if gate is not None else None
        db = torch.empty_like(beta) if beta is not None else None
        dh0 = torch.empty_like(initial_state) if initial_state is not None else None
        args = _lib.make_args(ctx.variant, query, key, value, gate, beta, None, ctx.scale, initial_state, None)
        grads = _lib.make_grads(d_out, d_final, dq, dk, dv, dg, db, dh0)
        # the saved workspace serves one backward; a second one (retain_graph) recomputes from the saved inputs
        saved, ctx.saved_ws = ctx.saved_ws, None
        _lib.chunk_backward(args, grads, device, saved)
        return None, dq, dk, dv, dg, db, None, dh0, None
