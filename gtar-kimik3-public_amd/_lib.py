"""ctypes binding of libgdr.so, the hand-written gfx950 HIP library behind every op in this package.

The library exposes the C ABI declared in include/gdr.h.  This module mirrors its two structs, loads the shared
object that sits next to this file (built in place by csrc/Makefile), converts torch tensors into strided views
(device pointer + dtype code + b/h/t element strides) and launches on torch's current HIP stream.

There is deliberately no fallback: if the library is missing or the tensors are not on the GPU, the call
raises.  The CPU restatement of the reference algorithm lives under oracle/ and is test infrastructure only.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY_PATH = os.path.join(_HERE, "libgdr.so")
ABI_VERSION = 8
PRO_NORM_QK, PRO_BETA_LOGITS, PRO_GATE_LOWRANK, PRO_CONV = 1, 2, 4, 8

KDA, GDN, GLA, DELTANET = 0, 1, 2, 3
F32, BF16, F16 = 0, 1, 2
_DTYPE_CODES = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}


class GdrTensor(ctypes.Structure):
    _fields_ = [
        ("ptr", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("stride_b", ctypes.c_int64),
        ("stride_h", ctypes.c_int64),
        ("stride_t", ctypes.c_int64),
    ]


class GdrArgs(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("variant", ctypes.c_int32),
        ("batch", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("seq_len", ctypes.c_int32),
        ("key_dim", ctypes.c_int32),
        ("value_dim", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("q", GdrTensor),
        ("k", GdrTensor),
        ("v", GdrTensor),
        ("gate", GdrTensor),
        ("beta", GdrTensor),
        ("out", GdrTensor),
        ("h0", ctypes.c_void_p),
        ("ht", ctypes.c_void_p),
        ("cu_seqlens", ctypes.c_void_p),
        ("n_seqs", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_int64),
    ]


class GdrPrologue(ctypes.Structure):
    _fields_ = [
        ("flags", ctypes.c_int32),
        ("rank", ctypes.c_int32),
        ("gate_lowrank", GdrTensor),
        ("gate_weight", ctypes.c_void_p),
        ("gate_bias", ctypes.c_void_p),
        ("a_log", ctypes.c_void_p),
        ("conv_size", ctypes.c_int32),
        ("conv_reserved", ctypes.c_int32),
        ("conv_weight", ctypes.c_void_p * 3),
        ("conv_state_in", ctypes.c_void_p * 3),
        ("conv_state_out", ctypes.c_void_p * 3),
    ]


class GdrAttentionArgs(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("batch", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("kv_heads", ctypes.c_int32),
        ("seq_len", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("n_seqs", ctypes.c_int32),
        ("q", GdrTensor),
        ("k", GdrTensor),
        ("v", GdrTensor),
        ("out", GdrTensor),
        ("cu_seqlens", ctypes.c_void_p),
        ("lse", ctypes.c_void_p),
    ]


class GdrAttentionGrads(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("d_out", GdrTensor),
        ("d_q", GdrTensor),
        ("d_k", GdrTensor),
        ("d_v", GdrTensor),
        ("delta", ctypes.c_void_p),
    ]


class GdrConvArgs(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("batch", ctypes.c_int32),
        ("seq_len", ctypes.c_int32),
        ("channels", ctypes.c_int32),
        ("kernel_size", ctypes.c_int32),
        ("n_seqs", ctypes.c_int32),
        ("apply_silu", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("x", GdrTensor),
        ("out", GdrTensor),
        ("weight", ctypes.c_void_p),
        ("state_in", ctypes.c_void_p),
        ("state_out", ctypes.c_void_p),
        ("cu_seqlens", ctypes.c_void_p),
    ]


class GdrNormGateArgs(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("batch", ctypes.c_int32),
        ("seq_len", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("value_dim", ctypes.c_int32),
        ("weight_dtype", ctypes.c_int32),
        ("eps", ctypes.c_float),
        ("reserved", ctypes.c_int32),
        ("x", GdrTensor),
        ("gate", GdrTensor),
        ("out", GdrTensor),
        ("weight", ctypes.c_void_p),
    ]


class GdrGrads(ctypes.Structure):
    _fields_ = [
        ("d_out", GdrTensor),
        ("d_final", ctypes.c_void_p),
        ("d_query", GdrTensor),
        ("d_key", GdrTensor),
        ("d_value", GdrTensor),
        ("d_gate", GdrTensor),
        ("d_beta", GdrTensor),
        ("d_initial", ctypes.c_void_p),
    ]


# Every symbol include/gdr.h declares, with its ctypes signature.
EXPORTS = {
    "gdr_chunk_bwd": (ctypes.c_int, [ctypes.POINTER(GdrArgs), ctypes.POINTER(GdrGrads), ctypes.c_void_p,
                                     ctypes.c_int64, ctypes.c_void_p]),
    "gdr_chunk_bwd_workspace_bytes": (ctypes.c_int64, [ctypes.POINTER(GdrArgs)]),
    "gdr_chunk_bwd_saved": (ctypes.c_int, [ctypes.POINTER(GdrArgs), ctypes.POINTER(GdrGrads), ctypes.c_void_p,
                                           ctypes.c_int64, ctypes.c_void_p]),
    "gdr_chunk_fwd_train": (ctypes.c_int, [ctypes.POINTER(GdrArgs), ctypes.c_void_p, ctypes.c_int64,
                                           ctypes.c_void_p]),
    "gdr_chunk_fwd": (ctypes.c_int, [ctypes.POINTER(GdrArgs), ctypes.c_void_p]),
    "gdr_chunk_fwd_fused": (ctypes.c_int, [ctypes.POINTER(GdrArgs), ctypes.POINTER(GdrPrologue), ctypes.c_void_p]),
    "gdr_chunk_fwd_noalloc": (ctypes.c_int, [ctypes.POINTER(GdrArgs), ctypes.c_void_p]),
    "gdr_chunk_workspace_bytes": (ctypes.c_int64, [ctypes.POINTER(GdrArgs)]),
    "gdr_recurrent_fwd": (ctypes.c_int, [ctypes.POINTER(GdrArgs), ctypes.c_void_p]),
    "gdr_recurrent_verify": (ctypes.c_int, [ctypes.POINTER(GdrArgs), ctypes.c_void_p, ctypes.c_void_p]),
    "gdr_recurrent_commit": (ctypes.c_int, [ctypes.POINTER(GdrArgs), ctypes.c_void_p, ctypes.c_void_p,
                                            ctypes.c_void_p]),
    "gdr_recurrent_commit_verify": (ctypes.c_int, [ctypes.POINTER(GdrArgs), ctypes.c_void_p, ctypes.c_void_p,
                                                   ctypes.POINTER(GdrArgs), ctypes.c_void_p, ctypes.c_void_p]),
    "gdr_attention_fwd": (ctypes.c_int, [ctypes.POINTER(GdrAttentionArgs), ctypes.c_void_p]),
    "gdr_attention_bwd": (ctypes.c_int, [ctypes.POINTER(GdrAttentionArgs), ctypes.POINTER(GdrAttentionGrads),
                                         ctypes.c_void_p]),
    "gdr_short_conv_fwd": (ctypes.c_int, [ctypes.POINTER(GdrConvArgs), ctypes.c_void_p]),
    "gdr_norm_gate_fwd": (ctypes.c_int, [ctypes.POINTER(GdrNormGateArgs), ctypes.c_void_p]),
    "gdr_last_error": (ctypes.c_char_p, []),
    "gdr_abi_version": (ctypes.c_int, []),
}

_lib = None
_lock = threading.Lock()


def load_library(path: str = LIBRARY_PATH) -> ctypes.CDLL:
    """Load libgdr.so once (after torch, so it binds to the HIP runtime torch already loaded)."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(path):
                raise RuntimeError(
                    f"libgdr.so not found at {path}; build it with `make -C {os.path.join(_HERE, 'csrc')}` "
                    "(or __graft_entry__.build()).  There is no fallback implementation."
                )
            lib = ctypes.CDLL(path)
            for name, (restype, argtypes) in EXPORTS.items():
                fn = getattr(lib, name)
                fn.restype = restype
                fn.argtypes = argtypes
            if lib.gdr_abi_version() != ABI_VERSION:
                raise RuntimeError(f"libgdr.so ABI {lib.gdr_abi_version()} != binding ABI {ABI_VERSION}; rebuild")
            _lib = lib
    return _lib


def _view(x: torch.Tensor | None, name: str) -> GdrTensor:
    view = GdrTensor()
    if x is None:
        return view
    if x.dtype not in _DTYPE_CODES:
        raise TypeError(f"{name}: unsupported dtype {x.dtype}")
    if x.dim() == 4:
        if x.shape[-1] > 1 and x.stride(-1) != 1:
            raise ValueError(f"{name}: the last dimension must be contiguous")
        sb, sh, st = x.stride(0), x.stride(1), x.stride(2)
    elif x.dim() == 3:
        sb, sh, st = x.stride(0), x.stride(1), x.stride(2)
    else:
        raise ValueError(f"{name}: expected 3 or 4 dimensions, got {tuple(x.shape)}")
    view.ptr = x.data_ptr()
    view.dtype = _DTYPE_CODES[x.dtype]
    view.stride_b, view.stride_h, view.stride_t = sb, sh, st
    return view


def make_args(variant, q, k, v, gate, beta, out, scale, h0, ht, cu_seqlens=None) -> GdrArgs:
    batch, heads, seq_len, key_dim = q.shape
    args = GdrArgs()
    args.abi_version = ABI_VERSION
    args.variant = variant
    args.batch, args.heads, args.seq_len, args.key_dim = batch, heads, seq_len, key_dim
    args.value_dim = v.shape[-1]
    args.scale = float(scale)
    args.q, args.k, args.v = _view(q, "query"), _view(k, "key"), _view(v, "value")
    args.gate, args.beta, args.out = _view(gate, "gate"), _view(beta, "beta"), _view(out, "out")
    args.h0 = h0.data_ptr() if h0 is not None else None
    args.ht = ht.data_ptr() if ht is not None else None
    if cu_seqlens is not None:
        args.cu_seqlens = cu_seqlens.data_ptr()
        args.n_seqs = cu_seqlens.numel() - 1
    return args


def chunk_workspace(args: GdrArgs, device: torch.device) -> torch.Tensor:
    """Allocate (from torch's caching allocator) and attach the chunk-mode workspace; keep the returned tensor
    alive until the launch has been enqueued."""
    lib = load_library()
    nbytes = lib.gdr_chunk_workspace_bytes(ctypes.byref(args))
    if nbytes < 0:
        raise RuntimeError(f"gdr_chunk_workspace_bytes failed ({nbytes}): {lib.gdr_last_error().decode()}")
    ws = torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)
    args.workspace = ws.data_ptr()
    args.workspace_bytes = int(nbytes)
    return ws


def launch(entry: str, args: GdrArgs, device: torch.device) -> None:
    lib = load_library()
    stream = torch.cuda.current_stream(device).cuda_stream
    rc = getattr(lib, entry)(ctypes.byref(args), ctypes.c_void_p(stream))
    if rc != 0:
        raise RuntimeError(f"{entry} failed ({rc}): {lib.gdr_last_error().decode()}")


def make_grads(d_out, d_final, d_query, d_key, d_value, d_gate, d_beta, d_initial) -> GdrGrads:
    grads = GdrGrads()
    grads.d_out = _view(d_out, "d_out")
    grads.d_final = d_final.data_ptr() if d_final is not None else None
    grads.d_query, grads.d_key, grads.d_value = (_view(d_query, "d_query"), _view(d_key, "d_key"),
                                                 _view(d_value, "d_value"))
    grads.d_gate, grads.d_beta = _view(d_gate, "d_gate"), _view(d_beta, "d_beta")
    grads.d_initial = d_initial.data_ptr() if d_initial is not None else None
    return grads


def bwd_workspace(args: GdrArgs, device: torch.device) -> torch.Tensor:
    """The chunk backward's workspace (gdr_chunk_bwd_workspace_bytes) from torch's caching allocator."""
    lib = load_library()
    nbytes = lib.gdr_chunk_bwd_workspace_bytes(ctypes.byref(args))
    if nbytes < 0:
        raise RuntimeError(f"gdr_chunk_bwd_workspace_bytes failed ({nbytes}): {lib.gdr_last_error().decode()}")
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def chunk_forward_train(args: GdrArgs, ws: torch.Tensor, device: torch.device) -> None:
    """Enqueue gdr_chunk_fwd_train: the forward's out / ht, and in `ws` what gdr_chunk_bwd_saved reads."""
    lib = load_library()
    stream = torch.cuda.current_stream(device).cuda_stream
    _check("gdr_chunk_fwd_train", lib.gdr_chunk_fwd_train(ctypes.byref(args), ctypes.c_void_p(ws.data_ptr()),
                                                          ctypes.c_int64(ws.numel()), ctypes.c_void_p(stream)))


def chunk_backward(args: GdrArgs, grads: GdrGrads, device: torch.device, saved: torch.Tensor | None = None) -> None:
    """Enqueue the chunk backward on torch's current stream: gdr_chunk_bwd_saved on `saved` (the workspace a
    gdr_chunk_fwd_train of the same args filled), else gdr_chunk_bwd on a fresh workspace (released to the
    allocator, which orders its reuse on that stream)."""
    lib = load_library()
    stream = torch.cuda.current_stream(device).cuda_stream
    if saved is not None:
        rc = lib.gdr_chunk_bwd_saved(ctypes.byref(args), ctypes.byref(grads), ctypes.c_void_p(saved.data_ptr()),
                                     ctypes.c_int64(saved.numel()), ctypes.c_void_p(stream))
        _check("gdr_chunk_bwd_saved", rc)
        return
    ws = bwd_workspace(args, device)
    rc = lib.gdr_chunk_bwd(ctypes.byref(args), ctypes.byref(grads), ctypes.c_void_p(ws.data_ptr()),
                           ctypes.c_int64(ws.numel()), ctypes.c_void_p(stream))
    _check("gdr_chunk_bwd", rc)


def _check(entry: str, rc: int) -> None:
    if rc != 0:
        raise RuntimeError(f"{entry} failed ({rc}): {load_library().gdr_last_error().decode()}")


def verify(args: GdrArgs, updates: torch.Tensor, device: torch.device) -> None:
    """Enqueue gdr_recurrent_verify on torch's current stream; `updates` is the f32 [B, H, T, V] record."""
    lib = load_library()
    stream = torch.cuda.current_stream(device).cuda_stream
    _check("gdr_recurrent_verify", lib.gdr_recurrent_verify(ctypes.byref(args), ctypes.c_void_p(updates.data_ptr()),
                                                            ctypes.c_void_p(stream)))


def commit(args: GdrArgs, updates: torch.Tensor, accepted: torch.Tensor | None, device: torch.device) -> None:
    """Enqueue gdr_recurrent_commit; `accepted` is a device int32 [B] tensor or None (all tokens)."""
    lib = load_library()
    stream = torch.cuda.current_stream(device).cuda_stream
    acc = ctypes.c_void_p(accepted.data_ptr()) if accepted is not None else None
    _check("gdr_recurrent_commit", lib.gdr_recurrent_commit(ctypes.byref(args), ctypes.c_void_p(updates.data_ptr()),
                                                            acc, ctypes.c_void_p(stream)))


def commit_verify(prev: GdrArgs, prev_updates: torch.Tensor, accepted: torch.Tensor | None, args: GdrArgs,
                  updates: torch.Tensor, device: torch.device) -> None:
    """Enqueue gdr_recurrent_commit_verify: commit `prev` (into prev.ht) and verify `args` from that state, one launch."""
    lib = load_library()
    stream = torch.cuda.current_stream(device).cuda_stream
    acc = ctypes.c_void_p(accepted.data_ptr()) if accepted is not None else None
    _check("gdr_recurrent_commit_verify",
           lib.gdr_recurrent_commit_verify(ctypes.byref(prev), ctypes.c_void_p(prev_updates.data_ptr()), acc,
                                           ctypes.byref(args), ctypes.c_void_p(updates.data_ptr()),
                                           ctypes.c_void_p(stream)))


def make_prologue(flags: int, gate_lowrank=None, gate_weight=None, gate_bias=None, a_log=None, conv_weights=None,
                  conv_states_in=None, conv_states_out=None) -> GdrPrologue:
    pro = GdrPrologue()
    pro.flags = flags
    if conv_weights is not None:
        pro.conv_size = conv_weights[0].shape[-1]
        for i in range(3):
            pro.conv_weight[i] = conv_weights[i].data_ptr()
            pro.conv_state_in[i] = conv_states_in[i].data_ptr() if conv_states_in is not None else None
            pro.conv_state_out[i] = conv_states_out[i].data_ptr() if conv_states_out is not None else None
    if gate_lowrank is not None:
        pro.rank = gate_lowrank.shape[-1]
        view = GdrTensor()
        view.ptr, view.dtype = gate_lowrank.data_ptr(), _DTYPE_CODES[gate_lowrank.dtype]
        view.stride_b, view.stride_h, view.stride_t = gate_lowrank.stride(0), 0, gate_lowrank.stride(1)
        pro.gate_lowrank = view
        pro.gate_weight = gate_weight.data_ptr()
        pro.gate_bias = gate_bias.data_ptr() if gate_bias is not None else None
        pro.a_log = a_log.data_ptr()
    return pro


def launch_fused(args: GdrArgs, pro: GdrPrologue, device: torch.device) -> None:
    """Enqueue gdr_chunk_fwd_fused on torch's current stream (args carries the workspace)."""
    lib = load_library()
    stream = torch.cuda.current_stream(device).cuda_stream
    _check("gdr_chunk_fwd_fused", lib.gdr_chunk_fwd_fused(ctypes.byref(args), ctypes.byref(pro),
                                                          ctypes.c_void_p(stream)))


def _view3(x: torch.Tensor, name: str) -> GdrTensor:
    """[B, T, C] view (stride_h unused)."""
    if x.dtype not in _DTYPE_CODES:
        raise TypeError(f"{name}: unsupported dtype {x.dtype}")
    view = GdrTensor()
    view.ptr, view.dtype = x.data_ptr(), _DTYPE_CODES[x.dtype]
    view.stride_b, view.stride_h, view.stride_t = x.stride(0), 0, x.stride(1)
    return view


def _attention_args(q, k, v, out, scale, cu_seqlens, lse) -> GdrAttentionArgs:
    args = GdrAttentionArgs()
    args.abi_version = ABI_VERSION
    args.batch, args.heads, args.seq_len, args.head_dim = q.shape[0], q.shape[1], q.shape[2], q.shape[3]
    args.kv_heads = k.shape[1]
    args.scale = float(scale)
    args.q, args.k, args.v, args.out = _view(q, "query"), _view(k, "key"), _view(v, "value"), _view(out, "out")
    if cu_seqlens is not None:
        args.cu_seqlens = cu_seqlens.data_ptr()
        args.n_seqs = cu_seqlens.numel() - 1
    args.lse = lse.data_ptr() if lse is not None else None
    return args


def attention(q, k, v, out, scale, cu_seqlens, device, lse=None) -> None:
    """Enqueue gdr_attention_fwd on torch's current stream (writing the row log-sum-exp into `lse`, fp32 [B, H, T],
    when given)."""
    args = _attention_args(q, k, v, out, scale, cu_seqlens, lse)
    lib = load_library()
    stream = torch.cuda.current_stream(device).cuda_stream
    _check("gdr_attention_fwd", lib.gdr_attention_fwd(ctypes.byref(args), ctypes.c_void_p(stream)))


def attention_bwd(q, k, v, out, lse, scale, cu_seqlens, d_out, d_q, d_k, d_v, delta, device) -> None:
    """Enqueue gdr_attention_bwd on torch's current stream: d_q, d_k, d_v from the forward's q, k, v, out and lse
    and the incoming d_out; `delta` (fp32 [B, H, T]) is scratch."""
    args = _attention_args(q, k, v, out, scale, cu_seqlens, lse)
    grads = GdrAttentionGrads()
    grads.abi_version = ABI_VERSION
    grads.d_out, grads.d_q = _view(d_out, "d_out"), _view(d_q, "d_q")
    grads.d_k, grads.d_v = _view(d_k, "d_k"), _view(d_v, "d_v")
    grads.delta = delta.data_ptr()
    lib = load_library()
    stream = torch.cuda.current_stream(device).cuda_stream
    _check("gdr_attention_bwd", lib.gdr_attention_bwd(ctypes.byref(args), ctypes.byref(grads),
                                                      ctypes.c_void_p(stream)))


def short_conv(x, out, weight, state_in, state_out, cu_seqlens, silu, device) -> None:
    """Enqueue gdr_short_conv_fwd on torch's current stream."""
    args = GdrConvArgs()
    args.abi_version = ABI_VERSION
    args.batch, args.seq_len, args.channels = x.shape
    args.kernel_size = weight.shape[-1]
    args.apply_silu = int(bool(silu))
    args.x, args.out = _view3(x, "x"), _view3(out, "out")
    args.weight = weight.data_ptr()
    args.state_in = state_in.data_ptr() if state_in is not None else None
    args.state_out = state_out.data_ptr() if state_out is not None else None
    if cu_seqlens is not None:
        args.cu_seqlens = cu_seqlens.data_ptr()
        args.n_seqs = cu_seqlens.numel() - 1
    lib = load_library()
    stream = torch.cuda.current_stream(device).cuda_stream
    _check("gdr_short_conv_fwd", lib.gdr_short_conv_fwd(ctypes.byref(args), ctypes.c_void_p(stream)))


def norm_gate(x, gate, weight, out, eps, device) -> None:
    """Enqueue gdr_norm_gate_fwd on torch's current stream; x, gate, out are [B, T, H, V] views."""
    args = GdrNormGateArgs()
    args.abi_version = ABI_VERSION
    args.batch, args.seq_len, args.heads, args.value_dim = x.shape
    args.weight_dtype = _DTYPE_CODES[weight.dtype]
    args.eps = float(eps)

    def bthv(t, name):
        if t.dtype not in _DTYPE_CODES:
            raise TypeError(f"{name}: unsupported dtype {t.dtype}")
        if t.shape[-1] > 1 and t.stride(-1) != 1:
            raise ValueError(f"{name}: the last dimension must be contiguous")
        view = GdrTensor()
        view.ptr, view.dtype = t.data_ptr(), _DTYPE_CODES[t.dtype]
        view.stride_b, view.stride_h, view.stride_t = t.stride(0), t.stride(2), t.stride(1)
        return view

    args.x, args.gate, args.out = bthv(x, "x"), bthv(gate, "gate"), bthv(out, "out")
    args.weight = weight.data_ptr()
    lib = load_library()
    stream = torch.cuda.current_stream(device).cuda_stream
    _check("gdr_norm_gate_fwd", lib.gdr_norm_gate_fwd(ctypes.byref(args), ctypes.c_void_p(stream)))
