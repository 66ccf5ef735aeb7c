"""Inference harness for the hybrid KDA / attention stack over packed sequences (the packed-prefill configuration).

The reference's KimiK3 model (src/models/kimi_k3.py:39-66) stacks blocks whose mixer is causal attention every
`attention_interval`-th layer and KDA otherwise, each block `h += mixer(rmsnorm(h)); h += swiglu(rmsnorm(h))`.  The
reference runs it on padded batches; this harness runs the same blocks on packed sequences (`cu_seqlens`) with the
package's gfx950 ops on the paths that must respect sequence boundaries or carry per-sequence state:

  * KDA mixer (src/layers/kimi_delta_attention.py:41-61): the three short convolutions (segment-aware), the q/k
    normalisation, the beta sigmoid, the low-rank gate and the op run as one `chunk_kimi_delta_attention_fused`
    call with a per-sequence state, and the output RMSNorm x SiLU gate is one `output_norm_gate` pass;
  * attention mixer (src/layers/attention.py:82-117, no rotary embedding, as KimiK3 passes none): `flash_attention`
    over the packed sequences.

Projections, RMSNorm and the SwiGLU MLP are plain PyTorch (hipBLASLt GEMMs and elementwise kernels).  Weights are
random (seeded), bf16, initialised as the reference initialises them.  This is a measurement harness for the op in
its surrounding stack, not a model implementation: no embedding, head, cache or training.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from .attention import flash_attention
from .epilogue import output_norm_gate
from .fused import chunk_kimi_delta_attention_fused


@dataclass
class StackConfig:
    """Defaults: configs/kimi_k3_0.6B.json's block shapes."""
    hidden_size: int = 1024
    intermediate_size: int = 3072
    num_layers: int = 4
    num_attention_heads: int = 16
    num_key_value_heads: int = 8
    head_dim: int = 128
    kda_num_heads: int = 16
    kda_head_dim: int = 128
    conv_size: int = 4
    attention_interval: int = 4
    rms_norm_eps: float = 1e-6


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm over the last dimension in fp32, returned in x's dtype (src/layers/rmsnorm.py:11-16)."""
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * weight.float()).to(x.dtype)


def init_weights(cfg: StackConfig, seed: int = 0, dtype=torch.bfloat16):
    """Seeded random weights per layer (CPU tensors), in the reference's initialisation: linear weights N(0, 0.02),
    A_log = log U[1, 16], decay bias = softplus^-1(dt) with dt log-uniform in [1e-3, 1e-1]
    (src/layers/kimi_delta_attention.py:32-34), depthwise conv weights U(-1/sqrt(W), 1/sqrt(W)) (nn.Conv1d's
    default for fan-in W), norm weights 1."""
    gen = torch.Generator().manual_seed(seed)
    lin = lambda out_f, in_f: (torch.randn(out_f, in_f, generator=gen) * 0.02).to(dtype)
    H, D = cfg.hidden_size, cfg.head_dim
    layers = []
    for i in range(cfg.num_layers):
        w = {"in_norm": torch.ones(H), "post_norm": torch.ones(H),
             "gate": lin(cfg.intermediate_size, H), "up": lin(cfg.intermediate_size, H),
             "down": lin(H, cfg.intermediate_size)}
        if (i + 1) % cfg.attention_interval == 0:
            w.update(attention=True, wq=lin(cfg.num_attention_heads * D, H), wk=lin(cfg.num_key_value_heads * D, H),
                     wv=lin(cfg.num_key_value_heads * D, H), q_norm=torch.ones(D), k_norm=torch.ones(D),
                     wo=lin(H, cfg.num_attention_heads * D))
        else:
            nh, hd, W = cfg.kda_num_heads, cfg.kda_head_dim, cfg.conv_size
            inner = nh * hd
            bound = 1.0 / math.sqrt(W)
            conv = lambda: ((torch.rand(inner, 1, W, generator=gen) * 2 - 1) * bound).to(dtype)
            dt = torch.exp(torch.empty(inner).uniform_(math.log(1e-3), math.log(1e-1), generator=gen))
            w.update(attention=False, wq=lin(inner, H), wk=lin(inner, H), wv=lin(inner, H), conv_q=conv(),
                     conv_k=conv(), conv_v=conv(), w_beta=lin(nh, H), w_decay0=lin(hd, H), w_decay1=lin(inner, hd),
                     b_decay1=dt + torch.log(-torch.expm1(-dt)), w_og0=lin(hd, H), w_og1=lin(inner, hd),
                     norm=torch.ones(hd), wo=lin(H, inner),
                     a_log=torch.log(torch.empty(nh).uniform_(1, 16, generator=gen)))
        layers.append(w)
    return layers


class HybridStack:
    """The stack on one GPU: `forward(hidden [1, T, H], cu_seqlens, kda_states)` -> (hidden, kda_states)."""

    def __init__(self, cfg: StackConfig, layers, device="cuda"):
        self.cfg = cfg
        self.layers = [{k: (v.to(device) if torch.is_tensor(v) else v) for k, v in w.items()} for w in layers]
        self.kda_op_events = []  # (start, stop) CUDA events around the KDA op calls of the last forward, if timed

    def _kda(self, x, w, cu, state, timed):
        cfg = self.cfg
        T = x.shape[0]
        nh, hd = cfg.kda_num_heads, cfg.kda_head_dim
        shape = (1, T, nh, hd)
        q = F.linear(x, w["wq"])[None].view(shape)  # the convolutions' inputs: the kernel convolves
        k = F.linear(x, w["wk"])[None].view(shape)
        v = F.linear(x, w["wv"])[None].view(shape)
        z = F.linear(x, w["w_decay0"])[None]
        beta = F.linear(x, w["w_beta"]).float()[None]  # logits
        if timed:
            ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            ev[0].record()
        out, state = chunk_kimi_delta_attention_fused(
            q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), z, w["w_decay1"], w["b_decay1"], w["a_log"],
            beta.transpose(1, 2), initial_state=state, output_final_state=True, cu_seqlens=cu,
            conv_weights=(w["conv_q"], w["conv_k"], w["conv_v"]))
        if timed:
            ev[1].record()
            self.kda_op_events.append(ev)
        gate = F.linear(F.linear(x, w["w_og0"]), w["w_og1"]).view(shape)  # pre-activation
        o = output_norm_gate(out.transpose(1, 2), gate, w["norm"], cfg.rms_norm_eps)  # [1, T, nh, hd]
        return F.linear(o.reshape(T, nh * hd).to(x.dtype), w["wo"]), state

    def _attention(self, x, w, cu):
        cfg = self.cfg
        T, D = x.shape[0], cfg.head_dim
        q = rms_norm(F.linear(x, w["wq"]).view(T, cfg.num_attention_heads, D), w["q_norm"], cfg.rms_norm_eps)
        k = rms_norm(F.linear(x, w["wk"]).view(T, cfg.num_key_value_heads, D), w["k_norm"], cfg.rms_norm_eps)
        v = F.linear(x, w["wv"]).view(T, cfg.num_key_value_heads, D)
        o = flash_attention(q.transpose(0, 1)[None], k.transpose(0, 1)[None], v.transpose(0, 1)[None],
                            cu_seqlens=cu)
        return F.linear(o[0].transpose(0, 1).reshape(T, -1), w["wo"])

    @torch.no_grad()
    def forward(self, hidden, cu_seqlens, kda_states=None, timed=False):
        """hidden [1, T, H] packed; cu_seqlens int32 [N + 1] on the device; kda_states: per KDA layer the
        [N, heads, K, V] fp32 states (None: zeros).  The residual stream is kept in fp32 and every block's input is
        its bf16 RMSNorm.  Returns the fp32 hidden states and the KDA layers' final states."""
        cfg = self.cfg
        self.kda_op_events = []
        h = hidden[0].float()
        states = list(kda_states) if kda_states is not None else [None] * len(self.layers)
        for i, w in enumerate(self.layers):
            x = rms_norm(h, w["in_norm"], cfg.rms_norm_eps).to(torch.bfloat16)
            if w["attention"]:
                y = self._attention(x, w, cu_seqlens)
            else:
                y, states[i] = self._kda(x, w, cu_seqlens, states[i], timed)
            h = h + y.float()
            x = rms_norm(h, w["post_norm"], cfg.rms_norm_eps).to(torch.bfloat16)
            h = h + F.linear(F.silu(F.linear(x, w["gate"])) * F.linear(x, w["up"]), w["down"]).float()
        return h[None], states
