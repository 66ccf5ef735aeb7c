"""Benchmark of the gfx950 gated delta-rule kernels on the headline configurations.

One JSON line on stdout:
  * value / ms_per_step: KDA chunkwise prefill at B=4, T=4096, H=16, dk=dv=128, chunk 64 (bf16 q/k/v, fp32
    per-channel gate, beta and state, initial state ~ N(0, 0.02)); one step = one call of
    chunk_kimi_delta_attention(..., output_final_state=True) with every input already resident in HBM.  A call
    is two launches on the caller's stream: the chunk-parallel preparation kernel and the state-scan kernel.
  * roofline: the call against HBM (its bound): algorithmic bytes per call (inputs read once, outputs written
    once) / average call time measured with HIP events on the launch stream; traffic = HBM bytes per call (both
    launches) from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary when it matches the current kernel
    source, else null.  mfma_frac reports the same call against the dense bf16 MFMA peak.
  * decode: the batch-256 KDA decode step (fp32 state [256,16,128,128] ~ N(0, 0.02), one token per sequence,
    1000 back-to-back steps, state handed from step to step as the reference API does), in state GB/s.
  * varlen: the packed-prefill configuration's KDA op (32 sequences, lengths ~U[256, 4096], cu_seqlens), with its
    HBM roofline and committed traffic.
  * verify: a speculative-decoding cycle at the decode configuration's state size (batch 256, 16 heads, 128 x 128
    fp32 state) on 8-token blocks: verify (gdr_recurrent_verify, no final state) then commit of a per-sequence
    accepted prefix drawn on the device (gdr_recurrent_commit), in algorithmic GB/s per kernel and per cycle.
  * fused: the prefill configuration from the KDA layer's pre-op tensors (q, k before normalisation, beta logits,
    the gate's rank-128 activations with decay_proj[1]'s weight and bias), as one gdr_chunk_fwd_fused call, beside
    the same preparation done in PyTorch followed by the plain op (what the reference layer runs).
  * stack: the packed-prefill configuration through the hybrid stack harness (3 KDA blocks and 1 attention block
    of the 0.6B model's shapes, random bf16 weights, 32 sequences with lengths ~U[256, 4096]): end-to-end tokens/s
    and the KDA op's share of the time.
  * attention: the stack's causal attention layer alone on the packed configuration (16 query / 8 key-value heads,
    head dim 128, bf16): ms per call, TFLOP/s over the causal FLOPs 4 H D L (L + 1) / 2 per sequence, and the
    fraction of dense bf16 MFMA peak; then its backward alone (gdr_attention_bwd), over 2.5x those FLOPs.
  * train: the prefill configuration under torch.autograd, the training forward (gdr_chunk_fwd_train) then the
    backward (gdr_chunk_bwd_saved), steps queued back to back, with the backward's algorithmic bytes and HBM
    fraction.
  * variants: the variant sweep configuration (Gated DeltaNet, GLA, DeltaNet and KDA at B=2, T=8192, H=16,
    dk=dv=128, bf16 q/k/v, fp32 gate/beta/state, no initial state): per op tokens/s, the HBM roofline with traffic
    and the bf16 MFMA fraction.  This leg runs first, so the headline leg meets the GPU at settled clocks.
  * cpu_baseline: the reference's CPU path for the op (fp32 token loop, restated in oracle/) timed on this
    host on a bounded sample of the same prefill workload; cpu_baselines_other_configs: the same loop on c1 (in
    full), the decode step (a bounded number of steps, per step) and each variant of the sweep (one full pass
    each).
Only one GPU is used; --gpus above 1 exits with a message.
"""

from __future__ import annotations

import argparse
import hashlib
import importlib
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PREFILL = dict(B=4, T=4096, H=16, K=128, V=128, chunk=64)
DECODE = dict(B=256, H=16, K=128, V=128, steps=1000)
VERIFY = dict(B=256, H=16, K=128, V=128, T=8, cycles=200)
VARLEN = dict(n_seqs=32, low=256, high=4096, H=16, K=128, V=128)
TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "hbm_traffic.json")


def delta_flops_per_token_head(C, K, V):
    """Causal FLOP count of the chunkwise delta rule per token and head: P, W and scores C*K each; U and the
    intra-chunk output C*V each; W S, K^T u and Q S 2*K*V each; the triangular inverse C^2/3."""
    return C * (3 * K + 2 * V) + 6 * K * V + C * C / 3


def prefill_bytes(B, T, H, K, V, **_):
    bf16, f32 = 2, 4
    reads = B * T * H * (2 * K * bf16 + V * bf16 + K * f32 + f32) + B * H * K * V * f32
    writes = B * T * H * V * bf16 + B * H * K * V * f32
    return reads + writes


def decode_bytes(B, H, K, V, **_):
    bf16, f32 = 2, 4
    state = 2 * B * H * K * V * f32
    io = B * H * (2 * K * bf16 + V * bf16 + K * f32 + f32 + V * bf16)
    return state + io


def source_hash(source):
    path = os.path.join(ROOT, "gtar-kimik3-public_amd", "csrc", source)
    return hashlib.sha256(open(path, "rb").read()).hexdigest()[:16]


def committed_traffic(workload):
    """HBM bytes per call of `workload` from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary, or None when
    the summary was taken on a different revision of any of the kernels' source files."""
    try:
        entry = json.load(open(TRAFFIC_SUMMARY))[workload]
        if entry["sources_sha256_16"] != [source_hash(src) for src in entry["sources"]]:
            return None
    except (OSError, ValueError, KeyError, TypeError):
        return None
    return entry.get("hbm_bytes_per_call")


def prefill_inputs(workloads, torch):
    cfg = PREFILL
    return workloads.make_inputs("kda", cfg["B"], cfg["T"], cfg["H"], cfg["K"], cfg["V"], seed=0, state_std=0.02,
                                 device=torch.device("cuda"))


def bench_prefill(gdr, inp, torch, steps, warmup):
    args = inp.args()

    def step():
        return gdr.chunk_kimi_delta_attention(*args, initial_state=inp.initial_state, output_final_state=True)

    with torch.no_grad():
        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(steps):
            step()
        stop.record(stream)
        torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps  # ms per step (one call: prep + scan launches)


VARIANT_SWEEP = dict(B=2, T=8192, H=16, K=128, V=128, chunk=64)
VARIANT_FNS = {"kda": "chunk_kimi_delta_attention", "gdn": "chunk_gated_deltanet",
               "gla": "chunk_gated_linear_attention", "deltanet": "chunk_deltanet"}


def variant_bytes(variant, B, T, H, K, V, h0=False, **_):
    """Algorithmic bytes of one chunk call: q, k, v (bf16) read and out (bf16) written per token and head, the gate
    (fp32 per channel for KDA and GLA, per head for GDN, none for DeltaNet) and beta (none for GLA) read, the final
    state written and, when given, the initial state read."""
    bf16, f32 = 2, 4
    gate = {"kda": K * f32, "gla": K * f32, "gdn": f32, "deltanet": 0}[variant]
    beta = 0 if variant == "gla" else f32
    per_token_head = 2 * K * bf16 + V * bf16 + gate + beta + V * bf16
    return B * T * H * per_token_head + (2 if h0 else 1) * B * H * K * V * f32


def variant_flops(variant, C, K, V):
    """Causal FLOP count per token and head: the delta rule (delta_flops_per_token_head) or, for GLA (no delta
    rule), the intra-chunk scores and output C*(K+V) plus the state products Q S and K^T V 4*K*V."""
    return C * (K + V) + 4 * K * V if variant == "gla" else delta_flops_per_token_head(C, K, V)


def bench_variants(gdr, workloads, torch, steps, warmup):
    """The variant sweep configuration: each op at B=2, T=8192, H=16, dk=dv=128, chunk 64 (bf16 q/k/v, fp32 gate,
    beta and state, no initial state), one call = the public chunk op with output_final_state=True."""
    cfg = VARIANT_SWEEP
    dev = torch.device("cuda")
    stream = torch.cuda.current_stream()
    out = {}
    for variant in ("gdn", "gla", "deltanet", "kda"):
        inp = workloads.make_inputs(variant, cfg["B"], cfg["T"], cfg["H"], cfg["K"], cfg["V"], seed=0, device=dev)
        fn = getattr(gdr, VARIANT_FNS[variant])
        args = inp.args()
        with torch.no_grad():
            for _ in range(warmup):
                fn(*args, output_final_state=True)
            torch.cuda.synchronize()
            start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record(stream)
            for _ in range(steps):
                fn(*args, output_final_state=True)
            stop.record(stream)
            torch.cuda.synchronize()
        ms = start.elapsed_time(stop) / steps
        tokens = cfg["B"] * cfg["T"]
        nbytes = variant_bytes(variant, **cfg)
        flops = variant_flops(variant, cfg["chunk"], cfg["K"], cfg["V"]) * tokens * cfg["H"]
        gbs = nbytes / (ms * 1e-3) / 1e9
        tflops = flops / (ms * 1e-3) / 1e12
        out[variant] = {"op": VARIANT_FNS[variant], "ms_per_call": round(ms, 4),
                        "tokens_per_s": round(tokens / (ms * 1e-3), 1), "algorithmic_bytes": nbytes,
                        "algorithmic_flops": flops, "tflops": round(tflops, 2),
                        "mfma_frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
                        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                     "frac": round(gbs / HBM_PEAK_GBS, 4),
                                     "traffic": committed_traffic(f"chunk_{variant}_prefill_c4")}}
    return {"workload": "chunk_prefill_variant_sweep", **cfg, "state": "fp32", "initial_state": None,
            "variants": out}


def bench_decode(gdr, workloads, torch, warmup):
    cfg = DECODE
    dev = torch.device("cuda")
    ring = [workloads.decode_inputs("kda", cfg["B"], cfg["H"], cfg["K"], cfg["V"], seed=100 + i, device=dev)
            for i in range(8)]
    state = workloads.decode_state(cfg["B"], cfg["H"], cfg["K"], cfg["V"], std=0.02, seed=7, device=dev)

    def run(n, state):
        for i in range(n):
            r = ring[i % 8]
            _, state = gdr.recurrent_kimi_delta_attention(*r.args(), initial_state=state, output_final_state=True)
        return state

    with torch.no_grad():
        state = run(warmup, state)
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        state = run(cfg["steps"], state)
        stop.record(stream)
        torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / cfg["steps"]
    gbs = decode_bytes(**cfg) / (ms * 1e-3) / 1e9
    return {"workload": "kda_decode_step", "B": cfg["B"], "H": cfg["H"], "K": cfg["K"], "V": cfg["V"],
            "steps": cfg["steps"], "us_per_step": round(ms * 1e3, 3), "value": round(gbs, 1),
            "unit": "GB/s (state + io bytes per step)", "tokens_per_s": round(cfg["B"] / (ms * 1e-3), 1),
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": committed_traffic("recurrent_kda_decode")}}


def verify_bytes(B, H, K, V, T, **_):
    """Algorithmic bytes of one verify call: the state read once; q, k, v, gate, beta read and out written per
    token; the fp32 update record written."""
    bf16, f32 = 2, 4
    io = B * H * T * (2 * K * bf16 + V * bf16 + K * f32 + f32 + V * bf16)
    return B * H * K * V * f32 + io + B * H * T * V * f32


def commit_bytes(accepted_tokens, B, H, K, V, **_):
    """Algorithmic bytes of one commit: the state read and written once, and k (bf16), the gate and the record row
    of each accepted token (accepted_tokens summed over the batch)."""
    bf16, f32 = 2, 4
    return 2 * B * H * K * V * f32 + accepted_tokens * H * (K * bf16 + K * f32 + V * f32)


def bench_verify(gdr, workloads, torch, warmup):
    cfg = VERIFY
    dev = torch.device("cuda")
    B, H, K, V, T = cfg["B"], cfg["H"], cfg["K"], cfg["V"], cfg["T"]
    ring = [workloads.make_inputs("kda", B, T, H, K, V, seed=200 + i, device=dev) for i in range(8)]
    gen = torch.Generator("cpu").manual_seed(3)
    counts = [torch.randint(0, T + 1, (B,), generator=gen, dtype=torch.int32) for _ in range(8)]
    accepted = [c.to(dev) for c in counts]
    state = workloads.decode_state(B, H, K, V, std=0.02, seed=9, device=dev)
    stream = torch.cuda.current_stream()

    def timed(fn, n):
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for i in range(n):
            fn(i)
        stop.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(stop) / n

    with torch.no_grad():
        blocks = [gdr.verify_kimi_delta_attention(*r.args(), initial_state=state)[2] for r in ring]
        verify_only = lambda i: gdr.verify_kimi_delta_attention(*ring[i % 8].args(), initial_state=state)
        commit_only = lambda i: blocks[i % 8].commit(accepted[i % 8])
        cur = [state]

        def cycle(i):
            _, _, block = gdr.verify_kimi_delta_attention(*ring[i % 8].args(), initial_state=cur[0])
            cur[0] = block.commit(accepted[i % 8])

        pending = [blocks[0]]

        def one_launch_cycle(i):  # commit of the previous block and verify of this one (gdr_recurrent_commit_verify)
            _, _, pending[0] = gdr.verify_kimi_delta_attention(*ring[i % 8].args(), pending=pending[0],
                                                               accepted=accepted[i % 8])

        for fn in (verify_only, commit_only, cycle, one_launch_cycle):
            for i in range(warmup):
                fn(i)
        torch.cuda.synchronize()
        v_ms = timed(verify_only, cfg["cycles"])
        c_ms = timed(commit_only, cfg["cycles"])
        y_ms = timed(cycle, cfg["cycles"])
        f_ms = timed(one_launch_cycle, cfg["cycles"])
    mean_accepted = sum(int(c.sum()) for c in counts) / len(counts)
    vb, cb = verify_bytes(**cfg), commit_bytes(mean_accepted, **cfg)
    fb = vb + cb - B * H * K * V * 4  # one launch reads the state once for both halves
    gbs = lambda nbytes, ms: nbytes / (ms * 1e-3) / 1e9
    return {"workload": "kda_verify_commit", "B": B, "H": H, "K": K, "V": V, "T": T, "cycles": cfg["cycles"],
            "mean_accepted_tokens": round(mean_accepted / B, 3),
            "us_verify": round(v_ms * 1e3, 2), "us_commit": round(c_ms * 1e3, 2), "us_cycle": round(y_ms * 1e3, 2),
            "verify_gbs": round(gbs(vb, v_ms), 1), "commit_gbs": round(gbs(cb, c_ms), 1),
            "accepted_tokens_per_s": round(mean_accepted / (y_ms * 1e-3), 1),
            "us_cycle_one_launch": round(f_ms * 1e3, 2), "one_launch_gbs": round(gbs(fb, f_ms), 1),
            "accepted_tokens_per_s_one_launch": round(mean_accepted / (f_ms * 1e-3), 1),
            "roofline": {"bound": "hbm", "achieved": round(gbs(vb + cb, y_ms), 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(gbs(vb + cb, y_ms) / HBM_PEAK_GBS, 4),
                         "traffic_verify": committed_traffic("recurrent_kda_verify"),
                         "traffic_commit": committed_traffic("recurrent_kda_commit"),
                         "traffic_one_launch": committed_traffic("recurrent_kda_commit_verify")}}


def fused_bytes(B, T, H, K, V, R=128, **_):
    """Algorithmic bytes of one fused-prologue call: q, k, v (bf16) and beta logits per token and head, z (bf16) per
    token, decay_proj[1]'s weight (bf16) and bias and A_log once, out (bf16), h0 and the final state."""
    bf16, f32 = 2, 4
    per_token_head = 2 * K * bf16 + V * bf16 + f32 + V * bf16
    return B * T * H * per_token_head + B * T * R * bf16 + H * K * (R * bf16 + f32) + H * f32 + 2 * B * H * K * V * f32


def bench_fused(gdr, torch, steps, warmup):
    import math
    cfg = dict(PREFILL, R=128)
    B, T, H, K, V, R = cfg["B"], cfg["T"], cfg["H"], cfg["K"], cfg["V"], cfg["R"]
    gen = torch.Generator("cpu").manual_seed(11)
    dev = "cuda"
    q = (torch.randn(B, T, H, K, generator=gen) * 3).bfloat16().to(dev).transpose(1, 2)
    k = (torch.randn(B, T, H, K, generator=gen) * 3).bfloat16().to(dev).transpose(1, 2)
    v = torch.randn(B, T, H, V, generator=gen).bfloat16().to(dev).transpose(1, 2)
    z = torch.randn(B, T, R, generator=gen).bfloat16().to(dev)
    w = (torch.randn(H * K, R, generator=gen) / math.sqrt(R)).bfloat16().to(dev)
    dt = torch.exp(torch.empty(H * K).uniform_(math.log(1e-3), math.log(1e-1), generator=gen))
    bias = (dt + torch.log(-torch.expm1(-dt))).to(dev)
    a_log = torch.log(torch.empty(H).uniform_(1, 16, generator=gen)).to(dev)
    logits = torch.randn(B, T, H, generator=gen).to(dev).transpose(1, 2)
    h0 = (torch.randn(B, H, K, V, generator=gen) * 0.02).to(dev)
    F = torch.nn.functional

    def fused():
        return gdr.chunk_kimi_delta_attention_fused(q, k, v, z, w, bias, a_log, logits, initial_state=h0,
                                                    output_final_state=True)

    def unfused():  # the reference layer's preparation (src/layers/kimi_delta_attention.py:45-49), then the op
        qn = F.normalize(q.float(), dim=-1).bfloat16()
        kn = F.normalize(k.float(), dim=-1).bfloat16()
        gate = -a_log.exp()[:, None] * F.softplus(F.linear(z, w, bias.bfloat16()).float().view(B, T, H, K))
        return gdr.chunk_kimi_delta_attention(qn, kn, v, gate.transpose(1, 2), logits.sigmoid(), initial_state=h0,
                                              output_final_state=True)

    # with the short convolutions: q, k, v are the convolutions' inputs [B, T, C] and the kernel convolves
    C = H * K
    xq, xk, xv = (x.transpose(1, 2).contiguous().view(B, T, C) for x in (q, k, v))
    bound = 1 / math.sqrt(4)
    cw = [((torch.rand(C, 1, 4, generator=gen) * 2 - 1) * bound).bfloat16().to(dev) for _ in range(3)]
    heads = lambda x: x.view(B, T, H, -1).transpose(1, 2)

    def fused_conv():
        return gdr.chunk_kimi_delta_attention_fused(heads(xq), heads(xk), heads(xv), z, w, bias, a_log, logits,
                                                    initial_state=h0, output_final_state=True, conv_weights=cw)

    def torch_conv_unfused():  # ShortConvolution (src/layers/short_convolution.py:11-15), the preparation, the op
        conv = lambda x, wt: F.silu(F.conv1d(x.transpose(1, 2), wt, padding=3, groups=C)[..., :T]).transpose(1, 2)
        qc, kc, vc = (heads(conv(x, wt)) for x, wt in zip((xq, xk, xv), cw))
        qn = F.normalize(qc.float(), dim=-1).bfloat16()
        kn = F.normalize(kc.float(), dim=-1).bfloat16()
        gate = -a_log.exp()[:, None] * F.softplus(F.linear(z, w, bias.bfloat16()).float().view(B, T, H, K))
        return gdr.chunk_kimi_delta_attention(qn, kn, vc, gate.transpose(1, 2), logits.sigmoid(), initial_state=h0,
                                              output_final_state=True)

    # the output epilogue on the op's output: RMSNorm x SiLU gate (src/layers/kimi_delta_attention.py:58-59)
    ogate = torch.randn(B, T, H, V, generator=gen).bfloat16().to(dev)
    nweight = torch.ones(V, device=dev)

    def short_conv():  # one standalone segment-free short convolution of the c2 q projection (gdr_short_conv_fwd)
        return gdr.short_convolution(xq, cw[0])

    def norm_gate():
        return gdr.output_norm_gate(o_out.transpose(1, 2), ogate, nweight, 1e-6)

    def torch_norm_gate():
        x = o_out.transpose(1, 2)
        xf = x.float()
        return nweight * (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)).to(x.dtype) * F.silu(ogate)

    stream = torch.cuda.current_stream()
    res = {}
    with torch.no_grad():
        o_out = fused()[0]
        for name, fn in (("fused", fused), ("torch_prologue_plus_op", unfused), ("fused_conv", fused_conv),
                         ("torch_conv_prologue_plus_op", torch_conv_unfused), ("norm_gate", norm_gate),
                         ("torch_norm_gate", torch_norm_gate), ("short_conv", short_conv)):
            for _ in range(warmup):
                fn()
            torch.cuda.synchronize()
            start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record(stream)
            for _ in range(steps):
                fn()
            stop.record(stream)
            torch.cuda.synchronize()
            res[name] = start.elapsed_time(stop) / steps
    nbytes = fused_bytes(**cfg)
    gbs = nbytes / (res["fused"] * 1e-3) / 1e9
    return {"workload": "kda_chunk_prefill_fused_prologue", **{x: cfg[x] for x in ("B", "T", "H", "K", "V", "R")},
            "ms_fused": round(res["fused"], 4), "ms_torch_prologue_plus_op": round(res["torch_prologue_plus_op"], 4),
            "ms_fused_with_conv": round(res["fused_conv"], 4),
            "ms_torch_conv_prologue_plus_op": round(res["torch_conv_prologue_plus_op"], 4),
            "us_norm_gate": round(res["norm_gate"] * 1e3, 2), "us_torch_norm_gate": round(res["torch_norm_gate"] * 1e3, 2),
            "us_short_conv": round(res["short_conv"] * 1e3, 2),
            "tokens_per_s": round(B * T / (res["fused"] * 1e-3), 1), "algorithmic_bytes": nbytes,
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4)}}


def bench_varlen(gdr, workloads, torch, steps, warmup):
    """The packed-prefill configuration's KDA op: 32 sequences with lengths ~U[256, 4096] (seeded) packed via
    cu_seqlens, H=16, dk=dv=128, per-sequence initial state ~ N(0, 0.02)."""
    cfg = VARLEN
    lengths = workloads.varlen_lengths(cfg["n_seqs"], cfg["low"], cfg["high"], seed=0)
    inp, cu = workloads.make_varlen_inputs("kda", lengths, cfg["H"], cfg["K"], cfg["V"], seed=0, device="cuda")
    args = inp.args()

    def step():
        return gdr.chunk_kimi_delta_attention(*args, initial_state=inp.initial_state, output_final_state=True,
                                              cu_seqlens=cu)

    with torch.no_grad():
        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(steps):
            step()
        stop.record(stream)
        torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / steps
    tokens = sum(lengths)
    nbytes = varlen_bytes(tokens, cfg["n_seqs"], cfg["H"], cfg["K"], cfg["V"])
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"workload": "kda_varlen_packed_prefill", "n_seqs": cfg["n_seqs"], "tokens": tokens, "H": cfg["H"],
            "K": cfg["K"], "V": cfg["V"], "ms_per_call": round(ms, 4), "tokens_per_s": round(tokens / (ms * 1e-3), 1),
            "algorithmic_bytes": nbytes,
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": committed_traffic("chunk_kda_prefill_varlen")},
            "note": "KDA op only (the layer stack around it is out of scope)"}


def varlen_bytes(tokens, n_seqs, H, K, V):
    """Algorithmic bytes of the packed KDA call: per token and head q, k (bf16), v (bf16), gate (fp32 per channel)
    and beta (fp32) read and out (bf16) written; per sequence and head the fp32 initial state read and the final
    state written."""
    bf16, f32 = 2, 4
    return tokens * H * (2 * K * bf16 + V * bf16 + K * f32 + f32 + V * bf16) + n_seqs * H * 2 * K * V * f32


def bench_attention(gdr, workloads, torch, steps, warmup):
    lengths = workloads.varlen_lengths(VARLEN["n_seqs"], VARLEN["low"], VARLEN["high"], seed=0)
    cu = torch.tensor([0] + list(torch.tensor(lengths).cumsum(0).tolist()), dtype=torch.int32, device="cuda")
    tokens, H, Hkv, D = int(cu[-1]), 16, 8, 128
    g = torch.Generator(device="cuda").manual_seed(0)
    q = torch.randn(1, H, tokens, D, device="cuda", generator=g).bfloat16()
    k, v = (torch.randn(1, Hkv, tokens, D, device="cuda", generator=g).bfloat16() for _ in range(2))
    stream = torch.cuda.current_stream()
    with torch.no_grad():
        for _ in range(warmup):
            gdr.flash_attention(q, k, v, cu_seqlens=cu)
        torch.cuda.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(steps):
            gdr.flash_attention(q, k, v, cu_seqlens=cu)
        stop.record(stream)
        torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / steps
    flops = sum(4 * H * D * n * (n + 1) / 2 for n in lengths)
    tflops = flops / (ms * 1e-3) / 1e12
    # The backward alone (gdr_attention_bwd: the dQ launch, then the dK / dV launch), replayed on one retained graph
    # with a fixed output gradient.  Its algorithmic FLOPs are the usual five causal products (S recomputed, dP, dV,
    # dK, dQ: 2.5x the forward's); the kernels form S and dP in both launches, seven products in all.
    leaves = [x.clone().requires_grad_() for x in (q, k, v)]
    out = gdr.flash_attention(*leaves, cu_seqlens=cu)
    d_out = torch.randn(out.shape, device="cuda", generator=g).bfloat16()
    for _ in range(warmup):
        torch.autograd.grad(out, leaves, d_out, retain_graph=True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(steps):
        torch.autograd.grad(out, leaves, d_out, retain_graph=True)
    stop.record(stream)
    torch.cuda.synchronize()
    bwd_ms = start.elapsed_time(stop) / steps
    bwd_tflops = 2.5 * flops / (bwd_ms * 1e-3) / 1e12
    return {"workload": "packed_causal_attention", "n_seqs": len(lengths), "tokens": tokens, "heads": H,
            "kv_heads": Hkv, "head_dim": D, "ms_per_call": round(ms, 4), "tflops": round(tflops, 1),
            "mfma_frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4), "backward_ms_per_call": round(bwd_ms, 4),
            "backward_tflops": round(bwd_tflops, 1), "backward_mfma_frac": round(bwd_tflops / MFMA_BF16_PEAK_TFLOPS, 4)}


def bench_stack(gdr, workloads, torch, steps, warmup):
    stack = importlib.import_module("gtar-kimik3-public_amd.stack")
    cfg = stack.StackConfig()
    model = stack.HybridStack(cfg, stack.init_weights(cfg, seed=0))
    lengths = workloads.varlen_lengths(VARLEN["n_seqs"], VARLEN["low"], VARLEN["high"], seed=0)
    cu = torch.tensor([0] + list(torch.tensor(lengths).cumsum(0).tolist()), dtype=torch.int32, device="cuda")
    tokens = int(cu[-1])
    hidden = torch.randn(1, tokens, cfg.hidden_size, generator=torch.Generator().manual_seed(1)).bfloat16().cuda()
    for _ in range(warmup):
        model.forward(hidden, cu)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    total, kda = 0.0, 0.0
    for _ in range(steps):
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        model.forward(hidden, cu, timed=True)
        stop.record(stream)
        torch.cuda.synchronize()
        total += start.elapsed_time(stop)
        kda += sum(a.elapsed_time(b) for a, b in model.kda_op_events)
    total, kda = total / steps, kda / steps
    return {"workload": "hybrid_stack_packed_prefill", "n_seqs": len(lengths), "tokens": tokens,
            "layers": f"{cfg.num_layers} ({cfg.num_layers - cfg.num_layers // cfg.attention_interval} KDA, "
                      f"{cfg.num_layers // cfg.attention_interval} attention)",
            "hidden": cfg.hidden_size, "ms_per_forward": round(total, 3), "tokens_per_s": round(tokens / (total * 1e-3), 1),
            "kda_op_ms": round(kda, 3), "kda_op_share": round(kda / total, 4),
            "note": "random bf16 weights; projections, block norms and MLP in PyTorch; attention, the KDA op with its "
                    "short convolutions and prologue fused in (kda_op_ms), and the KDA output norm-gate on this "
                    "package's kernels"}


def train_bytes(B, T, H, K, V, **_):
    """Algorithmic HBM bytes of one chunk backward: read q, k, v (bf16), gate (fp32), beta, dO (bf16), h0 and the
    final-state gradient; write dq, dk, dv (bf16), dgate, dbeta (fp32) and dh0."""
    per_token_head = 3 * K * 2 + V * 2 + K * 4 + 4 + V * 2 + (2 * K + V) * 2 + K * 4 + 4
    return B * T * H * per_token_head + 3 * B * H * K * V * 4


def bench_train(gdr, workloads, torch, steps, warmup):
    """The prefill configuration's KDA op under torch.autograd: the training forward (gdr_chunk_fwd_train, which
    keeps the records, states and u), then the backward (gdr_chunk_bwd_saved) for q, k, v, gate, beta and the
    initial state, with a random dO and final-state gradient."""
    cfg = PREFILL
    inp = workloads.make_inputs("kda", cfg["B"], cfg["T"], cfg["H"], cfg["K"], cfg["V"], seed=0, state_std=0.02,
                                device="cuda")
    leaves = [x.detach().clone().requires_grad_() for x in (inp.query, inp.key, inp.value, inp.gate, inp.beta,
                                                           inp.initial_state)]
    d_out = torch.randn(inp.value.shape, device="cuda").to(inp.value.dtype)
    d_final = torch.randn(inp.initial_state.shape, device="cuda")

    def forward():
        return gdr.chunk_kimi_delta_attention(*leaves[:5], initial_state=leaves[5], output_final_state=True)

    def clear_grads():
        # the gradients are written fresh each step (autograd would otherwise add them into .grad, which is
        # PyTorch's accumulation, not the op's backward)
        for x in leaves:
            x.grad = None

    def step():
        clear_grads()
        out, final = forward()
        torch.autograd.backward([out, final], [d_out, d_final])

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    # Steps are queued back to back, as a training loop runs them (the host stays ahead of the GPU), with one
    # synchronisation after the last: the events then time the GPU's work, not the host's dispatch of each step.
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    for e in ev:
        clear_grads()
        e[0].record(stream)
        out, final = forward()
        e[1].record(stream)
        torch.autograd.backward([out, final], [d_out, d_final])
        e[2].record(stream)
    torch.cuda.synchronize()
    fwd_ms = sum(e[0].elapsed_time(e[1]) for e in ev) / steps
    tot_ms = sum(e[0].elapsed_time(e[2]) for e in ev) / steps
    bwd_ms = tot_ms - fwd_ms
    tokens = cfg["B"] * cfg["T"]
    nbytes = train_bytes(**cfg)
    return {"workload": "kda_chunk_fwd_bwd", "B": cfg["B"], "T": cfg["T"], "H": cfg["H"], "K": cfg["K"],
            "V": cfg["V"], "ms_forward": round(fwd_ms, 4), "ms_backward": round(bwd_ms, 4),
            "tokens_per_s_fwd_bwd": round(tokens / (tot_ms * 1e-3), 1),
            "backward_algorithmic_bytes": nbytes, "backward_gbs": round(nbytes / (bwd_ms * 1e-3) / 1e9, 1),
            "backward_hbm_frac": round(nbytes / (bwd_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "backward_traffic": committed_traffic("chunk_kda_backward")}


def _timed_passes(fn, budget_s):
    passes, t0 = 0, time.perf_counter()
    while True:
        fn()
        passes += 1
        elapsed = time.perf_counter() - t0
        if elapsed >= budget_s:
            return passes, elapsed


def cpu_baseline(workloads, torch, budget_s):
    """The reference CPU path for the op (the fp32 token loop, restated in oracle/) on the full prefill workload,
    repeated until `budget_s`."""
    from oracle import gdr_oracle as oracle

    cfg = PREFILL
    inp = workloads.make_inputs("kda", cfg["B"], cfg["T"], cfg["H"], cfg["K"], cfg["V"], seed=0, state_std=0.02)
    passes, elapsed = _timed_passes(lambda: oracle.kda_reference(inp.query, inp.key, inp.value, inp.gate, inp.beta,
                                                                 None, inp.initial_state), budget_s)
    tokens = passes * cfg["B"] * cfg["T"]
    return {"value": round(tokens / elapsed, 1), "unit": "tokens/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"{passes} full pass(es) of the prefill workload (B=4 T=4096 H=16 dk=dv=128) through the "
                      f"reference's fp32 CPU token loop, {elapsed:.1f} s, {len(os.sched_getaffinity(0))} host "
                      "cores visible"}


def cpu_baselines_other(workloads, torch, budget_s):
    """The same CPU token loop on the other configurations: c1 (the reference's CPU-runnable case, fp32 B=1 T=256
    H=2 d=64) in full, repeated until `budget_s`; the batch-256 decode step over a bounded number of steps (about
    `budget_s`), reported per step; and each variant of the sweep configuration (B=2 T=8192 H=16 d=128) with its
    own update rule (the reference's unified loop, tests/bench_ops.py:52-66), one full pass each."""
    from oracle import gdr_oracle as oracle

    res = {"cores": torch.get_num_threads(), "host_cores_visible": len(os.sched_getaffinity(0)), "kind": "port"}
    c1 = workloads.make_inputs("kda", 1, 256, 2, 64, 64, seed=0, dtype=torch.float32)
    passes, elapsed = _timed_passes(lambda: oracle.kda_reference(c1.query, c1.key, c1.value, c1.gate, c1.beta),
                                    budget_s)
    res["c1_kda_fp32_B1_T256_H2_d64"] = {"tokens_per_s": round(passes * 256 / elapsed, 1),
                                         "ms_per_pass": round(elapsed / passes * 1e3, 2), "passes": passes}
    cfg = DECODE
    dec = workloads.decode_inputs("kda", cfg["B"], cfg["H"], cfg["K"], cfg["V"], seed=100)
    state = [workloads.decode_state(cfg["B"], cfg["H"], cfg["K"], cfg["V"], std=0.02, seed=7)]

    def step():
        _, state[0] = oracle.kda_reference(dec.query, dec.key, dec.value, dec.gate, dec.beta, None, state[0])

    steps, elapsed = _timed_passes(step, budget_s)
    res["c3_kda_decode_B256_H16_d128"] = {"ms_per_step": round(elapsed / steps * 1e3, 2), "steps": steps,
                                          "tokens_per_s": round(cfg["B"] * steps / elapsed, 1),
                                          "state_gb_per_s": round(decode_bytes(**cfg) * steps / elapsed / 1e9, 2)}
    vs = VARIANT_SWEEP
    for variant in ("gdn", "gla", "deltanet"):
        inp = workloads.make_inputs(variant, vs["B"], vs["T"], vs["H"], vs["K"], vs["V"], seed=0)
        t0 = time.perf_counter()
        oracle.recurrence(variant, inp.query, inp.key, inp.value, inp.gate, inp.beta, dtype=torch.float32)
        elapsed = time.perf_counter() - t0
        res[f"c4_{variant}_B2_T8192_H16_d128"] = {"tokens_per_s": round(vs["B"] * vs["T"] / elapsed, 1),
                                                  "s_per_pass": round(elapsed, 2)}
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=400,
                    help="untimed prefill calls before the timed ones (about 0.1 s at c2): right after the inputs are "
                         "built the GPU's clocks are still rising, and the first few tens of calls run up to 7 %% slower")
    ap.add_argument("--no-decode", action="store_true", help="skip the decode leg")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-verify", action="store_true", help="skip the speculative verify + commit leg")
    ap.add_argument("--no-fused", action="store_true", help="skip the fused-prologue prefill leg")
    ap.add_argument("--no-stack", action="store_true", help="skip the hybrid stack harness leg")
    ap.add_argument("--no-attention", action="store_true", help="skip the packed attention leg")
    ap.add_argument("--no-varlen", action="store_true", help="skip the packed varlen prefill leg")
    ap.add_argument("--no-train", action="store_true", help="skip the forward + backward (autograd) leg")
    ap.add_argument("--no-variants", action="store_true", help="skip the GDN / GLA / DeltaNet variant sweep leg")
    ap.add_argument("--cpu-budget", type=float, default=10.0, help="minimum seconds of CPU baseline work")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="after the GPU legs, copy a buffer of this many MiB three times (a plain copy kernel of "
                         "known size that calibrates rocprofv3's FETCH_SIZE / WRITE_SIZE counters)")
    opts = ap.parse_args()
    if opts.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this op family runs per (sequence, head) with no cross-GPU "
              "exchange, and multi-GPU runs are out of scope for this build.", file=sys.stderr)
        sys.exit(2)

    import torch

    gdr = importlib.import_module("gtar-kimik3-public_amd")
    workloads = importlib.import_module("gtar-kimik3-public_amd.workloads")
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)

    # The headline's inputs are built first, then the variant sweep (chunk calls of the same kernels at B=2, T=8192)
    # runs, and the headline leg follows with no idle gap.  After the GPU has idled, a stream of these calls runs
    # fast for a few calls, then up to 15 % slower for the next few tens of calls before it settles (power
    # management); the headline then measures the settled rate.  The headline leg itself is exactly `warmup`
    # untimed calls and then `steps` timed ones.
    prefill = prefill_inputs(workloads, torch)
    variants = None if opts.no_variants else bench_variants(gdr, workloads, torch, steps=50, warmup=200)
    ms = bench_prefill(gdr, prefill, torch, opts.steps, opts.warmup)
    del prefill
    cfg = PREFILL
    tokens = cfg["B"] * cfg["T"]
    nbytes = prefill_bytes(**cfg)
    flops = delta_flops_per_token_head(cfg["chunk"], cfg["K"], cfg["V"]) * tokens * cfg["H"]
    gbs = nbytes / (ms * 1e-3) / 1e9
    tflops = flops / (ms * 1e-3) / 1e12
    record = {
        "metric": "KDA prefill tokens/sec (% MFMA peak); decode-step state GB/s (% HBM peak)",
        "value": round(tokens / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": opts.steps,
        "warmup": opts.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "kda_chunk_prefill", **cfg, "state": "fp32", "gate": "fp32 per-channel"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": committed_traffic("chunk_kda_prefill")},
        "mfma_frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
        "tflops": round(tflops, 2),
        "algorithmic_bytes": nbytes,
        "algorithmic_flops": flops,
    }
    if variants is not None:
        record["variants"] = variants
    if not opts.no_decode:
        record["decode"] = bench_decode(gdr, workloads, torch, warmup=20)
    if not opts.no_verify:
        record["verify"] = bench_verify(gdr, workloads, torch, warmup=10)
    if not opts.no_fused:
        record["fused"] = bench_fused(gdr, torch, steps=20, warmup=100)
    if not opts.no_varlen:
        record["varlen"] = bench_varlen(gdr, workloads, torch, steps=10, warmup=50)
    if not opts.no_attention:
        record["attention"] = bench_attention(gdr, workloads, torch, steps=10, warmup=20)
    if not opts.no_stack:
        record["stack"] = bench_stack(gdr, workloads, torch, steps=5, warmup=2)
    if not opts.no_train:
        record["train"] = bench_train(gdr, workloads, torch, steps=10, warmup=50)
    if opts.copy_mib:
        src = torch.ones(opts.copy_mib * 2**18, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
    if not opts.no_cpu:
        record["cpu_baseline"] = cpu_baseline(workloads, torch, opts.cpu_budget)
        record["cpu_baselines_other_configs"] = cpu_baselines_other(workloads, torch, opts.cpu_budget / 4)
    print(json.dumps(record), flush=True)


if __name__ == "__main__":
    main()
