"""gdr_chunk_fwd_noalloc: the chunk forward on the library's own device scratch, called through the C ABI.

The entry point has no counterpart in the reference; it serves callers that cannot allocate device memory.  It
runs the same two launches as gdr_chunk_fwd with the workspace placed in a fixed per-GPU scratch array, so its
outputs must equal gdr_chunk_fwd's bit for bit.  Two calls in a row (the second on a smaller input) check that the
scratch keeps no state that a later call depends on; the size limit and the NULL-workspace rule are checked on the
host without a GPU.
"""

import ctypes

import pytest
import torch

from _helpers import lib, workloads

SCRATCH_BYTES = 128 << 20


def _fwd(entry, variant, inp, out_dtype=torch.bfloat16):
    """Run `entry` through the C ABI on torch's current stream; returns (out, final state)."""
    q, k, v = inp.query, inp.key, inp.value
    B, H, T, K = q.shape
    V = v.shape[-1]
    out = torch.empty(B, H, T, V, device=q.device, dtype=out_dtype)
    ht = torch.empty(B, H, K, V, device=q.device, dtype=torch.float32)
    args = lib.make_args(variant, q, k, v, inp.gate, inp.beta, out, K ** -0.5, inp.initial_state, ht)
    so = lib.load_library()
    keep = None
    if entry == "gdr_chunk_fwd":
        keep = lib.chunk_workspace(args, q.device)  # noqa: F841 (alive until the launch is enqueued)
    else:
        assert args.workspace is None
    stream = torch.cuda.current_stream(q.device).cuda_stream
    rc = getattr(so, entry)(ctypes.byref(args), ctypes.c_void_p(stream))
    assert rc == 0, so.gdr_last_error().decode()
    torch.cuda.synchronize()
    return out, ht


@pytest.mark.gpu
@pytest.mark.parametrize("variant,name", [(lib.KDA, "kda"), (lib.GDN, "gdn"), (lib.GLA, "gla"),
                                          (lib.DELTANET, "deltanet")])
def test_noalloc_matches_chunk_fwd_on_two_calls(variant, name):
    dev = torch.device("cuda")
    # first call: B=1 T=4096 H=16 d128 (1,024 records, 72.9 MB of the 128 MiB); second: smaller and ragged
    shapes = [(1, 4096, 16, 128, 128, 0), (2, 200, 4, 128, 64, 1)]
    for i, (B, T, H, K, V, seed) in enumerate(shapes):
        print(f"noalloc {name} call {i}: B={B} T={T} H={H} K={K} V={V}", flush=True)
        inp = workloads.make_inputs(name, B, T, H, K, V, seed=seed, state_std=0.02, device=dev)
        ref_o, ref_s = _fwd("gdr_chunk_fwd", variant, inp)
        out, state = _fwd("gdr_chunk_fwd_noalloc", variant, inp)
        assert torch.equal(out, ref_o), f"call {i}: out differs"
        assert torch.equal(state, ref_s), f"call {i}: final state differs"


@pytest.mark.gpu
def test_noalloc_varlen_and_fp32_out_match_chunk_fwd():
    dev = torch.device("cuda")
    lengths = [200, 0, 65, 1, 640]
    inp, cu = workloads.make_varlen_inputs("kda", lengths, 4, 128, 128, seed=3, device=dev)
    outs = []
    for entry in ("gdr_chunk_fwd", "gdr_chunk_fwd_noalloc"):
        q, k, v = inp.query, inp.key, inp.value
        out = torch.empty(v.shape, device=dev, dtype=torch.float32)
        ht = torch.empty_like(inp.initial_state)
        args = lib.make_args(lib.KDA, q, k, v, inp.gate, inp.beta, out, 0.125, inp.initial_state, ht, cu)
        keep = lib.chunk_workspace(args, dev) if entry == "gdr_chunk_fwd" else None  # noqa: F841
        so = lib.load_library()
        rc = getattr(so, entry)(ctypes.byref(args), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        assert rc == 0, so.gdr_last_error().decode()
        torch.cuda.synchronize()
        outs.append((out, ht))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])


@pytest.mark.gpu
def test_noalloc_under_graph_capture_matches_chunk_fwd():
    """gdr_chunk_fwd_noalloc captured in a torch.cuda.CUDAGraph (the callers it is for include code under graph
    capture): each replay, with eager work and a synchronisation between replays, equals eager gdr_chunk_fwd bit for
    bit.  The captured call allocates nothing, so its output buffers come from the graph's memory pool."""
    dev = torch.device("cuda")
    inp = workloads.make_inputs("kda", 1, 1000, 8, 128, 128, seed=5, state_std=0.02, device=dev)
    ref_o, ref_s = _fwd("gdr_chunk_fwd", lib.KDA, inp)
    so = lib.load_library()

    def launch(stream):
        q, k, v = inp.query, inp.key, inp.value
        out = torch.empty(v.shape, device=dev, dtype=torch.bfloat16)
        ht = torch.empty_like(inp.initial_state)
        args = lib.make_args(lib.KDA, q, k, v, inp.gate, inp.beta, out, 128 ** -0.5, inp.initial_state, ht)
        rc = so.gdr_chunk_fwd_noalloc(ctypes.byref(args), ctypes.c_void_p(stream.cuda_stream))
        assert rc == 0, so.gdr_last_error().decode()
        return out, ht

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        launch(side)  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        cap_o, cap_s = launch(torch.cuda.current_stream())
    for i in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(cap_o, ref_o) and torch.equal(cap_s, ref_s), f"replay {i}"
        _fwd("gdr_chunk_fwd", lib.KDA, inp)  # eager work between replays
        torch.cuda.synchronize()


def _host_args(B, T, H, K=128, V=128):
    """A gdr_args with placeholder (never dereferenced) pointers: the checks below fail before any device work."""
    args = lib.GdrArgs()
    args.abi_version = lib.ABI_VERSION
    args.variant = lib.KDA
    args.batch, args.heads, args.seq_len, args.key_dim, args.value_dim = B, H, T, K, V
    args.scale = K ** -0.5
    for name in ("q", "k", "v", "out"):
        view = getattr(args, name)
        view.ptr, view.dtype, view.stride_t = 0x1000, lib.BF16, K
    args.gate.ptr, args.gate.dtype, args.gate.stride_t = 0x1000, lib.F32, K
    args.beta.ptr, args.beta.dtype, args.beta.stride_t = 0x1000, lib.F32, 1
    return args


def test_noalloc_rejects_what_does_not_fit_without_a_gpu():
    so = lib.load_library()
    args = _host_args(4, 4096, 16)  # 291.5 MB of records
    assert so.gdr_chunk_workspace_bytes(ctypes.byref(args)) > SCRATCH_BYTES
    assert so.gdr_chunk_fwd_noalloc(ctypes.byref(args), None) == -2
    msg = so.gdr_last_error().decode()
    assert "gdr_chunk_fwd_noalloc" in msg and str(SCRATCH_BYTES) in msg, msg
    args = _host_args(1, 4096, 16)
    args.workspace = 0x100000
    assert so.gdr_chunk_fwd_noalloc(ctypes.byref(args), None) == -1
    assert "workspace must be NULL" in so.gdr_last_error().decode()
