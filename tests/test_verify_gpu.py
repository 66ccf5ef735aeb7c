"""Speculative-decoding verify (gdr_recurrent_verify) and prefix commit (gdr_recurrent_commit) on the GPU.

Parity: the verify outputs and final state against the fp64 token recurrence (out max-abs error <= 2e-2 * max|o|,
state relative Frobenius error <= 1e-2), and bit for bit against the recurrent op (the same kernel, which only adds
the record store).  The committed state after n accepted tokens against the recurrence over the first n tokens
(same tolerance), and bit for bit against the recurrent op run on those n tokens alone, which is the op-level form
of the reference's fork -> verify -> rollback -> replay equivalence (tests/test_speculative.py:844-893) and of its
full-accept commit equivalence (:896-936).  The one-launch cycle (gdr_recurrent_commit_verify) bit for bit against
commit followed by verify.
"""

import pytest
import torch

from _helpers import OUT_TOL, RECURRENT_FNS, STATE_TOL, gdr, oracle, oracle_args, out_error, state_error, workloads

pytestmark = pytest.mark.gpu

VERIFY_FNS = {
    "kda": gdr.verify_kimi_delta_attention,
    "gdn": gdr.verify_gated_deltanet,
    "gla": gdr.verify_gated_linear_attention,
    "deltanet": gdr.verify_deltanet,
}

SHAPES = [
    # (B, H, T, K, V): T = 1 + drafts
    (2, 4, 5, 128, 128),
    (3, 2, 8, 64, 64),
    (1, 2, 3, 128, 256),
    (2, 4, 17, 128, 128),  # three 8-token staging groups, the last one partial
    (64, 16, 8, 128, 128),  # wide 128-column slices (B * H * V / 128 >= 1024 workgroups)
]


def _prefix(inp, n):
    cut = lambda x: None if x is None else x[:, :, :n]
    return workloads.Inputs(cut(inp.query), cut(inp.key), cut(inp.value), cut(inp.gate), cut(inp.beta),
                            inp.initial_state)


@pytest.mark.parametrize("variant", oracle.VARIANTS)
@pytest.mark.parametrize("shape", SHAPES)
def test_verify_matches_oracle_and_recurrent(variant, shape):
    B, H, T, K, V = shape
    print(f"verify {variant} B={B} H={H} T={T} K={K} V={V}", flush=True)
    inp = workloads.make_inputs(variant, B, T, H, K, V, seed=11, state_std=0.5, device="cuda")
    with torch.no_grad():
        out, final, block = VERIFY_FNS[variant](*inp.args(), initial_state=inp.initial_state,
                                                output_final_state=True)
        rec_out, rec_final = RECURRENT_FNS[variant](*inp.args(), initial_state=inp.initial_state,
                                                    output_final_state=True)
    q, k, v, g, beta, h0 = oracle_args(inp)
    ref_o, ref_s = oracle.recurrence(variant, q, k, v, g, beta, None, h0)
    eo, es = out_error(out, ref_o), state_error(final, ref_s)
    print(f"  out err {eo:.2e}  state err {es:.2e}")
    assert eo <= OUT_TOL and es <= STATE_TOL
    assert torch.equal(out, rec_out) and torch.equal(final, rec_final)
    assert block.updates.shape == (B, H, T, V) and block.updates.dtype == torch.float32
    # accepting the whole block reproduces the verify's final state exactly
    assert torch.equal(block.commit(), final) and torch.equal(block.commit(T), final)


@pytest.mark.parametrize("variant", oracle.VARIANTS)
@pytest.mark.parametrize("T", [8, 17])  # 17: three groups of the 8-token staging, the last one partial
def test_commit_every_prefix(variant, T):
    B, H, K, V = 2, 3, 128, 64
    print(f"commit prefixes {variant} T={T}", flush=True)
    inp = workloads.make_inputs(variant, B, T, H, K, V, seed=12, state_std=0.5, device="cuda")
    with torch.no_grad():
        _, _, block = VERIFY_FNS[variant](*inp.args(), initial_state=inp.initial_state)
    assert torch.equal(block.commit(0), inp.initial_state)
    for n in range(1, T + 1):
        state = block.commit(n)
        part = _prefix(inp, n)
        q, k, v, g, beta, h0 = oracle_args(part)
        _, ref_s = oracle.recurrence(variant, q, k, v, g, beta, None, h0)
        es = state_error(state, ref_s)
        with torch.no_grad():
            _, replay = RECURRENT_FNS[variant](*part.args(), initial_state=part.initial_state,
                                               output_final_state=True)
        print(f"  n={n} state err {es:.2e}")
        assert es <= STATE_TOL
        assert torch.equal(state, replay), f"n={n}: commit differs from a replay of the accepted prefix"


@pytest.mark.parametrize("variant", oracle.VARIANTS)
def test_commit_per_sequence_counts_on_device(variant):
    B, H, T, K, V = 5, 2, 6, 64, 128
    print(f"commit per-sequence {variant}", flush=True)
    inp = workloads.make_inputs(variant, B, T, H, K, V, seed=13, state_std=0.5, device="cuda")
    with torch.no_grad():
        _, _, block = VERIFY_FNS[variant](*inp.args(), initial_state=inp.initial_state)
    counts = [3, 0, 6, -2, 11]  # out-of-range counts clamp to [0, T] on the device
    state = block.commit(torch.tensor(counts, dtype=torch.int32, device="cuda"))
    for b, c in enumerate(counts):
        n = min(max(c, 0), T)
        expect = block.commit(n)
        assert torch.equal(state[b], expect[b]), f"sequence {b} (count {c})"


@pytest.mark.parametrize("variant", oracle.VARIANTS)
def test_update_record(variant):
    """The record holds u_t = beta_t (v_t - k_t S_t) (v_t for GLA), S_t the decayed state before token t's write."""
    B, H, T, K, V = 2, 2, 4, 64, 64
    inp = workloads.make_inputs(variant, B, T, H, K, V, seed=14, state_std=0.5, device="cuda")
    with torch.no_grad():
        _, _, block = VERIFY_FNS[variant](*inp.args(), initial_state=inp.initial_state)
    q, k, v, g, beta, h0 = oracle_args(inp)
    if variant == "gla":
        assert torch.equal(block.updates.cpu(), v.float())
        return
    state = h0.double()
    for t in range(T):
        if g is not None:
            decay = g[:, :, t].double().exp()
            state = state * (decay[..., :, None] if g.dim() == 4 else decay[..., None, None])
        kt = k[:, :, t].double()
        u = beta[:, :, t, None].double() * (v[:, :, t].double() - torch.einsum("bhk,bhkv->bhv", kt, state))
        err = ((block.updates[:, :, t].double().cpu() - u).abs().max() / u.abs().max()).item()
        assert err <= 1e-3, f"t={t}: record error {err:.2e}"
        state = state + kt[..., :, None] * u[..., None, :]


def test_commit_in_place_and_zero_initial_state():
    B, H, T, K, V = 2, 2, 5, 128, 128
    inp = workloads.make_inputs("kda", B, T, H, K, V, seed=15, state_std=None, device="cuda")
    with torch.no_grad():
        _, final, block = gdr.verify_kimi_delta_attention(*inp.args(), output_final_state=True)
    assert torch.count_nonzero(block.commit(0)) == 0
    state = torch.randn(B, H, K, V, device="cuda")
    inp2 = workloads.make_inputs("kda", B, T, H, K, V, seed=16, device="cuda")
    with torch.no_grad():
        _, final2, block2 = gdr.verify_kimi_delta_attention(*inp2.args(), initial_state=state,
                                                            output_final_state=True)
    block2.commit(T, out=state)  # in place over the block's own initial state
    assert torch.equal(state, final2)


def test_cache_fork_verify_accept_equals_clean_run():
    """RecurrentCache: fork -> verify(1 + K) -> accept(n) leaves the state and length a clean run over the n accepted
    tokens would; rollback restores the forked state exactly (tests/test_speculative.py:784-841, 844-936)."""
    B, H, T, K, V = 1, 4, 5, 128, 128
    for n in (0, 1, T - 1, T):
        print(f"cache accept n={n}", flush=True)
        inp = workloads.make_inputs("kda", B, T, H, K, V, seed=17, state_std=0.5, device="cuda")
        cache = gdr.RecurrentCache(B, H, K, V, 8, 4, "cuda", torch.bfloat16)
        cache.update(inp.initial_state.clone(), 7)
        saved = cache.state.clone()
        cache.fork()
        with torch.no_grad():
            _, final, block = gdr.verify_kimi_delta_attention(*inp.args(), initial_state=cache.state,
                                                              output_final_state=True)
        cache.update(final, T)  # what the layer does after a verify forward
        cache.rollback()
        assert torch.equal(cache.state, saved) and cache.seq_len == 7
        cache.fork()
        cache.accept(n, block)
        assert cache.seq_len == 7 + n
        if n == 0:
            assert torch.equal(cache.state, saved)
            continue
        part = _prefix(inp, n)
        with torch.no_grad():
            _, clean = gdr.recurrent_kimi_delta_attention(*part.args(), initial_state=saved, output_final_state=True)
        assert torch.equal(cache.state, clean)


def _accept_counts(B, T):
    """Per-sequence accept counts on the device covering 0, T and values in between."""
    counts = [(3 * i) % (T + 1) for i in range(B)]
    counts[0], counts[-1] = 0, T
    return torch.tensor(counts, dtype=torch.int32, device="cuda")


@pytest.mark.parametrize("variant", oracle.VARIANTS)
@pytest.mark.parametrize("shape", [(2, 4, 8, 5, 128, 128), (3, 2, 3, 8, 64, 64), (64, 16, 8, 8, 128, 128),
                                   (2, 4, 17, 9, 128, 128), (3, 2, 9, 17, 64, 64)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_commit_verify_equals_commit_then_verify(variant, shape, dtype):
    """One launch per cycle against the two-launch cycle: out, the new record, the committed state and the final
    state bit for bit, with per-sequence accept counts on the device, a previous block of another length, and a
    previous block that started from a zero state."""
    B, H, Tp, T, K, V = shape
    fn = VERIFY_FNS[variant]
    acc = _accept_counts(B, Tp)
    for state_std in (0.5, None):
        print(f"commit-verify {variant} {dtype} B={B} H={H} Tp={Tp} T={T} K={K} V={V} h0={state_std}", flush=True)
        prev = workloads.make_inputs(variant, B, Tp, H, K, V, seed=21, dtype=dtype, state_std=state_std,
                                     device="cuda")
        nxt = workloads.make_inputs(variant, B, T, H, K, V, seed=22, dtype=dtype, device="cuda")
        with torch.no_grad():
            _, _, block = fn(*prev.args(), initial_state=prev.initial_state)
            committed = block.commit(acc)
            out_ref, final_ref, block_ref = fn(*nxt.args(), initial_state=committed, output_final_state=True)
            out, final, new_block = fn(*nxt.args(), output_final_state=True, pending=block, accepted=acc)
        assert torch.equal(new_block.initial_state, committed)
        assert torch.equal(out, out_ref) and torch.equal(final, final_ref)
        assert torch.equal(new_block.updates, block_ref.updates)


def test_commit_verify_chain_in_place():
    """Three cycles, each committing over the previous block's initial state in place, with int, None (all tokens)
    and zero accept counts, against the two-launch cycle; then a cycle whose blocks differ in dtype, which takes the
    two-launch path."""
    B, H, T, K, V = 4, 4, 6, 128, 128
    inputs = [workloads.make_inputs("kda", B, T, H, K, V, seed=30 + i, device="cuda") for i in range(4)]
    state0 = torch.randn(B, H, K, V, device="cuda") * 0.3
    fn = gdr.verify_kimi_delta_attention
    counts = (3, None, 0)
    with torch.no_grad():
        ref = []
        _, _, blk = fn(*inputs[0].args(), initial_state=state0.clone())
        for inp, n in zip(inputs[1:], counts):
            s = blk.commit(n)
            o, _, blk = fn(*inp.args(), initial_state=s)
            ref.append((o, s))
        s = state0.clone()
        _, _, blk = fn(*inputs[0].args(), initial_state=s)
        for (o_ref, s_ref), inp, n in zip(ref, inputs[1:], counts):
            print(f"in-place cycle accepted={n}", flush=True)
            o, _, blk = fn(*inp.args(), pending=blk, accepted=n, committed_out=blk.initial_state)
            assert blk.initial_state.data_ptr() == s.data_ptr()
            assert torch.equal(o, o_ref) and torch.equal(blk.initial_state, s_ref)
        f32 = workloads.make_inputs("kda", B, T, H, K, V, seed=40, dtype=torch.float32, device="cuda")
        o_mixed, _, _ = fn(*f32.args(), pending=blk, accepted=2)
        o_two, _, _ = fn(*f32.args(), initial_state=blk.commit(2))
    assert torch.equal(o_mixed, o_two)
