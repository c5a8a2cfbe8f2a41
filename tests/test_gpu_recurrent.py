"""GPU parity of the recurrent decode / spec-verify kernel (kda355_recurrent_launch) against the CPU oracle.

Bars (north star): output max-abs error beyond bf16 storage rounding <= 2e-2 x RMS(ref); states relative Frobenius
<= 1e-3; which pool rows are written is bit-exact (every other row bit-identical).
"""
import numpy as np
import pytest
import torch

from helpers import STATE_TOL, check_out, config_inputs, f32, gen, rel_frob

pytestmark = pytest.mark.gpu
D = 128


def _kda():
    import kda355
    return kda355


def _say(msg):
    print(f"[case] {msg}", flush=True)


def _cu_tokens(B, S):
    return np.arange(0, B * S + 1, S)


def _run_case(oracle, B, S, H, slots, seed, spec, raw=False, pad_rows=(), graph=False, qk_norms=False):
    kda = _kda()
    _say(f"recurrent B={B} S={S} H={H} slots={slots} spec={spec} raw={raw} pad={pad_rows} graph={graph} "
         f"qk_norms={qk_norms} seed={seed}")
    g = gen(seed)
    T = B * S
    q, k, v, gg, beta = config_inputs(T, H, g)
    if qk_norms:
        # rows of norm 1e-3 .. 10 (log-uniform): the in-kernel x rsqrt(|x|^2 + 1e-6) is not the identity on them
        for t in (q, k):
            t.copy_((t.float() * torch.exp(torch.empty(T, H, 1).uniform_(np.log(1e-3), np.log(10.0),
                                                                          generator=g))).bfloat16())
    pool = torch.randn(slots, H, D, D, generator=g) * 0.05
    perm = torch.randperm(slots - 1, generator=g)[: B * S] + 1
    idx = perm.view(B, S).to(torch.int32) if spec else perm[:B].to(torch.int32)
    for (n, t) in pad_rows:
        if spec:
            idx[n, t] = 0
        else:
            idx[n] = 0
    acc = torch.randint(1, S + 1, (B,), generator=g, dtype=torch.int32) if spec else None
    A_log = torch.rand(H, generator=g) * 2.0
    dt_bias = torch.randn(H * D, generator=g) * 0.5
    raw_g = torch.randn(T, H, D, generator=g).bfloat16()
    raw_beta = torch.randn(T, H, generator=g).bfloat16()
    dev = torch.device("cuda", 0)
    dq, dk, dv = (x[None].to(dev) for x in (q, k, v))
    dpool = pool.to(dev)
    didx = idx.to(dev)
    dacc = acc.to(dev) if spec else None
    cu = torch.arange(0, T + 1, S, dtype=torch.int32, device=dev)
    kw = dict(initial_state=dpool, cu_seqlens=cu, ssm_state_indices=didx, num_accepted_tokens=dacc)
    if raw:
        kw.update(raw_g=raw_g[None].to(dev), raw_beta=raw_beta[None].to(dev), A_log=A_log.to(dev),
                  dt_bias=dt_bias.to(dev), lower_bound=-5.0)
    else:
        kw.update(g=gg[None].to(dev), beta=beta[None].to(dev))
    if graph:
        out = torch.empty(1, T, H, D, dtype=torch.bfloat16, device=dev)
        kw["out"] = out
        kda.fused_recurrent_kda(dq, dk, dv, **kw)        # warm-up outside capture
        torch.cuda.synchronize()
        dpool.copy_(pool.to(dev))
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            kda.fused_recurrent_kda(dq, dk, dv, **kw)
        gr.replay()
    else:
        out, _ = kda.fused_recurrent_kda(dq, dk, dv, **kw)
    torch.cuda.synchronize()
    if raw:
        from oracle import oracle as O
        g_np = O.gate(f32(raw_g), f32(A_log), f32(dt_bias), -5.0)
        b_np = O.sigmoid(f32(raw_beta))
    else:
        g_np, b_np = f32(gg), f32(beta)
    ro, rpool, written = oracle.recurrent(f32(q), f32(k), f32(v), g_np, b_np, f32(pool), idx.numpy(),
                                          acc.numpy() if spec else None, precision=64)
    got_pool = dpool.cpu().numpy()
    check_out(out[0], ro, f"recurrent B={B} S={S} H={H}", _cu_tokens(B, S))
    for r in sorted(set(written)):
        e = rel_frob(got_pool[r], rpool[r])
        assert e <= STATE_TOL, f"pool row {r}: relF {e:.3e}"
    keep = np.ones(slots, bool)
    keep[list(set(written))] = False
    assert np.array_equal(got_pool[keep], f32(pool)[keep]), "rows outside the written set changed"
    return out, dpool


def test_plain_decode_small(oracle):
    _run_case(oracle, B=16, S=1, H=4, slots=40, seed=1, spec=False)


def test_plain_decode_padding_slot(oracle):
    _run_case(oracle, B=8, S=1, H=2, slots=20, seed=2, spec=False, pad_rows=[(3, 0)])


def test_spec_verify(oracle):
    _run_case(oracle, B=8, S=4, H=4, slots=64, seed=3, spec=True)


def test_spec_verify_padding_writes(oracle):
    _run_case(oracle, B=6, S=4, H=2, slots=40, seed=4, spec=True, pad_rows=[(0, 3), (2, 1)])


def test_raw_gate_beta(oracle):
    _run_case(oracle, B=8, S=2, H=4, slots=32, seed=5, spec=True, raw=True)
    _run_case(oracle, B=8, S=1, H=4, slots=32, seed=6, spec=False, raw=True)


def test_non_unit_qk_norms(oracle):
    """q / k rows of norms 1e-3 .. 10: the decode form x rsqrt(|x|^2 + 1e-6) (reference.py:159-160) shrinks the small
    ones below unit norm, which the oracle's decode form reproduces and the prefill clamp form would not."""
    _run_case(oracle, B=16, S=1, H=4, slots=40, seed=8, spec=False, qk_norms=True)
    _run_case(oracle, B=8, S=3, H=4, slots=40, seed=9, spec=True, qk_norms=True)


def test_graph_capture_replay(oracle):
    _run_case(oracle, B=32, S=1, H=8, slots=64, seed=7, spec=False, graph=True)


def test_graph_replay_new_indices_and_data(oracle):
    """Capture once, then replay after refilling inputs, indices and the pool in place (HANDOVER.md:72-73 rule)."""
    kda = _kda()
    B, H, slots = 16, 4, 48
    dev = torch.device("cuda", 0)
    _say(f"graph re-replay B={B} H={H}")
    g = gen(11)
    bufs = dict(q=torch.empty(1, B, H, D, dtype=torch.bfloat16, device=dev),
                k=torch.empty(1, B, H, D, dtype=torch.bfloat16, device=dev),
                v=torch.empty(1, B, H, D, dtype=torch.bfloat16, device=dev),
                g=torch.empty(1, B, H, D, device=dev), beta=torch.empty(1, B, H, device=dev))
    pool = torch.zeros(slots, H, D, D, device=dev)
    idx = torch.ones(B, dtype=torch.int32, device=dev)
    out = torch.empty(1, B, H, D, dtype=torch.bfloat16, device=dev)
    cu = torch.arange(0, B + 1, dtype=torch.int32, device=dev)

    def call():
        kda.fused_recurrent_kda(bufs["q"], bufs["k"], bufs["v"], bufs["g"], bufs["beta"], initial_state=pool,
                                cu_seqlens=cu, ssm_state_indices=idx, out=out)

    call()
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        call()
    for rep in range(3):
        q, k, v, gg, beta = config_inputs(B, H, g)
        p0 = torch.randn(slots, H, D, D, generator=g) * 0.05
        ix = (torch.randperm(slots - 1, generator=g)[:B] + 1).to(torch.int32)
        for name, x in (("q", q), ("k", k), ("v", v), ("g", gg), ("beta", beta)):
            bufs[name].copy_(x[None])
        pool.copy_(p0)
        idx.copy_(ix)
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        ro, rpool, written = oracle.recurrent(f32(q), f32(k), f32(v), f32(gg), f32(beta), f32(p0), ix.numpy(),
                                              precision=64)
        check_out(out[0], ro, f"replay {rep}", _cu_tokens(B, 1))
        got = pool.cpu().numpy()
        for r in written:
            assert rel_frob(got[r], rpool[r]) <= STATE_TOL, f"replay {rep}: row {r}"
        keep = np.ones(slots, bool)
        keep[written] = False
        assert np.array_equal(got[keep], f32(p0)[keep]), f"replay {rep}: unwritten rows changed"


def test_spec_scratch_commit(oracle):
    """Config-4 form: verify writes per-token states to a [B, S] scratch, then the accepted length is committed."""
    kda = _kda()
    B, S, H, slots = 8, 4, 4, 40
    dev = torch.device("cuda", 0)
    _say(f"spec scratch + commit B={B} S={S} H={H}")
    g = gen(21)
    q, k, v, gg, beta = config_inputs(B * S, H, g)
    pool = torch.randn(slots, H, D, D, generator=g) * 0.05
    pslot = (torch.randperm(slots - 1, generator=g)[:B] + 1).to(torch.int32)
    acc = torch.randint(1, S + 1, (B,), generator=g, dtype=torch.int32)
    dpool = pool.to(dev)
    scratch = torch.full((B * S, H, D, D), float("nan"), device=dev)
    sidx = torch.arange(B * S, dtype=torch.int32, device=dev).view(B, S)
    cu = torch.arange(0, B * S + 1, S, dtype=torch.int32, device=dev)
    read_idx = pslot.view(B, 1).repeat(1, S).contiguous().to(dev)   # every token reads the committed slot
    ones = torch.ones(B, dtype=torch.int32, device=dev)
    out, _ = kda.fused_recurrent_kda(q[None].to(dev), k[None].to(dev), v[None].to(dev), gg[None].to(dev),
                                     beta[None].to(dev), initial_state=dpool, cu_seqlens=cu,
                                     ssm_state_indices=read_idx, num_accepted_tokens=ones, write_pool=scratch,
                                     write_indices=sidx)
    kda.spec_commit(scratch, sidx, dpool, pslot.to(dev), acc.to(dev))
    torch.cuda.synchronize()
    # oracle: per-token states from the committed slot, then pool[slot] = state after token a-1
    S_in = f32(pool)[pslot.numpy()]
    from oracle import oracle as O
    ro, steps = O.recurrent_core(O.l2norm_rsqrt(f32(q)), O.l2norm_rsqrt(f32(k)), f32(v), f32(gg), f32(beta), S_in,
                                 D ** -0.5, precision=64)
    check_out(out[0], ro, "spec scratch", _cu_tokens(B, S))
    sc = scratch.cpu().numpy().reshape(B, S, H, D, D)
    for n in range(B):
        for t in range(S):
            assert rel_frob(sc[n, t], steps[n, t]) <= STATE_TOL
    got = dpool.cpu().numpy()
    for n in range(B):
        assert rel_frob(got[pslot[n]], steps[n, acc[n] - 1]) <= STATE_TOL
    keep = np.ones(slots, bool)
    keep[pslot.numpy()] = False
    assert np.array_equal(got[keep], f32(pool)[keep])


def test_errors_raise():
    kda = _kda()
    dev = torch.device("cuda", 0)
    q = torch.zeros(1, 4, 2, D, dtype=torch.bfloat16, device=dev)
    pool = torch.zeros(8, 2, D, D, device=dev)
    idx = torch.arange(1, 5, dtype=torch.int32, device=dev)
    cu = torch.arange(0, 5, dtype=torch.int32, device=dev)
    gg = torch.zeros(1, 4, 2, D, device=dev)
    beta = torch.zeros(1, 4, 2, device=dev)
    with pytest.raises(TypeError):
        kda.fused_recurrent_kda(q, q, q, gg.double(), beta, initial_state=pool, cu_seqlens=cu, ssm_state_indices=idx)
    with pytest.raises(ValueError):
        kda.fused_recurrent_kda(q, q, q, gg, beta, initial_state=pool, cu_seqlens=cu, ssm_state_indices=idx[::2])
    with pytest.raises(TypeError):
        kda.fused_recurrent_kda(q, q, q, gg, beta, initial_state=pool, cu_seqlens=cu, ssm_state_indices=idx.cpu())


@pytest.mark.parametrize("spec", [False, True])
def test_slot0_live_when_not_reserved(oracle, spec):
    """slot0_reserved=False makes slot 0 an ordinary pool row (read and written like any other); rows < 0 stay padding.
    Checked against the oracle's reserved-slot-0 semantics on the pool shifted by one row (kernel slot s = oracle
    slot s + 1, so the oracle's padding slot 0 is the kernel's -1)."""
    kda = _kda()
    B, S, H, slots = (6, 3, 2, 24) if spec else (8, 1, 2, 16)
    _say(f"recurrent slot0 live spec={spec} B={B} S={S}")
    g = gen(40 + spec)
    T = B * S
    q, k, v, gg, beta = config_inputs(T, H, g)
    pool = torch.randn(slots, H, D, D, generator=g) * 0.05
    perm = torch.randperm(slots, generator=g)[:B * S]
    perm[perm == 0] = perm[0].item()
    perm[0] = 0  # slot 0 is used
    idx = perm.view(B, S).to(torch.int32) if spec else perm[:B].to(torch.int32)
    if spec:
        idx[B - 1, 1] = -1  # a padding write row
    else:
        idx[B - 1] = -1     # a padding sequence
    acc = torch.randint(1, S + 1, (B,), generator=g, dtype=torch.int32) if spec else None
    dev = torch.device("cuda", 0)
    dpool = pool.to(dev)
    cu = torch.arange(0, T + 1, S, dtype=torch.int32, device=dev)
    out, _ = kda.fused_recurrent_kda(q[None].to(dev), k[None].to(dev), v[None].to(dev), gg[None].to(dev),
                                     beta[None].to(dev), initial_state=dpool, cu_seqlens=cu,
                                     ssm_state_indices=idx.to(dev),
                                     num_accepted_tokens=acc.to(dev) if spec else None, slot0_reserved=False)
    torch.cuda.synchronize()
    pool_o = np.concatenate([np.zeros((1, H, D, D), np.float32), f32(pool)])
    ro, rpool, written = oracle.recurrent(f32(q), f32(k), f32(v), f32(gg), f32(beta), pool_o, idx.numpy() + 1,
                                          acc.numpy() if spec else None, precision=64)
    assert 1 in set(written), "the oracle must write the kernel's slot 0 (its row 1)"
    check_out(out[0], ro, f"recurrent slot0 live spec={spec}", _cu_tokens(B, S))
    got = dpool.cpu().numpy()
    for r in sorted(set(written)):
        e = rel_frob(got[r - 1], rpool[r])
        assert e <= STATE_TOL, f"pool row {r - 1}: relF {e:.3e}"
    keep = np.ones(slots, bool)
    keep[[r - 1 for r in set(written)]] = False
    assert np.array_equal(got[keep], f32(pool)[keep]), "rows outside the written set changed"
