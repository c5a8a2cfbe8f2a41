"""GPU parity at the full sizes of BASELINE.json's configurations, through the same calls and kernel variants that
bench.py times.

* config 3: fused_recurrent_kda, B = 256, H = 32, a 4096-slot pool (8 GiB), captured and replayed (the launch writes
  512 MiB of state, above the streaming threshold: recurrent_kernel<..., NT = true>);
* config 4: spec verify B = 64 x S = 4 at H = 64 and 96 on a 1024-slot pool, per-token states to a [64, 4, H, 128,
  128] scratch, then the commit of the accepted lengths (verify writes 1 / 1.5 GiB: the streaming variant);
* config 2: one T = 131072 sequence at H = 32 on a 64-slot pool, 32 bf16 every-4096 checkpoint rows through a row
  table (the split plan: 8 pieces, scan, output fixup and checkpoint compose), then the same call in precise mode
  at half the output and state bars;
* config 1 serving form: the config-1 lengths at H = 32 through prefill_prepare / prefill with one checkpoint per
  sequence inside the later pieces (every split sequence in 2 pieces: the scan, fixup and checkpoint compose run in
  one tail launch), and the every-n bf16 variant.

Inputs are generated on the device from seeded generators (the full-size inputs are GBs); the oracle (fp64) runs on
the rows and heads it checks, copied back.  Rows outside the written set are compared on the device with saved
copies, so every other byte of the pools is checked bit for bit.
"""
import numpy as np
import pytest
import torch

from helpers import OUT_TOL, STATE_TOL, check_out, f32, rel_frob

pytestmark = pytest.mark.gpu
D = 128
C2_TRIP = 1.5e-2   # config 2's default-mode output excess, 1.2 x the measured 1.25e-2 (the bar is OUT_TOL)
DEV = torch.device("cuda", 0)


def _kda():
    import kda355
    return kda355


def _say(msg):
    print(f"[case] {msg}", flush=True)


def _synth(T, H, seed):
    """The configs' distributions on the device: q, k fp32 N(0,1) L2-normalized then bf16, v bf16 N(0,1),
    g = -softplus(N(0,1)) fp32, beta = sigmoid(N(0,1)) fp32."""
    gen = torch.Generator(device=DEV).manual_seed(seed)
    out = [torch.nn.functional.normalize(torch.randn(1, T, H, D, generator=gen, device=DEV), dim=-1).bfloat16()
           for _ in range(2)]
    out.append(torch.randn(1, T, H, D, generator=gen, device=DEV).bfloat16())
    out.append(-torch.nn.functional.softplus(torch.randn(1, T, H, D, generator=gen, device=DEV)))
    out.append(torch.sigmoid(torch.randn(1, T, H, generator=gen, device=DEV)))
    return out


def _heads(x, hs):
    """[1, T, H, ...] device tensor -> numpy [T, len(hs), ...] of the checked heads."""
    return np.ascontiguousarray(f32(x[0][:, hs]))


# ------------------------------------------------------------------------------------------------ config 3
def test_config3_decode_full_size_graph_replay(oracle):
    kda = _kda()
    B, H, slots = 256, 32, 4096
    _say(f"config 3: recurrent B={B} H={H} slots={slots}, graph replay x2")
    q, k, v = (torch.empty(1, B, H, D, dtype=torch.bfloat16, device=DEV) for _ in range(3))
    g = torch.empty(1, B, H, D, device=DEV)
    beta = torch.empty(1, B, H, device=DEV)
    pool = torch.empty(slots, H, D, D, device=DEV)
    idx = torch.ones(B, dtype=torch.int32, device=DEV)
    cu = torch.arange(0, B + 1, dtype=torch.int32, device=DEV)
    out = torch.empty(1, B, H, D, dtype=torch.bfloat16, device=DEV)

    def call():
        kda.fused_recurrent_kda(q, k, v, g, beta, initial_state=pool, cu_seqlens=cu, ssm_state_indices=idx, out=out)

    pool.zero_()
    call()
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        call()
    for rep in range(2):
        seed = 3 + 100 * rep
        for dst, src in zip((q, k, v, g, beta), _synth(B, H, seed)):
            dst.copy_(src)
        pool.normal_(0.0, 0.05, generator=torch.Generator(device=DEV).manual_seed(seed))
        ix = torch.randperm(slots - 1, generator=torch.Generator().manual_seed(seed))[:B] + 1
        idx.copy_(ix.to(torch.int32))
        before = pool.clone()
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        # the oracle on a compact pool: row 0 (padding), then the B read rows in order
        rows = ix.to(DEV)
        compact = np.zeros((B + 1, H, D, D), np.float32)
        compact[1:] = before[rows].cpu().numpy()
        ro, rpool, written = oracle.recurrent(f32(q[0]), f32(k[0]), f32(v[0]), f32(g[0]), f32(beta[0]), compact,
                                              np.arange(1, B + 1), precision=64)
        check_out(out[0], ro, f"config 3 replay {rep}", np.arange(B + 1))
        got = pool[rows].cpu().numpy()
        worst = max(rel_frob(got[n], rpool[n + 1]) for n in range(B))
        _say(f"config 3 replay {rep}: worst written-row relF {worst:.2e}")
        assert worst <= STATE_TOL
        before[rows] = pool[rows]
        assert torch.equal(pool, before), "rows outside the 256 written slots changed"


# ------------------------------------------------------------------------------------------------ config 4
@pytest.mark.parametrize("H", [64, 96])
def test_config4_spec_verify_and_commit_full_size(oracle, H):
    kda = _kda()
    B, S, slots = 64, 4, 1024
    T = B * S
    _say(f"config 4: spec verify B={B} S={S} H={H} slots={slots} + commit, graph")
    q, k, v, g, beta = _synth(T, H, 4 + H)
    pool = torch.empty(slots, H, D, D, device=DEV)
    pool.normal_(0.0, 0.05, generator=torch.Generator(device=DEV).manual_seed(4 + H))
    cpu = torch.Generator().manual_seed(4 + H)
    slot = torch.randperm(slots - 1, generator=cpu)[:B] + 1
    acc = torch.randint(1, S + 1, (B,), generator=cpu)
    read_idx = slot.view(B, 1).expand(B, S).contiguous().to(torch.int32).to(DEV)
    scratch = torch.full((T, H, D, D), float("nan"), device=DEV)
    scratch_idx = torch.arange(T, dtype=torch.int32, device=DEV).view(B, S)
    pool_idx = slot.to(torch.int32).to(DEV)
    accd = acc.to(torch.int32).to(DEV)
    cu = torch.arange(0, T + 1, S, dtype=torch.int32, device=DEV)
    out = torch.full((1, T, H, D), float("nan"), dtype=torch.bfloat16, device=DEV)
    before = pool.clone()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        kda.fused_recurrent_kda(q, k, v, g, beta, initial_state=pool, cu_seqlens=cu, ssm_state_indices=read_idx,
                                num_accepted_tokens=accd, out=out, write_pool=scratch, write_indices=scratch_idx)
        kda.spec_commit(scratch, scratch_idx, pool, pool_idx, accd)
    gr.replay()
    torch.cuda.synchronize()
    S_in = before[pool_idx.long()].cpu().numpy()
    ro, steps = oracle.recurrent_core(oracle.l2norm_rsqrt(f32(q[0])), oracle.l2norm_rsqrt(f32(k[0])), f32(v[0]),
                                      f32(g[0]), f32(beta[0]), S_in, D ** -0.5, precision=64)
    check_out(out[0], ro, f"config 4 H={H}", np.arange(0, T + 1, S))
    sc = scratch.view(B, S, H, D, D)
    worst = 0.0
    for n in range(B):
        got = sc[n].cpu().numpy()
        worst = max(worst, max(rel_frob(got[t], steps[n, t]) for t in range(S)))
    committed = pool[pool_idx.long()].cpu().numpy()
    worst_c = max(rel_frob(committed[n], steps[n, int(acc[n]) - 1]) for n in range(B))
    _say(f"config 4 H={H}: worst scratch relF {worst:.2e}, worst committed relF {worst_c:.2e}")
    assert worst <= STATE_TOL and worst_c <= STATE_TOL
    before[pool_idx.long()] = pool[pool_idx.long()]
    assert torch.equal(pool, before), "pool rows other than the 64 committed slots changed"


# ------------------------------------------------------------------------------------------------ config 2
def test_config2_full_size_every_n_bf16(oracle):
    kda = _kda()
    T, H, slots, every, nck = 131072, 32, 64, 4096, 32
    hs = [0, 13, 31]
    q, k, v, g, beta = _synth(T, H, 5)
    cpu = torch.Generator().manual_seed(5)
    slot = torch.randperm(slots, generator=cpu)[:1].to(torch.int32)
    pool = torch.empty(slots, H, D, D, device=DEV)
    pool.normal_(0.0, 0.02, generator=torch.Generator(device=DEV).manual_seed(5))
    ck_rows = torch.randperm(64, generator=cpu)[:nck].to(torch.int32)
    ck = torch.full((64, H, D, D), float("nan"), dtype=torch.bfloat16, device=DEV)
    meta = kda.plan(torch.tensor([0, T], dtype=torch.int64), H, ck_every=every, device=DEV)
    _say(f"config 2: T={T} H={H} every={every} bf16 rows, pieces={meta.split} ck tasks={meta.plan.num_ck_tasks}")
    assert meta.split[0] >= 2 and meta.plan.num_ck_tasks > 0 and meta.ck_rows == nck
    before = pool.clone()
    init = pool[slot.long()].clone()
    s0 = pool[slot.long()][0][hs].cpu().numpy()
    o, fin, ckr = kda.chunk_kda(q, k, v, g, beta, initial_state=pool, meta=meta, ssm_state_indices=slot.to(DEV),
                                state_checkpoints=ck, checkpoint_every_n_tokens=every,
                                checkpoint_state_indices=ck_rows.to(DEV))
    torch.cuda.synchronize()
    ro, rf, rrows, _ = oracle.checkpoints_every_n(_heads(q, hs), _heads(k, hs), _heads(v, hs), _heads(g, hs),
                                                 np.ascontiguousarray(f32(beta[0][:, hs])), [0, T], every,
                                                 initial_state=s0[None], precision=64)
    ex = check_out(o[0][:, hs], ro, "config 2", [0, T])
    # The worst element sits near 10 x RMS with a relative error of ~1.2e-3 of its own size (measured 1.25e-2; the
    # 99.99th percentile of the excess is 2.7e-3): a tripwire 20 % above it fails a precision regression here first.
    assert ex <= C2_TRIP, f"config 2: excess {ex:.3e} above the regression tripwire {C2_TRIP}"
    e = rel_frob(pool[int(slot)][hs].cpu().numpy(), rf[0])
    got = ck[ck_rows.long()][:, hs].float().cpu().numpy()
    worst = 0.0
    for j in range(nck):
        bound = rel_frob(oracle.bf16_round(rrows[j]), rrows[j]) + STATE_TOL
        ej = rel_frob(got[j], rrows[j])
        assert ej <= bound, f"checkpoint row {j}: relF {ej:.3e} > {bound:.3e}"
        worst = max(worst, ej)
    _say(f"config 2: final-state relF {e:.2e}, worst bf16 checkpoint relF {worst:.2e}")
    assert e <= STATE_TOL
    before[slot.long()] = pool[slot.long()]
    assert torch.equal(pool, before), "pool slots other than the sequence's changed"
    unlisted = sorted(set(range(64)) - set(ck_rows.tolist()))
    assert bool(torch.isnan(ck[unlisted].float()).all()), "checkpoint rows outside the row table changed"

    # precise mode (fp16 pairs in the solve and the state update) on the same inputs and plan: half the output bar
    # (measured 8.7e-3) and half the state bar (measured 2.3e-4)
    pool[slot.long()] = init
    o, fin = kda.chunk_kda(q, k, v, g, beta, initial_state=pool, meta=meta, ssm_state_indices=slot.to(DEV),
                           precise=True)
    torch.cuda.synchronize()
    ex = check_out(o[0][:, hs], ro, "config 2 precise", [0, T])
    e = rel_frob(pool[int(slot)][hs].cpu().numpy(), rf[0])
    _say(f"config 2 precise: final-state relF {e:.2e}")
    assert ex <= 0.5 * OUT_TOL and e <= 0.5 * STATE_TOL


# ------------------------------------------------------------------------------------------------ config 1, serving
def _c1_lens():
    rng = np.random.default_rng(1)
    return [int(x) for x in rng.integers(256, 8193, size=8)]


def _raw_inputs_dev(T, H, seed):
    gen = torch.Generator(device=DEV).manual_seed(seed)
    q, k, v, raw_g = (torch.randn(1, T, H, D, generator=gen, device=DEV).bfloat16() for _ in range(4))
    raw_b = torch.randn(1, T, H, generator=gen, device=DEV).bfloat16()
    A_log = torch.rand(H, generator=gen, device=DEV) * 2 - 1
    dt_bias = torch.randn(H * D, generator=gen, device=DEV) * 0.5
    return q, k, v, raw_g, raw_b, A_log, dt_bias


def test_config1_serving_two_piece_tail_with_checkpoints(oracle):
    """The config-1 layout through the serving call with a checkpoint per sequence placed inside the later piece of
    every split sequence: the plan splits each long sequence in 2 pieces, so the scan, the output fixup and the
    checkpoint compose run in one tail launch."""
    kda = _kda()
    lens = _c1_lens()
    H, N = 32, len(lens)
    T = sum(lens)
    hs = [0, 17, 31]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    ck_off = [64 * max(1, (L * 9 // 10) // 64) for L in lens]
    slots = 2 * N + 5
    perm = torch.randperm(slots - 1, generator=torch.Generator().manual_seed(7)) + 1
    sidx, cidx = perm[:N].to(torch.int32), perm[N:2 * N].to(torch.int32)
    hinit = [n % 3 != 1 for n in range(N)]
    cu_cpu = torch.tensor(cu, dtype=torch.int32)
    meta = kda.prefill_prepare(cu_cpu, H, torch.tensor(ck_off, dtype=torch.int32), cidx, device=DEV)
    pl = meta.plan
    _say(f"config 1 serving: pieces={meta.split} fix={pl.num_fix_tasks} ck tasks={pl.num_ck_tasks}")
    assert pl.num_split > 0 and pl.num_pieces == 2 * pl.num_split and pl.num_ck_tasks > 0
    q, k, v, raw_g, raw_b, A_log, dt_bias = _raw_inputs_dev(T, H, 11)
    pool = torch.empty(slots, H, D, D, device=DEV)
    pool.normal_(0.0, 0.05, generator=torch.Generator(device=DEV).manual_seed(12))
    for n in range(N):
        if not hinit[n]:
            pool[int(sidx[n])] = float("nan")
        pool[int(cidx[n])] = float("nan")
    before = pool.clone()
    pool0 = before[:, hs].cpu().numpy()
    out = torch.full((1, T, H, D), float("nan"), dtype=torch.bfloat16, device=DEV)
    kda.prefill(q, k, v, raw_g, raw_b, A_log, dt_bias, D ** -0.5, -5.0, pool, sidx.to(DEV),
                torch.tensor(hinit, dtype=torch.bool, device=DEV), cu_cpu.to(DEV), out,
                torch.tensor(ck_off, dtype=torch.int32, device=DEV), cidx.to(DEV), meta=meta)
    torch.cuda.synchronize()
    dtb = dt_bias.view(H, D)[hs].reshape(-1)
    ro, rnew = oracle.prefill_serving(_heads(q, hs), _heads(k, hs), _heads(v, hs), _heads(raw_g, hs),
                                      np.ascontiguousarray(f32(raw_b[0][:, hs])), f32(A_log[hs]), f32(dtb), -5.0,
                                      D ** -0.5, pool0, sidx.numpy(), np.array(hinit), cu, np.array(ck_off),
                                      cidx.numpy(), precision=64)
    check_out(out[0][:, hs], ro, "config 1 serving", cu)
    written = [int(s) for s in sidx] + [int(c) for c in cidx]
    got = pool[:, hs].cpu().numpy()
    worst = max(rel_frob(got[r], rnew[r]) for r in written)
    _say(f"config 1 serving: worst written-row relF {worst:.2e}")
    assert worst <= STATE_TOL
    before[written] = pool[written]
    assert torch.equal(pool, before), "pool rows outside the written set changed"


def test_config1_every_n_bf16_checkpoints(oracle):
    """The config-1 layout with every-1024 bf16 checkpoint rows (kda_prefill with the B200 serving keywords): rows of
    later pieces come from the tail launch's checkpoint compose."""
    kda = _kda()
    lens = _c1_lens()
    H, N, every = 32, len(lens), 1024
    T = sum(lens)
    hs = [0, 31]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    counts = [-(-L // every) for L in lens]
    C = int(sum(counts))
    meta = kda.plan(torch.tensor(cu), H, ck_every=every, device=DEV)
    _say(f"config 1 every-n: pieces={meta.split} ck tasks={meta.plan.num_ck_tasks} rows={C}")
    assert meta.plan.num_pieces == 2 * meta.plan.num_split and meta.plan.num_ck_tasks > 0
    q, k, v, raw_g, raw_b, A_log, dt_bias = _raw_inputs_dev(T, H, 13)
    P = N + 2
    pool = torch.empty(P, H, D, D, device=DEV)
    pool.normal_(0.0, 0.05, generator=torch.Generator(device=DEV).manual_seed(14))
    idx = torch.randperm(P, generator=torch.Generator().manual_seed(14))[:N].to(torch.int32)
    pool0 = pool[idx.long()][:, hs].cpu().numpy()
    ck = torch.full((C, H, D, D), float("nan"), dtype=torch.bfloat16, device=DEV)
    ccs = torch.tensor(np.concatenate([[0], np.cumsum(counts)]), dtype=torch.int64, device=DEV)
    o, fin, ckr = kda.kda_prefill(q, k, v, raw_g, raw_b, A_log, dt_bias, pool, torch.tensor(cu, device=DEV),
                                  meta=meta, ssm_state_indices=idx.to(DEV), state_checkpoints=ck,
                                  checkpoint_cu_starts=ccs, checkpoint_every_n_tokens=every)
    torch.cuda.synchronize()
    qn = oracle.l2norm_clamp(_heads(q, hs))
    kn = oracle.l2norm_clamp(_heads(k, hs))
    gl = oracle.gate(_heads(raw_g, hs), f32(A_log[hs]), f32(dt_bias.view(H, D)[hs].reshape(-1)), -5.0)
    bt = oracle.sigmoid(np.ascontiguousarray(f32(raw_b[0][:, hs])))
    ro, rf, rows, _ = oracle.checkpoints_every_n(qn, kn, _heads(v, hs), gl, bt, cu, every, initial_state=pool0,
                                                 normalize_qk=False, precision=64)
    check_out(o[0][:, hs], ro, "config 1 every-n", cu)
    got = ck[:, hs].float().cpu().numpy()
    for r in range(C):
        bound = rel_frob(oracle.bf16_round(rows[r]), rows[r]) + STATE_TOL
        assert rel_frob(got[r], rows[r]) <= bound, f"checkpoint row {r}"
    fin_got = pool[idx.long()][:, hs].cpu().numpy()
    for n in range(N):
        assert rel_frob(fin_got[n], rf[n]) <= STATE_TOL, f"final state of sequence {n}"
