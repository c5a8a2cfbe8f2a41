"""GPU parity of the chunked prefill (kda355_prefill_launch) against the fp64 CPU oracle.

Bars (north star): output max-abs error beyond bf16 storage rounding <= 2e-2 x RMS(ref); final / checkpoint states
relative Frobenius <= 1e-3 (bf16 checkpoint rows: <= the bf16 rounding of the reference row + 1e-3); which pool rows
are written is bit-exact and every other byte of the pool and of the output's parent buffer is unchanged.
"""
import math

import numpy as np
import pytest
import torch

from helpers import OUT_TOL, STATE_TOL, bf16_half_ulp, check_out, config_inputs, f32, gen, rel_frob

pytestmark = pytest.mark.gpu
D = 128
DEV = torch.device("cuda", 0)


def _kda():
    import kda355
    return kda355


def _say(msg):
    print(f"[case] {msg}", flush=True)


def _cu(lens):
    return np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)


def _check_out(got, ref, what, cu=None):
    return check_out(got, ref, what, cu)


def _list_meta(kda, lens, H, cus, chunk64=True, **kw):
    """A plan for `cus` CUs with more (sequence, head) items than CUs: chunk64 = True runs the 64-token kernel on its
    workgroup lists (one workgroup per CU walking several items), False the 32-token kernel (one workgroup per item, two
    per CU)."""
    meta = kda.plan(torch.tensor(_cu(lens)), H, device=DEV, num_cus=cus, chunk64=chunk64, **kw)
    assert meta.split == (0, 0) and int(meta.plan.chunk_grid) == cus, (meta.split, int(meta.plan.chunk_grid))
    return meta


def _plain_case(oracle, H, lens, seed, init=True, gscale=1.0, heads_checked=None, gmod=None, precise=False, cus=None,
                chunk64=True):
    kda = _kda()
    _say(f"plain H={H} lens={lens[:10]} init={init} seed={seed}" + (" precise" if precise else "") +
         (f" {'lists' if chunk64 else '32-token kernel'} on {cus} CUs" if cus else ""))
    g = gen(seed)
    T = int(sum(lens))
    q, k, v, gg, beta = config_inputs(T, H, g)
    gg = gg * gscale
    if gmod is not None:
        gg = gmod(gg, g)
    N = len(lens)
    h0 = torch.randn(N, H, D, D, generator=g) * 0.02 if init else None
    cu = torch.tensor(_cu(lens), dtype=torch.int32)
    meta = _list_meta(kda, lens, H, cus, chunk64) if cus else None
    o, fin = kda.chunk_kda(q[None].to(DEV), k[None].to(DEV), v[None].to(DEV), gg[None].to(DEV), beta[None].to(DEV),
                           initial_state=h0.to(DEV) if init else None, output_final_state=True, cu_seqlens=cu.to(DEV),
                           precise=precise, meta=meta)
    torch.cuda.synchronize()
    hs = list(range(H)) if heads_checked is None else heads_checked
    sel = lambda x: np.ascontiguousarray(f32(x)[:, hs])  # noqa: E731
    ro, rf = oracle.prefill_plain(sel(q), sel(k), sel(v), sel(gg), sel(beta), _cu(lens),
                                  initial_state=None if h0 is None else sel(h0), precision=64)
    _check_out(o[0][:, hs], ro, f"H={H} lens={lens[:6]}", _cu(lens))
    got = f32(fin)[:, hs]
    for n in range(N):
        e = rel_frob(got[n], rf[n])
        assert e <= STATE_TOL, f"H={H} seq {n} (len {lens[n]}): final state relF {e:.3e}"


def test_config0_single_sequence(oracle):
    _plain_case(oracle, 4, [1024], 0, init=False)


def test_varlen_with_initial_states(oracle):
    _plain_case(oracle, 4, [300, 64, 1, 1000, 77], 1)


def test_precise_mode_whole_and_split(oracle):
    """precise=True (fp16-pair operands in the solve and the state updates) on whole sequences and on a layout cut
    into pieces (later pieces carry their transition, whose update takes the pair too), and on a plan that chose the
    32-token kernel (which has no precise form: the launch runs the 64-token kernel on the plan's workgroup lists),
    against the fp64 oracle."""
    _plain_case(oracle, 4, [300, 64, 1, 1000, 77], 1, precise=True)
    _plain_case(oracle, 2, [8192, 300], 70, precise=True)
    _plain_case(oracle, 2, [600, 300, 130, 1, 0, 65, 700, 33], 71, precise=True, cus=4, chunk64=False)


def test_ragged_tiny_and_empty(oracle):
    _plain_case(oracle, 3, [1, 17, 33, 0, 1, 63, 65, 128, 2], 2)


@pytest.mark.parametrize("chunk64", [True, False], ids=["lists", "chunk32"])
def test_workgroup_lists_plain(oracle, chunk64):
    """Unsplit layouts with more (sequence, head) items than CUs.  lists: the 64-token kernel's workgroup lists, each
    workgroup walking its list in turn (the next item's rows prefetched in the last chunk of the one before, its start
    state loaded after that one's final state is stored).  chunk32: the 32-token kernel, one workgroup per item.
    Planned for 4 and 3 CUs: 10-27 items per CU mixing empty, one-token, ragged and multi-chunk sequences, with and
    without initial states, and at the bench's p_64x128 shape on the device's CUs (three two-chunk items per CU)."""
    _plain_case(oracle, 3, [1, 17, 33, 0, 1, 63, 65, 128, 2, 0, 300, 64, 200], 90, cus=4, chunk64=chunk64)
    _plain_case(oracle, 5, [130, 0, 777, 64, 1, 250, 64], 91, init=False, cus=3, chunk64=chunk64)
    cus = torch.cuda.get_device_properties(DEV).multi_processor_count
    _plain_case(oracle, 12, [128] * 64, 92, heads_checked=[0, 5, 11], cus=cus, chunk64=chunk64)


@pytest.mark.parametrize("chunk64", [True, False], ids=["lists", "chunk32"])
def test_workgroup_lists_random_layouts(oracle, chunk64):
    """Seeded random layouts with more items than CUs (empty, one-token and up to 12-chunk sequences; 2 to 7 CUs, so
    many items of mixed lengths per CU), with and without initial states, given gates; the 64-token kernel's workgroup
    lists and the 32-token kernel, against the oracle."""
    rng = np.random.default_rng(11)
    for i in range(3):
        N, H, cus = int(rng.integers(6, 16)), int(rng.integers(2, 6)), int(rng.integers(2, 8))
        lens = [int(x) for x in rng.integers(0, 768, size=N)]
        lens[int(rng.integers(0, N))] = 0
        lens[int(rng.integers(0, N))] = 1
        _plain_case(oracle, H, lens, 95 + i, init=bool(i % 2 == 0), cus=cus, chunk64=chunk64)


def test_chunk32_device_scale(oracle):
    """The 32-token kernel as the launch picks it on the device: unsplit layouts with more (sequence, head) items than
    CUs (512 and 720 items at H = 16, ragged, with empty, one-token and 31 / 32 / 33 / 63 / 64 / 65-token sequences,
    with and without initial states), against the oracle on a few heads; and with the gates, beta and q / k norms in
    the kernel (kda_prefill), against the 64-token kernel on the same plan (both within the north-star state bar of
    each other)."""
    kda = _kda()
    cus = torch.cuda.get_device_properties(DEV).multi_processor_count
    rng = np.random.default_rng(31)
    lens = [int(x) for x in rng.integers(100, 700, size=30)] + [0, 1]
    _plain_case(oracle, 16, lens, 120, heads_checked=[0, 5, 15], cus=cus, chunk64=False)
    lens = [int(x) for x in rng.integers(1, 300, size=39)] + [31, 32, 33, 63, 64, 65]
    _plain_case(oracle, 16, lens, 121, init=False, heads_checked=[3, 9], cus=cus, chunk64=False)
    H, lens = 16, [int(x) for x in rng.integers(50, 600, size=32)]
    T = sum(lens)
    _say(f"chunk32 against chunk64, gates in the kernel, H={H} N={len(lens)}")
    g = gen(122)
    q, k, v, raw_g, raw_b, A_log, dt_bias = _raw_inputs(g, T, H)
    h0 = (torch.randn(len(lens), H, D, D, generator=g) * 0.05).to(DEV)
    cu = torch.tensor(_cu(lens), dtype=torch.int32)
    res = {}
    for c64 in (True, False):
        meta = _list_meta(kda, lens, H, cus, c64)
        o, f = kda.kda_prefill(q[None].to(DEV), k[None].to(DEV), v[None].to(DEV), raw_g[None].to(DEV),
                               raw_b[None].to(DEV), A_log.to(DEV), dt_bias.to(DEV), h0.clone(), cu_seqlens=cu.to(DEV),
                               meta=meta)
        torch.cuda.synchronize()
        res[c64] = (f32(o[0]), f32(f))
    (o64, f64), (o32, f32_) = res[True], res[False]
    rel = float(np.linalg.norm(o32 - o64) / np.linalg.norm(o64))
    worst = max(rel_frob(f32_[n], f64[n]) for n in range(len(lens)))
    _say(f"  output relL2 {rel:.3e}, worst final-state relF {worst:.3e}")
    assert rel <= 2e-2 and worst <= STATE_TOL, (rel, worst)


def test_other_head_counts(oracle):
    for i, (H, lens) in enumerate([(1, [700]), (8, [37, 200]), (16, [129, 64])]):
        _plain_case(oracle, H, lens, 10 + i)


def test_slow_and_fast_decay(oracle):
    _plain_case(oracle, 2, [2048, 500], 20, gscale=0.01)   # long memory: cross-chunk state carries
    _plain_case(oracle, 2, [1000], 21, gscale=4.0)         # fast decay


def _deep_gates(gg, g):
    """-20 and -30 on random channels and tokens (a quarter of all values), the rest as given."""
    pick = torch.rand(gg.shape, generator=g)
    return torch.where(pick < 0.125, torch.full_like(gg, -20.0), torch.where(pick < 0.25, torch.full_like(gg, -30.0), gg))


def test_log_decay_below_range_is_clamped(oracle):
    """Given per-token log-decays far below KDA355_MIN_LOG_DECAY (-9): -20 and -30 on random channels and tokens (a
    quarter of all values), on a split layout (one long sequence in many pieces) and a whole one.  The kernel raises
    them to -9, a decay of e^-9 instead of a smaller one, which moves the state by less than 1.2e-4 of the affected
    channel; outputs and states stay finite and within the bars of the exact fp64 oracle."""
    _plain_case(oracle, 2, [6000, 300], 22, gmod=_deep_gates)
    _plain_case(oracle, 4, [700, 1], 23, gmod=_deep_gates)


def test_chunk32_decay_extremes(oracle):
    """The 32-token kernel (planned for 4 CUs: 16 items, one workgroup each) at the decay extremes the 64-token kernel
    is tested at: long memory (g x 0.01), fast decay (g x 4), and given log-decays of -20 / -30 raised to -9, on ragged
    sequences with empty, one-token and one-chunk-plus-one ones, against the fp64 oracle."""
    lens = [600, 300, 130, 1, 0, 65, 700, 33]
    _plain_case(oracle, 2, lens, 140, gscale=0.01, cus=4, chunk64=False)
    _plain_case(oracle, 2, lens, 141, gscale=4.0, cus=4, chunk64=False)
    _plain_case(oracle, 2, lens, 142, gmod=_deep_gates, cus=4, chunk64=False)


@pytest.mark.parametrize("chunk64", [None, False], ids=["plan", "chunk32"])
def test_raw_gate_lower_bound_below_range(oracle, chunk64):
    """kda_prefill with lower_bound = -20 and saturated gates (dt_bias 20..30, so g = lower_bound * sigmoid(.) reaches
    -20 on every channel): the in-kernel gate is raised to -9 like a given one, and the result matches the oracle.  plan:
    the launch's own plan (the long sequence in pieces); chunk32: more sequences, planned for 4 CUs as the 32-token
    kernel, one of them a single token.  Every final state meets the state bar against the oracle with its gates raised
    to -9 (the kernel's definition).  Against the exact oracle, the clamp adds e^-9 of the start state: relative to a
    state of many tokens that is ~1e-4, inside the bar.  After a single token whose update is small beside a start
    state of scale 0.25, it is 9.8e-4 on its own (measured on MI355X: both chunk kernels then read 1.028e-3 against
    the exact oracle and 3.0e-4 against the clamped one), so that sequence is held to the clamped oracle alone."""
    kda = _kda()
    H, lens = (2, [1100, 64]) if chunk64 is None else (2, [600, 500, 300, 64, 1])
    _say(f"kda_prefill lower_bound=-20, saturated gates, {'plan' if chunk64 is None else '32-token kernel'}")
    g = gen(33)
    T = sum(lens)
    q, k, v, raw_g, raw_b, A_log, dt_bias = _raw_inputs(g, T, H)
    A_log = torch.full((H,), 2.0)
    dt_bias = torch.linspace(20.0, 30.0, D).repeat(H)
    h0 = torch.randn(len(lens), H, D, D, generator=g) * 0.25
    cu = torch.tensor(_cu(lens), dtype=torch.int64)
    meta = None if chunk64 is None else _list_meta(kda, lens, H, 4, chunk64)
    o, fin = kda.kda_prefill(q[None].to(DEV), k[None].to(DEV), v[None].to(DEV), raw_g[None].to(DEV),
                             raw_b[None].to(DEV), A_log.to(DEV), dt_bias.to(DEV), h0.to(DEV), cu.to(DEV),
                             lower_bound=-20.0, meta=meta)
    torch.cuda.synchronize()
    qn, kn, vf, gl, bt = _oracle_gated(oracle, q, k, v, raw_g, raw_b, A_log, dt_bias, lb=-20.0)
    assert gl.min() < -19.0, "the case must drive the gate below the range"
    ro, rf, _ = oracle.chains(qn, kn, vf, gl, bt, _cu(lens), D ** -0.5, f32(h0), precision=64)
    _, rf9, _ = oracle.chains(qn, kn, vf, np.maximum(gl, -9.0), bt, _cu(lens), D ** -0.5, f32(h0), precision=64)
    _check_out(o[0], ro, "lower_bound=-20", _cu(lens))
    for n in range(len(lens)):
        got = f32(fin[n])
        e, e9 = rel_frob(got, rf[n]), rel_frob(got, rf9[n])
        assert np.isfinite(got).all() and e9 <= STATE_TOL, f"seq {n}: final state relF {e9:.3e} (gates at -9)"
        assert lens[n] == 1 or e <= STATE_TOL, f"seq {n}: final state relF {e:.3e}"


def test_config1_layout_subset_of_heads(oracle):
    """Config 1 (8 sequences, lengths U[256, 8192] from seed 1, H = 32); the oracle checks 4 of the 32 heads."""
    rng = np.random.default_rng(1)
    lens = [int(x) for x in rng.integers(256, 8193, size=8)]
    _plain_case(oracle, 32, lens, 1, heads_checked=[0, 9, 22, 31])


def _raw_inputs(g, T, H):
    q = torch.randn(T, H, D, generator=g).bfloat16()
    k = torch.randn(T, H, D, generator=g).bfloat16()
    v = torch.randn(T, H, D, generator=g).bfloat16()
    raw_g = torch.randn(T, H, D, generator=g).bfloat16()
    raw_b = torch.randn(T, H, generator=g).bfloat16()
    A_log = torch.log(torch.empty(H).uniform_(1.0, 16.0, generator=g))
    dt = torch.exp(torch.rand(H * D, generator=g) * (math.log(0.1) - math.log(0.001)) + math.log(0.001)).clamp(min=1e-4)
    dt_bias = dt + torch.log(-torch.expm1(-dt))
    return q, k, v, raw_g, raw_b, A_log, dt_bias


def _oracle_gated(oracle, q, k, v, raw_g, raw_b, A_log, dt_bias, lb=-5.0):
    qn, kn = oracle.l2norm_clamp(f32(q)), oracle.l2norm_clamp(f32(k))
    gl = oracle.gate(f32(raw_g), f32(A_log), f32(dt_bias), lb)
    bt = oracle.sigmoid(f32(raw_b))
    return qn, kn, f32(v), gl, bt


@pytest.mark.parametrize("gates", ["b200", "spectrum", "slow"])
def test_kda_prefill_raw_gates(oracle, gates):
    """kda_prefill (gates, beta sigmoid and norms in the kernel), including test_slowdecay's gate regimes."""
    kda = _kda()
    H, lens = 4, [1500, 64, 333]
    _say(f"kda_prefill gates={gates}")
    g = gen(30)
    T = sum(lens)
    q, k, v, raw_g, raw_b, A_log, dt_bias = _raw_inputs(g, T, H)
    if gates != "b200":
        lo, hi = (-14.0, 2.0) if gates == "spectrum" else (-12.0, -6.0)
        A_log = torch.zeros(H)
        dt_bias = torch.linspace(lo, hi, D).repeat(H)
    h0 = torch.randn(len(lens), H, D, D, generator=g) * 0.25
    cu = torch.tensor(_cu(lens), dtype=torch.int64)
    o, fin = kda.kda_prefill(q[None].to(DEV), k[None].to(DEV), v[None].to(DEV), raw_g[None].to(DEV),
                             raw_b[None].to(DEV), A_log.to(DEV), dt_bias.to(DEV), h0.to(DEV), cu.to(DEV))
    torch.cuda.synchronize()
    qn, kn, vf, gl, bt = _oracle_gated(oracle, q, k, v, raw_g, raw_b, A_log, dt_bias)
    ro, rf, _ = oracle.chains(qn, kn, vf, gl, bt, _cu(lens), D ** -0.5, f32(h0), precision=64)
    _check_out(o[0], ro, f"gates={gates}", _cu(lens))
    for n in range(len(lens)):
        assert rel_frob(f32(fin[n]), rf[n]) <= STATE_TOL, f"gates={gates} seq {n}"


def test_chunk_kda_gate_and_beta_in_kernel(oracle):
    """The fla keyword form of the in-kernel gate: chunk_kda(..., use_gate_in_kernel=True,
    use_beta_sigmoid_in_kernel=True, A_log=, dt_bias=, lower_bound=) runs the kernel kda_prefill runs (bit for bit) and
    matches the oracle; the gate may come in fp32 (converted to the kernel's bf16 raw form)."""
    kda = _kda()
    H, lens = 4, [700, 64, 129]
    _say("chunk_kda gate and beta in the kernel")
    g = gen(31)
    T = sum(lens)
    q, k, v, raw_g, raw_b, A_log, dt_bias = _raw_inputs(g, T, H)
    h0 = torch.randn(len(lens), H, D, D, generator=g) * 0.25
    cu = torch.tensor(_cu(lens), dtype=torch.int64).to(DEV)
    args = (q[None].to(DEV), k[None].to(DEV), v[None].to(DEV))
    o1, f1 = kda.chunk_kda(*args, raw_g[None].to(DEV), raw_b[None].to(DEV), initial_state=h0.to(DEV), cu_seqlens=cu,
                           use_gate_in_kernel=True, use_beta_sigmoid_in_kernel=True, A_log=A_log.to(DEV),
                           dt_bias=dt_bias.to(DEV), lower_bound=-5.0)
    o2, f2 = kda.chunk_kda(*args, raw_g[None].float().to(DEV), raw_b[None].to(DEV), initial_state=h0.to(DEV),
                           cu_seqlens=cu, use_gate_in_kernel=True, use_beta_sigmoid_in_kernel=True,
                           A_log=A_log.to(DEV), dt_bias=dt_bias.to(DEV), lower_bound=-5.0)
    o3, f3 = kda.kda_prefill(*args, raw_g[None].to(DEV), raw_b[None].to(DEV), A_log.to(DEV), dt_bias.to(DEV),
                             h0.to(DEV), cu, lower_bound=-5.0)
    torch.cuda.synchronize()
    assert torch.equal(o1, o3) and torch.equal(f1, f3), "chunk_kda's keyword form and kda_prefill differ"
    assert torch.equal(o1, o2) and torch.equal(f1, f2), "an fp32 raw gate holding bf16 values changed the result"
    qn, kn, vf, gl, bt = _oracle_gated(oracle, q, k, v, raw_g, raw_b, A_log, dt_bias)
    ro, rf, _ = oracle.chains(qn, kn, vf, gl, bt, _cu(lens), D ** -0.5, f32(h0), precision=64)
    _check_out(o1[0], ro, "chunk_kda in-kernel gate", _cu(lens))
    for n in range(len(lens)):
        assert rel_frob(f32(f1[n]), rf[n]) <= STATE_TOL, f"seq {n}"


def _pages(slots, H, taps, g):
    """vLLM hybrid page layout (kda/mi350x/CONTRACT.md:60-67): conv state then SSM state per padded page."""
    dim = H * D
    conv_bytes = taps * 3 * dim * 2
    page = -(-(conv_bytes + H * D * D * 4 + 4096) // 256) * 256
    raw = torch.randint(0, 256, (slots * page,), dtype=torch.uint8, generator=g).to(DEV)
    ssm = torch.as_strided(raw.view(torch.float32), (slots, H, D, D), (page // 4, D * D, D, 1), conv_bytes // 4)
    ssm.copy_((torch.randn(slots, H, D, D, generator=g) * 0.05).to(DEV))
    return raw, ssm


@pytest.mark.parametrize("cus,chunk64", [(None, True), (4, True), (4, False)], ids=["whole", "lists", "chunk32"])
def test_serving_pool_checkpoints_page_layout(oracle, cus, chunk64):
    """prefill_prepare + prefill on the page layout: has_initial_state with NaN rows, one checkpoint per sequence,
    strided raw_beta, out a slice behind 256 leading rows; only out and the named rows change.  cus = 4: 28 items for
    4 CUs, run as the 64-token kernel's workgroup lists (7 items per list, gates in the kernel: each item's dt_bias
    handed to the next) and as the 32-token kernel (one workgroup per item)."""
    kda = _kda()
    H = 4
    lens = [777, 64, 1, 130, 1024, 17, 255]
    hinit = [1, 0, 1, 0, 1, 1, 0]
    ck_off = [704, 64, 0, 0, 1024, 0, 192]
    _say(f"serving pool H={H} lens={lens} cus={cus} chunk64={chunk64}")
    g = gen(40)
    T, N = sum(lens), len(lens)
    q, k, v, raw_g, raw_b, A_log, dt_bias = _raw_inputs(g, T, H)
    slots = 3 * N + 5
    raw, ssm = _pages(slots, H, 3, g)
    perm = torch.randperm(slots - 1, generator=g) + 1
    sidx = perm[:N].to(torch.int32)
    cidx = torch.tensor([int(perm[N + n]) if ck_off[n] > 0 else -1 for n in range(N)], dtype=torch.int32)
    for n in range(N):                                   # rows that must not be read: NaN
        if not hinit[n]:
            ssm[int(sidx[n])] = float("nan")
        if ck_off[n] > 0:
            ssm[int(cidx[n])] = float("nan")
    before = raw.clone()
    pool0 = ssm.cpu().numpy().copy()
    Wp = 4 * H * D + D + H + 8                           # input projection row: beta is a strided column slice
    proj = torch.randn(T, Wp, generator=g).bfloat16().to(DEV)
    proj[:, 4 * H * D + D:4 * H * D + D + H] = raw_b.to(DEV)
    beta_view = proj[:, 4 * H * D + D:4 * H * D + D + H][None]
    parent = torch.full((1, 256 + T + 7, H, D), 3.0, dtype=torch.bfloat16, device=DEV)
    out = parent[:, 256:256 + T]
    parent_before = parent.clone()
    cu_cpu = torch.tensor(_cu(lens), dtype=torch.int32)
    meta = (kda.prefill_prepare(cu_cpu, H, torch.tensor(ck_off, dtype=torch.int32), cidx, device=DEV) if cus is None
            else _list_meta(kda, lens, H, cus, chunk64, checkpoint_offsets=torch.tensor(ck_off, dtype=torch.int32)))
    kda.prefill(q[None].to(DEV), k[None].to(DEV), v[None].to(DEV), raw_g[None].to(DEV), beta_view, A_log.to(DEV),
                dt_bias.to(DEV), D ** -0.5, -5.0, ssm, sidx.to(DEV), torch.tensor(hinit, dtype=torch.bool).to(DEV),
                cu_cpu.to(DEV), out, torch.tensor(ck_off, dtype=torch.int32).to(DEV), cidx.to(DEV), meta=meta)
    torch.cuda.synchronize()
    ro, rnew = oracle.prefill_serving(f32(q), f32(k), f32(v), f32(raw_g), f32(raw_b), f32(A_log), f32(dt_bias), -5.0,
                                      D ** -0.5, pool0, sidx.numpy(), np.array(hinit, bool), _cu(lens),
                                      np.array(ck_off), cidx.numpy(), precision=64)
    _check_out(out[0], ro, "serving", _cu(lens))
    got = ssm.cpu().numpy()
    written = [int(s) for s in sidx] + [int(c) for c in cidx if c >= 0]
    for r in written:
        e = rel_frob(got[r], rnew[r])
        assert e <= STATE_TOL, f"pool row {r}: relF {e:.3e}"
    # every byte outside out and the written rows unchanged
    exp_raw = before.clone()
    exp_ssm = torch.as_strided(exp_raw.view(torch.float32), ssm.shape, ssm.stride(), ssm.storage_offset())
    for r in written:
        exp_ssm[r] = ssm[r]
    assert torch.equal(raw, exp_raw), "bytes outside the written rows changed"
    assert torch.equal(parent[:, :256], parent_before[:, :256]) and torch.equal(parent[:, 256 + T:],
                                                                                  parent_before[:, 256 + T:])


def test_serving_no_sync_with_meta():
    """prefill() with a meta does not synchronize with the device (CONTRACT.md:48-50 host gate)."""
    kda = _kda()
    H, lens = 2, [100, 50]
    g = gen(41)
    T = sum(lens)
    q, k, v, raw_g, raw_b, A_log, dt_bias = _raw_inputs(g, T, H)
    pool = torch.zeros(4, H, D, D, device=DEV)
    cu = torch.tensor(_cu(lens), dtype=torch.int32)
    meta = kda.prefill_prepare(cu, H, device=DEV)
    args = [x[None].to(DEV) for x in (q, k, v, raw_g, raw_b)]
    out = torch.empty(1, T, H, D, dtype=torch.bfloat16, device=DEV)
    idx = torch.tensor([1, 2], dtype=torch.int32, device=DEV)
    hi = torch.zeros(2, dtype=torch.bool, device=DEV)
    cud, A, dtb = cu.to(DEV), A_log.to(DEV), dt_bias.to(DEV)
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        kda.prefill(*args, A, dtb, D ** -0.5, -5.0, pool, idx, hi, cud, out, meta=meta,
                    workspace=torch.empty(meta.workspace_bytes, dtype=torch.uint8, device=DEV))
    finally:
        torch.cuda.set_sync_debug_mode("default")
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()


@pytest.mark.parametrize("every,cus,chunk64", [(64, None, True), (256, None, True), (64, 4, True), (64, 4, False),
                                               (256, 4, False)])
def test_every_n_checkpoints_fp32_and_bf16(oracle, every, cus, chunk64):
    """B200 every-n rows (kda/b200/test_kda_b200.py:213-240): fp32 rows match the oracle; bf16 rows are exactly the
    fp32 rows rounded to nearest even; output and pool are identical across checkpoint dtypes.  cus = 4: 20 items for
    4 CUs, as the 64-token kernel's workgroup lists (chunk64) or the 32-token kernel, whose checkpoints fall after every
    second 32-token chunk."""
    kda = _kda()
    H, lens = 4, [300, 64, 1, 1000, 77]
    _say(f"every-n every={every} cus={cus} chunk64={chunk64}")
    meta = _list_meta(kda, lens, H, cus, chunk64, ck_every=every) if cus else None
    g = gen(50 + every)
    T, N = sum(lens), len(lens)
    q, k, v, raw_g, raw_b, A_log, dt_bias = _raw_inputs(g, T, H)
    P = N + 3
    pool0 = torch.randn(P, H, D, D, generator=g) * 0.25
    idx = torch.randperm(P, generator=g)[:N].to(torch.int32)
    counts = [-(-L // every) for L in lens]
    ccs = torch.tensor(_cu(counts), dtype=torch.int64)
    C = int(sum(counts))
    got = {}
    for dt in (torch.float32, torch.bfloat16):
        pool = pool0.clone().to(DEV)
        ck = torch.full((C, H, D, D), float("nan"), device=DEV, dtype=dt)
        res = kda.kda_prefill(q[None].to(DEV), k[None].to(DEV), v[None].to(DEV), raw_g[None].to(DEV),
                              raw_b[None].to(DEV), A_log.to(DEV), dt_bias.to(DEV), pool,
                              torch.tensor(_cu(lens)).to(DEV), ssm_state_indices=idx.to(DEV), state_checkpoints=ck,
                              checkpoint_cu_starts=ccs.to(DEV), checkpoint_every_n_tokens=every, meta=meta)
        torch.cuda.synchronize()
        assert len(res) == 3 and res[2] is ck and res[1] is pool
        got[dt] = (res[0].clone(), pool.clone(), ck)
    assert torch.equal(got[torch.float32][0], got[torch.bfloat16][0]), "output differs across checkpoint dtypes"
    assert torch.equal(got[torch.float32][1], got[torch.bfloat16][1]), "pool differs across checkpoint dtypes"
    assert torch.equal(got[torch.float32][2].to(torch.bfloat16), got[torch.bfloat16][2]), "bf16 rows != RNE(fp32 rows)"
    qn, kn, vf, gl, bt = _oracle_gated(oracle, q, k, v, raw_g, raw_b, A_log, dt_bias)
    S0 = f32(pool0)[idx.numpy()]
    ro, rf, rows, starts = oracle.checkpoints_every_n(qn, kn, vf, gl, bt, _cu(lens), every, initial_state=S0,
                                                      normalize_qk=False, precision=64)
    assert list(starts) == list(ccs.numpy())
    _check_out(got[torch.float32][0][0], ro, f"every={every}", _cu(lens))
    ck32 = f32(got[torch.float32][2])
    ck16 = f32(got[torch.bfloat16][2])
    for r in range(C):
        assert rel_frob(ck32[r], rows[r]) <= STATE_TOL, f"fp32 checkpoint row {r}"
        rne = oracle.bf16_round(rows[r])
        assert rel_frob(ck16[r], rows[r]) <= rel_frob(rne, rows[r]) + STATE_TOL, f"bf16 checkpoint row {r}"
    fin = f32(got[torch.float32][1])
    for n in range(N):
        assert rel_frob(fin[int(idx[n])], rf[n]) <= STATE_TOL


@pytest.mark.parametrize("kind", ["plan", "lists", "chunk32"])
def test_graph_capture_prefill(oracle, kind):
    """The launch is capturable: replay after refilling q/k/v/g/beta and the initial states in place.  plan: the
    device's own plan of two sequences (the longer cut into pieces: chunk, scan and tail launches in the graph); lists /
    chunk32: six sequences planned for 4 CUs, as the 64-token kernel's workgroup lists or the 32-token kernel."""
    kda = _kda()
    H, lens = (2, [200, 70]) if kind == "plan" else (2, [200, 70, 130, 1, 65, 300])
    T, N = sum(lens), len(lens)
    _say(f"prefill graph capture ({kind})")
    g = gen(60)
    cu = torch.tensor(_cu(lens), dtype=torch.int32)
    meta = kda.plan(cu, H, device=DEV) if kind == "plan" else _list_meta(kda, lens, H, 4, kind == "lists")
    ws = torch.empty(meta.workspace_bytes, dtype=torch.uint8, device=DEV)
    bufs = [torch.empty(1, T, H, D, dtype=torch.bfloat16, device=DEV) for _ in range(3)]
    gbuf = torch.empty(1, T, H, D, device=DEV)
    bbuf = torch.empty(1, T, H, device=DEV)
    h0 = torch.empty(N, H, D, D, device=DEV)
    out = torch.empty(1, T, H, D, dtype=torch.bfloat16, device=DEV)

    def call():
        return kda.chunk_kda(*bufs, gbuf, bbuf, initial_state=h0, meta=meta, out=out, workspace=ws)

    q, k, v, gg, beta = config_inputs(T, H, g)
    for b, x in zip(bufs, (q, k, v)):
        b.copy_(x[None])
    gbuf.copy_(gg[None])
    bbuf.copy_(beta[None])
    h0.zero_()
    call()
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        _, fin = call()
    for rep in range(2):
        q, k, v, gg, beta = config_inputs(T, H, g)
        init = torch.randn(N, H, D, D, generator=g) * 0.02
        for b, x in zip(bufs, (q, k, v)):
            b.copy_(x[None])
        gbuf.copy_(gg[None])
        bbuf.copy_(beta[None])
        h0.copy_(init)
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        ro, rf = oracle.prefill_plain(f32(q), f32(k), f32(v), f32(gg), f32(beta), _cu(lens), initial_state=f32(init),
                                      precision=64)
        _check_out(out[0], ro, f"replay {rep}", _cu(lens))
        for n in range(N):
            assert rel_frob(f32(fin[n]), rf[n]) <= STATE_TOL


def test_prefill_errors():
    kda = _kda()
    H, T = 2, 10
    q = torch.zeros(1, T, H, D, dtype=torch.bfloat16, device=DEV)
    g = torch.zeros(1, T, H, D, device=DEV)
    b = torch.zeros(1, T, H, device=DEV)
    cu = torch.tensor([0, T], dtype=torch.int32, device=DEV)
    with pytest.raises(TypeError):
        kda.chunk_kda(q, q, q, g.double(), b, cu_seqlens=cu)
    with pytest.raises(ValueError):
        kda.chunk_kda(q, q, q, g, b, cu_seqlens=cu, initial_state=torch.zeros(2, H, D, D, device=DEV))
    meta = kda.plan(torch.tensor([0, 5, T]), H, device=DEV)
    with pytest.raises(ValueError):                      # meta of another layout
        kda.chunk_kda(q[:, :5], q[:, :5], q[:, :5], g[:, :5], b[:, :5], meta=meta)
    with pytest.raises(TypeError):
        kda.chunk_kda(q.cpu(), q.cpu(), q.cpu(), g.cpu(), b.cpu())


# ------------------------------------------------------------------------------------------------ long-sequence split
def test_split_long_sequence_plain(oracle):
    """A sequence long enough to leave CUs idle is cut into pieces (later pieces from zero with their transition, then
    the scan and the output fixup); the short one stays whole.  Output and final states against the fp64 oracle; the split is visible in the plan."""
    kda = _kda()
    H, lens = 2, [8192, 300]
    meta = kda.plan(torch.tensor(_cu(lens)), H, device=DEV)
    assert meta.split[0] >= 4, f"expected a split layout, got {meta.split}"
    _say(f"split plain H={H} lens={lens} pieces={meta.split}")
    g = gen(70)
    T = sum(lens)
    q, k, v, gg, beta = config_inputs(T, H, g)
    h0 = torch.randn(len(lens), H, D, D, generator=g) * 0.02
    o, fin = kda.chunk_kda(q[None].to(DEV), k[None].to(DEV), v[None].to(DEV), gg[None].to(DEV), beta[None].to(DEV),
                           initial_state=h0.to(DEV), meta=meta)
    torch.cuda.synchronize()
    ro, rf = oracle.prefill_plain(f32(q), f32(k), f32(v), f32(gg), f32(beta), _cu(lens), initial_state=f32(h0),
                                  precision=64)
    _check_out(o[0], ro, "split plain", _cu(lens))
    for n in range(len(lens)):
        assert rel_frob(f32(fin[n]), rf[n]) <= STATE_TOL, f"split plain seq {n}"


def test_split_matches_whole_walk():
    """The same call planned for a full chip (no split) and for 256 CUs (split) agrees to rounding: both outputs are
    bf16, so each may sit half a bf16 ulp from its exact value and the two a full ulp apart before any compute error
    counts; the later pieces' outputs also pass through fp16 partials and fp16 correction operands."""
    kda = _kda()
    H, lens = 4, [4096, 1100]
    g = gen(71)
    T = sum(lens)
    q, k, v, gg, beta = (x[None].to(DEV) for x in config_inputs(T, H, g))
    h0 = (torch.randn(len(lens), H, D, D, generator=g) * 0.02).to(DEV)
    cu = torch.tensor(_cu(lens))
    whole = kda.plan(cu, H, device=DEV, num_cus=1)
    split = kda.plan(cu, H, device=DEV, num_cus=256)
    assert whole.split[0] == 0 and split.split[0] >= 2
    _say(f"split vs whole pieces={split.split}")
    o1, f1 = kda.chunk_kda(q, k, v, gg, beta, initial_state=h0, meta=whole)
    o2, f2 = kda.chunk_kda(q, k, v, gg, beta, initial_state=h0, meta=split)
    torch.cuda.synchronize()
    a, b = f32(o2).astype(np.float64), f32(o1).astype(np.float64)
    rms = math.sqrt(float((b * b).mean()))
    ex = float(np.max(np.abs(a - b) - 2 * bf16_half_ulp(b))) / rms
    assert ex <= OUT_TOL, f"split vs whole output excess {ex:.3e} beyond one bf16 ulp"
    assert rel_frob(a, b) <= 4e-3, f"split vs whole output relL2 {rel_frob(a, b):.3e}"
    assert rel_frob(f32(f2), f32(f1)) <= STATE_TOL


@pytest.mark.parametrize("gscale", [1.0, 0.01])
def test_split_long_scan_matches_whole_walk(gscale):
    """A chain of many pieces: the scan composes the final state through every piece's transition (fp16 MFMA
    products with the state as an fp16 hi/lo pair), so its rounding adds up over the pieces.  With the config gates (gscale 1) a piece's transition
    underflows to zero within a chunk or two; gscale 0.01 (log-decay ~ -0.007 per token and channel) keeps every
    transition and every start state live, which exercises the scan and the output fixup in full.  Outputs and final
    states against the unsplit walk of the same call."""
    kda = _kda()
    H, lens = 2, [32768]
    g = gen(72)
    q, k, v, gg, beta = config_inputs(sum(lens), H, g)
    q, k, v, gg, beta = (x[None].to(DEV) for x in (q, k, v, gg * gscale, beta))
    h0 = (torch.randn(len(lens), H, D, D, generator=g) * 0.02).to(DEV)
    cu = torch.tensor(_cu(lens))
    whole = kda.plan(cu, H, device=DEV, num_cus=1)
    split = kda.plan(cu, H, device=DEV, num_cus=256)
    assert whole.split[0] == 0 and split.split[0] >= 32, f"expected a long chain of pieces, got {split.split}"
    o1, f1 = kda.chunk_kda(q, k, v, gg, beta, initial_state=h0, meta=whole)
    o2, f2 = kda.chunk_kda(q, k, v, gg, beta, initial_state=h0, meta=split)
    torch.cuda.synchronize()
    err = rel_frob(f32(f2), f32(f1))
    a, b = f32(o2).astype(np.float64), f32(o1).astype(np.float64)
    rms = math.sqrt(float((b * b).mean()))
    ex = float(np.max(np.abs(a - b) - 2 * bf16_half_ulp(b))) / rms
    _say(f"long scan gscale={gscale} pieces={split.split} final-state rel frob {err:.3e} output excess {ex:.3e} "
         f"relL2 {rel_frob(a, b):.3e}")
    assert err <= STATE_TOL
    assert ex <= OUT_TOL, f"split vs whole output excess {ex:.3e} beyond one bf16 ulp"


def test_split_three_pieces_matches_whole_walk():
    """A launch whose split sequences have at most 3 pieces takes the lean scan (one operand set, four workgroups per
    CU): the reference's p96_loaded8k_0 shape (H = 96, one 8192-token sequence, planned as 52 + 52 + 24 chunks) with
    slow decay, against the unsplit walk of the same call."""
    kda = _kda()
    H, lens = 96, [8192]
    g = gen(73)
    q, k, v, gg, beta = config_inputs(sum(lens), H, g)
    q, k, v, gg, beta = (x[None].to(DEV) for x in (q, k, v, gg * 0.01, beta))
    h0 = (torch.randn(len(lens), H, D, D, generator=g) * 0.02).to(DEV)
    cu = torch.tensor(_cu(lens))
    whole = kda.plan(cu, H, device=DEV, num_cus=1)
    split = kda.plan(cu, H, device=DEV, num_cus=256)
    assert whole.split[0] == 0 and split.split == (3, 1), f"expected 3 pieces, got {split.split}"
    o1, f1 = kda.chunk_kda(q, k, v, gg, beta, initial_state=h0, meta=whole)
    o2, f2 = kda.chunk_kda(q, k, v, gg, beta, initial_state=h0, meta=split)
    torch.cuda.synchronize()
    err = rel_frob(f32(f2), f32(f1))
    a, b = f32(o2).astype(np.float64), f32(o1).astype(np.float64)
    rms = math.sqrt(float((b * b).mean()))
    ex = float(np.max(np.abs(a - b) - 2 * bf16_half_ulp(b))) / rms
    _say(f"three pieces H={H} final-state rel frob {err:.3e} output excess {ex:.3e}")
    assert err <= STATE_TOL
    assert ex <= OUT_TOL


@pytest.mark.parametrize("ckdt", [torch.float32, torch.bfloat16])
def test_split_pool_every_n_checkpoints(oracle, ckdt):
    """Split sequence with the B200 every-n rows into an explicit row table (configuration 2's form) on a paged pool:
    rows that fall in later pieces are composed from their (local state, transition) pairs once the start is known."""
    kda = _kda()
    H, lens, every = 4, [4096], 256
    g = gen(72)
    T = sum(lens)
    q, k, v, gg, beta = config_inputs(T, H, g)
    P = 6
    pool0 = torch.randn(P, H, D, D, generator=g) * 0.05
    slot = torch.tensor([3], dtype=torch.int32)
    nck = T // every
    rows = torch.randperm(nck + 4, generator=g)[:nck].to(torch.int32)
    ck = torch.full((nck + 4, H, D, D), float("nan"), dtype=ckdt, device=DEV)
    pool = pool0.clone().to(DEV)
    meta = kda.plan(torch.tensor(_cu(lens)), H, ck_every=every, device=DEV)
    assert meta.split[0] >= 2
    _say(f"split pool every-n dtype={ckdt} pieces={meta.split}")
    o, fin, ckr = kda.chunk_kda(q[None].to(DEV), k[None].to(DEV), v[None].to(DEV), gg[None].to(DEV), beta[None].to(DEV),
                                initial_state=pool, meta=meta, ssm_state_indices=slot.to(DEV), state_checkpoints=ck,
                                checkpoint_every_n_tokens=every, checkpoint_state_indices=rows.to(DEV))
    torch.cuda.synchronize()
    ro, rf, rrows, _ = oracle.checkpoints_every_n(f32(q), f32(k), f32(v), f32(gg), f32(beta), _cu(lens), every,
                                                 initial_state=f32(pool0)[slot.numpy()], precision=64)
    _check_out(o[0], ro, "split every-n", _cu(lens))
    assert rel_frob(f32(pool[3]), rf[0]) <= STATE_TOL
    untouched = [i for i in range(P) if i != 3]
    assert torch.equal(pool[untouched].cpu(), pool0[untouched]), "other pool slots changed"
    got = f32(ck)
    written = set(rows.tolist())
    for j in range(nck):
        ref = rrows[j]
        if ckdt == torch.bfloat16:
            assert rel_frob(got[rows[j]], ref) <= rel_frob(oracle.bf16_round(ref), ref) + STATE_TOL, f"row {j}"
        else:
            assert rel_frob(got[rows[j]], ref) <= STATE_TOL, f"row {j}"
    for i in range(nck + 4):
        if i not in written:
            assert np.isnan(got[i]).all(), f"checkpoint row {i} should be untouched"


def test_split_random_layouts_raw_gates_every_n(oracle):
    """Seeded random layouts planned for 32 or 64 CUs, so that the longer sequences are cut into pieces, through the
    gate-in-kernel call on a pool with every-n checkpoints (rows in later pieces are composed after the scan): output,
    final pool rows and every fp32 checkpoint row against the oracle."""
    kda = _kda()
    rng = np.random.default_rng(17)
    for i in range(3):
        N, H, cus, every = int(rng.integers(2, 6)), int(rng.integers(1, 5)), int(rng.choice([32, 64])), 128
        lens = [int(x) for x in rng.integers(1, 2600, size=N)]
        lens[0] = int(rng.integers(2048, 4096))
        g = gen(300 + i)
        T = sum(lens)
        q, k, v, raw_g, raw_b, A_log, dt_bias = _raw_inputs(g, T, H)
        P = N + 2
        pool0 = torch.randn(P, H, D, D, generator=g) * 0.1
        idx = torch.randperm(P, generator=g)[:N].to(torch.int32)
        counts = [-(-L // every) for L in lens]
        ccs = torch.tensor(_cu(counts), dtype=torch.int64)
        C = int(sum(counts))
        meta = kda.plan(torch.tensor(_cu(lens)), H, ck_every=every, device=DEV, num_cus=cus)
        _say(f"split random {i}: H={H} lens={lens} cus={cus} pieces={meta.split}")
        assert meta.split[1] >= 1, "the layout is meant to be split"
        pool = pool0.clone().to(DEV)
        ck = torch.full((C, H, D, D), float("nan"), device=DEV)
        res = kda.kda_prefill(q[None].to(DEV), k[None].to(DEV), v[None].to(DEV), raw_g[None].to(DEV),
                              raw_b[None].to(DEV), A_log.to(DEV), dt_bias.to(DEV), pool,
                              torch.tensor(_cu(lens)).to(DEV), ssm_state_indices=idx.to(DEV), state_checkpoints=ck,
                              checkpoint_cu_starts=ccs.to(DEV), checkpoint_every_n_tokens=every, meta=meta)
        torch.cuda.synchronize()
        qn, kn, vf, gl, bt = _oracle_gated(oracle, q, k, v, raw_g, raw_b, A_log, dt_bias)
        ro, rf, rows, _ = oracle.checkpoints_every_n(qn, kn, vf, gl, bt, _cu(lens), every,
                                                     initial_state=f32(pool0)[idx.numpy()], normalize_qk=False,
                                                     precision=64)
        _check_out(res[0][0], ro, f"split random {i}", _cu(lens))
        fin = f32(pool)
        for n in range(N):
            assert rel_frob(fin[int(idx[n])], rf[n]) <= STATE_TOL, f"case {i} seq {n}: final state"
        got = f32(ck)
        for r in range(C):
            assert rel_frob(got[r], rows[r]) <= STATE_TOL, f"case {i} checkpoint row {r}"


ONE_CHUNK_LENS = [1024, 200, 130, 64]  # at H = 4 the plan cuts the first three into one-chunk pieces


def _one_chunk_plan_ok(meta, lens):
    # every split sequence in pieces of one chunk: as many pieces as chunks
    nch = [-(-n // 64) for n in lens]
    assert meta.split == (sum(nch[:3]), 3), f"expected one-chunk pieces, got {meta.split}"


def test_split_one_chunk_pieces_serving(oracle):
    """Pieces of a single chunk (short sequences spread over idle CUs): the serving path with single checkpoints at
    the ends of later pieces (chunks 10, 2, 2, and the whole one-chunk sequence), partial last chunks (200 and 130
    tokens), has_initial_state mixed; outputs and pool rows against the fp64 oracle, other rows untouched."""
    kda = _kda()
    H, lens = 4, ONE_CHUNK_LENS
    hinit = [1, 0, 1, 1]
    ck_off = [640, 128, 128, 64]
    g = gen(74)
    T, N = sum(lens), len(lens)
    q, k, v, raw_g, raw_b, A_log, dt_bias = _raw_inputs(g, T, H)
    slots = 2 * N + 3
    raw, ssm = _pages(slots, H, 3, g)
    perm = torch.randperm(slots - 1, generator=g) + 1
    sidx = perm[:N].to(torch.int32)
    cidx = perm[N:2 * N].to(torch.int32)
    for n in range(N):
        if not hinit[n]:
            ssm[int(sidx[n])] = float("nan")
        ssm[int(cidx[n])] = float("nan")
    pool0 = ssm.cpu().numpy().copy()
    cu_cpu = torch.tensor(_cu(lens), dtype=torch.int32)
    meta = kda.prefill_prepare(cu_cpu, H, torch.tensor(ck_off, dtype=torch.int32), cidx, device=DEV)
    _one_chunk_plan_ok(meta, lens)
    _say(f"one-chunk pieces serving H={H} lens={lens} pieces={meta.split}")
    out = torch.empty(1, T, H, D, dtype=torch.bfloat16, device=DEV)
    kda.prefill(q[None].to(DEV), k[None].to(DEV), v[None].to(DEV), raw_g[None].to(DEV), raw_b[None].to(DEV),
                A_log.to(DEV), dt_bias.to(DEV), D ** -0.5, -5.0, ssm, sidx.to(DEV),
                torch.tensor(hinit, dtype=torch.bool).to(DEV), cu_cpu.to(DEV), out,
                torch.tensor(ck_off, dtype=torch.int32).to(DEV), cidx.to(DEV), meta=meta)
    torch.cuda.synchronize()
    ro, rnew = oracle.prefill_serving(f32(q), f32(k), f32(v), f32(raw_g), f32(raw_b), f32(A_log), f32(dt_bias), -5.0,
                                      D ** -0.5, pool0, sidx.numpy(), np.array(hinit, bool), _cu(lens),
                                      np.array(ck_off), cidx.numpy(), precision=64)
    _check_out(out[0], ro, "one-chunk serving", _cu(lens))
    got = ssm.cpu().numpy()
    written = [int(s) for s in sidx] + [int(c) for c in cidx]
    for r in written:
        e = rel_frob(got[r], rnew[r])
        assert e <= STATE_TOL, f"pool row {r}: relF {e:.3e}"
    for r in range(slots):
        if r not in written:
            assert np.array_equal(got[r], pool0[r], equal_nan=True), f"pool row {r} should be untouched"


def test_split_one_chunk_pieces_every_n(oracle):
    """One-chunk pieces with a checkpoint row at every chunk boundary (every = 64 tokens): every row after a
    sequence's first chunk is composed from a later piece's (local state, transition) pair."""
    kda = _kda()
    H, lens, every = 4, ONE_CHUNK_LENS, 64
    g = gen(75)
    T, N = sum(lens), len(lens)
    q, k, v, gg, beta = config_inputs(T, H, g)
    P = N + 3
    pool0 = torch.randn(P, H, D, D, generator=g) * 0.05
    slot = (torch.randperm(P, generator=g)[:N]).to(torch.int32)
    nck = sum(-(-n // every) for n in lens)
    rows = torch.randperm(nck + 4, generator=g)[:nck].to(torch.int32)
    ck = torch.full((nck + 4, H, D, D), float("nan"), dtype=torch.float32, device=DEV)
    pool = pool0.clone().to(DEV)
    meta = kda.plan(torch.tensor(_cu(lens)), H, ck_every=every, device=DEV)
    _one_chunk_plan_ok(meta, lens)
    _say(f"one-chunk pieces every-n pieces={meta.split}")
    o, fin, ckr = kda.chunk_kda(q[None].to(DEV), k[None].to(DEV), v[None].to(DEV), gg[None].to(DEV), beta[None].to(DEV),
                                initial_state=pool, meta=meta, ssm_state_indices=slot.to(DEV), state_checkpoints=ck,
                                checkpoint_every_n_tokens=every, checkpoint_state_indices=rows.to(DEV))
    torch.cuda.synchronize()
    ro, rf, rrows, _ = oracle.checkpoints_every_n(f32(q), f32(k), f32(v), f32(gg), f32(beta), _cu(lens), every,
                                                 initial_state=f32(pool0)[slot.numpy()], precision=64)
    _check_out(o[0], ro, "one-chunk every-n", _cu(lens))
    for n in range(N):
        assert rel_frob(f32(pool[int(slot[n])]), rf[n]) <= STATE_TOL, f"final state {n}"
    untouched = [i for i in range(P) if i not in set(slot.tolist())]
    assert torch.equal(pool[untouched].cpu(), pool0[untouched]), "other pool slots changed"
    got = f32(ck)
    for j in range(nck):
        assert rel_frob(got[rows[j]], rrows[j]) <= STATE_TOL, f"row {j}"
    written = set(rows.tolist())
    for i in range(nck + 4):
        if i not in written:
            assert np.isnan(got[i]).all(), f"checkpoint row {i} should be untouched"


def test_split_serving_single_checkpoints(oracle):
    """Split sequences on the serving path with one checkpoint each, at chunk boundaries the plan puts inside or at
    the end of first and later pieces (chunks 48, 127 in a partial last chunk, 3, 16); has_initial_state mixed."""
    kda = _kda()
    H = 2
    lens = [8192, 8155, 300, 8192]
    hinit = [1, 0, 1, 1]
    ck_off = [3072, 8128, 192, 1024]                     # chunks 48, 127, 3, 16
    g = gen(73)
    T, N = sum(lens), len(lens)
    q, k, v, raw_g, raw_b, A_log, dt_bias = _raw_inputs(g, T, H)
    slots = 2 * N + 3
    raw, ssm = _pages(slots, H, 3, g)
    perm = torch.randperm(slots - 1, generator=g) + 1
    sidx = perm[:N].to(torch.int32)
    cidx = perm[N:2 * N].to(torch.int32)
    for n in range(N):
        if not hinit[n]:
            ssm[int(sidx[n])] = float("nan")
        ssm[int(cidx[n])] = float("nan")
    pool0 = ssm.cpu().numpy().copy()
    cu_cpu = torch.tensor(_cu(lens), dtype=torch.int32)
    meta = kda.prefill_prepare(cu_cpu, H, torch.tensor(ck_off, dtype=torch.int32), cidx, device=DEV)
    assert meta.split[1] >= 3, f"expected the three long sequences split, got {meta.split}"
    _say(f"split serving single checkpoints H={H} lens={lens} pieces={meta.split}")
    out = torch.empty(1, T, H, D, dtype=torch.bfloat16, device=DEV)
    kda.prefill(q[None].to(DEV), k[None].to(DEV), v[None].to(DEV), raw_g[None].to(DEV), raw_b[None].to(DEV),
                A_log.to(DEV), dt_bias.to(DEV), D ** -0.5, -5.0, ssm, sidx.to(DEV),
                torch.tensor(hinit, dtype=torch.bool).to(DEV), cu_cpu.to(DEV), out,
                torch.tensor(ck_off, dtype=torch.int32).to(DEV), cidx.to(DEV), meta=meta)
    torch.cuda.synchronize()
    ro, rnew = oracle.prefill_serving(f32(q), f32(k), f32(v), f32(raw_g), f32(raw_b), f32(A_log), f32(dt_bias), -5.0,
                                      D ** -0.5, pool0, sidx.numpy(), np.array(hinit, bool), _cu(lens),
                                      np.array(ck_off), cidx.numpy(), precision=64)
    _check_out(out[0], ro, "split serving", _cu(lens))
    got = ssm.cpu().numpy()
    for r in [int(s) for s in sidx] + [int(c) for c in cidx]:
        e = rel_frob(got[r], rnew[r])
        assert e <= STATE_TOL, f"pool row {r}: relF {e:.3e}"
