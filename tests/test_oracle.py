"""Pins of the CPU oracle (oracle/oracle.py + oracle/kda_oracle.c) by checks that do not retype its formulas:
closed forms, invariants, an independent dense product-form construction and an independent chunked (WY) evaluation.
Each check is chosen so that a plausible mistake (dropped term, wrong sign, transposed state, decay on the wrong axis,
decay applied after the read, off-by-one in a checkpoint) fails it.  CPU only.
"""
import math

import numpy as np
import pytest
import torch

from helpers import config_inputs, f32, gen

D = 128


def _unit(rng, shape):
    x = rng.standard_normal((*shape, D))
    return x / np.linalg.norm(x, axis=-1, keepdims=True)


def _rand_case(rng, T, H=1, gscale=1.0):
    q = _unit(rng, (T, H)).astype(np.float32)
    k = _unit(rng, (T, H)).astype(np.float32)
    v = rng.standard_normal((T, H, D)).astype(np.float32)
    g = (-np.log1p(np.exp(rng.standard_normal((T, H, D)))) * gscale).astype(np.float32)
    beta = (1 / (1 + np.exp(-rng.standard_normal((T, H))))).astype(np.float32)
    return q, k, v, g, beta


# ---------------------------------------------------------------------------------------------- elementwise pins
def test_bf16_round_matches_torch(oracle):
    x = torch.randn(100000, generator=gen(0)) * 10.0 ** torch.randint(-8, 8, (100000,), generator=gen(1))
    assert np.array_equal(oracle.bf16_round(x.numpy()), x.bfloat16().float().numpy())


def test_gate_special_values(oracle):
    H = 3
    A_log = np.array([0.0, 1.0, -2.0], np.float32)
    dt = np.linspace(-1, 1, H * D).astype(np.float32)
    # raw_g = -dt_bias -> sigmoid(0) = 1/2 -> g = lb / 2 exactly
    raw = np.broadcast_to(-dt.reshape(H, D), (2, H, D)).copy()
    assert np.array_equal(oracle.gate(raw, A_log, dt, -5.0), np.full((2, H, D), -2.5, np.float32))
    # saturation: raw -> +large gives lb, -large gives 0
    big = np.full((1, H, D), 1e4, np.float32)
    assert np.allclose(oracle.gate(big, A_log, dt, -5.0), -5.0)
    assert np.allclose(oracle.gate(-big, A_log, dt, -5.0), 0.0, atol=1e-30)
    # exp(A_log) multiplies the argument: doubling A (A_log += ln 2) equals doubling (raw + dt)
    r = np.random.default_rng(0).standard_normal((4, H, D)).astype(np.float32)
    a = oracle.gate(r, A_log + np.float32(math.log(2.0)), dt, -5.0)
    b = oracle.gate(2 * r + dt.reshape(H, D), A_log, dt, -5.0)
    assert np.allclose(a, b, rtol=1e-5, atol=1e-6)


def test_norms(oracle):
    x = np.random.default_rng(1).standard_normal((50, D)).astype(np.float32) * 3
    y = oracle.l2norm_clamp(x)
    assert np.allclose(np.linalg.norm(y, axis=1), 1.0, atol=1e-6)
    tiny = np.full((1, D), 1e-9, np.float32)                  # ||x|| < eps -> x / eps
    assert np.allclose(oracle.l2norm_clamp(tiny), tiny / 1e-6, rtol=1e-6)
    z = oracle.l2norm_rsqrt(x, mult=D ** -0.5)
    assert np.allclose(np.linalg.norm(z, axis=1), D ** -0.5, rtol=1e-5)
    zero = np.zeros((1, D), np.float32)                       # rsqrt(0 + eps) * 0 = 0, no NaN
    assert np.array_equal(oracle.l2norm_rsqrt(zero), zero)


@pytest.mark.parametrize("c", [1e-3, 1e-7])
def test_norm_forms_in_recurrences(oracle, c):
    """One token, zero state, beta = 1, g = 0, q = k = c e_0: o = scale v (k^ . q^).  The prefill form
    x / max(|x|, 1e-6) (reference.py:59-60) gives k^ . q^ = (c / max(c, 1e-6))^2; the decode form
    x rsqrt(|x|^2 + 1e-6) (reference.py:159-160), which vLLM's fused_recurrent_kda and the decode kernels use, gives
    c^2 / (c^2 + 1e-6).  At c = 1e-3 the two differ by 2x, so a recurrence on the wrong form fails."""
    H, scale = 1, 0.25
    x = np.zeros((1, H, D), np.float32)
    x[..., 0] = c
    v = np.random.default_rng(2).standard_normal((1, H, D)).astype(np.float32)
    z = np.zeros((1, H, D), np.float32)
    one = np.ones((1, H), np.float32)
    pre = min(1.0, c / 1e-6) ** 2
    dec = c * c / (c * c + 1e-6)
    o_p, _ = oracle.prefill_plain(x, x, v, z, one, [0, 1], scale=scale, precision=64)
    assert np.allclose(o_p, scale * v * pre, rtol=1e-5, atol=1e-12)
    pool = np.zeros((2, H, D, D), np.float32)
    o_d, _, _ = oracle.recurrent(x, x, v, z, one, pool, np.array([1]), scale=scale, precision=64)
    assert np.allclose(o_d, scale * v * dec, rtol=1e-5, atol=1e-12)


# ---------------------------------------------------------------------------------------------- recurrence pins
@pytest.mark.parametrize("prec", [32, 64])
def test_pure_decay_closed_form(oracle, prec):
    """beta = 0: S_t = diag(exp(Gamma_t)) S_0 on the KEY axis, o_t[v] = scale * sum_k S0[v, k] exp(Gamma_t[k]) q_t[k]
    (pins the decay axis, the V-major layout and the scale)."""
    rng = np.random.default_rng(2)
    T, H = 40, 2
    q, k, v, g, _ = _rand_case(rng, T, H, gscale=0.1)
    beta = np.zeros((T, H), np.float32)
    S0 = rng.standard_normal((1, H, D, D)).astype(np.float32)
    out, fin, _ = oracle.chains(q, k, v, g, beta, [0, T], 0.37, S0, precision=prec)
    Gam = np.cumsum(g.astype(np.float64), axis=0)              # [T, H, K]
    for h in range(H):
        ref_fin = S0[0, h].astype(np.float64) * np.exp(Gam[-1, h])[None, :]
        assert np.allclose(fin[0, h], ref_fin, rtol=5e-5 if prec == 32 else 1e-6, atol=1e-7)   # stored as fp32
        ref_o = 0.37 * np.einsum("vk,tk->tv", S0[0, h].astype(np.float64), np.exp(Gam[:, h]) * q[:, h])
        assert np.allclose(out[:, h], ref_o, rtol=5e-4 if prec == 32 else 1e-6, atol=1e-6 if prec == 32 else 1e-9)


def test_recall_beta_one(oracle):
    """beta = 1, q = k: the delta rule writes v_t exactly under key k_t, so o_t = scale * v_t whatever the decay and
    the history (pins the sign of u, decay-before-read and the output after the update)."""
    rng = np.random.default_rng(3)
    T = 30
    q, k, v, g, _ = _rand_case(rng, T)
    beta = np.ones((T, 1), np.float32)
    S0 = rng.standard_normal((1, 1, D, D)).astype(np.float32)
    out, _, _ = oracle.chains(k, k, v, g, beta, [0, T], 0.5, S0, precision=64)
    assert np.allclose(out, 0.5 * v, atol=1e-6)


def test_orthonormal_keys_associative_memory(oracle):
    """g = 0, beta = 1, orthonormal keys, zero start: S = sum_j k_j v_j^T, i.e. V-major S[v, k] = sum_j v_j[v] k_j[k],
    and every stored value is recalled exactly (S^T k_j = v_j)."""
    rng = np.random.default_rng(4)
    m = 24
    Qm, _ = np.linalg.qr(rng.standard_normal((D, m)))
    k = Qm.T.astype(np.float32)[:, None, :]
    v = rng.standard_normal((m, 1, D)).astype(np.float32)
    z = np.zeros((m, 1, D), np.float32)
    out, fin, _ = oracle.chains(k, k, v, z, np.ones((m, 1), np.float32), [0, m], 1.0, None, precision=64)
    ref = np.einsum("jv,jk->vk", v[:, 0].astype(np.float64), k[:, 0].astype(np.float64))
    assert np.allclose(fin[0, 0], ref, atol=1e-6)
    recall = fin[0, 0].astype(np.float64) @ k[:, 0].T.astype(np.float64)
    assert np.allclose(recall.T, v[:, 0], atol=1e-5)


def test_affine_linearity(oracle):
    """For fixed (q, k, g, beta) the map (S_0, v) -> (o, S_T) is linear."""
    rng = np.random.default_rng(5)
    T = 50
    q, k, v1, g, beta = _rand_case(rng, T)
    v2 = rng.standard_normal(v1.shape).astype(np.float32)
    S1 = rng.standard_normal((1, 1, D, D)).astype(np.float32)
    S2 = rng.standard_normal((1, 1, D, D)).astype(np.float32)
    a, b = 0.75, -1.25
    o1, f1, _ = oracle.chains(q, k, v1, g, beta, [0, T], 0.1, S1, precision=64)
    o2, f2, _ = oracle.chains(q, k, v2, g, beta, [0, T], 0.1, S2, precision=64)
    o3, f3, _ = oracle.chains(q, k, a * v1 + b * v2, g, beta, [0, T], 0.1, a * S1 + b * S2, precision=64)
    assert np.allclose(o3, a * o1 + b * o2, atol=1e-5)
    assert np.allclose(f3, a * f1 + b * f2, atol=1e-5)


def test_dense_product_form(oracle):
    """Independent construction: S_t = (I - beta_t k_t k_t^T) diag(e^{g_t}) S_{t-1} + beta_t k_t v_t^T as explicit
    128 x 128 matrix products (K-major), o_t = scale S_t^T q_t."""
    rng = np.random.default_rng(6)
    T = 7
    q, k, v, g, beta = _rand_case(rng, T)
    S0 = rng.standard_normal((1, 1, D, D)).astype(np.float32)
    out, fin, _ = oracle.chains(q, k, v, g, beta, [0, T], 0.25, S0, precision=64)
    S = S0[0, 0].T.astype(np.float64)
    I = np.eye(D)
    for t in range(T):
        kt = k[t, 0].astype(np.float64)
        A = (I - beta[t, 0] * np.outer(kt, kt)) @ np.diag(np.exp(g[t, 0].astype(np.float64)))
        S = A @ S + beta[t, 0] * np.outer(kt, v[t, 0])
        assert np.allclose(out[t, 0], 0.25 * S.T @ q[t, 0], atol=1e-6)
    assert np.allclose(fin[0, 0], S.T, atol=1e-6)


def _wy_chunked(q, k, v, g, beta, S0, scale, C=64):
    """Chunked WY form in fp64 (gamma = inclusive cumsum, T = (I + A_kk)^-1), S K-major."""
    T = q.shape[0]
    S = S0.copy()
    out = np.zeros((T, D))
    for c0 in range(0, T, C):
        c1 = min(T, c0 + C)
        n = c1 - c0
        Q, K, V = q[c0:c1], k[c0:c1], v[c0:c1]
        G = np.cumsum(g[c0:c1], 0)
        B = beta[c0:c1]
        E = np.exp(G[:, None, :] - G[None, :, :])
        ii, jj = np.arange(n)[:, None], np.arange(n)[None, :]
        Akk = np.einsum("id,jd,ijd->ij", K, K, E) * B[:, None] * (ii > jj)
        Aqk = np.einsum("id,jd,ijd->ij", Q, K, E) * (ii >= jj)
        Tm = np.linalg.inv(np.eye(n) + Akk)
        W = Tm @ (B[:, None] * K * np.exp(G))
        U = Tm @ (B[:, None] * V)
        Vp = U - W @ S
        out[c0:c1] = scale * ((Q * np.exp(G)) @ S + Aqk @ Vp)
        S = np.exp(G[-1])[:, None] * S + (K * np.exp(G[-1] - G)).T @ Vp
    return out, S


def test_chunked_wy_equivalence(oracle):
    """The token recurrence equals the chunk-64 WY form (an algebraically different evaluation) to fp64 rounding,
    including a partial last chunk."""
    rng = np.random.default_rng(7)
    T = 64 * 3 + 23
    q, k, v, g, beta = _rand_case(rng, T, gscale=0.3)
    S0 = rng.standard_normal((1, 1, D, D)).astype(np.float32) * 0.1
    out, fin, _ = oracle.chains(q, k, v, g, beta, [0, T], D ** -0.5, S0, precision=64)
    wo, wS = _wy_chunked(*(x[:, 0].astype(np.float64) for x in (q, k, v, g)), beta[:, 0].astype(np.float64),
                         S0[0, 0].T.astype(np.float64), D ** -0.5)
    assert np.allclose(out[:, 0], wo, atol=1e-6, rtol=1e-6)
    assert np.allclose(fin[0, 0], wS.T, atol=1e-6, rtol=1e-6)


def test_fp32_vs_fp64(oracle):
    rng = np.random.default_rng(8)
    T = 300
    q, k, v, g, beta = _rand_case(rng, T, H=2)
    S0 = (rng.standard_normal((1, 2, D, D)) * 0.02).astype(np.float32)
    o32, f32_, _ = oracle.chains(q, k, v, g, beta, [0, T], D ** -0.5, S0, precision=32)
    o64, f64, _ = oracle.chains(q, k, v, g, beta, [0, T], D ** -0.5, S0, precision=64)
    assert np.linalg.norm(o32 - o64) / np.linalg.norm(o64) < 1e-5
    assert np.linalg.norm(f32_ - f64) / np.linalg.norm(f64) < 1e-5


def test_varlen_independence(oracle):
    """Sequences of a packed batch are independent: each equals its own single-sequence run."""
    rng = np.random.default_rng(9)
    lens = [5, 70, 1, 33]
    cu = np.concatenate([[0], np.cumsum(lens)])
    q, k, v, g, beta = _rand_case(rng, int(cu[-1]), H=2)
    S0 = rng.standard_normal((4, 2, D, D)).astype(np.float32) * 0.1
    out, fin, _ = oracle.chains(q, k, v, g, beta, cu, 0.3, S0, precision=64)
    for n in range(4):
        sl = slice(cu[n], cu[n + 1])
        o1, f1, _ = oracle.chains(q[sl], k[sl], v[sl], g[sl], beta[sl], [0, lens[n]], 0.3, S0[n:n + 1], precision=64)
        assert np.array_equal(out[sl], o1) and np.array_equal(fin[n], f1[0])


# ---------------------------------------------------------------------------------------------- checkpoint pins
def test_snapshot_segment_chaining(oracle):
    """A snapshot after o tokens equals the final state of a run over the first o tokens, and resuming from it
    reproduces the rest exactly (kda/b200/test_kda_b200.py:38-55 chaining)."""
    rng = np.random.default_rng(10)
    T = 200
    q, k, v, g, beta = _rand_case(rng, T, H=2)
    S0 = rng.standard_normal((1, 2, D, D)).astype(np.float32) * 0.1
    sa = np.array([[0, 64, 128, -1]])
    out, fin, snaps = oracle.chains(q, k, v, g, beta, [0, T], 0.3, S0, snap_at=sa, precision=32)
    assert np.array_equal(snaps[0, 0], S0[0])
    for j, o in enumerate([64, 128], start=1):
        _, f_head, _ = oracle.chains(q[:o], k[:o], v[:o], g[:o], beta[:o], [0, o], 0.3, S0, precision=32)
        assert np.array_equal(snaps[0, j], f_head[0])
        o_tail, f_tail, _ = oracle.chains(q[o:], k[o:], v[o:], g[o:], beta[o:], [0, T - o], 0.3, f_head,
                                          precision=32)
        assert np.array_equal(o_tail, out[o:]) and np.array_equal(f_tail, fin)


def test_every_n_rows(oracle):
    """Every-n rows: row j of sequence i = state before token j*n, ceil(len/n) rows per sequence."""
    rng = np.random.default_rng(11)
    lens = [130, 64, 1, 65]
    cu = np.concatenate([[0], np.cumsum(lens)])
    q, k, v, g, beta = _rand_case(rng, int(cu[-1]))
    S0 = rng.standard_normal((4, 1, D, D)).astype(np.float32)
    o, fin, rows, starts = oracle.checkpoints_every_n(q, k, v, g, beta, cu, 64, scale=0.3, initial_state=S0,
                                                     normalize_qk=False)
    assert list(starts) == [0, 3, 4, 5, 7]
    for n in range(4):
        for j in range(starts[n + 1] - starts[n]):
            t = j * 64
            sl = slice(cu[n], cu[n] + t)
            _, f, _ = oracle.chains(q[sl], k[sl], v[sl], g[sl], beta[sl], [0, t], 0.3, S0[n:n + 1])
            assert np.array_equal(rows[starts[n] + j], f[0])


def test_serving_slots_and_checkpoint(oracle):
    """reference.py:25-101 slot rules: a row without has_initial_state is never read (NaN stays harmless), final
    states land in state_indices rows, the checkpoint row holds the state after o tokens, nothing else changes."""
    g = gen(12)
    H, lens = 2, [128, 70, 3]
    cu = np.concatenate([[0], np.cumsum(lens)])
    T = int(cu[-1])
    q = torch.randn(T, H, D, generator=g).bfloat16()
    k = torch.randn(T, H, D, generator=g).bfloat16()
    v = torch.randn(T, H, D, generator=g).bfloat16()
    raw_g = torch.randn(T, H, D, generator=g).bfloat16()
    raw_b = torch.randn(T, H, generator=g).bfloat16()
    A_log = torch.rand(H, generator=g)
    dt = torch.randn(H * D, generator=g)
    cache = (torch.randn(10, H, D, D, generator=g) * 0.1).numpy()
    cache[4] = np.nan                                         # row of a sequence without an initial state
    cache[7] = np.nan                                         # checkpoint row: write-only
    idx = np.array([2, 4, 6])
    hinit = np.array([True, False, True])
    ck_off, ck_idx = np.array([64, 0, 0]), np.array([7, -1, -1])
    o, new = oracle.prefill_serving(f32(q), f32(k), f32(v), f32(raw_g), f32(raw_b), f32(A_log), f32(dt), -5.0,
                                    D ** -0.5, cache, idx, hinit, cu, ck_off, ck_idx)
    assert np.isfinite(o).all() and np.isfinite(new[[2, 4, 6, 7]]).all()
    untouched = [0, 1, 3, 5, 8, 9]
    assert np.array_equal(new[untouched], cache[untouched])
    # the checkpoint row is the first 64 tokens of sequence 0 from cache[2]
    qn, kn = oracle.l2norm_clamp(f32(q)), oracle.l2norm_clamp(f32(k))
    gl = oracle.gate(f32(raw_g), f32(A_log), f32(dt), -5.0)
    bt = oracle.sigmoid(f32(raw_b))
    _, f, _ = oracle.chains(qn[:64], kn[:64], f32(v)[:64], gl[:64], bt[:64], [0, 64], D ** -0.5, cache[2:3])
    assert np.array_equal(new[7], f[0])


# ---------------------------------------------------------------------------------------------- decode pins
def test_recurrent_core_matches_chain(oracle):
    """The decode core (V-major loops) and the prefill chain (K-major loops) are two codings of one recurrence."""
    rng = np.random.default_rng(13)
    B, S, H = 3, 5, 2
    q, k, v, g, beta = _rand_case(rng, B * S, H)
    S_in = rng.standard_normal((B, H, D, D)).astype(np.float32)
    out, steps = oracle.recurrent_core(q, k, v, g, beta, S_in, 0.3, precision=64)
    cu = np.arange(0, B * S + 1, S)
    o2, fin, snaps = oracle.chains(q, k, v, g, beta, cu, 0.3, S_in, snap_at=np.tile(np.arange(1, S + 1), (B, 1)),
                                   precision=64)
    assert np.allclose(out, o2, atol=1e-6)
    assert np.allclose(steps, snaps, atol=1e-5)


def test_spec_slot_mapping(oracle):
    """beta = 0, g = 0: the state never changes, so every written row equals the read row; the read row is
    idx[n, a-1], written rows are idx[n, t] > 0, everything else stays (reference.py:135-143,168-171)."""
    rng = np.random.default_rng(14)
    B, S, H, slots = 4, 3, 1, 20
    q, k, v, _, _ = _rand_case(rng, B * S, H)
    z = np.zeros((B * S, H, D), np.float32)
    pool = rng.standard_normal((slots, H, D, D)).astype(np.float32)
    idx = np.array([[1, 2, 3], [4, 0, 5], [6, 7, 8], [9, 10, 0]])
    acc = np.array([3, 1, 2, 2])
    out, new, written = oracle.recurrent(q, k, v, z, np.zeros((B * S, H), np.float32), pool, idx, acc)
    assert sorted(written) == [1, 2, 3, 4, 5, 6, 7, 8, 9, 10]
    read = [3, 4, 7, 10]
    for n in range(B):
        for t in range(S):
            if idx[n, t] > 0:
                assert np.array_equal(new[idx[n, t]], pool[read[n]])
    rest = [r for r in range(slots) if r not in written]
    assert np.array_equal(new[rest], pool[rest])


def test_decode_full_closed_forms(oracle):
    """Fused decode (reference.py:104-181): one-hot conv weights make the conv a tap selector, the conv cache
    keeps the last 3 inputs (plain) / 2 history taps + S inputs (spec), RMSNorm output has unit mean square."""
    rng = np.random.default_rng(15)
    H, B, S, slots = 2, 3, 1, 6
    dim = H * D
    C = 3 * dim
    x = oracle.bf16_round(rng.standard_normal((B * S, C)).astype(np.float32))
    conv = oracle.bf16_round(rng.standard_normal((slots, 3, C)).astype(np.float32))
    w = np.zeros((3, 4, dim), np.float32)
    w[:, 3, :] = 1.0                                          # tap 3 = the current input
    gate_in = rng.standard_normal((B * S, H, D)).astype(np.float32)
    beta_in = rng.standard_normal((B * S, H)).astype(np.float32)
    og = np.full((B * S, dim), 30.0, np.float32)              # sigmoid(30) = 1 in fp32
    A_log = np.zeros(H, np.float32)
    dt = np.zeros(dim, np.float32)
    nw = np.ones(D, np.float32)
    ssm = rng.standard_normal((slots, H, D, D)).astype(np.float32) * 0.1
    idx = np.array([1, 3, 5])
    out, conv_new, ssm_new = oracle.decode_full(x, conv, w, gate_in, beta_in, og, A_log, dt, nw, ssm, idx, None,
                                                1e-12, -5.0)
    for n in range(B):
        # conv cache: the last 3 inputs = 2 old taps + this token
        assert np.array_equal(conv_new[idx[n], :2], conv[idx[n], 1:])
        assert np.array_equal(conv_new[idx[n], 2], x[n])
    ms = (out.reshape(B, H, D).astype(np.float64) ** 2).mean(-1)
    assert np.allclose(ms, 1.0, rtol=2e-2)
    # spec: S = 2, accepted a: history taps [a-1, a+2), afterwards [0, 4) = taps a, a+1 then the 2 inputs
    S = 2
    conv4 = oracle.bf16_round(rng.standard_normal((slots, 4, C)).astype(np.float32))
    x2 = oracle.bf16_round(rng.standard_normal((B * S, C)).astype(np.float32))
    idx2 = np.array([[1, 2], [3, 4], [5, 0]])
    acc = np.array([1, 2, 1])
    out2, cnew2, _ = oracle.decode_full(x2, conv4, w, np.repeat(gate_in, 2, 0), np.repeat(beta_in, 2, 0),
                                        np.repeat(og, 2, 0), A_log, dt, nw, ssm, idx2, acc, 1e-6, -5.0)
    for n in range(B):
        a = acc[n]
        c = idx2[n, 0]
        assert np.array_equal(cnew2[c, :2], conv4[c, a:a + 2])
        assert np.array_equal(cnew2[c, 2:4], x2[n * S:(n + 1) * S])


def test_decode_full_conv_groups_taps_silu(oracle):
    """Conv orientation pin (reference.py:144-157): conv_weight[group, tap, channel] with one-hot taps per group.
    q and k select the same current input (so k_hat . q_hat = 1), v selects a history tap; beta = 1, no decay, zero
    state: o = v / sqrt(128) and the gated RMSNorm output is SiLU(v_tap) / RMS(SiLU(v_tap)).  A transposed weight
    layout, a reversed tap order, a wrong spec history offset or a missing SiLU all change which values come out."""
    rng = np.random.default_rng(16)
    H, slots = 1, 8
    dim = H * D
    C = 3 * dim
    w = np.zeros((3, 4, dim), np.float32)
    w[0, 3] = 1.0                                             # q: the current input
    w[1, 3] = 1.0                                             # k: the current input
    w[2, 1] = 1.0                                             # v: window row t + 1
    nw = np.ones(D, np.float32)
    A_log = np.zeros(H, np.float32)
    dt = np.zeros(dim, np.float32)
    ssm = np.zeros((slots, H, D, D), np.float32)

    def expect(vt):
        sv = vt * (1.0 / (1.0 + np.exp(-vt.astype(np.float64))))
        return sv / np.sqrt((sv * sv).mean())

    for spec, S, acc in ((False, 1, None), (True, 2, np.array([2, 1]))):
        B = 2
        T = B * S
        taps = 2 + S if spec else 3
        conv = oracle.bf16_round(rng.standard_normal((slots, taps, C)).astype(np.float32))
        x = oracle.bf16_round(rng.standard_normal((T, C)).astype(np.float32))
        x[:, dim:2 * dim] = x[:, :dim]
        gate_in = np.full((T, H, D), -100.0, np.float32)      # sigmoid -> 0: g = 0
        beta_in = np.full((T, H), 30.0, np.float32)           # sigmoid(30) = 1 in fp32
        og = np.full((T, dim), 30.0, np.float32)
        idx = np.array([[3, 4], [5, 6]]) if spec else np.array([3, 5])
        out, _, _ = oracle.decode_full(x, conv, w, gate_in, beta_in, og, A_log, dt, nw, ssm, idx, acc, 1e-12, -5.0)
        for n in range(B):
            cs = idx[n, 0] if spec else idx[n]
            start = acc[n] - 1 if spec else 0
            vt = conv[cs, start + 1, 2 * dim:]                # window row 1 = history tap start + 1
            got = out[n * S].astype(np.float64)
            assert np.allclose(got, expect(vt), rtol=1.6e-2, atol=1e-2), (spec, n)


def test_decode_full_gated_rmsnorm(oracle):
    """Gated RMSNorm pin (reference.py:172-175): y = bf16(o) rsqrt(mean(bf16(o)^2) + eps) norm_weight sigmoid(og).
    The conv-orientation case above fixes o = SiLU(v_tap) / sqrt(128) (beta = 1, no decay, zero state, k^ . q^ = 1).
    Here sigmoid(og) takes the exact values 1/2 (og = 0), 1 (og = 30) and ~0 (og = -30) across channels, the weight
    is a per-channel ramp, and the history taps are small so that mean(o^2) ~ eps: dropping the gate or the weight,
    moving eps outside the rsqrt or dropping it changes the result by >= 30 %."""
    rng = np.random.default_rng(17)
    H, slots, B = 1, 6, 3
    dim = H * D
    C = 3 * dim
    w = np.zeros((3, 4, dim), np.float32)
    w[0, 3] = 1.0
    w[1, 3] = 1.0
    w[2, 1] = 1.0                                             # v: window row 1 (history tap 1 in plain decode)
    A_log = np.zeros(H, np.float32)
    dt = np.zeros(dim, np.float32)
    ssm = np.zeros((slots, H, D, D), np.float32)
    conv = oracle.bf16_round((rng.standard_normal((slots, 3, C)) * 0.2).astype(np.float32))
    x = oracle.bf16_round(rng.standard_normal((B, C)).astype(np.float32))
    x[:, dim:2 * dim] = x[:, :dim]
    gate_in = np.full((B, H, D), -100.0, np.float32)
    beta_in = np.full((B, H), 30.0, np.float32)
    og = np.tile(np.array([0.0, 30.0, -30.0, 0.0], np.float32), (B, dim // 4))
    nw = np.linspace(0.25, 2.0, D).astype(np.float32)
    idx = np.array([1, 3, 5])
    sv = conv[idx, 1, 2 * dim:].astype(np.float64)
    o = oracle.bf16_round(sv / (1.0 + np.exp(-sv)) / math.sqrt(D)).astype(np.float64)   # bf16(o)
    ms = (o * o).mean(-1, keepdims=True)
    eps = float(np.median(ms))
    out, _, _, (ob, fac) = oracle.decode_full(x, conv, w, gate_in, beta_in, og, A_log, dt, nw, ssm, idx, None, eps,
                                              -5.0, aux=True)
    sig = 1.0 / (1.0 + np.exp(-og.astype(np.float64)))
    expect = o / np.sqrt(ms + eps) * nw * sig
    # the checker's view (bf16(o) and the per-element norm factor) matches the closed form as well
    assert np.allclose(ob, o, rtol=8e-3, atol=0)
    assert np.allclose(fac, nw * sig / np.sqrt(ms + eps), rtol=2e-2)
    got = out.astype(np.float64)
    scale = np.abs(expect).max()
    assert np.allclose(got, expect, rtol=1.6e-2, atol=1e-2 * scale)
    # the alternatives this must tell apart
    for wrong in (o / np.sqrt(ms) * nw * sig, (o / np.sqrt(ms) + eps) * nw * sig, o / np.sqrt(ms + eps) * sig,
                  o / np.sqrt(ms + eps) * nw):
        assert np.abs(got - wrong).max() > 0.3 * scale


def test_config0_shapes(oracle):
    """Config 0 (T = 1024, H = 4, zero initial state) runs and is finite; fp32 agrees with fp64."""
    q, k, v, gg, beta = config_inputs(1024, 4, gen(0))
    o32, f32_ = oracle.prefill_plain(f32(q), f32(k), f32(v), f32(gg), f32(beta), [0, 1024], precision=32)
    o64, f64 = oracle.prefill_plain(f32(q), f32(k), f32(v), f32(gg), f32(beta), [0, 1024], precision=64)
    assert o32.shape == (1024, 4, D) and f32_.shape == (1, 4, D, D)
    assert np.isfinite(o32).all() and np.isfinite(f32_).all()
    assert np.linalg.norm(f32_ - f64) / np.linalg.norm(f64) < 1e-5
