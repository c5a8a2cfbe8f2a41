"""CPU oracle for KDA: the reference's semantics restated (numpy + the C core in kda_oracle.c).

TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels and the CPU baseline timed by bench.py.  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module.  The product (kda355) never does.

Every function works on numpy float32 arrays that hold exactly the values the device sees (bf16 tensors are
passed as their fp32 widening).  Paths cite caoshiyi/eat-kernels:

  gate / beta / norms ........ kda/mi350x/reference.py:19-22, 59-63, 159-163
  prefill_plain .............. kda/mi350x_plain/reference.py:14-39 and the fla `chunk_kda` plain call as the
                               reference invokes it (kda/b200/bench.py:108-117), with use_gate_in_kernel=False
                               and use_beta_sigmoid_in_kernel=False (g and beta used as given)
  prefill_serving ............ kda/mi350x/reference.py:25-101 (paged pool, has_initial_state, one checkpoint
                               row per sequence)
  checkpoints_every_n ........ kda/b200/kda_b200.py:19-22 and kda/b200/test_kda_b200.py:38-55 (row j = state
                               before token j*n)
  recurrent .................. kda/mi350x/reference.py:135-171 (decode / spec-verify slot semantics, recurrent
                               core only: vLLM's fused_recurrent_kda call, kda/mi350x/benchmark/vllm_reference/
                               kda.py:488-502)
  decode_full ................ kda/mi350x/reference.py:104-181 (conv1d + SiLU + norms + recurrence + gated RMSNorm)

Parity pins (tests/test_oracle.py): closed forms (pure decay at beta = 0, V-major layout at g = beta = 0,
associative recall at beta = 1 with orthonormal keys), affine structure (linearity in (S0, v)), segment chaining
(checkpoints), fp32 vs fp64 agreement, an independent chunked WY-form evaluation, and a brute-force dense
construction of the tiny case.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

D = 128
CHUNK = 64
_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "_build" / "libkda_oracle.so"
_lib = None


def lib():
    """The compiled C core (built by oracle/Makefile; __graft_entry__.build() runs it)."""
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            raise RuntimeError(f"oracle library missing: {_LIB_PATH} (run `make -C oracle`)")
        L = ctypes.CDLL(str(_LIB_PATH))
        P = ctypes.c_void_p
        L.kdao_prefill.argtypes = [P, P, P, P, P, ctypes.c_int64, ctypes.c_int, P, ctypes.c_int, ctypes.c_double,
                                   P, P, P, P, ctypes.c_int, P, ctypes.c_int, ctypes.c_int]
        L.kdao_prefill.restype = ctypes.c_int
        L.kdao_recurrent.argtypes = [P, P, P, P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_double,
                                     P, P, P, ctypes.c_int, ctypes.c_int]
        L.kdao_recurrent.restype = ctypes.c_int
        L.kdao_gate.argtypes = [P, P, P, ctypes.c_float, ctypes.c_int64, ctypes.c_int, P]
        L.kdao_l2norm_clamp.argtypes = [P, ctypes.c_int64, ctypes.c_float, P]
        L.kdao_l2norm_rsqrt.argtypes = [P, ctypes.c_int64, ctypes.c_float, ctypes.c_float, P]
        L.kdao_sigmoid.argtypes = [P, ctypes.c_int64, P]
        L.kdao_max_threads.restype = ctypes.c_int
        _lib = L
    return _lib


def _f32(x):
    return np.ascontiguousarray(x, dtype=np.float32)


def _p(a):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else None


# ------------------------------------------------------------------------------------------------ elementwise
def gate(raw_g, A_log, dt_bias, lower_bound):
    """reference.py:19-22: lb * sigmoid(exp(A_log[h]) * (raw_g + dt_bias[h, k])), raw_g [T, H, 128]."""
    raw_g = _f32(raw_g)
    T, H = raw_g.shape[0], raw_g.shape[1]
    out = np.empty_like(raw_g)
    lib().kdao_gate(_p(raw_g), _p(_f32(A_log)), _p(_f32(dt_bias)), float(lower_bound), T, H, _p(out))
    return out


def sigmoid(x):
    x = _f32(x)
    out = np.empty_like(x)
    lib().kdao_sigmoid(_p(x), x.size, _p(out))
    return out


def l2norm_clamp(x, eps=1e-6):
    """F.normalize(x, dim=-1, eps) (reference.py:59-60) over rows of 128."""
    x = _f32(x)
    out = np.empty_like(x)
    lib().kdao_l2norm_clamp(_p(x), x.size // D, float(eps), _p(out))
    return out


def l2norm_rsqrt(x, mult=1.0, eps=1e-6):
    """x * rsqrt(sum x^2 + eps) * mult (reference.py:159-160)."""
    x = _f32(x)
    out = np.empty_like(x)
    lib().kdao_l2norm_rsqrt(_p(x), x.size // D, float(eps), float(mult), _p(out))
    return out


def bf16_round(x):
    """Round-to-nearest-even to bf16, returned widened to fp32 (torch's .bfloat16() on finite values)."""
    x = _f32(x)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = (r & 0xFFFFFFFF).astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), x, out)


# ------------------------------------------------------------------------------------------------ prefill
def chains(q, k, v, g, beta, cu_seqlens, scale, initial_state=None, snap_at=None, precision=32, nthreads=0):
    """Token recurrence over every (sequence, head) (kdao_prefill).

    q, k: [T, H, 128] normalized; v [T, H, 128]; g [T, H, 128] log-decay; beta [T, H] activated;
    initial_state [N, H, 128, 128] V-major or None (zeros); snap_at [N, M] token counts (-1 = none).
    Returns (out [T, H, 128] fp32, final [N, H, 128, 128] V-major, snaps [N, M, H, 128, 128] or None)."""
    q, k, v, g, beta = map(_f32, (q, k, v, g, beta))
    T, H = q.shape[0], q.shape[1]
    cu = np.ascontiguousarray(cu_seqlens, dtype=np.int64)
    N = cu.size - 1
    out = np.zeros((T, H, D), np.float32)
    fin = np.empty((N, H, D, D), np.float32)
    S0 = _f32(initial_state) if initial_state is not None else None
    sa = snaps = None
    M = 0
    if snap_at is not None:
        sa = np.ascontiguousarray(snap_at, dtype=np.int64).reshape(N, -1)
        M = sa.shape[1]
        snaps = np.full((N, M, H, D, D), np.nan, np.float32)
    rc = lib().kdao_prefill(_p(q), _p(k), _p(v), _p(g), _p(beta), T, H, _p(cu), N, float(scale), _p(S0), _p(fin),
                            _p(out), _p(sa), M, _p(snaps), int(precision), int(nthreads))
    if rc != 0:
        raise ValueError("kdao_prefill: bad arguments")
    return out, fin, snaps


def prefill_plain(q, k, v, g, beta, cu_seqlens, scale=None, initial_state=None, normalize_qk=True, precision=32):
    """The plain call as the configs use it: fla chunk_kda(q, k, v, g, beta, scale, initial_state, cu_seqlens) with
    use_qk_l2norm_in_kernel=True, g a log-decay and beta already activated (reference recurrence
    kda/mi350x_plain/reference.py:20-39 after its gate / sigmoid lines).  Returns (o fp32 [T, H, 128], final)."""
    if scale is None:
        scale = D ** -0.5
    if normalize_qk:
        q, k = l2norm_clamp(q), l2norm_clamp(k)
    o, fin, _ = chains(q, k, v, g, beta, cu_seqlens, scale, initial_state, precision=precision)
    return o, fin


def checkpoints_every_n(q, k, v, g, beta, cu_seqlens, every, scale=None, initial_state=None, normalize_qk=True,
                        precision=32):
    """B200 every-n checkpoints (kda/b200/kda_b200.py:19-22): sequence i's row j (j < ceil(len_i / n)) is its state
    before token j * n.  Returns (o, final, rows [sum_i ceil(len_i/n), H, 128, 128], row_starts [N+1])."""
    if scale is None:
        scale = D ** -0.5
    if normalize_qk:
        q, k = l2norm_clamp(q), l2norm_clamp(k)
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    N = cu.size - 1
    lens = cu[1:] - cu[:-1]
    counts = [-(-int(L) // every) for L in lens]
    M = max(counts) if counts else 0
    sa = np.full((N, max(M, 1)), -1, np.int64)
    for n, c in enumerate(counts):
        sa[n, :c] = np.arange(c) * every
    o, fin, snaps = chains(q, k, v, g, beta, cu, scale, initial_state, snap_at=sa, precision=precision)
    starts = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    H = q.shape[1]
    rows = np.empty((int(starts[-1]), H, D, D), np.float32)
    for n, c in enumerate(counts):
        rows[starts[n]:starts[n] + c] = snaps[n, :c]
    return o, fin, rows, starts


def prefill_serving(q, k, v, raw_g, raw_beta, A_log, dt_bias, lower_bound, scale, state_cache, state_indices,
                    has_initial_state, cu_seqlens, checkpoint_offsets=None, checkpoint_state_indices=None,
                    precision=32):
    """reference.py:25-101.  state_cache [slots, H, 128, 128] (numpy, any slot layout); returns (o [T, H, 128] fp32,
    new_cache) where new_cache is a copy with the final states and the checkpoint rows written."""
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    N = cu.size - 1
    lens = cu[1:] - cu[:-1]
    idx = np.asarray(state_indices, dtype=np.int64)
    hinit = np.asarray(has_initial_state, dtype=bool)
    qn, kn = l2norm_clamp(q), l2norm_clamp(k)
    gl = gate(raw_g, A_log, dt_bias, lower_bound)
    bt = sigmoid(raw_beta)
    H = qn.shape[1]
    S0 = np.zeros((N, H, D, D), np.float32)
    for n in range(N):               # reference.py:79-82: the row is read only when has_initial_state[n]
        if hinit[n]:
            S0[n] = state_cache[idx[n]]
    sa = np.full((N, 1), -1, np.int64)
    ck_rows = {}
    if checkpoint_offsets is not None and checkpoint_state_indices is not None:
        for n, (o, r) in enumerate(zip(np.asarray(checkpoint_offsets).tolist(),
                                       np.asarray(checkpoint_state_indices).tolist())):
            if o > 0 and r >= 0:     # reference.py:55-57
                assert o % CHUNK == 0 and o <= lens[n], f"invalid checkpoint offset {o} for length {lens[n]}"
                sa[n, 0] = o
                ck_rows[n] = r
    out, fin, snaps = chains(qn, kn, v, gl, bt, cu, scale, S0, snap_at=sa, precision=precision)
    new = np.array(state_cache, copy=True)
    for n, r in ck_rows.items():     # reference.py:96-98
        new[r] = snaps[n, 0]
    for n in range(N):               # reference.py:99-100
        new[idx[n]] = fin[n]
    return out, new


# ------------------------------------------------------------------------------------------------ decode
def recurrent_core(q, k, v, g, beta, S_in, scale, precision=32, nthreads=0):
    """kdao_recurrent: B sequences x S tokens.  q/k/v/g [B*S, H, 128] (q, k normalized), beta [B*S, H],
    S_in [B, H, 128, 128] V-major.  Returns (out [B*S, H, 128], steps [B, S, H, 128, 128])."""
    q, k, v, g, beta, S_in = map(_f32, (q, k, v, g, beta, S_in))
    B, H = S_in.shape[0], S_in.shape[1]
    S = q.shape[0] // max(B, 1)
    out = np.empty((B * S, H, D), np.float32)
    steps = np.empty((B, S, H, D, D), np.float32)
    rc = lib().kdao_recurrent(_p(q), _p(k), _p(v), _p(g), _p(beta), B, S, H, float(scale), _p(S_in), _p(steps),
                              _p(out), int(precision), int(nthreads))
    if rc != 0:
        raise ValueError("kdao_recurrent: bad arguments")
    return out, steps


def recurrent(q, k, v, g, beta, pool, state_indices, num_accepted_tokens=None, scale=None, normalize_qk=True,
              precision=32):
    """vLLM fused_recurrent_kda slot semantics on a state pool (reference.py:135-143, 164-171):
      plain (state_indices [B]): read and write pool[state_indices[n]];
      spec  (state_indices [B, S], num_accepted_tokens [B]): start from pool[state_indices[n, a-1]], write the
            state after token t to pool[state_indices[n, t]] when that slot is > 0.
    Slot 0 is the reserved padding slot: a sequence whose read slot is <= 0 is neither read nor written (its
    output rows are zero).  normalize_qk uses the decode form x * rsqrt(sum x^2 + 1e-6) (reference.py:159-160, the
    form of vLLM's fused_recurrent_kda with use_qk_l2norm_in_kernel), not the prefill clamp x / max(|x|, 1e-6);
    scale multiplies q after it.  Returns (out [B*S, H, 128] fp32, new_pool, written_rows)."""
    if scale is None:
        scale = D ** -0.5
    q, k, v, g, beta = map(_f32, (q, k, v, g, beta))
    if normalize_qk:
        q, k = l2norm_rsqrt(q), l2norm_rsqrt(k)
    idx = np.asarray(state_indices, dtype=np.int64)
    spec = num_accepted_tokens is not None
    B = idx.shape[0]
    S = idx.shape[1] if spec else 1
    if spec:
        a = np.clip(np.asarray(num_accepted_tokens, dtype=np.int64), 1, S)
        rd = idx[np.arange(B), a - 1]
    else:
        rd = idx
    H = q.shape[1]
    S_in = np.zeros((B, H, D, D), np.float32)
    live = rd > 0
    for n in range(B):
        if live[n]:
            S_in[n] = pool[rd[n]]
    out, steps = recurrent_core(q, k, v, g, beta, S_in, scale, precision)
    new = np.array(pool, copy=True)
    written = []
    for n in range(B):
        if not live[n]:
            out[n * S:(n + 1) * S] = 0.0
            continue
        if spec:
            for t in range(S):
                if idx[n, t] > 0:
                    new[idx[n, t]] = steps[n, t]
                    written.append(int(idx[n, t]))
        else:
            new[rd[n]] = steps[n, S - 1]
            written.append(int(rd[n]))
    return out, new, written


def decode_full(mixed_qkv, conv_state, conv_weight, gate_in, beta_in, out_gate, A_log, dt_bias, norm_weight,
                ssm_state, state_indices, num_accepted_tokens, norm_eps, lower_bound, precision=32, aux=False):
    """reference.py:104-181 (fused conv1d + SiLU + KDA + gated RMSNorm decode / spec verify).

    mixed_qkv [T, 3*H*128] (bf16 values), conv_state [slots, taps, 3*H*128] (bf16 values), conv_weight
    [3, 4, H*128], gate_in [T, H, 128], beta_in [T, H], out_gate [T, H*128], A_log [H], dt_bias [H*128],
    norm_weight [128], ssm_state [slots, H, 128, 128].  Returns (out [T, H*128] bf16-rounded fp32, conv_new,
    ssm_new).  Rows <= 0 are padding: a sequence whose read row or conv row (idx[n, 0] in spec) is padding gets zero
    output and writes nothing (the reference kernel's slot rule, kda/mi350x/kda/decode/kda_v14_b.cu:1013-1042);
    spec writes skip padding rows (reference.py:168-171).  aux=True also returns (bf16(o) [T, H*128], the per-element
    factor rstd * norm_weight * sigmoid(out_gate) [T, H*128]) of the gated RMSNorm, from which a checker can bound
    what one step of the intermediate bf16(o) rounding moves each output element."""
    W = 4
    T, C = mixed_qkv.shape
    dim = C // 3
    H = dim // D
    idx = np.asarray(state_indices, dtype=np.int64)
    spec = num_accepted_tokens is not None
    B = idx.shape[0]
    S = T // B
    ar = np.arange(B)
    if spec:
        acc = np.clip(np.asarray(num_accepted_tokens, dtype=np.int64), 1, S)
        read_slot = idx[ar, acc - 1]
        cslot = idx[:, 0]
        start = acc - 1
    else:
        read_slot = idx
        cslot = read_slot
        start = np.zeros(B, np.int64)
    taps = start[:, None] + np.arange(W - 1)[None, :]
    hist = conv_state[cslot[:, None], taps]                       # [B, 3, C]   reference.py:144-145
    x = _f32(mixed_qkv).reshape(B, S, C)
    window = np.concatenate([hist, x], axis=1)                    # [B, 3 + S, C]
    w = _f32(conv_weight).transpose(1, 0, 2).reshape(W, C)        # reference.py:148
    conv_out = np.empty((B, S, C), np.float32)
    for t in range(S):                                            # reference.py:156-157
        c = np.zeros((B, C), np.float32)
        for j in range(W):
            c = c + window[:, t + j] * w[j]
        conv_out[:, t] = c * (1.0 / (1.0 + np.exp(-c)))
    qkv = conv_out.reshape(T, C)
    q = l2norm_rsqrt(qkv[:, :dim].reshape(T, H, D), mult=D ** -0.5)
    k = l2norm_rsqrt(qkv[:, dim:2 * dim].reshape(T, H, D))
    v = np.ascontiguousarray(qkv[:, 2 * dim:].reshape(T, H, D))
    g = gate(_f32(gate_in).reshape(T, H, D), A_log, dt_bias, lower_bound)
    b = sigmoid(beta_in)
    S_in = np.zeros((B, H, D, D), np.float32)
    live = (read_slot > 0) & (cslot > 0)                          # kda/mi350x/kda/decode/kda_v14_b.cu:1035
    for n in range(B):
        if live[n]:
            S_in[n] = ssm_state[read_slot[n]]
    o, steps = recurrent_core(q, k, v, g, b, S_in, 1.0, precision)
    ob = bf16_round(o)                                            # reference.py:172-175
    rstd = 1.0 / np.sqrt((ob * ob).mean(-1, keepdims=True) + np.float32(norm_eps))
    og = _f32(out_gate).reshape(T, H, D)
    fac = rstd * _f32(norm_weight) * (1.0 / (1.0 + np.exp(-og)))
    y = ob * fac
    out = bf16_round(y.reshape(T, dim))
    conv_new = np.array(conv_state, copy=True)
    ssm_new = np.array(ssm_state, copy=True)
    ob = ob.reshape(T, dim)
    fac = fac.reshape(T, dim)
    for n in range(B):
        if not live[n]:
            out[n * S:(n + 1) * S] = 0.0
            ob[n * S:(n + 1) * S] = 0.0                           # no norm applies to a dead sequence's rows
            fac[n * S:(n + 1) * S] = 0.0
            continue
        if spec:
            for t in range(S):
                if idx[n, t] > 0:
                    ssm_new[idx[n, t]] = steps[n, t]
            conv_new[cslot[n], :W - 2 + S] = window[n, 1:]        # reference.py:176-177
        else:
            ssm_new[read_slot[n]] = steps[n, S - 1]
            # reference.py:178-180 (taps [0, 3); more taps, which kernel_v13_a.py:711-712 accepts, stay as they are)
            conv_new[cslot[n], :W - 1] = window[n, -(W - 1):]
    if aux:
        return out, conv_new, ssm_new, (ob, fac)
    return out, conv_new, ssm_new


def max_threads():
    return int(lib().kdao_max_threads())


__all__ = ["gate", "sigmoid", "l2norm_clamp", "l2norm_rsqrt", "bf16_round", "chains", "prefill_plain",
           "checkpoints_every_n", "prefill_serving", "recurrent_core", "recurrent", "decode_full", "max_threads"]
