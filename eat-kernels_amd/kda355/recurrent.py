"""Recurrent KDA decode / speculative verify (host side of kda355_recurrent_launch).

    o, pool = fused_recurrent_kda(q, k, v, g, beta, initial_state=pool, cu_seqlens=cu,
                                  ssm_state_indices=idx, num_accepted_tokens=acc)

Mirrors the call vLLM's Kimi layer makes (kda/mi350x/benchmark/vllm_reference/kda.py:488-502, 560-575) and the fla
`fused_recurrent_kda` keyword form: q, k, v [1, T, H, 128] bf16 with T = B * S packed uniformly (only
len(cu_seqlens) is used: B = len - 1, S = T / B, kda/mi350x/docs/HANDOVER.md:88); the gate is either `g` (fp32
log-decay) or `raw_g` + A_log + dt_bias + lower_bound (bf16, activated in the kernel); beta is either `beta` (fp32,
activated) or `raw_beta` (bf16 logits).  The state pool initial_state [slots, H, 128, 128] fp32 (value-major, any slot
stride, rows dense) is updated in place:
  * plain decode (ssm_state_indices [B]): read and write pool[idx[n]];
  * spec verify (ssm_state_indices [B, S], num_accepted_tokens [B]): start from pool[idx[n, a-1]] and write the state
    after token t to pool[idx[n, t]] (kda/mi350x/reference.py:135-143, 168-171).
Slot 0 is the reserved padding slot (never read, never written); out-of-range slots are treated the same way.
Errors follow the reference validator (kda/mi350x/kda/decode/kernel_v13_a.py:697-735): TypeError for a wrong dtype or
device, ValueError for a wrong shape or stride.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib

D = 128


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _stream(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _need(name, t, dtype, device):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"kda355: {name} must be a tensor")
    if t.dtype != dtype:
        raise TypeError(f"kda355: {name} must be {dtype}, got {t.dtype}")
    if t.device != device:
        raise TypeError(f"kda355: {name} must be on {device}, got {t.device}")


def _rows_dense(name, t, inner):
    """Last `inner` dims contiguous (the row / slot stride is honoured)."""
    exp = 1
    for d in range(t.dim() - 1, t.dim() - 1 - inner, -1):
        if t.size(d) != 1 and t.stride(d) != exp:
            raise ValueError(f"kda355: {name} must be dense within a row")
        exp *= t.size(d)


def _pool_view(name, pool, H, device):
    _need(name, pool, torch.float32, device)
    if pool.dim() != 4 or tuple(pool.shape[1:]) != (H, D, D):
        raise ValueError(f"kda355: {name} must be [slots, {H}, 128, 128], got {tuple(pool.shape)}")
    _rows_dense(name, pool, 3)
    return pool.stride(0) if pool.size(0) > 1 else H * D * D


def fused_recurrent_kda(q, k, v, g=None, beta=None, scale=None, initial_state=None, inplace_final_state=True,
                        cu_seqlens=None, ssm_state_indices=None, num_accepted_tokens=None,
                        use_qk_l2norm_in_kernel=True, out=None, *, raw_g=None, raw_beta=None, A_log=None,
                        dt_bias=None, lower_bound=-5.0, write_pool=None, write_indices=None, slot0_reserved=True):
    """Returns (o [1, T, H, 128] bf16, initial_state) -- the pool is updated in place.

    write_pool / write_indices: optional separate destination of the per-token states of a spec verify (the
    intermediate-state scratch of a verify step whose accepted length is committed later by spec_commit); by default
    the per-token states go to initial_state[ssm_state_indices[n, t]] as in the reference."""
    if not inplace_final_state:
        raise ValueError("kda355: only the in-place pool form is supported (inplace_final_state=True)")
    if q.dim() != 4 or q.shape[0] != 1 or q.shape[3] != D:
        raise ValueError(f"kda355: q must be [1, T, H, 128], got {tuple(q.shape)}")
    dev = q.device
    if dev.type != "cuda":
        raise TypeError("kda355: tensors must be on a GPU")
    T, H = q.shape[1], q.shape[2]
    for name, t in (("q", q), ("k", k), ("v", v)):
        _need(name, t, torch.bfloat16, dev)
        if tuple(t.shape) != (1, T, H, D):
            raise ValueError(f"kda355: {name} must be [1, {T}, {H}, 128], got {tuple(t.shape)}")
        _rows_dense(name, t, 2)
    if q.stride(1) != k.stride(1) or q.stride(1) != v.stride(1):
        raise ValueError("kda355: q, k, v must share one token stride")
    if cu_seqlens is None:
        B = 1
    else:
        B = cu_seqlens.numel() - 1
    if B < 1 or T % B:
        raise ValueError(f"kda355: T = {T} is not B x S for B = {B}")
    S = T // B
    flags = _lib.REC_NORMALIZE_QK if use_qk_l2norm_in_kernel else 0
    if slot0_reserved:
        flags |= _lib.REC_SLOT0_RESERVED
    if (g is None) == (raw_g is None):
        raise ValueError("kda355: pass exactly one of g / raw_g")
    if g is not None:
        _need("g", g, torch.float32, dev)
        gt = g
    else:
        _need("raw_g", raw_g, torch.bfloat16, dev)
        gt = raw_g
        flags |= _lib.REC_RAW_GATE
        _need("A_log", A_log, torch.float32, dev)
        _need("dt_bias", dt_bias, torch.float32, dev)
        if A_log.numel() != H or dt_bias.numel() != H * D or not A_log.is_contiguous() or not dt_bias.is_contiguous():
            raise ValueError("kda355: A_log must be [H] and dt_bias [H*128], contiguous")
    if tuple(gt.shape) != (1, T, H, D):
        raise ValueError(f"kda355: gate must be [1, {T}, {H}, 128], got {tuple(gt.shape)}")
    _rows_dense("gate", gt, 2)
    if (beta is None) == (raw_beta is None):
        raise ValueError("kda355: pass exactly one of beta / raw_beta")
    if beta is not None:
        _need("beta", beta, torch.float32, dev)
        bt = beta
    else:
        _need("raw_beta", raw_beta, torch.bfloat16, dev)
        bt = raw_beta
        flags |= _lib.REC_RAW_BETA
    if tuple(bt.shape) != (1, T, H) or bt.stride(2) != 1:
        raise ValueError(f"kda355: beta must be [1, {T}, {H}] with dense heads, got {tuple(bt.shape)}")
    pool = initial_state
    pss = _pool_view("initial_state", pool, H, dev)
    idx = ssm_state_indices
    spec = num_accepted_tokens is not None
    _need("ssm_state_indices", idx, torch.int32, dev)
    if tuple(idx.shape) != ((B, S) if spec else (B,)) or not idx.is_contiguous():
        raise ValueError(f"kda355: ssm_state_indices must be contiguous int32 {(B, S) if spec else (B,)}, "
                         f"got {tuple(idx.shape)}")
    if spec:
        _need("num_accepted_tokens", num_accepted_tokens, torch.int32, dev)
        if tuple(num_accepted_tokens.shape) != (B,) or not num_accepted_tokens.is_contiguous():
            raise ValueError(f"kda355: num_accepted_tokens must be contiguous int32 ({B},)")
    if out is None:
        out = torch.empty(1, T, H, D, dtype=torch.bfloat16, device=dev)
    else:
        _need("out", out, torch.bfloat16, dev)
        if tuple(out.shape) != (1, T, H, D):
            raise ValueError(f"kda355: out must be [1, {T}, {H}, 128], got {tuple(out.shape)}")
        _rows_dense("out", out, 2)
    a = _lib.KdaRecurrentArgs()
    a.q, a.k, a.v, a.g, a.beta = _ptr(q), _ptr(k), _ptr(v), _ptr(gt), _ptr(bt)
    a.A_log, a.dt_bias = _ptr(A_log), _ptr(dt_bias)
    a.read_pool = _ptr(pool)
    a.read_idx = _ptr(idx)
    a.read_idx_stride = S if spec else 1
    a.num_accepted = _ptr(num_accepted_tokens) if spec else None
    a.out = _ptr(out)
    a.qkv_row_stride, a.g_row_stride, a.beta_row_stride, a.out_row_stride = q.stride(1), gt.stride(1), bt.stride(1), out.stride(1)
    a.read_slot_stride, a.read_slots = pss, pool.shape[0]
    if spec:
        flags |= _lib.REC_PER_TOKEN
        wp = pool if write_pool is None else write_pool
        wi = idx if write_indices is None else write_indices
        wss = _pool_view("write_pool", wp, H, dev)
        _need("write_indices", wi, torch.int32, dev)
        if tuple(wi.shape) != (B, S) or not wi.is_contiguous():
            raise ValueError(f"kda355: write_indices must be contiguous int32 ({B}, {S})")
        if slot0_reserved and write_pool is None:
            flags |= _lib.REC_WRITE_SLOT0_RESERVED
        a.write_pool, a.write_idx = _ptr(wp), _ptr(wi)
        a.write_slot_stride, a.write_slots = wss, wp.shape[0]
    a.B, a.S, a.H = B, S, H
    a.scale = float(D ** -0.5 if scale is None else scale)
    a.lower_bound = float(lower_bound)
    a.flags = flags
    _lib.check(_lib.lib().kda355_recurrent_launch(ctypes.byref(a), _stream(dev)), "fused_recurrent_kda")
    return out, pool


def spec_commit(scratch, scratch_indices, pool, pool_indices, num_accepted_tokens, slot0_reserved=True):
    """pool[pool_indices[n]] = scratch[scratch_indices[n, a-1]] with a = num_accepted_tokens[n] (clamped to 1..S)."""
    dev = pool.device
    B, S = scratch_indices.shape
    H = pool.shape[1]
    sss = _pool_view("scratch", scratch, H, dev)
    pss = _pool_view("pool", pool, H, dev)
    for name, t, shp in (("scratch_indices", scratch_indices, (B, S)), ("pool_indices", pool_indices, (B,)),
                         ("num_accepted_tokens", num_accepted_tokens, (B,))):
        _need(name, t, torch.int32, dev)
        if tuple(t.shape) != shp or not t.is_contiguous():
            raise ValueError(f"kda355: {name} must be contiguous int32 {shp}")
    a = _lib.KdaSpecCommitArgs()
    a.scratch, a.pool = _ptr(scratch), _ptr(pool)
    a.scratch_idx, a.pool_idx, a.num_accepted = _ptr(scratch_indices), _ptr(pool_indices), _ptr(num_accepted_tokens)
    a.scratch_slot_stride, a.scratch_slots, a.pool_slot_stride, a.pool_slots = sss, scratch.shape[0], pss, pool.shape[0]
    a.B, a.S, a.H = B, S, H
    a.flags = _lib.REC_SLOT0_RESERVED if slot0_reserved else 0
    _lib.check(_lib.lib().kda355_spec_commit_launch(ctypes.byref(a), _stream(dev)), "spec_commit")
    return pool
