"""Chunked KDA prefill (host side of kda355_prefill_plan / kda355_prefill_launch).

Three surfaces, each mirroring a reference interface:

  * chunk_kda(q, k, v, g, beta, scale, initial_state, output_final_state, cu_seqlens, ...) -> (o, final_state)
      the fla plain call as the reference invokes it (kda/b200/bench.py:108-117, kda/mi350x_plain/bench.py:83-92);
      g / beta are used as given unless use_gate_in_kernel / use_beta_sigmoid_in_kernel ask for the raw forms.
  * kda_prefill(q, k, v, raw_g, raw_beta, A_log, dt_bias, initial_state, cu_seqlens, scale, lower_bound, meta,
                **serving_kwargs) -> (out, new_state[, checkpoints])
      kda/mi350x_plain/kda_mi350x.py:37-46 (gates in the kernel), plus the B200 serving keywords
      (kda/b200/kda_b200.py:15-24): ssm_state_indices (pool form), state_checkpoints / checkpoint_cu_starts /
      checkpoint_every_n_tokens (every-n rows, fp32 or bf16).
  * prefill_prepare(cu_seqlens_cpu, num_heads, checkpoint_offsets, checkpoint_state_indices, device) -> meta
    prefill(q, k, v, raw_g, raw_beta, A_log, dt_bias, scale, lower_bound, state_cache, state_indices,
            has_initial_state, cu_seqlens, out, checkpoint_offsets, checkpoint_state_indices, meta) -> None
      the vLLM-ROCm Kimi serving convention (kda/mi350x/kda/kernel.py:100-147, kda/mi350x/CONTRACT.md:14-50): paged
      fp32 pool read / written in place, has_initial_state, one checkpoint row per sequence, strided raw_beta,
      output into the caller's slice, no host synchronization inside prefill().
Errors: TypeError for dtype / device, ValueError for shapes, strides and a meta from another layout (the reference
raises RuntimeError from TORCH_CHECK at kda/mi350x/kda/prefill/main.cpp:145-174; a ValueError is a RuntimeError-free
subclass of Exception, so callers catching Exception see both).
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib

D = 128
CHUNK = 64

PF_NORMALIZE_QK = 1
PF_RAW_GATE = 2
PF_RAW_BETA = 4
PF_POOL = 8
PF_CK_SINGLE = 16
PF_CK_EVERY = 32
PF_PRECISE = 64  # KDA355_PF_PRECISE: the solve's and state update's fp16 operands as fp16 pairs (precise=True)
PF_CHUNK64 = 128  # KDA355_PF_CHUNK64: keep the 64-token kernel (and its workgroup lists) on layouts with more items than CUs


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


class PrefillMeta:
    """Schedule of one batch layout: the host plan, its device table and the layout it was made for."""

    def __init__(self, plan, tables, num_heads, ck_every, any_ck, lens, chunk64=False):
        self.plan = plan
        self.lens = lens            # host int64 [N] sequence lengths
        self.tables = tables
        self.H = num_heads
        self.N = plan.N
        self.T = plan.T
        self.ck_every = ck_every
        self.any_ck = any_ck
        self.chunk64 = bool(chunk64)  # launches keep the 64-token kernel (KDA355_PF_CHUNK64)

    @property
    def workspace_bytes(self):
        return int(self.plan.workspace_bytes)

    @property
    def ck_rows(self):
        return int(self.plan.ck_rows)

    @property
    def split(self):
        """(pieces, split sequences): 0 pieces when no sequence is split."""
        return int(self.plan.num_pieces), int(self.plan.num_split)

    def as_tensors(self):
        """(plan, plan_table): the host plan as a CPU uint8 tensor (the KdaPrefillPlan bytes, then an int32 flag for
        planned checkpoints and the sequence lengths as int64) and its device table -- the metadata tensors that the
        torch.ops entry points take where vLLM's chunk op takes chunk_indices / chunk_offsets."""
        head = bytes(self.plan) + np.array([int(self.any_ck), int(self.chunk64)], np.int32).tobytes()
        raw = head + np.ascontiguousarray(self.lens, np.int64).tobytes()
        return torch.frombuffer(bytearray(raw), dtype=torch.uint8), self.tables

    @classmethod
    def from_tensors(cls, plan_bytes, plan_table):
        """Inverse of as_tensors; checks that the pair belongs together as far as the bytes allow."""
        n = ctypes.sizeof(_lib.KdaPrefillPlan)
        if not isinstance(plan_bytes, torch.Tensor) or plan_bytes.dtype != torch.uint8 or plan_bytes.device.type != "cpu":
            raise TypeError("kda355: plan must be the CPU uint8 tensor of PrefillMeta.as_tensors()")
        if not isinstance(plan_table, torch.Tensor) or plan_table.dtype != torch.int32:
            raise TypeError("kda355: plan_table must be the int32 table of PrefillMeta.as_tensors()")
        raw = plan_bytes.contiguous().numpy().tobytes()
        if len(raw) < n + 8:
            raise ValueError("kda355: plan is too short to hold a prefill plan")
        pl = _lib.KdaPrefillPlan.from_buffer_copy(raw[:n])
        any_ck = int(np.frombuffer(raw[n:n + 4], np.int32)[0]) != 0
        chunk64 = int(np.frombuffer(raw[n + 4:n + 8], np.int32)[0]) != 0
        lens = np.frombuffer(raw[n + 8:], np.int64).copy()
        if lens.size != pl.N or int(lens.sum()) != pl.T or plan_table.numel() != pl.table_words:
            raise ValueError("kda355: plan and plan_table do not come from one PrefillMeta.as_tensors() call")
        return cls(pl, plan_table, int(pl.H), int(pl.ck_every), any_ck, lens, chunk64)


def plan(cu_seqlens, num_heads, checkpoint_offsets=None, ck_every=0, device=None, num_cus=None, chunk64=None):
    """Host-only schedule from the layout (never the data); one H2D copy of the table when device is a GPU.
    num_cus: CUs to fill (default: the device's); when the (sequence, head) chains alone leave CUs idle or the longest
    chains would finish well after the rest, long sequences are split into pieces of >= 2 chunks (later pieces run
    from a zero state carrying their transition; a scan and an output fixup complete them, with a workspace).  An
    unsplit layout with more (sequence, head) items than CUs runs the 32-token kernel (two workgroups per CU) when the
    plan's schedule model says it finishes first.  chunk64: None leaves that choice to the plan; True keeps the
    64-token kernel (and its workgroup lists); False takes the 32-token kernel for any unsplit layout (a comparison and
    test switch)."""
    cu = np.ascontiguousarray(torch.as_tensor(cu_seqlens).detach().cpu().numpy(), dtype=np.int64)
    N = cu.size - 1
    if N < 1:
        raise ValueError("kda355: cu_seqlens needs at least 2 entries")
    ck = None
    if checkpoint_offsets is not None:
        ck = np.ascontiguousarray(torch.as_tensor(checkpoint_offsets).detach().cpu().numpy(), dtype=np.int32)
        if ck.size != N:
            raise ValueError("kda355: checkpoint_offsets must have N entries")
    pin = _lib.KdaPrefillPlanIn()
    pin.cu_seqlens = ctypes.c_void_p(cu.ctypes.data)
    pin.ck_offsets = ctypes.c_void_p(ck.ctypes.data) if ck is not None else None
    pin.N, pin.H, pin.ck_every = N, int(num_heads), int(ck_every)
    if num_cus is None and device is not None and torch.device(device).type == "cuda":
        num_cus = torch.cuda.get_device_properties(torch.device(device)).multi_processor_count
    pin.num_cus = int(num_cus or 0)
    pl = _lib.KdaPrefillPlan()
    L = _lib.lib()
    # one planning pass in the common case: a table of this many words holds every layout up to a few hundred pieces;
    # a larger one reports its size (table_words is set before the capacity check) and is planned again
    cap = 8192 + 32 * (N + int(cu[-1]) // 64)
    tab = np.zeros(cap, np.int32)
    rc = L.kda355_prefill_plan(ctypes.byref(pin), ctypes.byref(pl), ctypes.c_void_p(tab.ctypes.data), cap)
    if rc != 0 and int(pl.table_words) > cap:
        tab = np.zeros(int(pl.table_words), np.int32)
        rc = L.kda355_prefill_plan(ctypes.byref(pin), ctypes.byref(pl), ctypes.c_void_p(tab.ctypes.data), tab.size)
    _lib.check(rc, "prefill_plan")
    t = torch.from_numpy(tab[:int(pl.table_words)])
    if device is not None and torch.device(device).type == "cuda":
        t = t.to(device)
    any_ck = ck is not None and bool(np.any(ck > 0))
    if chunk64 is False and int(pl.num_split) == 0:
        pl.chunk32 = 1
    return PrefillMeta(pl, t, int(num_heads), int(ck_every), any_ck, np.diff(cu), chunk64 is True)


def _need(name, t, dtype, device):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"kda355: {name} must be a tensor")
    if t.dtype != dtype:
        raise TypeError(f"kda355: {name} must be {dtype}, got {t.dtype}")
    if t.device != device:
        raise TypeError(f"kda355: {name} must be on {device}, got {t.device}")


def _tok_rows(name, t, T, H, last):
    """[1, T, H, last] (or [1, T, H]) with dense heads; returns the token stride."""
    shape = (1, T, H, last) if last else (1, T, H)
    if tuple(t.shape) != shape:
        raise ValueError(f"kda355: {name} must be {list(shape)}, got {list(t.shape)}")
    if last:
        if (t.stride(3) != 1 and last > 1) or (t.stride(2) != last and H > 1):
            raise ValueError(f"kda355: {name} must be dense within a token")
    elif t.stride(2) != 1 and H > 1:
        raise ValueError(f"kda355: {name} rows must be dense over heads")
    return t.stride(1) if T > 1 else H * max(last, 1)


def _pool_stride(name, pool, H):
    if pool.dim() != 4 or tuple(pool.shape[1:]) != (H, D, D):
        raise ValueError(f"kda355: {name} must be [slots, {H}, 128, 128], got {list(pool.shape)}")
    if pool.stride(3) != 1 or pool.stride(2) != D or pool.stride(1) != D * D:
        raise ValueError(f"kda355: {name} rows must be dense")
    return pool.stride(0) if pool.shape[0] > 1 else H * D * D


def _launch(meta, q, k, v, gt, bt, out, flags, scale, lower_bound, A_log=None, dt_bias=None, pool=None, idx=None,
            has_init=None, init=None, final=None, ck_pool=None, ck_idx=None, ck_bf16=False, workspace=None):
    dev = q.device
    T, H = q.shape[1], q.shape[2]
    if meta.T != T or meta.H != H:
        raise ValueError(f"kda355: meta was prepared for another layout (T/H {meta.T}/{meta.H} vs {T}/{H})")
    if meta.tables.device != dev:
        raise ValueError("kda355: meta was prepared for another device")
    static = isinstance(workspace, str)
    if static:
        # kda355_prefill_launch_noalloc: the library's static device scratch, no allocation in the call
        if workspace != "static":
            raise ValueError("kda355: workspace must be a uint8 device tensor, None or 'static'")
        workspace = None
    elif workspace is None:
        workspace = torch.empty(max(meta.workspace_bytes, 256), dtype=torch.uint8, device=dev)
    elif workspace.numel() * workspace.element_size() < meta.workspace_bytes or workspace.device != dev:
        raise ValueError("kda355: workspace too small or on another device")
    a = _lib.KdaPrefillArgs()
    a.q, a.k, a.v, a.g, a.beta = _ptr(q), _ptr(k), _ptr(v), _ptr(gt), _ptr(bt)
    a.A_log, a.dt_bias = _ptr(A_log), _ptr(dt_bias)
    a.out = _ptr(out)
    a.qkv_row_stride = q.stride(1) if T > 1 else H * D
    a.g_row_stride = gt.stride(1) if T > 1 else H * D
    a.beta_row_stride = bt.stride(1) if T > 1 else H
    a.out_row_stride = out.stride(1) if T > 1 else H * D
    if pool is not None:
        a.state_pool, a.state_idx, a.has_initial_state = _ptr(pool), _ptr(idx), _ptr(has_init)
        a.state_slot_stride, a.state_slots = _pool_stride("state_cache", pool, H), pool.shape[0]
        flags |= PF_POOL
    else:
        a.initial_state, a.final_state = _ptr(init), _ptr(final)
    if ck_pool is not None:
        a.ck_pool, a.ck_idx = _ptr(ck_pool), _ptr(ck_idx)
        a.ck_slot_stride, a.ck_slots = _pool_stride("checkpoint pool", ck_pool, H), ck_pool.shape[0]
        a.ck_dtype = 1 if ck_bf16 else 0
    a.tables = _ptr(meta.tables)
    a.workspace = _ptr(workspace)
    a.T, a.N, a.H = T, meta.N, H
    a.scale, a.lower_bound = float(scale), float(lower_bound)
    a.flags = flags | (PF_CHUNK64 if getattr(meta, "chunk64", False) else 0)
    a.plan = ctypes.pointer(meta.plan)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    if static:
        _lib.check(_lib.noalloc_lib().kda355_prefill_launch_noalloc(ctypes.byref(a), stream), "prefill_noalloc")
    else:
        _lib.check(_lib.lib().kda355_prefill_launch(ctypes.byref(a), stream), "prefill")


def _check_qkv(q, k, v):
    if not isinstance(q, torch.Tensor) or q.dim() != 4 or q.shape[0] != 1 or q.shape[3] != D:
        raise ValueError(f"kda355: q must be [1, T, H, 128], got {list(getattr(q, 'shape', []))}")
    dev = q.device
    if dev.type != "cuda":
        raise TypeError("kda355: tensors must be on a GPU")
    T, H = q.shape[1], q.shape[2]
    strides = []
    for name, t in (("q", q), ("k", k), ("v", v)):
        _need(name, t, torch.bfloat16, dev)
        strides.append(_tok_rows(name, t, T, H, D))
    if len(set(strides)) != 1:
        raise ValueError("kda355: q, k, v must share one token stride")
    return dev, T, H


def _gates(dev, T, H, g, beta, raw_gate, raw_beta, A_log, dt_bias):
    """Validates the gate / beta inputs; returns (g, beta, A_log, dt_bias, flags)."""
    flags = 0
    if raw_gate:
        if not isinstance(g, torch.Tensor):
            raise TypeError("kda355: the gate must be a tensor")
        if g.dtype != torch.bfloat16:
            g = g.bfloat16()
        _need("raw_g", g, torch.bfloat16, dev)
        flags |= PF_RAW_GATE
        if A_log is None or dt_bias is None:
            raise ValueError("kda355: the in-kernel gate needs A_log and dt_bias")
        _need("A_log", A_log, torch.float32, dev)
        _need("dt_bias", dt_bias, torch.float32, dev)
        if A_log.numel() != H or dt_bias.numel() != H * D:
            raise ValueError("kda355: A_log must be [H] and dt_bias [H*128]")
        A_log, dt_bias = A_log.reshape(-1).contiguous(), dt_bias.reshape(-1).contiguous()
    else:
        _need("g", g, torch.float32, dev)
        A_log = dt_bias = None
    _tok_rows("g", g, T, H, D)
    if raw_beta:
        if not isinstance(beta, torch.Tensor):
            raise TypeError("kda355: beta must be a tensor")
        if beta.dtype != torch.bfloat16:
            beta = beta.bfloat16()
        _need("raw_beta", beta, torch.bfloat16, dev)
        flags |= PF_RAW_BETA
    else:
        _need("beta", beta, torch.float32, dev)
    _tok_rows("beta", beta, T, H, 0)
    return g, beta, A_log, dt_bias, flags


def _run_plain(q, k, v, g, beta, scale, initial_state, cu_seqlens, lower_bound, meta, out, workspace, flags, A_log,
               dt_bias, ssm_state_indices, state_checkpoints, checkpoint_cu_starts, checkpoint_every_n_tokens,
               checkpoint_state_indices):
    """The plain call with the B200 serving keywords (kda/b200/kda_b200.py:15-24).  Returns (out, final, ck, meta)."""
    dev, T, H = q.device, q.shape[1], q.shape[2]
    every = int(checkpoint_every_n_tokens or 0)
    if every:
        if every % CHUNK:
            raise ValueError("kda355: checkpoint_every_n_tokens must be a multiple of 64")
        if state_checkpoints is None or (checkpoint_cu_starts is None) == (checkpoint_state_indices is None):
            raise ValueError("kda355: every-n checkpoints need state_checkpoints and exactly one of "
                             "checkpoint_cu_starts / checkpoint_state_indices")
    if meta is None or meta.ck_every != every:
        if meta is not None and cu_seqlens is None:
            cu_seqlens = torch.as_tensor(np.concatenate([[0], np.cumsum(meta.lens)]))
        cu = torch.tensor([0, T], dtype=torch.int64) if cu_seqlens is None else cu_seqlens
        meta = plan(cu, H, ck_every=every, device=dev)
    N = meta.N
    if out is None:
        out = torch.empty(1, T, H, D, dtype=torch.bfloat16, device=dev)
    else:
        _need("out", out, torch.bfloat16, dev)
        _tok_rows("out", out, T, H, D)
    ck = {}
    if every:
        if state_checkpoints.dtype not in (torch.float32, torch.bfloat16) or state_checkpoints.device != dev:
            raise TypeError("kda355: state_checkpoints must be fp32 or bf16 on the device")
        if checkpoint_state_indices is not None:
            # explicit row table: row checkpoint_state_indices[r] receives the r-th checkpoint (sequence-major)
            _need("checkpoint_state_indices", checkpoint_state_indices, torch.int32, dev)
            if checkpoint_state_indices.dim() != 1 or not checkpoint_state_indices.is_contiguous() or \
                    checkpoint_state_indices.numel() < meta.ck_rows:
                raise ValueError(f"kda355: checkpoint_state_indices must be a contiguous int32 tensor of >= "
                                 f"{meta.ck_rows} rows")
            ck_idx = checkpoint_state_indices
        else:
            starts = checkpoint_cu_starts.to(device=dev, dtype=torch.int64)
            counts = (meta.lens + every - 1) // every
            ck_idx = _ck_row_table(starts[:-1], counts, dev)
        ck = dict(ck_pool=state_checkpoints, ck_idx=ck_idx, ck_bf16=state_checkpoints.dtype == torch.bfloat16)
        flags |= PF_CK_EVERY
    if ssm_state_indices is not None:
        pool = initial_state
        _need("initial_state", pool, torch.float32, dev)
        _need("ssm_state_indices", ssm_state_indices, torch.int32, dev)
        if ssm_state_indices.dim() != 1 or ssm_state_indices.numel() != N or not ssm_state_indices.is_contiguous():
            raise ValueError("kda355: ssm_state_indices must be a contiguous int32 [N] tensor")
        has_init = torch.ones(N, dtype=torch.bool, device=dev)
        _launch(meta, q, k, v, g, beta, out, flags, scale, lower_bound, A_log, dt_bias, pool=pool,
                idx=ssm_state_indices, has_init=has_init, workspace=workspace, **ck)
        final = pool
    else:
        init = None
        if initial_state is not None and initial_state.numel():
            _need("initial_state", initial_state, torch.float32, dev)
            if tuple(initial_state.shape) != (N, H, D, D):
                raise ValueError(f"kda355: initial_state must be [{N}, {H}, 128, 128], got {list(initial_state.shape)}")
            init = initial_state.contiguous()
        final = torch.empty(N, H, D, D, dtype=torch.float32, device=dev)
        _launch(meta, q, k, v, g, beta, out, flags, scale, lower_bound, A_log, dt_bias, init=init, final=final,
                workspace=workspace, **ck)
    return out, final, (state_checkpoints if every else None), meta


def chunk_kda(q, k, v, g, beta, scale=None, initial_state=None, output_final_state=True, cu_seqlens=None,
              use_qk_l2norm_in_kernel=True, use_gate_in_kernel=False, use_beta_sigmoid_in_kernel=False,
              A_log=None, dt_bias=None, lower_bound=-5.0, state_v_first=True, meta=None, out=None, workspace=None,
              *, ssm_state_indices=None, state_checkpoints=None, checkpoint_cu_starts=None,
              checkpoint_every_n_tokens=0, checkpoint_state_indices=None, precise=False, **unused):
    """fla chunk_kda plain call. q, k, v [1, T, H, 128] bf16; g [1, T, H, 128] (fp32 log-decay, or the raw gate with
    use_gate_in_kernel); beta [1, T, H] (fp32 activated, or logits with use_beta_sigmoid_in_kernel); initial_state
    [N, H, 128(V), 128(K)] fp32 or None; cu_seqlens [N+1] (None: one sequence).  meta: a plan(...) result for this
    layout (skips the host read of cu_seqlens).  workspace: a uint8 device tensor of >= meta.workspace_bytes, None
    (allocated per call when the layout needs one), or "static" (kda355_prefill_launch_noalloc: the library's static
    device scratch of 256 MiB, no allocation; calls on one GPU must not overlap).  Returns (o [1, T, H, 128] bf16, final_state [N, H, 128, 128] fp32
    or None).

    Serving keywords (the B200 contract, kda/b200/kda_b200.py:15-24):
      ssm_state_indices int32 [N]: initial_state is a pool [P, H, 128, 128]; sequence i reads and updates slot
          ssm_state_indices[i] in place (every other slot is untouched) and the returned final state is the pool;
      state_checkpoints fp32 / bf16 [C, H, 128, 128] with checkpoint_every_n_tokens n (a multiple of 64) and either
          checkpoint_cu_starts int64 [N+1] (row checkpoint_cu_starts[i] + j = state before token j*n of sequence i,
          j < ceil(len_i / n)) or checkpoint_state_indices int32 [>= rows] (the r-th such state, sequence-major, goes to
          row checkpoint_state_indices[r]); bf16 rows are the fp32 states rounded to nearest even.
    With checkpoints the call returns (o, final_state, state_checkpoints).
    precise=True (no counterpart in fla): the kernel carries the solve's and the state update's fp16 operands as fp16
    pairs, which about halves the state error on chunks of nearly parallel keys with beta ~ 1 at ~11 % more time."""
    if not state_v_first:
        raise ValueError("kda355: only the value-first state layout [N, H, V, K] is supported (state_v_first=True)")
    dev, T, H = _check_qkv(q, k, v)
    if scale is None:
        scale = D ** -0.5
    g, beta, A_log, dt_bias, flags = _gates(dev, T, H, g, beta, use_gate_in_kernel, use_beta_sigmoid_in_kernel,
                                            A_log, dt_bias)
    if use_qk_l2norm_in_kernel:
        flags |= PF_NORMALIZE_QK
    if precise:
        flags |= PF_PRECISE
    out, final, ck, _ = _run_plain(q, k, v, g, beta, scale, initial_state, cu_seqlens, lower_bound, meta, out,
                                   workspace, flags, A_log, dt_bias, ssm_state_indices, state_checkpoints,
                                   checkpoint_cu_starts, checkpoint_every_n_tokens, checkpoint_state_indices)
    if ck is not None:
        return out, final, ck
    return out, (final if output_final_state else None)


def kda_prefill(q, k, v, raw_g, raw_beta, A_log, dt_bias, initial_state, cu_seqlens=None, scale=None,
                lower_bound=-5.0, meta=None, *, ssm_state_indices=None, state_checkpoints=None,
                checkpoint_cu_starts=None, checkpoint_every_n_tokens=0, checkpoint_state_indices=None, precise=False):
    """kda/mi350x_plain/kda_mi350x.py:37-46 (gates, beta sigmoid and q/k norm in the kernel) with the B200 serving
    keywords of chunk_kda (kda/b200/kda_b200.py:15-24).  raw_g [1, T, H, 128] bf16, raw_beta [1, T, H] bf16 logits,
    A_log [H], dt_bias [H*128] fp32.  precise: as chunk_kda.  Returns (output, final_state) or (output, final_state,
    state_checkpoints)."""
    dev, T, H = _check_qkv(q, k, v)
    if scale is None:
        scale = D ** -0.5
    _need("raw_g", raw_g, torch.bfloat16, dev)
    _need("raw_beta", raw_beta, torch.bfloat16, dev)
    g, beta, A_log, dt_bias, flags = _gates(dev, T, H, raw_g, raw_beta, True, True, A_log, dt_bias)
    out, final, ck, _ = _run_plain(q, k, v, g, beta, scale, initial_state, cu_seqlens, lower_bound, meta, None, None,
                                   flags | PF_NORMALIZE_QK | (PF_PRECISE if precise else 0), A_log, dt_bias,
                                   ssm_state_indices, state_checkpoints,
                                   checkpoint_cu_starts, checkpoint_every_n_tokens, checkpoint_state_indices)
    return (out, final, ck) if ck is not None else (out, final)


def _ck_row_table(starts, counts, dev):
    """Flattened row ids starts[n] + j, j < counts[n] (device int32)."""
    counts_t = torch.as_tensor(counts, device=dev)
    rep = torch.repeat_interleave(starts, counts_t)
    base = torch.repeat_interleave(torch.cumsum(counts_t, 0) - counts_t, counts_t)
    j = torch.arange(int(counts_t.sum()), device=dev) - base
    return (rep + j).to(torch.int32).contiguous()


# ------------------------------------------------------------------------------------------------ serving
def prefill_prepare(cu_seqlens, num_heads, checkpoint_offsets=None, checkpoint_state_indices=None, device=None):
    """kda/mi350x/kda/kernel.py:100-110: per-step schedule from host copies of the layout, shared by every layer.
    Offsets that are not positive multiples of 64 within their sequence plan no checkpoint (the reference's
    prepare_prod rule, kda/mi350x/kda/prefill/main.cpp:110-118)."""
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    offs = checkpoint_offsets if (checkpoint_offsets is not None and checkpoint_state_indices is not None) else None
    return plan(cu_seqlens, num_heads, checkpoint_offsets=offs, device=dev)


def prefill(q, k, v, raw_g, raw_beta, A_log, dt_bias, scale, lower_bound, state_cache, state_indices,
            has_initial_state, cu_seqlens, out, checkpoint_offsets=None, checkpoint_state_indices=None, meta=None,
            workspace=None, *, precise=False):
    """kda/mi350x/kda/kernel.py:131-147 (contract kda/mi350x/CONTRACT.md:32-50).  In place: writes `out` and the pool
    rows state_indices[n] (final states) and checkpoint_state_indices[n] (state after checkpoint_offsets[n] tokens);
    nothing else.  No host synchronization when meta is given.  precise: as chunk_kda (no counterpart in the
    reference)."""
    dev, T, H = _check_qkv(q, k, v)
    if meta is None:
        meta = prefill_prepare(cu_seqlens, H, checkpoint_offsets, checkpoint_state_indices, dev)
    _need("raw_g", raw_g, torch.bfloat16, dev)
    _tok_rows("raw_g", raw_g, T, H, D)
    _need("raw_beta", raw_beta, torch.bfloat16, dev)
    _tok_rows("raw_beta", raw_beta, T, H, 0)
    _need("A_log", A_log, torch.float32, dev)
    _need("dt_bias", dt_bias, torch.float32, dev)
    if A_log.numel() != H or dt_bias.numel() != H * D or not A_log.is_contiguous() or not dt_bias.is_contiguous():
        raise ValueError("kda355: A_log must be contiguous [H] and dt_bias contiguous [H*128]")
    _need("state_cache", state_cache, torch.float32, dev)
    _need("state_indices", state_indices, torch.int32, dev)
    _need("has_initial_state", has_initial_state, torch.bool, dev)
    N = meta.N
    if state_indices.dim() != 1 or state_indices.numel() != N or not state_indices.is_contiguous():
        raise ValueError("kda355: state_indices must be a contiguous int32 [N] tensor")
    if has_initial_state.numel() != N or not has_initial_state.is_contiguous():
        raise ValueError("kda355: has_initial_state must be a contiguous bool [N] tensor")
    _need("out", out, torch.bfloat16, dev)
    _tok_rows("out", out, T, H, D)
    ck_given = checkpoint_offsets is not None and checkpoint_state_indices is not None
    if meta.any_ck and not ck_given:
        raise ValueError("kda355: meta was prepared with checkpoints but no checkpoint tensors were passed")
    flags = PF_NORMALIZE_QK | PF_RAW_GATE | PF_RAW_BETA | (PF_PRECISE if precise else 0)
    ck_pool = ck_idx = None
    if ck_given and meta.any_ck:
        _need("checkpoint_state_indices", checkpoint_state_indices, torch.int32, dev)
        if checkpoint_state_indices.numel() != N or not checkpoint_state_indices.is_contiguous():
            raise ValueError("kda355: checkpoint_state_indices must be a contiguous int32 [N] tensor")
        ck_pool, ck_idx = state_cache, checkpoint_state_indices
        flags |= PF_CK_SINGLE
    _launch(meta, q, k, v, raw_g, raw_beta, out, flags, scale, lower_bound, A_log, dt_bias, pool=state_cache,
            idx=state_indices, has_init=has_initial_state, ck_pool=ck_pool, ck_idx=ck_idx, workspace=workspace)
