"""Fused KDA decode / speculative verify step of the vLLM-ROCm Kimi layer (host side of kda355_decode_launch).

    decode(mixed_qkv, conv_state, conv_weight, gate, beta, out_gate, A_log, dt_bias, norm_weight, ssm_state,
           state_indices, num_accepted_tokens, cu_seqlens, norm_eps, lower_bound, out)

Same signature and argument meaning as the reference's `kernel.decode` (kda/mi350x/kda/kernel.py:212-216; semantics
kda/mi350x/reference.py:104-181): one call runs the width-4 causal conv + SiLU with the rolling bf16 conv cache, the
q/k norms, the gate and beta activations, the gated delta rule on the fp32 state pool and the gated RMSNorm, for
B sequences of S <= 16 tokens (T = B * S rows).  With num_accepted_tokens it is a spec verify; without, every token
is decoded in order and the final state written back (S = 1 is plain decode; the reference serves S > 1 through its
fallback path, kda/mi350x/kda/decode/kernel_v13_a.py:746-750, and so does this kernel directly).  conv_state
and ssm_state are updated in place and may be strided views into one paged byte pool (the slot stride is honoured,
rows must be dense).  Slot rows <= 0 are padding (zero output rows, nothing written).  `out` is written and returned.

Errors follow the reference validator (kda/mi350x/kda/decode/kernel_v13_a.py:697-735): TypeError for a wrong dtype or
device, ValueError for a wrong shape or stride.  Nothing data dependent is checked on the host, so the call is
capturable in a HIP graph.

Small launches (B * H <= 64) split each state over 4 workgroups, which needs a workspace of KDA355_DECODE_WS_BYTES
whose counters (its first 256 bytes) are zero before its first launch; every launch leaves them zero.  The keyword
`workspace` selects it: by default
the device's own (zeroed once, on the first call outside graph capture; a call captured before any eager call runs
whole states), None for whole states, or a caller's uint8 tensor.  Launches that may run at the same time on one GPU
(several streams) must not share a workspace.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib

D = 128
MAX_S = 16
WS_BYTES = 16640  # KDA355_DECODE_WS_BYTES
_DEFAULT = object()
_ws_by_device = {}


def default_workspace(device):
    """The device's default decode workspace (zeroed when first made), or None while a graph is being captured and
    there is none yet (making one then would record its zeroing into the graph)."""
    key = torch.device(device).index if torch.device(device).index is not None else torch.cuda.current_device()
    ws = _ws_by_device.get(key)
    if ws is None:
        if torch.cuda.is_current_stream_capturing():
            return None
        ws = torch.zeros(WS_BYTES, dtype=torch.uint8, device=torch.device("cuda", key))
        _ws_by_device[key] = ws
    return ws


def _chk(name, t, dtype, shape, device, rows_only=False):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"kda355 decode: {name} must be a tensor")
    if t.dtype != dtype or t.device != device:
        raise TypeError(f"kda355 decode: {name} must be {dtype} on {device}, got {t.dtype} on {t.device}")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"kda355 decode: {name} must have shape {tuple(shape)}, got {tuple(t.shape)}")
    dense = t[0].is_contiguous() if (rows_only and t.shape[0]) else t.is_contiguous()
    if not dense:
        raise ValueError(f"kda355 decode: {name} must be contiguous" + (" within a row / slot" if rows_only else ""))


def _slot_stride(t, per_slot):
    return t.stride(0) if t.shape[0] > 1 else per_slot


def decode(mixed_qkv, conv_state, conv_weight, gate, beta, out_gate, A_log, dt_bias, norm_weight, ssm_state,
           state_indices, num_accepted_tokens, cu_seqlens, norm_eps, lower_bound, out, *, workspace=_DEFAULT):
    if not isinstance(cu_seqlens, torch.Tensor):
        raise TypeError("kda355 decode: cu_seqlens must be a tensor")
    return decode_batch(mixed_qkv, conv_state, conv_weight, gate, beta, out_gate, A_log, dt_bias, norm_weight,
                        ssm_state, state_indices, num_accepted_tokens, cu_seqlens.numel() - 1, norm_eps, lower_bound,
                        out, workspace=workspace)


def decode_batch(mixed_qkv, conv_state, conv_weight, gate, beta, out_gate, A_log, dt_bias, norm_weight, ssm_state,
                 state_indices, num_accepted_tokens, B, norm_eps, lower_bound, out, *, workspace=_DEFAULT):
    """decode() with the batch size B given directly (only the length of cu_seqlens is ever used: every sequence has
    the same S = T / B tokens)."""
    if not isinstance(mixed_qkv, torch.Tensor) or mixed_qkv.dim() != 2:
        raise ValueError("kda355 decode: mixed_qkv must be [T, 3 * H * 128]")
    dev = mixed_qkv.device
    if dev.type != "cuda":
        raise TypeError("kda355 decode: tensors must be on a GPU")
    T, C = mixed_qkv.shape
    if C % (3 * D):
        raise ValueError(f"kda355 decode: mixed_qkv width {C} is not 3 * H * 128")
    dim = C // 3
    H = dim // D
    B = int(B)
    spec = num_accepted_tokens is not None
    if B < 1 or T % B:
        raise ValueError(f"kda355 decode: T = {T} is not B x S for B = {B}")
    S = T // B
    if S > MAX_S:
        raise ValueError(f"kda355 decode: S = {S} tokens per sequence exceeds {MAX_S}")
    taps = (2 + S) if spec else 3
    _chk("mixed_qkv", mixed_qkv, torch.bfloat16, (T, 3 * dim), dev, True)
    if conv_state.dim() != 3 or conv_state.shape[1] < taps or conv_state.shape[2] != 3 * dim:
        raise ValueError(f"kda355 decode: conv_state must be [slots, >= {taps}, {3 * dim}], got {tuple(conv_state.shape)}")
    _chk("conv_state", conv_state, torch.bfloat16, None, dev, True)
    _chk("conv_weight", conv_weight, torch.float32, (3, 4, dim), dev)
    if not gate.is_contiguous():
        gate = gate.contiguous()  # the reference's kernel.decode makes the same copy
    _chk("gate", gate, torch.bfloat16, (T, H, D), dev)
    _chk("beta", beta, torch.bfloat16, (T, H), dev, True)
    _chk("out_gate", out_gate, torch.bfloat16, (T, dim), dev, True)
    _chk("A_log", A_log, torch.float32, (H,), dev)
    _chk("dt_bias", dt_bias, torch.float32, (dim,), dev)
    _chk("norm_weight", norm_weight, torch.float32, (D,), dev)
    if ssm_state.dim() != 4 or tuple(ssm_state.shape[1:]) != (H, D, D):
        raise ValueError(f"kda355 decode: ssm_state must be [slots, {H}, 128, 128], got {tuple(ssm_state.shape)}")
    _chk("ssm_state", ssm_state, torch.float32, None, dev, True)
    _chk("out", out, torch.bfloat16, (T, dim), dev)
    for name, t in (("state_indices", state_indices), ("num_accepted_tokens", num_accepted_tokens)):
        if t is not None and t.device != dev:
            raise TypeError(f"kda355 decode: {name} must be on {dev}, got {t.device}")
    if state_indices.dtype != torch.int32 or tuple(state_indices.shape) != ((B, S) if spec else (B,)):
        raise ValueError(f"kda355 decode: state_indices must be int32 {(B, S) if spec else (B,)}, "
                         f"got {state_indices.dtype} {tuple(state_indices.shape)}")
    if spec and (num_accepted_tokens.dtype != torch.int32 or tuple(num_accepted_tokens.shape) != (B,)):
        raise ValueError(f"kda355 decode: num_accepted_tokens must be int32 ({B},), "
                         f"got {num_accepted_tokens.dtype} {tuple(num_accepted_tokens.shape)}")
    idx = state_indices.contiguous()
    acc = num_accepted_tokens.contiguous() if spec else None
    if workspace is _DEFAULT:
        workspace = default_workspace(dev)
    elif workspace is not None:
        if not isinstance(workspace, torch.Tensor) or workspace.device != dev:
            raise TypeError(f"kda355 decode: workspace must be a tensor on {dev}")
        if not workspace.is_contiguous() or workspace.numel() * workspace.element_size() < WS_BYTES:
            raise ValueError(f"kda355 decode: workspace must be contiguous with >= {WS_BYTES} bytes")

    a = _lib.KdaDecodeArgs()
    a.mixed_qkv, a.conv_state, a.conv_weight = mixed_qkv.data_ptr(), conv_state.data_ptr(), conv_weight.data_ptr()
    a.gate, a.beta, a.out_gate = gate.data_ptr(), beta.data_ptr(), out_gate.data_ptr()
    a.A_log, a.dt_bias, a.norm_weight = A_log.data_ptr(), dt_bias.data_ptr(), norm_weight.data_ptr()
    a.ssm_state, a.state_indices = ssm_state.data_ptr(), idx.data_ptr()
    a.num_accepted = acc.data_ptr() if spec else None
    a.out = out.data_ptr()
    a.mixed_row_stride, a.gate_row_stride = mixed_qkv.stride(0), gate.stride(0)
    a.beta_row_stride, a.out_gate_row_stride, a.out_row_stride = beta.stride(0), out_gate.stride(0), out.stride(0)
    a.conv_slot_stride = _slot_stride(conv_state, conv_state.shape[1] * 3 * dim)
    a.conv_tap_stride = conv_state.stride(1) if conv_state.shape[1] > 1 else 3 * dim
    a.conv_slots, a.conv_taps = conv_state.shape[0], conv_state.shape[1]
    a.ssm_slot_stride, a.ssm_slots = _slot_stride(ssm_state, H * D * D), ssm_state.shape[0]
    a.B, a.S, a.H = B, S, H
    a.norm_eps, a.lower_bound = float(norm_eps), float(lower_bound)
    a.flags = 0
    a.workspace = workspace.data_ptr() if workspace is not None else None
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    _lib.check(_lib.lib().kda355_decode_launch(ctypes.byref(a), stream), "decode")
    return out
