"""torch.library registration of the kda355 entry points: torch.ops.kda355.*.

An engine that swaps kernels through the op registry (vLLM's `torch.ops._C.fused_kda_*`, the benchmark's
`torch.ops.kda_sota.*` / `torch.ops.kda_decode_sota.*`) gets the same calls here, and dynamo / torch.compile sees
registered ops with mutation annotations and fake implementations instead of opaque Python:

  fused_kda_decode     vLLM's ROCm Kimi fused decode op, argument for argument, with the schema of
                       kda/mi350x/benchmark/baselines/decode/vllm_hip/bindings.cpp:20-32 (as the benchmark calls it,
                       kda/mi350x/benchmark/baselines/decode/sota_decode.py:57-65).
  fused_kda_prefill    vLLM's prologue + chunk op pair (kda/mi350x/benchmark/baselines/prefill/bindings.cpp:40-58) as
                       one op: the prologue's raw inputs and the chunk op's state and checkpoint arguments, under the
                       same names, types and mutation annotations.  The pair's intermediates (qg, w, u, kg_t, aqk,
                       decay) and its group workspace do not exist in the fused kernel; its chunk_indices /
                       chunk_offsets metadata is the host plan here (plan, plan_table: PrefillMeta.as_tensors()).
  prefill              the reference's serving prefill, kda/mi350x/kda/kernel.py:131-147.
  decode               the reference's fused decode / spec verify, kda/mi350x/kda/kernel.py:212-216.
  fused_recurrent_kda  vLLM's fused_recurrent_kda on a state pool as the Kimi layer calls it
                       (kda/mi350x/benchmark/vllm_reference/kda.py:488-502).
  spec_commit          copies each sequence's accepted per-token state into its pool row.

Every op is implemented for the CUDA dispatch key only and calls the HIP kernels of libkda355.so; on CPU tensors the
dispatcher raises.  Importing this module registers the ops once per process.
"""
from __future__ import annotations

import importlib

import torch

from .decode import decode as _decode_fn, decode_batch as _decode_batch

# the package re-exports functions named like their modules (kda355.prefill, kda355.decode), so the modules are
# looked up by their full names
_prefill = importlib.import_module(__package__ + ".prefill")
_recurrent = importlib.import_module(__package__ + ".recurrent")

D = 128
NAMESPACE = "kda355"

SCHEMAS = {
    "fused_kda_decode":
        "fused_kda_decode(Tensor x, Tensor weight, Tensor? bias, Tensor! conv_state, Tensor raw_g, Tensor raw_beta, "
        "Tensor A_log, Tensor dt_bias, Tensor state_indices, Tensor! state, Tensor! out, float? lower_bound=None, "
        "Tensor? output_gate=None, Tensor? norm_weight=None, float norm_eps=1e-5) -> ()",
    "fused_kda_prefill":
        "fused_kda_prefill(Tensor q, Tensor k, Tensor v, Tensor raw_g, Tensor raw_beta, Tensor A_log, Tensor dt_bias, "
        "Tensor! out, Tensor cu_seqlens, float scale, float lower_bound, Tensor? initial_state=None, "
        "Tensor(a!)? final_state=None, Tensor(c!)? checkpoint_state=None, Tensor? checkpoint_offsets=None, "
        "Tensor? checkpoint_state_indices=None, Tensor(d!)? state_cache=None, Tensor? state_indices=None, "
        "Tensor? has_initial_state=None, Tensor? plan=None, Tensor? plan_table=None, Tensor(e!)? workspace=None) -> ()",
    "prefill":
        "prefill(Tensor q, Tensor k, Tensor v, Tensor raw_g, Tensor raw_beta, Tensor A_log, Tensor dt_bias, "
        "float scale, float lower_bound, Tensor(a!) state_cache, Tensor state_indices, Tensor has_initial_state, "
        "Tensor cu_seqlens, Tensor(b!) out, Tensor? checkpoint_offsets=None, Tensor? checkpoint_state_indices=None, "
        "Tensor? plan=None, Tensor? plan_table=None, Tensor(c!)? workspace=None) -> ()",
    "decode":
        "decode(Tensor mixed_qkv, Tensor(a!) conv_state, Tensor conv_weight, Tensor gate, Tensor beta, "
        "Tensor out_gate, Tensor A_log, Tensor dt_bias, Tensor norm_weight, Tensor(b!) ssm_state, "
        "Tensor state_indices, Tensor? num_accepted_tokens, Tensor cu_seqlens, float norm_eps, float lower_bound, "
        "Tensor(c!) out) -> ()",
    "fused_recurrent_kda":
        "fused_recurrent_kda(Tensor q, Tensor k, Tensor v, Tensor raw_g, Tensor raw_beta, Tensor A_log, "
        "Tensor dt_bias, float lower_bound, Tensor(a!) initial_state, Tensor cu_seqlens, Tensor ssm_state_indices, "
        "Tensor? num_accepted_tokens, Tensor(b!) out, float? scale=None, bool use_qk_l2norm_in_kernel=True, "
        "Tensor(c!)? write_pool=None, Tensor? write_indices=None) -> ()",
    "spec_commit":
        "spec_commit(Tensor scratch, Tensor scratch_indices, Tensor(a!) pool, Tensor pool_indices, "
        "Tensor num_accepted_tokens, bool slot0_reserved=True) -> ()",
}


def _meta(plan, plan_table):
    if (plan is None) != (plan_table is None):
        raise ValueError("kda355: pass plan and plan_table together (PrefillMeta.as_tensors())")
    return None if plan is None else _prefill.PrefillMeta.from_tensors(plan, plan_table)


def _fused_kda_decode(x, weight, bias, conv_state, raw_g, raw_beta, A_log, dt_bias, state_indices, state, out,
                      lower_bound=None, output_gate=None, norm_weight=None, norm_eps=1e-5):
    """Plain decode, one token per sequence (T = B = state_indices.numel()), as vLLM's op: x [T, 3 * H * 128] the
    projected q|k|v rows; weight the conv taps; conv_state [slots, 3 * H * 128, taps], a view whose tap-major
    transpose has dense rows (the pool layout of kda/mi350x/reference.py:104-181); raw_g [1, T, H, 128];
    raw_beta [1, T, H]; state [slots, H, 128, 128] fp32; out [1, T, H, 128] and output_gate [T, H, 128] bf16.
    The kernel implements the bounded gate and the gated RMSNorm, so lower_bound, output_gate and norm_weight are
    required and a conv bias is rejected."""
    if bias is not None:
        raise ValueError("kda355 fused_kda_decode: the KDA conv has no bias (bias must be None)")
    if lower_bound is None:
        raise ValueError("kda355 fused_kda_decode: lower_bound is required (the gate is lower_bound * sigmoid(...))")
    if output_gate is None or norm_weight is None:
        raise ValueError("kda355 fused_kda_decode: output_gate and norm_weight are required (fused gated RMSNorm)")
    if x.dim() != 2 or raw_g.dim() != 4 or raw_beta.dim() != 3 or out.dim() != 4 or output_gate.dim() != 3:
        raise ValueError("kda355 fused_kda_decode: expected x [T, C], raw_g [1, T, H, 128], raw_beta [1, T, H], "
                         "out [1, T, H, 128], output_gate [T, H, 128]")
    if conv_state.dim() != 3:
        raise ValueError("kda355 fused_kda_decode: conv_state must be [slots, 3 * H * 128, taps]")
    T = x.shape[0]
    B = state_indices.numel()
    if B != T:
        raise ValueError(f"kda355 fused_kda_decode: one token per sequence (T = {T}, {B} state indices)")
    H = raw_beta.shape[2]
    try:
        out2 = out[0].view(T, H * D)
        og2 = output_gate.view(T, H * D)
    except RuntimeError as e:
        raise ValueError(f"kda355 fused_kda_decode: out / output_gate must have dense rows ({e})") from None
    _decode_batch(x, conv_state.transpose(1, 2), weight, raw_g[0], raw_beta[0], og2, A_log, dt_bias, norm_weight,
                  state, state_indices, None, B, norm_eps, lower_bound, out2)


def _fused_kda_prefill(q, k, v, raw_g, raw_beta, A_log, dt_bias, out, cu_seqlens, scale, lower_bound,
                       initial_state=None, final_state=None, checkpoint_state=None, checkpoint_offsets=None,
                       checkpoint_state_indices=None, state_cache=None, state_indices=None, has_initial_state=None,
                       plan=None, plan_table=None, workspace=None):
    """Semantics of vLLM's chunk_kda_prefill with the fused backend (kda/mi350x_plain/sota/vllm_reference/
    kda_prefill.py:27-140 and kda_chunk.py:192-294): q / k L2-normalized in the kernel, the bounded gate and
    sigmoid(beta) applied in the kernel.  State: either state_cache + state_indices + has_initial_state (read and
    written in place; initial_state / final_state must then be None) or the dense initial_state / final_state
    [N, H, 128, 128].  Checkpoints: checkpoint_offsets [N] (0 or a non-multiple of 64: none) into checkpoint_state,
    at row checkpoint_state_indices[n] (< 0: none) or, without them, at row n.  A given plan fixes the checkpoint
    offsets (they are planned on the host): pass the plan made with the same offsets."""
    meta = _meta(plan, plan_table)
    dev, T, H = _prefill._check_qkv(q, k, v)
    ck = checkpoint_state is not None and checkpoint_offsets is not None
    if meta is None:
        meta = _prefill.plan(cu_seqlens, H, checkpoint_offsets=checkpoint_offsets if ck else None, device=dev)
    if meta.any_ck and not ck:
        raise ValueError("kda355: the plan was prepared with checkpoints but checkpoint_state / offsets are missing")
    N = meta.N
    if state_cache is not None:
        if initial_state is not None or final_state is not None:
            raise ValueError("kda355: state_cache replaces initial_state / final_state")
        if state_indices is None or has_initial_state is None:
            raise ValueError("kda355: state_cache needs state_indices and has_initial_state")
    g, beta, A_log, dt_bias, flags = _prefill._gates(dev, T, H, raw_g, raw_beta, True, True, A_log, dt_bias)
    flags |= _prefill.PF_NORMALIZE_QK
    _prefill._need("out", out, torch.bfloat16, dev)
    _prefill._tok_rows("out", out, T, H, D)
    kw = {}
    if ck and meta.any_ck:
        if checkpoint_state_indices is None:
            ck_idx = torch.arange(N, dtype=torch.int32, device=dev)
        else:
            _prefill._need("checkpoint_state_indices", checkpoint_state_indices, torch.int32, dev)
            if checkpoint_state_indices.numel() != N or not checkpoint_state_indices.is_contiguous():
                raise ValueError("kda355: checkpoint_state_indices must be a contiguous int32 [N] tensor")
            ck_idx = checkpoint_state_indices
        _prefill._need("checkpoint_state", checkpoint_state, torch.float32, dev)
        kw.update(ck_pool=checkpoint_state, ck_idx=ck_idx)
        flags |= _prefill.PF_CK_SINGLE
    if state_cache is not None:
        _prefill._need("state_cache", state_cache, torch.float32, dev)
        _prefill._need("state_indices", state_indices, torch.int32, dev)
        _prefill._need("has_initial_state", has_initial_state, torch.bool, dev)
        if state_indices.numel() != N or not state_indices.is_contiguous():
            raise ValueError("kda355: state_indices must be a contiguous int32 [N] tensor")
        if has_initial_state.numel() != N or not has_initial_state.is_contiguous():
            raise ValueError("kda355: has_initial_state must be a contiguous bool [N] tensor")
        kw.update(pool=state_cache, idx=state_indices, has_init=has_initial_state)
    else:
        init = None
        if initial_state is not None:
            _prefill._need("initial_state", initial_state, torch.float32, dev)
            if tuple(initial_state.shape) != (N, H, D, D) or not initial_state.is_contiguous():
                raise ValueError(f"kda355: initial_state must be a contiguous [{N}, {H}, 128, 128] tensor")
            init = initial_state
        if final_state is None:
            final_state = torch.empty(N, H, D, D, dtype=torch.float32, device=dev)
        else:
            _prefill._need("final_state", final_state, torch.float32, dev)
            if tuple(final_state.shape) != (N, H, D, D) or not final_state.is_contiguous():
                raise ValueError(f"kda355: final_state must be a contiguous [{N}, {H}, 128, 128] tensor")
        kw.update(init=init, final=final_state)
    _prefill._launch(meta, q, k, v, g, beta, out, flags, scale, lower_bound, A_log, dt_bias, workspace=workspace,
                     **kw)


def _prefill_op(q, k, v, raw_g, raw_beta, A_log, dt_bias, scale, lower_bound, state_cache, state_indices,
                has_initial_state, cu_seqlens, out, checkpoint_offsets=None, checkpoint_state_indices=None, plan=None,
                plan_table=None, workspace=None):
    _prefill.prefill(q, k, v, raw_g, raw_beta, A_log, dt_bias, scale, lower_bound, state_cache, state_indices,
                     has_initial_state, cu_seqlens, out, checkpoint_offsets, checkpoint_state_indices,
                     meta=_meta(plan, plan_table), workspace=workspace)


def _decode_op(mixed_qkv, conv_state, conv_weight, gate, beta, out_gate, A_log, dt_bias, norm_weight, ssm_state,
               state_indices, num_accepted_tokens, cu_seqlens, norm_eps, lower_bound, out):
    _decode_fn(mixed_qkv, conv_state, conv_weight, gate, beta, out_gate, A_log, dt_bias, norm_weight, ssm_state,
               state_indices, num_accepted_tokens, cu_seqlens, norm_eps, lower_bound, out)


def _fused_recurrent_op(q, k, v, raw_g, raw_beta, A_log, dt_bias, lower_bound, initial_state, cu_seqlens,
                        ssm_state_indices, num_accepted_tokens, out, scale=None, use_qk_l2norm_in_kernel=True,
                        write_pool=None, write_indices=None):
    _recurrent.fused_recurrent_kda(q, k, v, scale=scale, initial_state=initial_state, cu_seqlens=cu_seqlens,
                                   ssm_state_indices=ssm_state_indices, num_accepted_tokens=num_accepted_tokens,
                                   use_qk_l2norm_in_kernel=use_qk_l2norm_in_kernel, out=out, raw_g=raw_g,
                                   raw_beta=raw_beta, A_log=A_log, dt_bias=dt_bias, lower_bound=lower_bound,
                                   write_pool=write_pool, write_indices=write_indices)


def _spec_commit_op(scratch, scratch_indices, pool, pool_indices, num_accepted_tokens, slot0_reserved=True):
    _recurrent.spec_commit(scratch, scratch_indices, pool, pool_indices, num_accepted_tokens, slot0_reserved)


_IMPLS = {
    "fused_kda_decode": _fused_kda_decode,
    "fused_kda_prefill": _fused_kda_prefill,
    "prefill": _prefill_op,
    "decode": _decode_op,
    "fused_recurrent_kda": _fused_recurrent_op,
    "spec_commit": _spec_commit_op,
}


def _fake(*args, **kwargs):
    """Every op writes only into tensors it was given and returns nothing."""
    return None


def _registered():
    try:
        getattr(getattr(torch.ops, NAMESPACE), "fused_kda_decode")
        return True
    except (AttributeError, RuntimeError):
        return False


def _register():
    if _registered():  # the package imported a second time under another path: the ops already exist
        return None
    lib = torch.library.Library(NAMESPACE, "DEF")
    for name, schema in SCHEMAS.items():
        lib.define(schema)
        lib.impl(name, _IMPLS[name], "CUDA")
        torch.library.register_fake(f"{NAMESPACE}::{name}", _fake, lib=lib)
    return lib


_LIBRARY = _register()
