"""torch.ops.kda355.* registration (kda355/ops.py), without a GPU: the schemas against the vLLM op schemas they stand
in for, the plan <-> tensor round trip, fake-tensor tracing and the loud failure on CPU tensors."""
import numpy as np
import pytest
import torch

D = 128

# The op schemas the registrations stand in for, as the reference registers them (interface data):
# kda/mi350x/benchmark/baselines/decode/vllm_hip/bindings.cpp:22-27 and .../prefill/bindings.cpp:42-57.
VLLM_DECODE = (
    "fused_kda_decode(Tensor x, Tensor weight, Tensor? bias, Tensor! conv_state, Tensor raw_g, Tensor raw_beta, "
    "Tensor A_log, Tensor dt_bias, Tensor state_indices, Tensor! state, Tensor! out, float? lower_bound=None, "
    "Tensor? output_gate=None, Tensor? norm_weight=None, float norm_eps=1e-5) -> ()")
VLLM_PROLOGUE = (
    "fused_kda_prologue(Tensor q, Tensor k, Tensor v, Tensor raw_g, Tensor raw_beta, Tensor A_log, Tensor dt_bias, "
    "Tensor! qg, Tensor! w, Tensor! u, Tensor! kg_t, Tensor! aqk, Tensor! decay, Tensor cu_seqlens, "
    "Tensor chunk_indices, Tensor? conv_weight, Tensor(e!)? conv_state, Tensor? conv_state_indices, "
    "Tensor? conv_has_initial_state, float scale, float lower_bound) -> ()")
VLLM_CHUNK = (
    "fused_kda_chunk(Tensor qg, Tensor w, Tensor u, Tensor kg_t, Tensor aqk, Tensor decay, Tensor? initial_state, "
    "Tensor(a!)? final_state, Tensor! out, Tensor cu_seqlens, Tensor chunk_offsets, float scale, "
    "Tensor(b!)? group_state, int groups, Tensor(c!)? checkpoint_state=None, Tensor? checkpoint_offsets=None, "
    "Tensor? checkpoint_state_indices=None, Tensor(d!)? state_cache=None, Tensor? state_indices=None, "
    "Tensor? has_initial_state=None) -> ()")
# the pair's intermediates and grouping, which the fused kernel does not have, and the prologue's conv operands
# (documented there as unused: kda/mi350x_plain/sota/vllm_reference/kda_chunk.py:76-82)
NOT_IN_FUSED = {"qg", "w", "u", "kg_t", "aqk", "decay", "chunk_indices", "chunk_offsets", "group_state", "groups",
                "conv_weight", "conv_state", "conv_state_indices", "conv_has_initial_state"}


def _ops():
    import kda355
    return kda355.ops


def _args(schema):
    """name -> (type, written, default) of a parsed schema's arguments."""
    out = {}
    for a in schema.arguments:
        w = a.alias_info is not None and a.alias_info.is_write
        out[a.name] = (str(a.type), w, a.default_value if a.has_default_value() else "<none>")
    return out


def _schema(name):
    return getattr(torch.ops.kda355, name).default._schema


def test_all_ops_registered():
    ops = _ops()
    for name in ops.SCHEMAS:
        s = _schema(name)
        assert s.name == f"kda355::{name}"
        assert len(s.returns) == 0, f"{name} writes into its arguments and returns nothing"


def test_fused_kda_decode_schema_is_vllms():
    _ops()
    ours, ref = _schema("fused_kda_decode"), torch._C.parse_schema(VLLM_DECODE)
    assert [a.name for a in ours.arguments] == [a.name for a in ref.arguments]
    assert _args(ours) == _args(ref)


def test_fused_kda_prefill_schema_covers_the_pair():
    _ops()
    ours = _args(_schema("fused_kda_prefill"))
    want = {}
    for s in (VLLM_PROLOGUE, VLLM_CHUNK):
        for name, sig in _args(torch._C.parse_schema(s)).items():
            if name not in NOT_IN_FUSED:
                want[name] = sig
    # out is written by the chunk op (Tensor!); the same mutable annotation here
    for name, (typ, written, default) in want.items():
        assert name in ours, f"fused_kda_prefill lacks {name}"
        assert ours[name][:2] == (typ, written), f"{name}: {ours[name]} vs vLLM {(typ, written, default)}"
    extra = set(ours) - set(want)
    assert extra == {"plan", "plan_table", "workspace"}, extra


def _layout():
    lens = [4096, 300, 64, 1000, 1]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    ck = np.array([2048, 256, 0, 100, 0], np.int32)
    return cu, ck


def test_plan_tensor_round_trip():
    import kda355
    from kda355.prefill import PrefillMeta
    cu, ck = _layout()
    meta = kda355.plan(torch.as_tensor(cu), 4, checkpoint_offsets=torch.as_tensor(ck), num_cus=256)
    plan, table = meta.as_tensors()
    assert plan.dtype == torch.uint8 and plan.device.type == "cpu"
    back = PrefillMeta.from_tensors(plan, table)
    assert bytes(back.plan) == bytes(meta.plan)
    assert back.tables is table and back.any_ck == meta.any_ck and back.H == 4 and back.N == 5
    assert np.array_equal(back.lens, meta.lens)
    assert back.workspace_bytes == meta.workspace_bytes and back.split == meta.split and back.chunk64 == meta.chunk64


def test_plan_tensor_mismatch_rejected():
    import kda355
    from kda355.prefill import PrefillMeta
    cu, ck = _layout()
    a = kda355.plan(torch.as_tensor(cu), 4, checkpoint_offsets=torch.as_tensor(ck), num_cus=256)
    b = kda355.plan(torch.tensor([0, 64, 128]), 4, num_cus=256)
    pa, ta = a.as_tensors()
    pb, tb = b.as_tensors()
    with pytest.raises(ValueError):
        PrefillMeta.from_tensors(pa, tb)
    with pytest.raises(ValueError):
        PrefillMeta.from_tensors(pa[:16], ta)
    with pytest.raises(TypeError):
        PrefillMeta.from_tensors(pa.to(torch.int32), ta)
    with pytest.raises(ValueError):
        _ops()._meta(pa, None)


def test_ops_trace_under_fake_tensors():
    """The fake implementations let dynamo / AOT tracing run the ops on fake CUDA tensors (no kernel is called)."""
    _ops()
    from torch._subclasses.fake_tensor import FakeTensorMode
    H, B, T = 2, 3, 3
    with FakeTensorMode():
        dev = "cuda"
        pool = torch.empty(8, H, D, D, device=dev)
        idx = torch.zeros(B, dtype=torch.int32, device=dev)
        conv = torch.empty(8, 3 * H * D, 3, dtype=torch.bfloat16, device=dev)
        x = torch.empty(T, 3 * H * D, dtype=torch.bfloat16, device=dev)
        out = torch.empty(1, T, H, D, dtype=torch.bfloat16, device=dev)
        assert torch.ops.kda355.fused_kda_decode(
            x, torch.empty(3, 4, H * D, device=dev), None, conv, torch.empty(1, T, H, D, device=dev),
            torch.empty(1, T, H, device=dev), torch.empty(H, device=dev), torch.empty(H * D, device=dev), idx, pool,
            out, -5.0, torch.empty(T, H, D, device=dev), torch.empty(D, device=dev), 1e-5) is None
        assert torch.ops.kda355.spec_commit(pool, idx.view(B, 1), pool, idx, idx) is None


def test_cpu_tensors_fail_loudly():
    _ops()
    pool = torch.zeros(8, 2, D, D)
    idx = torch.zeros(3, 2, dtype=torch.int32)
    with pytest.raises(NotImplementedError):
        torch.ops.kda355.spec_commit(pool, idx, pool, idx[:, 0].contiguous(), idx[:, 0].contiguous())
