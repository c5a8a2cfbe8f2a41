"""The torch.ops.kda355.* registrations on the GPU: each op against the CPU oracle, and bit for bit against the Python
entry point it wraps (the same kernels), in the argument forms of the ops they stand in for (vLLM's fused_kda_decode
as kda/mi350x/benchmark/baselines/decode/sota_decode.py:57-65 calls it; the fused prologue + chunk pair with the
state cache or dense initial / final states and a staging checkpoint buffer, kda/mi350x_plain/sota/vllm_reference/
kda_chunk.py:192-294); plus a CUDA-graph capture and a torch.compile (aot_eager, fullgraph) trace of the ops."""
import pytest
import torch

from test_gpu_contract import DEV, LB, SCALE, Serving
from test_gpu_decode import NORM_EPS, Case, _check, _device_args

pytestmark = pytest.mark.gpu
D = 128
_MIX = [(4096, 1, 2048), (300, 1, 256), (64, 1, 0), (1000, 1, 512), (17, 1, 0)]


def _kda():
    import kda355
    return kda355


def _say(msg):
    print(f"[case] {msg}", flush=True)


def _vllm_decode(d, c):
    """torch.ops.kda355.fused_kda_decode in the benchmark's vLLM call form (sota_decode.py:57-65)."""
    T, H = c.T, c.H
    torch.ops.kda355.fused_kda_decode(d["mixed"], d["conv_weight"], None, d["conv"].transpose(1, 2),
                                      d["gate"].unsqueeze(0), d["beta"].unsqueeze(0), d["A_log"], d["dt_bias"],
                                      d["idx"], d["ssm"], d["out"].view(1, T, H, D), LB,
                                      d["out_gate"].view(T, H, D), d["norm_weight"], NORM_EPS)


def _pools_equal(a, b):
    if "raw" in a:
        return torch.equal(a["raw"], b["raw"])
    return torch.equal(a["conv"], b["conv"]) and torch.equal(a["ssm"], b["ssm"])


def test_op_fused_kda_decode_vllm_form(oracle):
    kda = _kda()
    _say("fused_kda_decode B=16 H=12 pages")
    c = Case(B=16, S=1, H=12, seed=71, spec=False)
    d = _device_args(c, DEV)
    _vllm_decode(d, c)
    torch.cuda.synchronize()
    _check(c, d, oracle, "op fused_kda_decode: ")
    e = _device_args(c, DEV)
    kda.decode(e["mixed"], e["conv"], e["conv_weight"], e["gate"], e["beta"], e["out_gate"], e["A_log"],
               e["dt_bias"], e["norm_weight"], e["ssm"], e["idx"], None, e["cu"], NORM_EPS, LB, e["out"])
    torch.cuda.synchronize()
    assert torch.equal(d["out"], e["out"]) and _pools_equal(d, e), "op and kda355.decode differ"


def test_op_fused_kda_decode_rejects_unsupported_forms():
    _kda()
    c = Case(B=4, S=1, H=4, seed=72, spec=False, pages=False)
    d = _device_args(c, DEV)
    T, H = c.T, c.H
    args = [d["mixed"], d["conv_weight"], None, d["conv"].transpose(1, 2), d["gate"].unsqueeze(0),
            d["beta"].unsqueeze(0), d["A_log"], d["dt_bias"], d["idx"], d["ssm"], d["out"].view(1, T, H, D)]
    with pytest.raises(ValueError, match="lower_bound"):
        torch.ops.kda355.fused_kda_decode(*args, None, d["out_gate"].view(T, H, D), d["norm_weight"], NORM_EPS)
    with pytest.raises(ValueError, match="bias"):
        bad = list(args)
        bad[2] = torch.zeros(3 * H * D, device=DEV)
        torch.ops.kda355.fused_kda_decode(*bad, LB, d["out_gate"].view(T, H, D), d["norm_weight"], NORM_EPS)
    with pytest.raises(ValueError, match="norm"):
        torch.ops.kda355.fused_kda_decode(*args, LB, None, None, NORM_EPS)


def test_op_decode_spec_verify(oracle):
    _kda()
    _say("decode op spec B=8 S=4 H=4")
    c = Case(B=8, S=4, H=4, seed=73, spec=True)
    d = _device_args(c, DEV)
    torch.ops.kda355.decode(d["mixed"], d["conv"], d["conv_weight"], d["gate"], d["beta"], d["out_gate"], d["A_log"],
                            d["dt_bias"], d["norm_weight"], d["ssm"], d["idx"], d["acc"], d["cu"], NORM_EPS, LB,
                            d["out"])
    torch.cuda.synchronize()
    _check(c, d, oracle, "op decode: ")


def test_op_decode_graph_replay(oracle):
    """The op captured once in a CUDA graph and replayed on new inputs copied into the captured buffers."""
    _kda()
    cases = [Case(B=8, S=1, H=4, seed=80 + i, spec=False, pages=False) for i in range(3)]
    d = _device_args(cases[0], DEV)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        _vllm_decode(d, cases[0])
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    _check(cases[0], d, oracle, "op eager warm-up: ")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _vllm_decode(d, cases[0])
    for c in cases[1:]:
        src = _device_args(c, DEV)
        for k in ("mixed", "conv", "ssm", "gate", "beta", "out_gate", "conv_weight", "A_log", "dt_bias",
                  "norm_weight", "idx", "out"):
            d[k].copy_(src[k])
        graph.replay()
        torch.cuda.synchronize()
        _check(c, d, oracle, "op graph replay: ")


def test_op_decode_torch_compile(oracle):
    """dynamo + AOT functionalization trace the op as one mutating node (fullgraph) with the same results."""
    _kda()
    c = Case(B=8, S=1, H=4, seed=91, spec=False, pages=False)

    def step(mixed, conv, w, gate, beta, A_log, dt_bias, idx, ssm, out, og, nw):
        T, H = gate.shape[0], gate.shape[1]
        torch.ops.kda355.fused_kda_decode(mixed, w, None, conv.transpose(1, 2), gate.unsqueeze(0),
                                          beta.unsqueeze(0), A_log, dt_bias, idx, ssm, out.view(1, T, H, D), LB,
                                          og.view(T, H, D), nw, NORM_EPS)
        return out

    compiled = torch.compile(step, backend="aot_eager", fullgraph=True)
    outs = []
    for fn in (step, compiled):
        d = _device_args(c, DEV)
        fn(d["mixed"], d["conv"], d["conv_weight"], d["gate"], d["beta"], d["A_log"], d["dt_bias"], d["idx"],
           d["ssm"], d["out"], d["out_gate"], d["norm_weight"])
        torch.cuda.synchronize()
        outs.append(d)
    _check(c, outs[1], oracle, "compiled op: ")
    assert torch.equal(outs[0]["out"], outs[1]["out"]) and _pools_equal(outs[0], outs[1])


def _serving_tensors(c, kda):
    cu_cpu = torch.tensor(c.cu, dtype=torch.int32)
    return dict(cu_cpu=cu_cpu, cu=cu_cpu.to(DEV), sidx=c.sidx.to(DEV), cidx=c.cidx.to(DEV), ck=c.ck_off.to(DEV),
                hinit=torch.tensor(c.hinit, dtype=torch.bool, device=DEV))


def test_op_prefill_plan_tensors_no_sync(oracle):
    kda = _kda()
    _say("prefill op with plan tensors H=4")
    c = Serving(4, _MIX, 4242)
    t = _serving_tensors(c, kda)
    plan, table = kda.prefill_prepare(t["cu_cpu"], c.H, c.ck_off, c.cidx, device=DEV).as_tensors()
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        torch.ops.kda355.prefill(c.q, c.k, c.v, c.raw_g, c.raw_b, c.A_log, c.dt_bias, SCALE, LB, c.ssm, t["sidx"],
                                 t["hinit"], t["cu"], c.out, t["ck"], t["cidx"], plan, table)
    finally:
        torch.cuda.set_sync_debug_mode(0)
    torch.cuda.synchronize()
    c.verify(oracle, what="op prefill")
    ref = Serving(4, _MIX, 4242)
    ref.run(kda)
    assert torch.equal(c.out, ref.out) and torch.equal(c.raw, ref.raw), "op and kda355.prefill differ"


def test_op_fused_kda_prefill_cache_and_dense_states(oracle):
    """vLLM's two state forms through one op: the paged cache (checkpoints into the cache rows), then dense
    initial / final states with a staging checkpoint buffer indexed by sequence -- the same numbers bit for bit."""
    kda = _kda()
    _say("fused_kda_prefill state cache H=4")
    c = Serving(4, _MIX, 4343)
    t = _serving_tensors(c, kda)
    torch.ops.kda355.fused_kda_prefill(c.q, c.k, c.v, c.raw_g, c.raw_b, c.A_log, c.dt_bias, c.out, t["cu"], SCALE, LB,
                                       checkpoint_state=c.ssm, checkpoint_offsets=t["ck"],
                                       checkpoint_state_indices=t["cidx"], state_cache=c.ssm, state_indices=t["sidx"],
                                       has_initial_state=t["hinit"])
    torch.cuda.synchronize()
    c.verify(oracle, what="op fused_kda_prefill cache")

    _say("fused_kda_prefill dense states H=4")
    e = Serving(4, _MIX, 4343)
    N = e.N
    init = e.ssm[e.sidx.long()].contiguous()
    final = torch.full_like(init, float("nan"))
    staging = torch.full_like(init, float("nan"))
    plan, table = kda.plan(t["cu_cpu"], e.H, checkpoint_offsets=e.ck_off, device=DEV).as_tensors()
    torch.ops.kda355.fused_kda_prefill(e.q, e.k, e.v, e.raw_g, e.raw_b, e.A_log, e.dt_bias, e.out, t["cu"], SCALE, LB,
                                       initial_state=init, final_state=final, checkpoint_state=staging,
                                       checkpoint_offsets=t["ck"], plan=plan, plan_table=table)
    torch.cuda.synchronize()
    assert torch.equal(e.out, c.out), "dense-state output differs from the state-cache output"
    assert torch.equal(final, c.ssm[c.sidx.long()]), "final states differ from the cache rows"
    for n in range(N):
        if int(c.cidx[n]) >= 0:
            assert torch.equal(staging[n], c.ssm[int(c.cidx[n])]), f"checkpoint of sequence {n} differs"
        else:
            assert bool(torch.isnan(staging[n]).all()), f"staging row {n} written without a checkpoint"


def test_op_recurrent_spec_and_commit():
    """fused_recurrent_kda (spec verify into a scratch) then spec_commit: ops and Python entry points agree bit for
    bit (their parity against the oracle is covered by the recurrent tests)."""
    kda = _kda()
    B, S, H, slots = 6, 4, 4, 40
    g = torch.Generator(device=DEV).manual_seed(5)
    T = B * S
    q, k, v, rg = (torch.randn(1, T, H, D, generator=g, device=DEV).bfloat16() for _ in range(4))
    rb = torch.randn(1, T, H, generator=g, device=DEV).bfloat16()
    A_log = torch.rand(H, generator=g, device=DEV) * 2 - 1
    dt_bias = torch.randn(H * D, generator=g, device=DEV) * 0.5
    pool0 = torch.randn(slots, H, D, D, generator=g, device=DEV) * 0.05
    idx = (torch.randperm(slots - 1, device=DEV)[:B * S] + 1).to(torch.int32).view(B, S)
    sidx = torch.arange(1, B * S + 1, dtype=torch.int32, device=DEV).view(B, S)  # scratch row 0 unused
    acc = torch.tensor([1, 4, 2, 3, 4, 1], dtype=torch.int32, device=DEV)
    cu = torch.arange(0, T + 1, S, dtype=torch.int32, device=DEV)
    res = []
    for use_op in (False, True):
        pool, scratch = pool0.clone(), torch.zeros(B * S + 1, H, D, D, device=DEV)
        out = torch.empty(1, T, H, D, dtype=torch.bfloat16, device=DEV)
        if use_op:
            torch.ops.kda355.fused_recurrent_kda(q, k, v, rg, rb, A_log, dt_bias, LB, pool, cu, idx, acc, out,
                                                 write_pool=scratch, write_indices=sidx)
            torch.ops.kda355.spec_commit(scratch, sidx, pool, idx[:, 0].contiguous(), acc)
        else:
            kda.fused_recurrent_kda(q, k, v, initial_state=pool, cu_seqlens=cu, ssm_state_indices=idx,
                                    num_accepted_tokens=acc, out=out, raw_g=rg, raw_beta=rb, A_log=A_log,
                                    dt_bias=dt_bias, lower_bound=LB, write_pool=scratch, write_indices=sidx)
            kda.spec_commit(scratch, sidx, pool, idx[:, 0].contiguous(), acc)
        torch.cuda.synchronize()
        assert torch.isfinite(out.float()).all()
        res.append((out, pool, scratch))
    assert all(torch.equal(a, b) for a, b in zip(*res)), "ops and Python entry points differ"
    assert not torch.equal(res[0][1], pool0), "the commit wrote nothing"
