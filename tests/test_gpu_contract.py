"""The reference eval's correctness gates for the serving prefill (kda/mi350x/benchmark/eval_kda_mi350x.py), run
against the fp64 CPU oracle:

* the contract cases (gate_prefill_contract, :625-666): head counts 1 .. 128 on a ragged mix with edge checkpoints,
  64 ragged sequences, 256 x 64 tokens, one token, a checkpoint at 64, meta=None, a contiguous pool, a 64K-token
  sequence with a checkpoint at 32768, and a batch of more than 2^31 elements (H = 96, 176 x 1024 tokens);
* the numerics probes (NUMERIC_PROBES, :715-758): slow decay over 16K tokens, a wide decay spectrum, saturated gates,
  deep-layer statistics (beta ~ 1, chunk-aligned q / k / v, larger states) at H = 12 and 96, one-hot keys, and
  rescaled q / k / v (x 1e-3 / 1e3 / 1e3);
* the integration flow on one page pool (gate_integration, :796-880): prefill (cold, warm, with checkpoints) ->
  three spec-verify steps -> a next-turn prefill resuming from the accepted slots -> a new request resuming from a
  checkpoint row (prefix hit).

Inputs follow the eval's PrefillCase (:273-345): q, k, v, raw_g ~ N(0, 1) bf16, raw_beta a column slice of an
input projection, A_log ~ U(-1, 1), dt_bias ~ N(0, 0.5^2), pool rows ~ N(0, 0.05^2) on the vLLM page layout, lower
bound -5, scale 128^-1/2; cold sequences' slots and checkpoint rows are poisoned with NaN (write-only).

Bars: the north-star bars (output max-abs beyond bf16 rounding <= 2e-2 x RMS; written rows relative Frobenius
<= 1e-3) plus the eval's per-sequence relative L2 <= 2e-2, for the contract cases and the numerics probes alike (the
eval itself holds the probes' pool rows to relative L2 <= 2e-2, P_RTOL, twenty times looser).  Every byte outside
`out` and the written rows is compared with a saved copy.
"""
import random
import zlib

import numpy as np
import pytest
import torch

from helpers import STATE_TOL, check_out, decode_rounding_allowance, f32, rel_frob

pytestmark = pytest.mark.gpu
D = 128
DEV = torch.device("cuda", 0)
LB = -5.0
SCALE = D ** -0.5
P_RTOL = 2e-2
LEAD = 256  # output rows before the prefill's slice in the caller's buffer (decode tokens first)


def _kda():
    import kda355
    return kda355


def _say(msg):
    print(f"[case] {msg}", flush=True)


class Serving:
    """One serving prefill call: layout, device inputs, page pool (or a dense pool) and its snapshot."""

    def __init__(self, H, seqs, seed, pages=True, gates=None, taps=10):
        gates = gates or {}
        self.H, self.seqs = H, seqs
        N = len(seqs)
        lens = [s[0] for s in seqs]
        self.N, self.T = N, sum(lens)
        T = self.T
        self.cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
        gen = torch.Generator(device=DEV).manual_seed(seed)
        slots = 2 * N + 9
        self.slots = slots
        dim = H * D
        if pages:
            conv_bytes = taps * 3 * dim * 2
            page = -(-(conv_bytes + H * D * D * 4 + 4096) // 256) * 256
            self.raw = torch.randint(0, 256, (slots * page,), dtype=torch.uint8, generator=gen, device=DEV)
            self.ssm = torch.as_strided(self.raw.view(torch.float32), (slots, H, D, D), (page // 4, D * D, D, 1),
                                        conv_bytes // 4)
        else:
            self.raw = None
            self.ssm = torch.empty(slots, H, D, D, device=DEV)
        cpu = torch.Generator().manual_seed(seed)
        perm = (torch.randperm(slots - 1, generator=cpu) + 1).to(torch.int32)
        self.sidx = perm[:N].contiguous()
        self.cidx = torch.tensor([int(perm[N + n]) if s[2] > 0 else -1 for n, s in enumerate(seqs)], dtype=torch.int32)
        self.hinit = [bool(s[1]) for s in seqs]
        self.ck_off = torch.tensor([s[2] for s in seqs], dtype=torch.int32)
        self.q, self.k, self.v, self.raw_g = (torch.randn(1, T, H, D, generator=gen, device=DEV).bfloat16()
                                              for _ in range(4))
        Wp = -(-(4 * dim + D + H) // 16) * 16
        self.P = torch.randn(T, Wp, generator=gen, device=DEV).bfloat16()
        self.raw_b = self.P[:, 4 * dim + D:4 * dim + D + H][None]
        self.A_log = torch.rand(H, generator=gen, device=DEV) * 2 - 1
        self.dt_bias = torch.randn(H * D, generator=gen, device=DEV) * 0.5
        self.ssm.copy_(torch.randn(slots, H, D, D, generator=gen, device=DEV) * 0.05)
        # the eval's gate settings (eval_kda_mi350x.py:309-334)
        if "q_scale" in gates:
            self.q.mul_(gates["q_scale"])
        if "k_scale" in gates:
            self.k.mul_(gates["k_scale"])
        if "v_scale" in gates:
            self.v.mul_(gates["v_scale"])
        if "a_log" in gates:
            self.A_log.fill_(gates["a_log"])
        if "dt_range" in gates:
            lo, hi = gates["dt_range"]
            self.dt_bias.copy_(torch.linspace(lo, hi, D, device=DEV).repeat(H))
        if "beta_logit" in gates:
            self.raw_b.fill_(gates["beta_logit"])
        if "aligned" in gates:           # q / k / v of a 64-token chunk share a direction
            nc = -(-T // 64)
            for t in (self.q, self.k, self.v):
                base = torch.randn(nc, 1, H, D, generator=gen, device=DEV)
                noise = torch.randn(nc, 64, H, D, generator=gen, device=DEV) * gates["aligned"]
                t.copy_((base + noise).reshape(nc * 64, H, D)[:T].unsqueeze(0))
        if "state_scale" in gates:
            self.ssm.mul_(gates["state_scale"] / 0.05)
        if "one_hot_k" in gates:
            idx = torch.randint(0, 4, (T, H), generator=gen, device=DEV)
            self.k.copy_(torch.nn.functional.one_hot(idx, D).unsqueeze(0).to(self.k.dtype))
        for n in range(N):               # write-only rows: poisoned
            if not self.hinit[n]:
                self.ssm[int(self.sidx[n])] = float("nan")
            if int(self.cidx[n]) >= 0:
                self.ssm[int(self.cidx[n])] = float("nan")
        self.big_out = torch.full((1, LEAD + T, H, D), float("nan"), dtype=torch.bfloat16, device=DEV)
        self.out = self.big_out[:, LEAD:]
        self.written = sorted(set(self.sidx.tolist()) | {int(c) for c in self.cidx.tolist() if c >= 0})
        self.snap = (self.raw if self.raw is not None else self.ssm).clone()

    def run(self, kda, meta_none=False, precise=False):
        cu_cpu = torch.tensor(self.cu, dtype=torch.int32)
        meta = None if meta_none else kda.prefill_prepare(cu_cpu, self.H, self.ck_off, self.cidx, device=DEV)
        kda.prefill(self.q, self.k, self.v, self.raw_g, self.raw_b, self.A_log, self.dt_bias, SCALE, LB, self.ssm,
                    self.sidx.to(DEV), torch.tensor(self.hinit, dtype=torch.bool, device=DEV), cu_cpu.to(DEV),
                    self.out, self.ck_off.to(DEV), self.cidx.to(DEV), meta=meta, precise=precise)
        torch.cuda.synchronize()
        return meta

    def verify(self, oracle, hs=None, state_tol=STATE_TOL, what=""):
        """Checks heads hs (all by default) against the fp64 oracle; untouched bytes on the device, all heads."""
        H = self.H
        hs = list(range(H)) if hs is None else hs
        snap_ssm = (torch.as_strided(self.snap.view(torch.float32), self.ssm.shape, self.ssm.stride(),
                                     self.ssm.storage_offset()) if self.raw is not None else self.snap)
        pool0 = snap_ssm[:, hs].cpu().numpy()
        sel = lambda x: np.ascontiguousarray(f32(x[0][:, hs]))  # noqa: E731
        dtb = self.dt_bias.view(H, D)[hs].reshape(-1)
        ro, rnew = oracle.prefill_serving(sel(self.q), sel(self.k), sel(self.v), sel(self.raw_g), sel(self.raw_b),
                                          f32(self.A_log[hs]), f32(dtb), LB, SCALE, pool0, self.sidx.numpy(),
                                          np.array(self.hinit), self.cu, self.ck_off.numpy(), self.cidx.numpy(),
                                          precision=64)
        check_out(self.out[0][:, hs], ro, what, self.cu)
        got = self.ssm[:, hs].cpu().numpy()
        worst = 0.0
        for r in self.written:
            assert np.isfinite(got[r]).all(), f"{what}: pool row {r} not finite"
            worst = max(worst, rel_frob(got[r], rnew[r]))
        _say(f"{what}: worst written-row relF {worst:.2e}")
        assert worst <= state_tol, f"{what}: written-row relF {worst:.3e} > {state_tol}"
        assert bool(torch.isnan(self.big_out[:, :LEAD].float()).all()), f"{what}: wrote outside its output slice"
        exp = self.snap.clone()
        if self.raw is not None:
            e_ssm = torch.as_strided(exp.view(torch.float32), self.ssm.shape, self.ssm.stride(),
                                     self.ssm.storage_offset())
            e_ssm[self.written] = self.ssm[self.written]
            assert torch.equal(self.raw, exp), f"{what}: bytes outside the written rows changed"
        else:
            exp[self.written] = self.ssm[self.written]
            assert torch.equal(self.ssm, exp), f"{what}: unwritten pool rows changed"


# ------------------------------------------------------------------------------------------------ contract cases
_MIX = [(777, 1, 704), (64, 0, 64), (1, 1, 0), (130, 0, 0), (1024, 1, 1024), (17, 1, 0), (255, 0, 192)]


def _contract_cases(seed=1):
    rng = random.Random(seed)
    cases = [(f"heads_h{H}", H, _MIX, {}) for H in (1, 4, 8, 16, 24, 32, 48, 128)]
    ragged = []
    for _ in range(64):
        n = rng.randint(1, 300)
        ck = 64 * rng.randint(1, n // 64) if n >= 64 and rng.random() < 0.6 else 0
        ragged.append((n, int(rng.random() < 0.8), ck))
    cases.append(("ragged64_h12", 12, ragged, {}))
    cases.append(("many256x64_h12", 12, [(64, int(rng.random() < 0.8), 64 * (rng.random() < 0.3)) for _ in range(256)],
                  {}))
    cases.append(("tiny_h12", 12, [(1, 0, 0)], {}))
    cases.append(("ck_at_64_h12", 12, [(4096, 1, 64), (65, 0, 64), (128, 1, 128)], {}))
    cases.append(("meta_none_h12", 12, [(3000, 1, 2048), (100, 0, 64), (5000, 1, 0)], {"meta_none": True}))
    cases.append(("contiguous_pool_h12", 12, [(2000, 1, 1024), (300, 0, 256)], {"contiguous": True}))
    cases.append(("long64k_h12", 12, [(65536, 1, 32768)], {"heads": [0, 5, 11]}))
    cases.append(("int64_extent_h96", 96,
                  [(1024, int(rng.random() < 0.8), 1024 * (rng.random() < 0.3)) for _ in range(176)],
                  {"heads": [0, 95]}))
    return cases


_CONTRACT = _contract_cases()


@pytest.mark.parametrize("case", _CONTRACT, ids=[c[0] for c in _CONTRACT])
def test_prefill_contract(oracle, case):
    name, H, seqs, flags = case
    _say(f"contract {name}: H={H} N={len(seqs)} T={sum(s[0] for s in seqs)}")
    c = Serving(H, seqs, 7919 + zlib.crc32(name.encode()) % 1000, pages=not flags.get("contiguous"))
    if name == "int64_extent_h96":
        assert c.T * H * D > 2 ** 31, "the case must exceed 2^31 elements"
    c.run(_kda(), meta_none=flags.get("meta_none", False))
    c.verify(oracle, hs=flags.get("heads"), what=name)


# ------------------------------------------------------------------------------------------------ numerics probes
_PROBES = [
    ("slow_decay_16k", 12, [(16384, 1, 8192)], {"a_log": 0.0, "dt_range": (-12.0, -6.0)}),
    ("spectrum_4x4k", 12, [(4096, 1, 2048)] * 4, {"a_log": 0.0, "dt_range": (-14.0, 2.0)}),
    ("saturated", 12, [(2048, 1, 1024), (777, 0, 0)], {"a_log": 2.0, "dt_range": (20.0, 30.0)}),
    ("deep_layer", 12, [(4096, 1, 3072), (1500, 1, 1024)], {"a_log": 0.0, "dt_range": (-12.0, -4.0),
                                                            "beta_logit": 6.0, "aligned": 0.3, "state_scale": 0.5}),
    ("deep_layer_h96", 96, [(2048, 1, 1024), (300, 0, 256)], {"a_log": 0.0, "dt_range": (-12.0, -4.0),
                                                              "beta_logit": 6.0, "aligned": 0.3, "state_scale": 0.5}),
    ("one_hot_keys", 12, [(1024, 1, 512), (200, 0, 0)], {"one_hot_k": True, "beta_logit": 4.0}),
    ("rescaled", 12, [(1024, 1, 1024), (513, 1, 512)], {"q_scale": 1e-3, "k_scale": 1e3, "v_scale": 1e3}),
]


@pytest.mark.parametrize("probe", _PROBES, ids=[p[0] for p in _PROBES])
def test_numerics_probe(oracle, probe):
    """Written pool rows at the north-star state bar (1e-3); the worst, deep_layer, measures 9.3e-4."""
    name, H, seqs, gates = probe
    _say(f"numerics probe {name}: H={H} seqs={[s[0] for s in seqs]} gates={gates}")
    c = Serving(H, seqs, 31 + len(name), gates=gates)
    c.run(_kda())
    c.verify(oracle, state_tol=STATE_TOL, what=name)


PRECISE_STATE_TOL = 0.5 * STATE_TOL


@pytest.mark.parametrize("probe", _PROBES, ids=[p[0] for p in _PROBES])
def test_numerics_probe_precise(oracle, probe):
    """precise=True (fp16-pair operands in the solve and the state update): every probe's written rows at half the
    north-star bar (5e-4); deep_layer measures 4.9e-4 there."""
    name, H, seqs, gates = probe
    _say(f"numerics probe (precise) {name}: H={H} seqs={[s[0] for s in seqs]} gates={gates}")
    c = Serving(H, seqs, 31 + len(name), gates=gates)
    c.run(_kda(), precise=True)
    c.verify(oracle, state_tol=PRECISE_STATE_TOL, what=f"{name} (precise)")


# ------------------------------------------------------------------------------------------------ integration
def test_integration_prefill_spec_decode_prefix_hit(oracle):
    """One page pool and conv cache through prefill -> 3 spec-verify steps -> next-turn prefill -> prefix hit
    (eval_kda_mi350x.py:796-880).  After each step the written rows are reset to the oracle's (so each step is
    checked on its own), as the eval does."""
    kda = _kda()
    H, S, B, W = 12, 8, 3, 4
    dim = H * D
    taps = 2 + S
    slots = 64
    gen = torch.Generator(device=DEV).manual_seed(555)
    conv_bytes = taps * 3 * dim * 2
    page = -(-(conv_bytes + H * D * D * 4 + 4096) // 256) * 256
    raw = torch.randint(0, 256, (slots * page,), dtype=torch.uint8, generator=gen, device=DEV)
    conv = torch.as_strided(raw.view(torch.bfloat16), (slots, taps, 3 * dim), (page // 2, 3 * dim, 1), 0)
    ssm = torch.as_strided(raw.view(torch.float32), (slots, H, D, D), (page // 4, D * D, D, 1), conv_bytes // 4)
    conv.copy_(torch.randn(conv.shape, generator=gen, device=DEV).bfloat16())
    ssm.copy_(torch.randn(ssm.shape, generator=gen, device=DEV) * 0.05)
    A_log = torch.rand(H, generator=gen, device=DEV) * 2 - 1
    dt_bias = torch.randn(dim, generator=gen, device=DEV) * 0.5
    conv_w = torch.randn(3, W, dim, generator=gen, device=DEV) * 0.4
    norm_w = 1 + torch.randn(D, generator=gen, device=DEV) * 0.1
    spec_idx = torch.arange(1, 1 + B * S, dtype=torch.int32, device=DEV).view(B, S)
    Wp = -(-(4 * dim + D + H) // 16) * 16

    def prefill_step(lens, has_init, slots_n, ck_off, ck_rows, tag):
        T = sum(lens)
        q, k, v, rg = (torch.randn(1, T, H, D, generator=gen, device=DEV).bfloat16() for _ in range(4))
        P = torch.randn(T, Wp, generator=gen, device=DEV).bfloat16()
        rb = P[:, 4 * dim + D:4 * dim + D + H][None]
        cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
        cu_cpu = torch.tensor(cu, dtype=torch.int32)
        co, cr = torch.tensor(ck_off, dtype=torch.int32), torch.tensor(ck_rows, dtype=torch.int32)
        si = torch.tensor(slots_n, dtype=torch.int32)
        out = torch.empty(1, T, H, D, dtype=torch.bfloat16, device=DEV)
        pool0 = ssm.cpu().numpy()
        meta = kda.prefill_prepare(cu_cpu, H, co, cr, device=DEV)
        kda.prefill(q, k, v, rg, rb, A_log, dt_bias, SCALE, LB, ssm, si.to(DEV),
                    torch.tensor(has_init, dtype=torch.bool, device=DEV), cu_cpu.to(DEV), out, co.to(DEV), cr.to(DEV),
                    meta=meta)
        torch.cuda.synchronize()
        ro, rnew = oracle.prefill_serving(f32(q[0]), f32(k[0]), f32(v[0]), f32(rg[0]), f32(rb[0]), f32(A_log),
                                          f32(dt_bias), LB, SCALE, pool0, si.numpy(), np.array(has_init), cu,
                                          co.numpy(), cr.numpy(), precision=64)
        check_out(out[0], ro, tag, cu)
        rows = sorted(set(slots_n) | {r for r in ck_rows if r >= 0})
        got = ssm.cpu().numpy()
        worst = max(rel_frob(got[r], rnew[r]) for r in rows)
        _say(f"{tag}: worst written-row relF {worst:.2e}")
        assert worst <= STATE_TOL, f"{tag}: pool row relF {worst:.3e}"
        ssm[rows] = torch.from_numpy(rnew[rows]).to(DEV)      # continue from the oracle's state

    def decode_step(acc, tag):
        T = B * S
        P = torch.randn(T, Wp, generator=gen, device=DEV).bfloat16()
        mq, og, beta = P[:, :3 * dim], P[:, 3 * dim:4 * dim], P[:, 4 * dim + D:4 * dim + D + H]
        gate = torch.randn(T, H, D, generator=gen, device=DEV).bfloat16()
        nat = torch.tensor(acc, dtype=torch.int32, device=DEV)
        cu = torch.arange(0, T + 1, S, dtype=torch.long, device=DEV)
        out = torch.empty(T, dim, dtype=torch.bfloat16, device=DEV)
        conv0, ssm0 = conv.cpu(), ssm.cpu().numpy()
        kda.decode(mq, conv, conv_w, gate, beta, og, A_log, dt_bias, norm_w, ssm, spec_idx, nat, cu, 1e-5, LB, out)
        torch.cuda.synchronize()
        ro, rconv, rssm, (ob, fac) = oracle.decode_full(f32(mq), f32(conv0), f32(conv_w), f32(gate), f32(beta),
                                                        f32(og), f32(A_log), f32(dt_bias), f32(norm_w), ssm0,
                                                        spec_idx.cpu().numpy(), np.array(acc), 1e-5, LB,
                                                        precision=64, aux=True)
        check_out(out, ro, tag, np.arange(0, T + 1, S), allow=decode_rounding_allowance(ro, ob, fac))
        assert np.array_equal(f32(conv), rconv), f"{tag}: conv cache differs from the reference rule"
        rows = sorted(int(x) for x in spec_idx.flatten().tolist())
        got = ssm.cpu().numpy()
        worst = max(rel_frob(got[r], rssm[r]) for r in rows)
        _say(f"{tag}: worst written-row relF {worst:.2e}")
        assert worst <= STATE_TOL
        ssm[rows] = torch.from_numpy(rssm[rows]).to(DEV)

    heads = spec_idx[:, 0].tolist()
    prefill_step([1500, 64, 777], [False, True, True], heads, [1024, 64, 0], [40, 41, -1], "prefill-1")
    decode_step([1, 1, 1], "verify-1")
    decode_step([5, 3, 8], "verify-2")
    resume = [int(spec_idx[n, a - 1]) for n, a in enumerate([4, 1, 6])]
    decode_step([4, 1, 6], "verify-3")
    prefill_step([640, 1300, 90], [True, True, True], resume, [0, 1024, 64], [-1, 42, 43], "prefill-2")
    ssm[50] = ssm[40]                                         # prefix hit: the caller copies a checkpoint row
    prefill_step([2048], [True], [50], [2048], [44], "prefill-3 (prefix hit)")
