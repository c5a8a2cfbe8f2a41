"""GPU parity of the fused decode / spec-verify step (kda355.decode -> kda355_decode_launch) against the CPU oracle
(oracle.decode_full, the restatement of kda/mi350x/reference.py:104-181).

Inputs follow the reference eval's DecodeCase (kda/mi350x/benchmark/eval_kda_mi350x.py:463-491): the vLLM page
layout (one raw byte pool per slot: conv state [taps, 3*H*128] bf16, then the fp32 SSM state, pages padded to 256 B
with 4 KiB of padding; eval_kda_mi350x.py:183-202) and column slices of one input projection for mixed_qkv /
out_gate / beta (eval_kda_mi350x.py:265-270).

Bars: output max-abs error beyond bf16 storage rounding <= 2e-2 x RMS(ref); written SSM rows relative Frobenius
<= 1e-3; the conv cache bit-exact; every other byte of the page pool (unwritten slots, page padding) bit-identical.
"""
import numpy as np
import pytest
import torch

from helpers import STATE_TOL, check_out, decode_rounding_allowance, f32, gen, rel_frob

pytestmark = pytest.mark.gpu
D = 128
W = 4
PAGE_PAD = 4096
NORM_EPS = 1e-5
LB = -5.0


def _say(msg):
    print(f"[case] {msg}", flush=True)


class Case:
    """Seeded CPU inputs of one decode call; `raw` is the page pool (or None with dense pools)."""

    def __init__(self, B, S, H, seed, spec, pages=True, extra_taps=0, pad=(), hostile_dead=False, slots=None):
        g = gen(seed)
        dim = H * D
        T = B * S
        self.B, self.S, self.H, self.T, self.spec = B, S, H, T, spec
        taps = (W - 2 + S if spec else W - 1) + extra_taps
        slots = slots or 2 * B * S + 16
        self.slots, self.taps = slots, taps
        if pages:
            conv_bytes = taps * 3 * dim * 2
            page = -(-(conv_bytes + H * D * D * 4 + PAGE_PAD) // 256) * 256
            self.raw = torch.randint(0, 256, (slots * page,), dtype=torch.uint8, generator=g)
            self.page, self.conv_bytes = page, conv_bytes
            conv, ssm = self.views(self.raw)
            conv.copy_(torch.randn(conv.shape, generator=g).bfloat16())
            ssm.copy_(torch.randn(ssm.shape, generator=g) * 0.05)
            Wp = -(-(4 * dim + D + H) // 16) * 16
            P = torch.randn(T, Wp, generator=g).bfloat16()
            self.P = P
            self.mixed, self.out_gate, self.beta = P[:, :3 * dim], P[:, 3 * dim:4 * dim], P[:, 4 * dim + D:4 * dim + D + H]
        else:
            self.raw = None
            self.conv = torch.randn(slots, taps, 3 * dim, generator=g).bfloat16()
            self.ssm = torch.randn(slots, H, D, D, generator=g) * 0.05
            self.mixed = torch.randn(T, 3 * dim, generator=g).bfloat16()
            self.out_gate = torch.randn(T, dim, generator=g).bfloat16()
            self.beta = torch.randn(T, H, generator=g).bfloat16()
        self.gate = torch.randn(T, H, D, generator=g).bfloat16()
        self.conv_weight = torch.randn(3, W, dim, generator=g) * 0.4
        self.A_log = torch.rand(H, generator=g) * 2 - 1
        self.dt_bias = torch.randn(dim, generator=g) * 0.5
        self.norm_weight = 1 + torch.randn(D, generator=g) * 0.1
        perm = (torch.randperm(slots - 1, generator=g)[: B * S] + 1).to(torch.int32)
        self.idx = perm.view(B, S).clone() if spec else perm[:B].clone()
        for p in pad:
            self.idx[p] = 0
        self.acc = torch.randint(1, S + 1, (B,), generator=g, dtype=torch.int32) if spec else None
        if hostile_dead:
            # dead sequences' out_gate rows are NaN and some norm weights negative: their output rows must still be +0
            for n in self.dead():
                self.out_gate[n * S:(n + 1) * S] = float("nan")
            self.norm_weight[::3] *= -1.0

    def dead(self):
        """Sequences whose read or conv row is padding (decode_kernel's slot rule): zero output, no writes."""
        idx = self.idx.numpy()
        out = []
        for n in range(self.B):
            if self.spec:
                a = int(np.clip(self.acc[n], 1, self.S))
                rd, cs = idx[n, a - 1], idx[n, 0]
            else:
                rd = cs = idx[n]
            if not (0 < rd < self.slots and 0 < cs < self.slots):
                out.append(n)
        return out

    def views(self, raw):
        dim = self.H * D
        conv = torch.as_strided(raw.view(torch.bfloat16), (self.slots, self.taps, 3 * dim), (self.page // 2, 3 * dim, 1), 0)
        ssm = torch.as_strided(raw.view(torch.float32), (self.slots, self.H, D, D), (self.page // 4, D * D, D, 1),
                               self.conv_bytes // 4)
        return conv, ssm

    def pools(self):
        return self.views(self.raw) if self.raw is not None else (self.conv, self.ssm)

    def oracle(self, O):
        conv, ssm = self.pools()
        return O.decode_full(f32(self.mixed), f32(conv), f32(self.conv_weight), f32(self.gate), f32(self.beta),
                             f32(self.out_gate), f32(self.A_log), f32(self.dt_bias), f32(self.norm_weight), f32(ssm),
                             self.idx.numpy(), self.acc.numpy() if self.spec else None, NORM_EPS, LB, precision=64,
                             aux=True)

    def written(self):
        """(ssm rows written, conv slots written) per the reference's slot rules."""
        idx = self.idx.numpy()
        rows, cslots = set(), set()
        for n in range(self.B):
            if self.spec:
                a = int(np.clip(self.acc[n], 1, self.S))
                rd, cs = idx[n, a - 1], idx[n, 0]
                if rd > 0 and cs > 0:
                    rows |= {int(r) for r in idx[n] if r > 0}
                    cslots.add(int(cs))
            elif idx[n] > 0:
                rows.add(int(idx[n]))
                cslots.add(int(idx[n]))
        return rows, cslots


def _device_args(c, dev):
    """Device copies with the same layouts (the page pool is copied whole, its views rebuilt on the device)."""
    d = {}
    if c.raw is not None:
        d["raw"] = c.raw.to(dev)
        d["conv"], d["ssm"] = c.views(d["raw"])
        P = c.P.to(dev)
        dim = c.H * D
        d["mixed"], d["out_gate"], d["beta"] = P[:, :3 * dim], P[:, 3 * dim:4 * dim], P[:, 4 * dim + D:4 * dim + D + c.H]
    else:
        d["conv"], d["ssm"] = c.conv.to(dev), c.ssm.to(dev)
        d["mixed"], d["out_gate"], d["beta"] = c.mixed.to(dev), c.out_gate.to(dev), c.beta.to(dev)
    for k in ("gate", "conv_weight", "A_log", "dt_bias", "norm_weight", "idx"):
        d[k] = getattr(c, k).to(dev)
    d["acc"] = c.acc.to(dev) if c.spec else None
    d["cu"] = torch.arange(0, c.T + 1, c.S, dtype=torch.int32, device=dev)
    d["out"] = torch.full((c.T, c.H * D), float("nan"), dtype=torch.bfloat16, device=dev)
    return d


def _call(kda, d, **kw):
    return kda.decode(d["mixed"], d["conv"], d["conv_weight"], d["gate"], d["beta"], d["out_gate"], d["A_log"],
                      d["dt_bias"], d["norm_weight"], d["ssm"], d["idx"], d["acc"], d["cu"], NORM_EPS, LB, d["out"], **kw)


def _check(c, d, O, tag=""):
    ro, rconv, rssm, (ob, fac) = c.oracle(O)
    check_out(d["out"], ro, f"{tag}decode B={c.B} S={c.S} H={c.H}", np.arange(0, c.T + 1, c.S),
              allow=decode_rounding_allowance(ro, ob, fac))
    bits = d["out"].view(torch.int16).cpu()
    for n in c.dead():
        assert bool((bits[n * c.S:(n + 1) * c.S] == 0).all()), f"{tag}dead sequence {n}: output rows not +0"
    rows, cslots = c.written()
    conv, ssm = d["conv"].cpu(), d["ssm"].cpu()
    assert np.array_equal(f32(conv), rconv), f"{tag}conv cache differs from the reference rule"
    got = f32(ssm)
    for r in sorted(rows):
        e = rel_frob(got[r], rssm[r])
        assert e <= STATE_TOL, f"{tag}ssm row {r}: relF {e:.3e}"
    _, ssm0 = c.pools()
    keep = np.ones(c.slots, bool)
    keep[sorted(rows)] = False
    assert np.array_equal(got[keep], f32(ssm0)[keep]), f"{tag}unwritten ssm rows changed"
    if c.raw is not None:
        # every byte outside the conv / ssm views (page padding) is untouched
        raw = d["raw"].cpu()
        mask = torch.ones(raw.numel(), dtype=torch.bool)
        pg = c.page
        for s in range(c.slots):
            mask[s * pg: s * pg + c.conv_bytes + c.H * D * D * 4] = False
        assert torch.equal(raw[mask], c.raw[mask]), f"{tag}page padding changed"


def _run(oracle, call_kw=None, **kw):
    import kda355
    _say("decode " + " ".join(f"{k}={v}" for k, v in kw.items()) + (f" {list(call_kw)}" if call_kw else ""))
    c = Case(**kw)
    d = _device_args(c, torch.device("cuda", 0))
    _call(kda355, d, **(call_kw or {}))
    torch.cuda.synchronize()
    _check(c, d, oracle)
    return c, d


def test_plain_decode_pages(oracle):
    _run(oracle, B=16, S=1, H=4, seed=1, spec=False)


def test_plain_decode_dense_pools(oracle):
    _run(oracle, B=8, S=1, H=2, seed=2, spec=False, pages=False)


def test_plain_decode_padding_slot(oracle):
    _run(oracle, B=8, S=1, H=2, seed=3, spec=False, pad=[(2,), (5,)])


def test_sliced_decode_dead_rows_stay_zero(oracle):
    """Launches of at most 64 (sequence, head) pairs split each state over 4 workgroups, the last of which finishes
    the gated RMSNorm of the head.  Dead sequences (padding read or conv row) with NaN out_gate rows and negative norm
    weights: their output rows stay +0, as in the whole-state path."""
    _run(oracle, B=6, S=2, H=2, seed=15, spec=False, pad=[(1,), (4,)], hostile_dead=True)
    _run(oracle, B=6, S=1, H=2, seed=17, spec=False, pad=[(1,), (4,)], hostile_dead=True)
    _run(oracle, B=6, S=3, H=2, seed=16, spec=True, pad=[(2, 0), (3, 1)], hostile_dead=True)


def test_plain_decode_extra_taps(oracle):
    """A conv cache with more taps than plain decode needs: taps beyond 3 are left alone."""
    _run(oracle, B=4, S=1, H=2, seed=4, spec=False, extra_taps=2)


def test_plain_multi_token(oracle):
    """Several tokens per sequence without num_accepted_tokens: decoded in order, final state and last 3 inputs kept."""
    _run(oracle, B=4, S=3, H=2, seed=11, spec=False)


def test_spec_verify_pages(oracle):
    _run(oracle, B=8, S=4, H=4, seed=5, spec=True)


def test_spec_verify_s8(oracle):
    """Config-4 token count (S = 8: 7 drafts + 1) at a small batch."""
    _run(oracle, B=6, S=8, H=2, seed=6, spec=True)


def test_spec_verify_streaming_size(oracle):
    """A launch that writes more state than the streaming threshold (8 x 8 x 96 states of 64 KiB = 403 MB > 384 MiB):
    the kernel variant with streaming stores, which forms each token's operands inside the walk."""
    _run(oracle, B=8, S=8, H=96, seed=12, spec=True, pages=False)


def test_spec_verify_whole_state_workgroups(oracle):
    """A launch above the slicing size (9 x 32 = 288 > 64 (sequence, head) pairs): one workgroup per whole state (the
    launches of at most 64 pairs above split each state over 4 workgroups of 32 rows)."""
    _run(oracle, B=9, S=4, H=32, seed=13, spec=True, pages=False)


def test_sliced_decode_workspace(oracle):
    """A caller's workspace: two sliced launches in a row share it and leave its counters (the first 256 bytes) zero
    (the last slice of every (sequence, head) resets its counter), and the same calls without a workspace run whole
    states; all against the oracle."""
    import importlib
    dec = importlib.import_module("kda355.decode")
    dev = torch.device("cuda", 0)
    ws = torch.zeros(dec.WS_BYTES, dtype=torch.uint8, device=dev)
    for spec, S in ((False, 1), (False, 3), (True, 4)):
        for rep in range(2):
            _run(oracle, call_kw={"workspace": ws}, B=5, S=S, H=3, seed=40 + 2 * S + rep, spec=spec)
            assert int(ws[:256].count_nonzero()) == 0, f"workspace counters not zero after spec={spec} S={S} call {rep}"
        _run(oracle, call_kw={"workspace": None}, B=5, S=S, H=3, seed=60 + S, spec=spec)


def test_plain_decode_whole_state_workgroups(oracle):
    _run(oracle, B=9, S=1, H=32, seed=14, spec=False)


def test_spec_verify_padding(oracle):
    """Padding write rows (skipped) and a sequence whose conv row idx[n, 0] is padding (dead: zero output)."""
    _run(oracle, B=6, S=4, H=2, seed=7, spec=True, pad=[(0, 3), (2, 1), (4, 0)])


def test_spec_verify_dense_pools(oracle):
    _run(oracle, B=4, S=3, H=4, seed=8, spec=True, pages=False)


def test_graph_replay_new_data(oracle):
    """One capture replayed over new inputs, indices and pool contents written in place between replays."""
    import kda355
    O = oracle
    dev = torch.device("cuda", 0)
    c = Case(B=8, S=4, H=2, seed=9, spec=True)
    d = _device_args(c, dev)
    _say("decode graph replay B=8 S=4 H=2")
    _call(kda355, d)
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        _call(kda355, d)
    for rep in range(3):
        c2 = Case(B=8, S=4, H=2, seed=100 + rep, spec=True)
        d["raw"].copy_(c2.raw)
        d["mixed"].copy_(c2.mixed)
        d["out_gate"].copy_(c2.out_gate)
        d["beta"].copy_(c2.beta)
        for k in ("gate", "conv_weight", "A_log", "dt_bias", "norm_weight", "idx"):
            d[k].copy_(getattr(c2, k))
        d["acc"].copy_(c2.acc)
        d["out"].fill_(float("nan"))
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        _check(c2, d, O, tag=f"replay {rep}: ")


def test_config3_shape_one_step(oracle):
    """Config-3 width (H = 32) at a batch the oracle finishes in seconds."""
    _run(oracle, B=4, S=1, H=32, seed=10, spec=False)


# The reference eval's held-out decode shapes (kda/mi350x/benchmark/eval_kda_mi350x.py:761-793): (H, B, S), S = 1 plain
# decode, S > 1 spec verify with uniform accepted lengths; each captured and replayed, replayed again on new data,
# indices and pool contents, and called eagerly; every fourth shape also on dense pools.
_HELDOUT = {
    "h_d_h12_b8": (12, 8, 1), "h_d_h12_b200": (12, 200, 1), "h_s2_h12_b8": (12, 8, 2), "h_s4_h12_b40": (12, 40, 4),
    "h_s8_h12_b100": (12, 100, 8), "h_s8_h12_b256": (12, 256, 8), "h_d_h24_b16": (24, 16, 1), "h_s5_h24_b33": (24, 33, 5),
    "h_s6_h16_b4": (16, 4, 6), "h_s6_h16_b48": (16, 48, 6), "h_d_h16_b512": (16, 512, 1), "h_s3_h8_b96": (8, 96, 3),
    "h_d_h8_b7": (8, 7, 1), "h_s8_h48_b12": (48, 12, 8), "h_d_h96_b64": (96, 64, 1), "h_s3_h96_b5": (96, 5, 3),
    "h_s7_h12_b1": (12, 1, 7),
}


def _load(d, c):
    """Copy case c's inputs, indices and pools into the device buffers d (same shapes and layouts)."""
    if c.raw is not None:
        d["raw"].copy_(c.raw)
        d["mixed"].copy_(c.mixed)
        d["out_gate"].copy_(c.out_gate)
        d["beta"].copy_(c.beta)
    else:
        for k, x in (("conv", c.conv), ("ssm", c.ssm), ("mixed", c.mixed), ("out_gate", c.out_gate),
                     ("beta", c.beta)):
            d[k].copy_(x)
    for k in ("gate", "conv_weight", "A_log", "dt_bias", "norm_weight", "idx"):
        d[k].copy_(getattr(c, k))
    if c.spec:
        d["acc"].copy_(c.acc)
    d["out"].fill_(float("nan"))


@pytest.mark.parametrize("name", list(_HELDOUT))
def test_heldout_decode_shape(oracle, name):
    import kda355
    H, B, S = _HELDOUT[name]
    i = list(_HELDOUT).index(name)
    dev = torch.device("cuda", 0)
    slots = B * S + 16
    for pages in ((True, False) if i % 4 == 0 else (True,)):
        _say(f"held-out {name}: H={H} B={B} S={S} {'pages' if pages else 'dense'}")
        cases = [Case(B=B, S=S, H=H, seed=13 * i + r, spec=S > 1, pages=pages, slots=slots) for r in range(3)]
        d = _device_args(cases[0], dev)
        _call(kda355, d)
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            _call(kda355, d)
        for r, c in enumerate(cases[:2]):
            _load(d, c)
            torch.cuda.synchronize()
            gr.replay()
            torch.cuda.synchronize()
            _check(c, d, oracle, tag=f"{name} replay {r}: ")
        _load(d, cases[2])
        _call(kda355, d)
        torch.cuda.synchronize()
        _check(cases[2], d, oracle, tag=f"{name} eager: ")
