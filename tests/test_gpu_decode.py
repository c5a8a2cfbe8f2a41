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

from helpers import OUT_TOL, STATE_TOL, f32, gen, out_err, rel_frob

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

    def __init__(self, B, S, H, seed, spec, pages=True, extra_taps=0, pad=()):
        g = gen(seed)
        dim = H * D
        T = B * S
        self.B, self.S, self.H, self.T, self.spec = B, S, H, T, spec
        taps = (W - 2 + S if spec else W - 1) + extra_taps
        slots = 2 * B * S + 16
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
                             self.idx.numpy(), self.acc.numpy() if self.spec else None, NORM_EPS, LB, precision=64)

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


def _call(kda, d):
    return kda.decode(d["mixed"], d["conv"], d["conv_weight"], d["gate"], d["beta"], d["out_gate"], d["A_log"],
                      d["dt_bias"], d["norm_weight"], d["ssm"], d["idx"], d["acc"], d["cu"], NORM_EPS, LB, d["out"])


def _check(c, d, O, tag=""):
    ro, rconv, rssm = c.oracle(O)
    ex, rawe, rel = out_err(f32(d["out"]), ro)
    assert ex <= OUT_TOL, f"{tag}output excess {ex:.3e} (raw {rawe:.3e}, relL2 {rel:.3e})"
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


def _run(oracle, **kw):
    import kda355
    _say("decode " + " ".join(f"{k}={v}" for k, v in kw.items()))
    c = Case(**kw)
    d = _device_args(c, torch.device("cuda", 0))
    _call(kda355, d)
    torch.cuda.synchronize()
    _check(c, d, oracle)
    return c, d


def test_plain_decode_pages(oracle):
    _run(oracle, B=16, S=1, H=4, seed=1, spec=False)


def test_plain_decode_dense_pools(oracle):
    _run(oracle, B=8, S=1, H=2, seed=2, spec=False, pages=False)


def test_plain_decode_padding_slot(oracle):
    _run(oracle, B=8, S=1, H=2, seed=3, spec=False, pad=[(2,), (5,)])


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
    """A launch above the slicing size (9 x 32 = 288 > 64 (sequence, head) pairs): one workgroup per whole state and
    the gated RMSNorm inside the decode kernel (the launches of at most 64 pairs above split each state over 4
    workgroups of 32 rows and finish the norm in a second kernel)."""
    _run(oracle, B=9, S=4, H=32, seed=13, spec=True, pages=False)


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
