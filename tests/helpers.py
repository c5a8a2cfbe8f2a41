"""Shared test helpers: seeded CPU inputs (BASELINE.json distributions), tolerance metrics."""
from __future__ import annotations

import math

import numpy as np
import torch

D = 128


def gen(seed):
    return torch.Generator().manual_seed(seed)


def qk_unit_bf16(shape, g):
    """fp32 N(0,1), L2-normalized per (token, head) in fp32, then bf16 (the configs' q / k)."""
    x = torch.randn(*shape, D, generator=g)
    return torch.nn.functional.normalize(x, dim=-1).bfloat16()


def config_inputs(T, H, g, N0=None):
    """q, k, v bf16 [T, H, 128]; g fp32 -softplus(N(0,1)); beta fp32 sigmoid(N(0,1)) (CPU tensors)."""
    q = qk_unit_bf16((T, H), g)
    k = qk_unit_bf16((T, H), g)
    v = torch.randn(T, H, D, generator=g).bfloat16()
    gg = -torch.nn.functional.softplus(torch.randn(T, H, D, generator=g))
    beta = torch.sigmoid(torch.randn(T, H, generator=g))
    return q, k, v, gg, beta


def f32(t):
    return t.detach().float().cpu().numpy()


def bf16_half_ulp(x):
    """Half a bf16 ulp at |x| (the rounding bound of storing x in bf16)."""
    a = np.abs(np.asarray(x, np.float64))
    e = np.floor(np.log2(np.maximum(a, 1e-38)))
    return np.ldexp(1.0, (e - 8).astype(np.int64))


def out_err(got_bf16, ref):
    """(excess, raw, relL2): excess = max(|got - ref| - half_ulp_bf16(ref)) / RMS(ref) -- the max-abs error beyond the
    bf16 storage rounding the output format itself imposes; raw = max|got - ref| / RMS(ref)."""
    g = np.asarray(got_bf16, np.float64)
    r = np.asarray(ref, np.float64)
    rms = math.sqrt(float((r * r).mean())) or 1e-30
    d = np.abs(g - r)
    excess = float(np.max(d - bf16_half_ulp(r), initial=0.0)) / rms
    raw = float(d.max(initial=0.0)) / rms
    rel = float(np.linalg.norm(g - r) / max(np.linalg.norm(r), 1e-30))
    return excess, raw, rel


def rel_frob(got, ref):
    g = np.asarray(got, np.float64)
    r = np.asarray(ref, np.float64)
    return float(np.linalg.norm(g - r) / max(np.linalg.norm(r), 1e-30))


OUT_TOL = 2e-2     # max-abs error <= 2e-2 x RMS(ref) (bf16 output)
REL_TOL = 2e-2     # relative L2 error of each sequence's output (kda/mi350x/benchmark/eval_kda_mi350x.py:80-82)
STATE_TOL = 1e-3   # relative Frobenius error of fp32 final / checkpoint states


def seq_rel(got, ref, cu):
    """Largest relative L2 error over the sequences [cu[n], cu[n+1]) (token axis first), the reference eval's
    metric (eval_kda_mi350x.py:154-156, 327-331); sequences with an all-zero reference are skipped."""
    g = np.asarray(got, np.float64)
    r = np.asarray(ref, np.float64)
    worst = 0.0
    for a, b in zip(list(cu[:-1]), list(cu[1:])):
        if b <= a:
            continue
        nr = np.linalg.norm(r[a:b])
        if nr == 0.0:
            continue
        worst = max(worst, float(np.linalg.norm(g[a:b] - r[a:b]) / nr))
    return worst


def check_out(got, ref, what, cu=None, allow=None):
    """Both output bars, asserted and printed: the max-abs error beyond bf16 storage rounding <= OUT_TOL x RMS(ref),
    and the relative L2 error of every sequence (or of the whole output when cu is None) <= REL_TOL.  The raw
    max-abs / RMS is printed beside them.  allow: a per-element rounding allowance replacing half a bf16 ulp of the
    reference (for outputs whose reference formula rounds to bf16 more than once, see decode_rounding_allowance)."""
    g = f32(got) if isinstance(got, torch.Tensor) else np.asarray(got)
    ex, raw, rel = out_err(g, ref)
    if allow is not None:
        r = np.asarray(ref, np.float64)
        rms = math.sqrt(float((r * r).mean())) or 1e-30
        ex = float(np.max(np.abs(g.astype(np.float64) - r) - np.asarray(allow, np.float64), initial=0.0)) / rms
    worst = seq_rel(g, ref, cu) if cu is not None else rel
    print(f"[err] {what}: excess {ex:.2e} raw max-abs/RMS {raw:.2e} relL2 {rel:.2e} worst-seq relL2 {worst:.2e}",
          flush=True)
    assert ex <= OUT_TOL, f"{what}: output excess {ex:.3e} > {OUT_TOL} (raw {raw:.3e}, relL2 {rel:.3e})"
    assert worst <= REL_TOL, f"{what}: per-sequence relL2 {worst:.3e} > {REL_TOL}"
    return ex


def decode_rounding_allowance(ref_out, ob, fac):
    """The fused decode's reference rounds twice (kda/mi350x/reference.py:172-175): o -> bf16(o), then
    y = bf16(o) * fac -> bf16.  An fp32 o within a few fp32 ulps of a bf16 rounding boundary of o rounds to the
    neighbouring bf16 value on some elements, which moves y by fac * ulp(bf16(o)) before the output rounding.  The
    allowance per element is exactly that one step plus half a bf16 ulp of the output; the max-abs bar applies to the
    error beyond it.  ob = bf16(o_ref) and fac from oracle.decode_full(..., aux=True)."""
    ob = np.abs(np.asarray(ob, np.float64))
    step = 2.0 * bf16_half_ulp(ob)
    return np.abs(np.asarray(fac, np.float64)) * step + bf16_half_ulp(ref_out)
