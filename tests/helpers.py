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
STATE_TOL = 1e-3   # relative Frobenius error of fp32 final / checkpoint states
