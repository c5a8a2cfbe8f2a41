"""The operator helpers of the reference's serving module (kda/mi350x/kda/kernel.py:113-128,153-209), kept only so
that callers which invoke them keep working.  None of them has anything to act on here: the kernels never wait on
other workgroups (no relay, mailboxes or claim counters), nothing is compiled at run time, and the prefill's decay
range is handled inside the kernel (a log-decay below -9 is raised to -9).  Each helper returns the reference's
result shape and changes nothing.
"""
from __future__ import annotations

import warnings

from . import _lib


def decode_warmup(device=None):
    """kernel.py:187-190.  Loads libkda355.so; there is nothing to compile or probe.  Returns {"library", "device"}."""
    _lib.lib()
    return {"library": str(_lib.LIB_PATH), "device": device}


def decode_cotenant_mode(mode=""):
    """kernel.py:193-196.  Has no effect: this build has one decode launch form per shape, and none of them waits for
    other workgroups to be resident.  Warns when a mode is requested; always returns ""."""
    if mode:
        warnings.warn(f"kda355: decode_cotenant_mode({mode!r}) has no effect (one launch form per shape)",
                      RuntimeWarning, stacklevel=2)
    return ""


def decode_health(heal=False):
    """kernel.py:199-209.  No decode state lives outside the caller's pools, so every count is zero."""
    return {"ok": True, "stale_words": 0, "raised_flags": 0, "ghost_events": 0, "claim_misaligned": 0,
            "claim_healed": 0, "healed": 0}


def prefill_health(device=None, sync=False, acknowledge=False):
    """kernel.py:153-177.  No relay, so no handoff can time out.  sync=True still waits for the device."""
    if sync:
        import torch
        torch.cuda.synchronize(device)
    return {"ok": True, "relay": "off", "relay_state": "absent", "serial": 0, "faults": []}


def prefill_range_guard(on=None):
    """kernel.py:113-128.  There is no fp32 recompute path to switch; the kernel raises every log-decay below -9 to
    -9 instead (a state change below 1.2e-4 relative on the affected channel).  Returns False; warns if asked to turn
    a guard on."""
    if on:
        warnings.warn("kda355: no fp32 range-guard recompute; log-decays below -9 are raised to -9 in the kernel",
                      RuntimeWarning, stacklevel=2)
    return False
