"""kda355_prefill_launch_noalloc (the static-scratch variant of kda355_prefill_launch) against the caller-workspace
entry point, through the C ABI: two calls in a row on split layouts (the only ones with a workspace), the second
smaller than the first, each bit-identical to the workspace launch of the same plan (same kernels, same schedule),
outputs and final states; and a layout whose workspace exceeds the scratch is rejected with KDA355_EINVAL."""
import ctypes

import numpy as np
import pytest
import torch

from helpers import config_inputs, gen

pytestmark = pytest.mark.gpu
D = 128
DEV = torch.device("cuda", 0)


def _case(lens, H, seed):
    import kda355
    g = gen(seed)
    T = int(sum(lens))
    q, k, v, gg, beta = (x[None].to(DEV) for x in config_inputs(T, H, g))
    h0 = (torch.randn(len(lens), H, D, D, generator=g) * 0.02).to(DEV)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int64)
    meta = kda355.plan(cu, H, device=DEV)
    assert meta.workspace_bytes > 0, "the case must use a workspace"
    return q, k, v, gg, beta, h0, meta


def test_noalloc_matches_workspace_launch():
    import kda355
    from kda355 import _lib
    for i, (lens, H) in enumerate([([4096, 300], 4), ([2048], 2)]):
        print(f"[case] no-alloc call {i}: lens={lens} H={H}", flush=True)
        q, k, v, gg, beta, h0, meta = _case(lens, H, 80 + i)
        assert meta.workspace_bytes <= _lib.NOALLOC_SCRATCH_BYTES
        o1, f1 = kda355.chunk_kda(q, k, v, gg, beta, initial_state=h0, meta=meta)
        o2 = torch.full_like(o1, float("nan"))
        o2, f2 = kda355.chunk_kda(q, k, v, gg, beta, initial_state=h0, meta=meta, out=o2, workspace="static")
        torch.cuda.synchronize()
        assert torch.equal(o1, o2), f"call {i}: output differs from the workspace launch"
        assert torch.equal(f1, f2), f"call {i}: final states differ from the workspace launch"
