"""kda355: MI355X-native (gfx950) KDA -- Kimi Delta Attention, head dim 128 -- behind the reference's API surfaces.

    from kda355 import chunk_kda, kda_prefill                      # plain prefill calls (fla / reference forms)
    from kda355 import prefill_prepare, prefill                    # vLLM-ROCm Kimi serving prefill (paged pool)
    from kda355 import fused_recurrent_kda, spec_commit           # decode / speculative verify on a state pool
    from kda355 import decode                                      # vLLM-ROCm fused decode (conv + KDA + gated norm)
    from kda355 import decode_warmup, prefill_health, ...          # the reference's operator helpers (no-ops here)
    torch.ops.kda355.{fused_kda_decode, fused_kda_prefill, prefill, decode, fused_recurrent_kda, spec_commit}
                                                                   # the same kernels as registered torch ops

Every entry point runs the hand-written HIP kernels of libkda355.so (include/kda355.h).  There is no CPU or PyTorch
fallback: calling on CPU tensors raises TypeError, and a missing library raises RuntimeError.
"""
from ._lib import LIB_PATH, lib  # noqa: F401
from .prefill import chunk_kda, kda_prefill, plan, prefill, prefill_prepare  # noqa: F401
from .recurrent import fused_recurrent_kda, spec_commit  # noqa: F401
from .decode import decode  # noqa: F401
from .health import (decode_cotenant_mode, decode_health, decode_warmup, prefill_health,  # noqa: F401
                     prefill_range_guard)
from . import ops  # noqa: F401  (registers torch.ops.kda355.*)

__all__ = ["chunk_kda", "kda_prefill", "plan", "prefill", "prefill_prepare", "fused_recurrent_kda", "spec_commit", "decode",
           "decode_warmup", "decode_cotenant_mode", "decode_health", "prefill_health", "prefill_range_guard",
           "lib", "LIB_PATH"]
