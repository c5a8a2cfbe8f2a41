"""The reference eval's co-tenant gate (kda/mi350x/benchmark/eval_kda_mi350x.py:883-976): a kernel on another stream
holds 3/4 of the CUs with all their LDS for a few seconds (tests/cotenant/hog.hip, bounded by the wall clock); a
serving prefill (p12_loaded16k_1), an eager spec-verify decode and a graph replay of it (s8_h12_b64) launched beside
it must finish well before the co-tenant leaves (no workgroup of ours waits for another to be resident) and match the
oracle to the usual bars."""
import ctypes
import time
from pathlib import Path

import pytest
import torch

from test_gpu_contract import DEV, LB, SCALE, Serving
from test_gpu_decode import Case, _call, _check, _device_args

pytestmark = pytest.mark.gpu
HOG = Path(__file__).resolve().parent / "cotenant" / "libhog.so"
HOG_SECONDS = 4.0  # the eval's co-tenant duration (eval_kda_mi350x.py:945)
FINISH_S = 1.5  # the eval's bar: finished this long after launch, i.e. not waiting for the co-tenant to leave
# p12_loaded16k_1 (kda/mi350x/benchmark/eval_kda_mi350x.py:92-115): (tokens, has_initial_state, checkpoint offset)
P12_LOADED16K_1 = [(3008, 1, 3008), (1536, 1, 1536), (256, 1, 64), (128, 0, 0), (1600, 1, 832), (640, 1, 0),
                   (576, 1, 0), (512, 1, 0), (448, 1, 0), (2560, 1, 2560), (320, 1, 256), (4288, 1, 3712)]


def _say(msg):
    print(f"[case] {msg}", flush=True)


def _hog():
    if not HOG.exists():
        raise RuntimeError(f"{HOG} is not built (make -C tests/cotenant, or __graft_entry__.build())")
    lib = ctypes.CDLL(str(HOG))
    lib.kda355_test_hog.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_double, ctypes.c_void_p, ctypes.c_void_p]
    lib.kda355_test_hog.restype = ctypes.c_int
    return lib


def _beside_hog(lib, fn):
    """Runs fn on the current stream while the hog holds 3/4 of the CUs; returns seconds from fn's launch to its end."""
    cus = torch.cuda.get_device_properties(DEV).multi_processor_count
    blocks = cus * 3 // 4
    started = torch.zeros(blocks * 64, dtype=torch.int32, device=DEV)
    side = torch.cuda.Stream(device=DEV)
    torch.cuda.synchronize()
    t_launch = time.perf_counter()
    rc = lib.kda355_test_hog(blocks, 160 * 1024, HOG_SECONDS, ctypes.c_void_p(started.data_ptr()),
                             ctypes.c_void_p(side.cuda_stream))
    assert rc == 0, f"hog launch failed: HIP error {rc}"
    while int(started.sum()) < blocks * 64 and time.perf_counter() - t_launch < 2.0:
        time.sleep(0.01)
    resident = int(started.sum()) // 64
    t0 = time.perf_counter()
    left = HOG_SECONDS - (t0 - t_launch)  # co-tenant time still ahead when fn starts (an upper bound)
    if resident != blocks or left <= FINISH_S:
        side.synchronize()  # let the co-tenant finish before failing
    assert resident == blocks, f"only {resident} of {blocks} co-tenant workgroups became resident"
    assert left > FINISH_S, f"the co-tenant had only {left:.2f} s left when the call started (needs > {FINISH_S})"
    fn()
    torch.cuda.current_stream().synchronize()
    dt = time.perf_counter() - t0
    side.synchronize()
    _say(f"{resident} of {blocks} co-tenant workgroups resident, {left:.2f} s of co-tenant time left at the call; "
         f"finished {dt * 1e3:.1f} ms after launch")
    return dt


def test_cotenant_prefill(oracle):
    import kda355
    lib = _hog()
    _say("co-tenant: prefill p12_loaded16k_1")
    c = Serving(12, P12_LOADED16K_1, 913)
    cu_cpu = torch.tensor(c.cu, dtype=torch.int32)
    meta = kda355.prefill_prepare(cu_cpu, c.H, c.ck_off, c.cidx, device=DEV)
    ws = torch.empty(max(meta.workspace_bytes, 256), dtype=torch.uint8, device=DEV)
    sidx, hinit = c.sidx.to(DEV), torch.tensor(c.hinit, dtype=torch.bool, device=DEV)
    cu, ck, cidx = cu_cpu.to(DEV), c.ck_off.to(DEV), c.cidx.to(DEV)

    def call():  # no device-wide synchronize inside: that would wait for the co-tenant too
        kda355.prefill(c.q, c.k, c.v, c.raw_g, c.raw_b, c.A_log, c.dt_bias, SCALE, LB, c.ssm, sidx, hinit, cu, c.out,
                       ck, cidx, meta=meta, workspace=ws)

    dt = _beside_hog(lib, call)
    c.verify(oracle, what="prefill beside the co-tenant")
    assert dt < FINISH_S, f"prefill took {dt:.2f} s beside the co-tenant"


def test_cotenant_decode_eager_and_graph(oracle):
    import kda355
    lib = _hog()
    _say("co-tenant: decode s8_h12_b64 eager")
    c = Case(B=64, S=8, H=12, seed=914, spec=True)
    d = _device_args(c, DEV)
    dt = _beside_hog(lib, lambda: _call(kda355, d))
    _check(c, d, oracle, "eager decode beside the co-tenant: ")
    assert dt < FINISH_S, f"decode took {dt:.2f} s beside the co-tenant"

    _say("co-tenant: decode s8_h12_b64 graph replay")
    c2 = Case(B=64, S=8, H=12, seed=915, spec=True)
    d2 = _device_args(c2, DEV)
    keep = {k: v.clone() for k, v in d2.items() if isinstance(v, torch.Tensor)}
    s = torch.cuda.Stream(device=DEV)
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        _call(kda355, d2)  # warm-up outside the capture
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _call(kda355, d2)
    torch.cuda.synchronize()  # nothing else runs yet
    for k, v in keep.items():  # the captured buffers back to the case's inputs
        d2[k].copy_(v)
    torch.cuda.synchronize()
    dt = _beside_hog(lib, graph.replay)
    _check(c2, d2, oracle, "graph replay beside the co-tenant: ")
    assert dt < FINISH_S, f"graph replay took {dt:.2f} s beside the co-tenant"
