"""The C ABI library loads on a machine without a GPU, exports every entry point include/kda355.h declares, and
rejects invalid arguments with KDA355_EINVAL before touching the device."""
import ctypes
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def _declared():
    text = (ROOT / "include" / "kda355.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(kda355_\w+)\s*\(", text, re.M)))


def test_header_lists_entry_points():
    names = _declared()
    assert "kda355_recurrent_launch" in names and "kda355_last_error" in names


def test_library_exports_every_declared_symbol():
    from kda355 import _lib
    L = _lib.lib()
    missing = [n for n in _declared() if not hasattr(L, n)]
    assert not missing, f"not exported: {missing}"
    assert L.kda355_version() >= 100


def test_invalid_arguments_rejected_without_gpu():
    from kda355 import _lib
    L = _lib.lib()
    a = _lib.KdaRecurrentArgs()
    a.B, a.S, a.H = 4, 1, 2                              # pointers left null
    assert L.kda355_recurrent_launch(ctypes.byref(a), None) == _lib.EINVAL
    assert b"null" in L.kda355_last_error()
    a.S = 0
    assert L.kda355_recurrent_launch(ctypes.byref(a), None) == _lib.EINVAL
    c = _lib.KdaSpecCommitArgs()
    c.B, c.S, c.H = 2, 2, 1
    assert L.kda355_spec_commit_launch(ctypes.byref(c), None) == _lib.EINVAL
    d = _lib.KdaDecodeArgs()
    d.B, d.S, d.H, d.conv_taps = 4, 1, 2, 3             # pointers left null
    assert L.kda355_decode_launch(ctypes.byref(d), None) == _lib.EINVAL
    assert b"null" in L.kda355_last_error()
    d.S = 17                                            # beyond the 16-token verify window
    assert L.kda355_decode_launch(ctypes.byref(d), None) == _lib.EINVAL


def test_struct_layout_matches_header():
    """ctypes mirrors of the argument structs have the size the C compiler gives them."""
    import subprocess
    import tempfile
    from kda355 import _lib
    src = '#include "kda355.h"\n#include <stdio.h>\nint main(){printf("%zu %zu %zu %zu %zu %zu\\n", ' \
          'sizeof(KdaRecurrentArgs), sizeof(KdaSpecCommitArgs), sizeof(KdaPrefillPlanIn), sizeof(KdaPrefillPlan), ' \
          'sizeof(KdaPrefillArgs), sizeof(KdaDecodeArgs));return 0;}\n'
    with tempfile.TemporaryDirectory() as d:
        (Path(d) / "m.c").write_text(src)
        subprocess.run(["gcc", "-I", str(ROOT / "include"), str(Path(d) / "m.c"), "-o", str(Path(d) / "m")],
                       check=True)
        sizes = subprocess.run([str(Path(d) / "m")], capture_output=True, text=True, check=True).stdout.split()
    mirrors = [_lib.KdaRecurrentArgs, _lib.KdaSpecCommitArgs, _lib.KdaPrefillPlanIn, _lib.KdaPrefillPlan,
               _lib.KdaPrefillArgs, _lib.KdaDecodeArgs]
    assert [int(x) for x in sizes] == [ctypes.sizeof(m) for m in mirrors]


def test_prefill_plan_host_only():
    """The schedule is built on the host from the layout alone: chunk counts, every-n row counts, bad layouts."""
    import numpy as np
    from kda355 import _lib
    L = _lib.lib()
    cu = np.array([0, 100, 100, 300, 4396], np.int64)
    pin = _lib.KdaPrefillPlanIn()
    pin.cu_seqlens = ctypes.c_void_p(cu.ctypes.data)
    pin.N, pin.H, pin.ck_every = 4, 8, 128
    pin.num_cus = 64                                     # 32 chains, 9 chunks per CU at balance: 64 > 1.25 x 9
    pl = _lib.KdaPrefillPlan()
    assert L.kda355_prefill_plan(ctypes.byref(pin), ctypes.byref(pl), None, 0) == 0
    assert pl.num_chunks == 2 + 0 + 4 + 64 and pl.T == 4396 and pl.ck_rows == 1 + 0 + 2 + 32
    # the 64-chunk sequence is cut into 4 pieces of 16 (the minimum piece); pieces 2..4 each keep one 16 KiB R tile
    # per chunk and head, every piece a start / local-state / transition slot per head, and the every-2-chunk rows
    # inside pieces 2..4 (chunks 18, 20, .., 62: 8 + 8 + 7) a (local state, transition) pair per head
    assert (pl.num_pieces, pl.num_split, pl.num_chains, pl.num_fix_tasks, pl.num_ck_tasks) == (4, 1, 7, 24, 23)
    assert L.kda355_prefill_workspace_bytes(ctypes.byref(pl)) == (3 * 4 + 2 * 23) * 8 * 65536 + 48 * 8 * 16384
    pin.num_cus = 4                                      # 140 chunks per CU: nothing is split, no workspace
    assert L.kda355_prefill_plan(ctypes.byref(pin), ctypes.byref(pl), None, 0) == 0
    assert pl.num_pieces == 0 and L.kda355_prefill_workspace_bytes(ctypes.byref(pl)) == 0
    tab = np.zeros(pl.table_words, np.int32)
    assert L.kda355_prefill_plan(ctypes.byref(pin), ctypes.byref(pl), ctypes.c_void_p(tab.ctypes.data), tab.size) == 0
    assert L.kda355_prefill_plan(ctypes.byref(pin), ctypes.byref(pl), ctypes.c_void_p(tab.ctypes.data), 3) == _lib.EINVAL
    bad = np.array([0, 10, 5], np.int64)
    pin.cu_seqlens, pin.N = ctypes.c_void_p(bad.ctypes.data), 2
    assert L.kda355_prefill_plan(ctypes.byref(pin), ctypes.byref(pl), None, 0) == _lib.EINVAL
    assert b"non-decreasing" in L.kda355_last_error()
    pin.cu_seqlens, pin.N, pin.ck_every = ctypes.c_void_p(cu.ctypes.data), 4, 100
    assert L.kda355_prefill_plan(ctypes.byref(pin), ctypes.byref(pl), None, 0) == _lib.EINVAL


def test_prefill_plan_splits_long_sequences():
    """With idle CUs, long sequences are cut into pieces of >= 16 chunks; short ones and full chips are not split."""
    import numpy as np
    from kda355 import _lib
    L = _lib.lib()

    def plan(lens, H, cus):
        cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
        pin = _lib.KdaPrefillPlanIn()
        pin.cu_seqlens = ctypes.c_void_p(cu.ctypes.data)
        pin.N, pin.H, pin.num_cus = len(lens), H, cus
        pl = _lib.KdaPrefillPlan()
        assert L.kda355_prefill_plan(ctypes.byref(pin), ctypes.byref(pl), None, 0) == 0
        tab = np.zeros(pl.table_words, np.int32)
        assert L.kda355_prefill_plan(ctypes.byref(pin), ctypes.byref(pl), ctypes.c_void_p(tab.ctypes.data), tab.size) == 0
        return pl, tab

    pl, tab = plan([131072], 32, 256)                    # configuration 2: 2048 chunks x 32 heads on 256 CUs
    assert (pl.num_pieces, pl.num_split, pl.num_chains, pl.num_fix_tasks) == (8, 1, 8, 7 * 256 // 2)
    assert pl.workspace_bytes == 3 * 8 * 32 * 128 * 128 * 4 + 7 * 256 * 32 * 64 * 128 * 2
    final = tab[20:20 + 13 * 8].reshape(8, 13)
    assert sorted(final[:, 6]) == list(range(0, 2048, 256)) and set(final[:, 1]) == {256}   # first chunk, count
    assert sorted(final[:, 7].tolist()) == [1] * 7 + [4]   # pieces 2..8 run from zero; piece 1 hands over its end
    lens1 = [4011, 4318, 6249, 7799, 532, 1400, 6787, 7785]   # configuration 1: 256 chains on 256 CUs
    pl, tab = plan(lens1, 32, 256)
    # 611 chunks x 32 heads = 77 per CU at balance, but the longest chain has 122 chunks: the long sequences are cut
    # into pieces of >= 16 chunks, none longer than 64, covering every chunk once
    counts = tab[20:20 + 13 * pl.num_chains].reshape(-1, 13)
    assert pl.num_split >= 2 and pl.num_pieces > pl.num_split
    assert counts[:, 1].max() <= 64 and counts[counts[:, 1] < 16, 1].tolist() in ([], [9]) and counts[:, 1].sum() == 611
    assert list(counts[:, 1]) == sorted(counts[:, 1], reverse=True)                         # longest first
    pl, _ = plan(lens1, 32, 64)                          # a quarter of the CUs: 306 chunks per CU, nothing is split
    assert pl.num_pieces == 0
    pl, _ = plan([1000, 900], 2, 256)                    # 16 chunks: too short to split
    assert pl.num_pieces == 0
    pl, _ = plan([2048, 500], 2, 256)                    # 32 chunks -> 2 pieces of 16
    assert (pl.num_pieces, pl.num_split) == (2, 1)
    # the plan is made on the host for every serving step: a large batch with one long outlier stays cheap
    import time
    rng = np.random.default_rng(0)
    lens = list(rng.integers(64, 2048, size=255)) + [65536]
    t0 = time.perf_counter()
    pl, _ = plan(lens, 32, 256)
    assert pl.num_split == 1 and time.perf_counter() - t0 < 0.05


def test_prefill_plan_schedules_both_checkpoint_kinds():
    """Later pieces get compose tasks for the single checkpoint and for every-n rows alike (the launch's mode picks
    one; a plan made without flags must still cover both): 8192 tokens in 8 pieces of 16 chunks, single checkpoint at
    chunk 40 (inside piece 3), every-n rows every 8 chunks (row j is the state after 8 j chunks: rows 0..2 belong to
    the first piece, which writes them itself; rows 3..15 fall in pieces 2..8)."""
    import numpy as np
    from kda355 import _lib
    L = _lib.lib()
    cu = np.array([0, 8192], np.int64)
    ck = np.array([40 * 64], np.int32)
    pin = _lib.KdaPrefillPlanIn()
    pin.cu_seqlens, pin.ck_offsets = ctypes.c_void_p(cu.ctypes.data), ctypes.c_void_p(ck.ctypes.data)
    pin.N, pin.H, pin.num_cus, pin.ck_every = 1, 2, 256, 8 * 64
    pl = _lib.KdaPrefillPlan()
    assert L.kda355_prefill_plan(ctypes.byref(pin), ctypes.byref(pl), None, 0) == 0
    tab = np.zeros(pl.table_words, np.int32)
    assert L.kda355_prefill_plan(ctypes.byref(pin), ctypes.byref(pl), ctypes.c_void_p(tab.ctypes.data), tab.size) == 0
    assert (pl.num_pieces, pl.num_split) == (8, 1)
    off_ckc, nck = tab[13], tab[14]                      # header: compose list offset and length
    tasks = tab[off_ckc:off_ckc + 4 * nck].reshape(nck, 4)
    kinds = tasks[:, 3].tolist()
    assert kinds.count(1) == 1 and kinds.count(2) == 13 and nck == pl.num_ck_tasks == 14
    assert tasks[tasks[:, 3] == 1, 0].tolist() == [0]    # the single checkpoint of sequence 0
    assert sorted(tasks[tasks[:, 3] == 2, 0].tolist()) == list(range(3, 16))   # every-n rows in later pieces
    assert pl.workspace_bytes == (3 * 8 + 2 * 14) * 2 * 65536 + 7 * 16 * 2 * 16384


def test_decode_rejects_host_tensors():
    """The fused decode wrapper raises TypeError for CPU tensors (the reference validator's device rule,
    kda/mi350x/kda/decode/kernel_v13_a.py:705-707), before any device call."""
    import pytest
    import torch
    import kda355
    H, B = 1, 2
    dim = H * 128
    t = torch.zeros
    with pytest.raises(TypeError):
        kda355.decode(t(B, 3 * dim, dtype=torch.bfloat16), t(4, 3, 3 * dim, dtype=torch.bfloat16), t(3, 4, dim),
                      t(B, H, 128, dtype=torch.bfloat16), t(B, H, dtype=torch.bfloat16), t(B, dim, dtype=torch.bfloat16),
                      t(H), t(dim), t(128), t(4, H, 128, 128), t(B, dtype=torch.int32), None,
                      torch.arange(B + 1, dtype=torch.int32), 1e-5, -5.0, t(B, dim, dtype=torch.bfloat16))
