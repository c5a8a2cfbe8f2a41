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
    """libkda355.so exports every declared entry point but the no-allocation one, which libkda355_noalloc.so exports
    (so that only its callers hold its static scratch)."""
    from kda355 import _lib
    L, NL = _lib.lib(), _lib.noalloc_lib()
    missing = [n for n in _declared() if not hasattr(NL if n in _lib.NOALLOC_SYMBOLS else L, n)]
    assert not missing, f"not exported: {missing}"
    assert set(_lib.NOALLOC_SYMBOLS) <= set(_declared())
    assert L.kda355_version() >= 100


def test_noalloc_rejects_oversized_layout():
    """kda355_prefill_launch_noalloc rejects a plan whose workspace exceeds its static scratch (config 2's layout needs
    ~1 GB) with KDA355_EINVAL before any device call; the plan is made on the host."""
    import kda355
    from kda355 import _lib
    T, H = 131072, 32
    meta = kda355.plan(np.array([0, T], np.int64), H, device=None)
    assert meta.workspace_bytes > _lib.NOALLOC_SCRATCH_BYTES
    a = _lib.KdaPrefillArgs()
    fake = ctypes.c_void_p(1 << 20)                      # never dereferenced: the call is rejected first
    for f in ("q", "k", "v", "g", "beta", "out", "tables", "final_state"):
        setattr(a, f, fake)
    a.T, a.N, a.H = T, 1, H
    a.plan = ctypes.pointer(meta.plan)
    assert _lib.noalloc_lib().kda355_prefill_launch_noalloc(ctypes.byref(a), None) == _lib.EINVAL
    assert b"static scratch" in _lib.lib().kda355_last_error()


def test_prefill_rejects_oversized_row_strides():
    """Row strides of 2^21 elements or more (the kernels address a chunk's rows with 32-bit offsets) are rejected with
    KDA355_EINVAL before any device call; a stride just below passes that check and the call fails on the next one
    (a pool slot stride that is not a multiple of 4, on purpose), still before any device call."""
    import kda355
    from kda355 import _lib
    L = _lib.lib()
    T, H = 256, 2
    meta = kda355.plan(np.array([0, T], np.int64), H, device=None)
    a = _lib.KdaPrefillArgs()
    fake = ctypes.c_void_p(1 << 20)                      # never dereferenced: the call is rejected first
    for f in ("q", "k", "v", "g", "beta", "out", "tables", "final_state"):
        setattr(a, f, fake)
    a.T, a.N, a.H = T, 1, H
    a.plan = ctypes.pointer(meta.plan)
    a.qkv_row_stride, a.g_row_stride, a.beta_row_stride, a.out_row_stride = H * 128, H * 128, H, 1 << 21
    assert L.kda355_prefill_launch(ctypes.byref(a), None) == _lib.EINVAL
    assert b"row strides" in L.kda355_last_error()
    a.out_row_stride, a.qkv_row_stride = H * 128, (1 << 21) + 8
    assert L.kda355_prefill_launch(ctypes.byref(a), None) == _lib.EINVAL
    assert b"row strides" in L.kda355_last_error()
    a.qkv_row_stride, a.flags = (1 << 21) - 8, 8          # KDA355_PF_POOL
    a.state_pool, a.state_idx, a.has_initial_state, a.state_slot_stride = fake, fake, fake, 3
    assert L.kda355_prefill_launch(ctypes.byref(a), None) == _lib.EINVAL
    assert b"state pool misaligned" in L.kda355_last_error()


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


def _plan(lens, H, cus, every=0, ck=None):
    """kda355_prefill_plan over a layout of sequence lengths: (plan, table, the cu array the table refers to)."""
    import numpy as np
    from kda355 import _lib
    L = _lib.lib()
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    pin = _lib.KdaPrefillPlanIn()
    pin.cu_seqlens = ctypes.c_void_p(cu.ctypes.data)
    if ck is not None:
        ck = np.asarray(ck, np.int32)
        pin.ck_offsets = ctypes.c_void_p(ck.ctypes.data)
    pin.N, pin.H, pin.num_cus, pin.ck_every = len(lens), H, cus, every
    pl = _lib.KdaPrefillPlan()
    assert L.kda355_prefill_plan(ctypes.byref(pin), ctypes.byref(pl), None, 0) == 0
    tab = np.zeros(pl.table_words, np.int32)
    assert L.kda355_prefill_plan(ctypes.byref(pin), ctypes.byref(pl), ctypes.c_void_p(tab.ctypes.data), tab.size) == 0
    return pl, tab


def _check_pieces(pl, tab, lens, H, every=0, ck_chunk=None):
    """The invariants of a split plan, from its tables: every sequence's chunks are covered once, in order; a split
    sequence is a first piece (flag 4: hands over its end state) followed by later pieces (flag 1: run from zero) of
    >= 1 chunk; fixup tasks = one per group of <= 2 chunks of a later piece; compose tasks = one per checkpoint that
    falls strictly inside a later piece (every-n row j: the state after j * every chunks, j * every < chunks of the
    sequence; single: the state after ck_chunk[n] chunks); the workspace = (3 slots per piece + 2 per compose task)
    states per head + one 16 KiB R tile per later-piece chunk and head."""
    ch = tab[20:20 + 13 * pl.num_chains].reshape(-1, 13)
    nch = [(x + 63) // 64 for x in lens]
    fix = ck_rows = ck_single = r_chunks = 0
    for n, c in enumerate(nch):
        pieces = sorted((int(f), int(k), int(fl)) for s, k, _, _, _, _, f, fl, *_ in ch if s == n)
        assert [f for f, _, _ in pieces] == list(np.cumsum([0] + [k for _, k, _ in pieces])[:-1])
        assert sum(k for _, k, _ in pieces) == c
        if len(pieces) == 1:
            assert pieces[0][2] == 2                      # a whole sequence: writes its final state
            continue
        assert pieces[0][2] == 4 and all(fl == 1 for _, _, fl in pieces[1:])
        assert all(k >= 1 for _, k, _ in pieces)
        for f, k, _ in pieces[1:]:
            fix += (k + 1) // 2
            r_chunks += k
            if every:
                ck_rows += sum(1 for j in range(1, c + 1) if f < j * every <= f + k and j * every < c)
            if ck_chunk is not None and f < ck_chunk[n] <= f + k:
                ck_single += 1
    split = [n for n in range(len(nch)) if sum(1 for r in ch if r[0] == n) > 1]
    assert pl.num_split == len(split) and pl.num_pieces == sum(1 for r in ch if r[0] in split)
    assert pl.num_fix_tasks == fix and pl.num_ck_tasks == ck_rows + ck_single
    assert pl.workspace_bytes == ((3 * pl.num_pieces + 2 * pl.num_ck_tasks) * H * 65536 + r_chunks * H * 16384
                                  if pl.num_pieces else 0)
    return ch


import numpy as np  # noqa: E402  (used by the plan helpers above)


def test_prefill_plan_host_only():
    """The schedule is built on the host from the layout alone: chunk counts, every-n row counts, bad layouts."""
    from kda355 import _lib
    L = _lib.lib()
    lens = [100, 0, 200, 4296]
    pl, tab = _plan(lens, 8, 64, every=128)              # 32 chains, 9 chunks per CU at balance on 64 CUs
    assert pl.num_chunks == 2 + 0 + 4 + 68 and pl.T == 4596 and pl.ck_rows == 1 + 0 + 2 + 34
    # the 68-chunk sequence (its last chunk 8 tokens) is cut into pieces; the others run whole
    ch = _check_pieces(pl, tab, lens, 8, every=2)
    assert pl.num_split == 1 and pl.num_pieces >= 4
    assert L.kda355_prefill_workspace_bytes(ctypes.byref(pl)) == pl.workspace_bytes
    pl, tab = _plan(lens, 8, 4, every=128)               # 140 chunks per CU: nothing is split, no workspace
    assert pl.num_pieces == 0 and L.kda355_prefill_workspace_bytes(ctypes.byref(pl)) == 0
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    pin = _lib.KdaPrefillPlanIn()
    pin.cu_seqlens, pin.N, pin.H, pin.num_cus, pin.ck_every = ctypes.c_void_p(cu.ctypes.data), 4, 8, 4, 128
    small = np.zeros(3, np.int32)
    assert L.kda355_prefill_plan(ctypes.byref(pin), ctypes.byref(pl), ctypes.c_void_p(small.ctypes.data), 3) == _lib.EINVAL
    bad = np.array([0, 10, 5], np.int64)
    pin.cu_seqlens, pin.N = ctypes.c_void_p(bad.ctypes.data), 2
    assert L.kda355_prefill_plan(ctypes.byref(pin), ctypes.byref(pl), None, 0) == _lib.EINVAL
    assert b"non-decreasing" in L.kda355_last_error()
    pin.cu_seqlens, pin.N, pin.ck_every = ctypes.c_void_p(cu.ctypes.data), 4, 100
    assert L.kda355_prefill_plan(ctypes.byref(pin), ctypes.byref(pl), None, 0) == _lib.EINVAL


def _lists(pl, tab, H):
    """The workgroup lists of a plan: per list, the (chain entry, head) items and their chunk counts."""
    G, off = int(pl.chunk_grid), int(tab[17])
    starts = tab[off:off + G + 1]
    items = tab[off + G + 1:off + G + 1 + int(starts[-1])]
    nch = lambda it: int(tab[20 + 13 * (int(it) // H) + 1])  # noqa: E731
    return [[(int(it), nch(it)) for it in items[starts[b]:starts[b + 1]]] for b in range(G)]


def test_prefill_plan_workgroup_lists():
    """Unsplit layouts with more (chain, head) items than CUs get workgroup lists when the list schedule is shorter
    (one workgroup per CU walks its items in turn): the lists partition the items and each runs longest first.
    Layouts that fit the CUs, split layouts and layouts the lists would not shorten keep one workgroup per item."""
    pl, tab = _plan([128] * 64, 12, 256)                 # the reference's p_64x128: 768 two-chunk items
    assert pl.num_split == 0 and pl.chunk_grid == 256
    ls = _lists(pl, tab, 12)
    assert sorted(it for lst in ls for it, _ in lst) == list(range(768)) and {len(lst) for lst in ls} == {3}
    lens, H = [130, 0, 777, 64, 1, 250, 64], 5       # mixed lengths, an empty sequence, on 3 CUs
    pl, tab = _plan(lens, H, 3)
    assert pl.num_split == 0 and pl.chunk_grid == 3
    ls = _lists(pl, tab, H)
    assert sorted(it for lst in ls for it, _ in lst) == list(range(len(lens) * H))
    for lst in ls:
        assert [c for _, c in lst] == sorted((c for _, c in lst), reverse=True)
    loads = [sum(c for _, c in lst) for lst in ls]
    assert max(loads) - min(loads) <= 13                 # within one longest item
    for lens, H, cus in (([131072], 32, 256), ([704, 1216, 512], 96, 256), ([100] * 10, 4, 256)):
        pl, tab = _plan(lens, H, cus)                    # split / no gain (p96_light8k_0) / fits the CUs
        assert pl.chunk_grid == 0 and tab[17] == 0


def test_prefill_plan_chunk32_choice():
    """The 32-token kernel (two workgroups per CU) is chosen for unsplit layouts with more items than CUs when the
    plan's schedule model has it finish first: items of similar length that keep both workgroups of a CU busy; not
    when a few long chains would run alone on their CUs (p96_loaded8k_1, p96_light8k_0) or pairs of unequal items
    would leave the longer alone (a ragged 256-1023-token layout), nor for split layouts or layouts that fit the CUs.
    Each case is one the model was fitted on, timed on MI355X with both kernels."""
    for lens, H in (([512] * 32, 12), ([512] * 32, 16), ([1024] * 32, 16), ([256] * 64, 16), ([2048] * 16, 32),
                    ([128] * 64, 12), ([128] * 128, 12)):
        pl, _ = _plan(lens, H, 256)
        assert pl.num_split == 0 and pl.chunk32 == 1, (lens[:2], H)
    for lens, H in (([384, 1344, 3008, 2176, 320, 832], 96), ([704, 1216, 512], 96),
                    ([256 + (97 * i) % 768 for i in range(32)], 16), ([131072], 32), ([8192] * 8, 32),
                    ([100] * 10, 4)):
        pl, _ = _plan(lens, H, 256)
        assert pl.chunk32 == 0, (lens[:2], H)
    rng = np.random.default_rng(9)
    for _ in range(40):
        N, H, cus = int(rng.integers(1, 40)), int(rng.integers(1, 9)), int(rng.choice([2, 3, 8, 32, 256]))
        pl, _ = _plan([int(x) for x in rng.integers(0, 1500, size=N)], H, cus)
        assert pl.chunk32 in (0, 1) and (pl.chunk32 == 0 or (pl.num_split == 0 and pl.num_chains * H > cus))


def test_prefill_plan_workgroup_lists_random_layouts():
    """Planner invariants over seeded random layouts and CU counts: a plan with workgroup lists splits nothing, has
    more items than lists, and its lists partition the items, each longest first; a plan without lists has no list
    section."""
    rng = np.random.default_rng(7)
    with_lists = 0
    for _ in range(60):
        N, H, cus = int(rng.integers(1, 40)), int(rng.integers(1, 9)), int(rng.choice([2, 3, 8, 32, 64, 256]))
        lens = [int(x) for x in rng.integers(0, 1500, size=N)]
        lens[int(rng.integers(0, N))] = 0
        pl, tab = _plan(lens, H, cus)
        if pl.chunk_grid == 0:
            assert tab[17] == 0
            continue
        with_lists += 1
        assert pl.num_split == 0 and pl.chunk_grid == cus < pl.num_chains * H
        ls = _lists(pl, tab, H)
        assert sorted(it for lst in ls for it, _ in lst) == list(range(pl.num_chains * H))
        for lst in ls:
            assert [c for _, c in lst] == sorted((c for _, c in lst), reverse=True)
    assert with_lists >= 10


def test_prefill_plan_splits_long_sequences():
    """With idle CUs, long sequences are cut into pieces of >= 2 chunks; full chips are not split."""
    pl, tab = _plan([131072], 32, 256)                   # configuration 2: 2048 chunks x 32 heads on 256 CUs
    assert (pl.num_pieces, pl.num_split, pl.num_chains, pl.num_fix_tasks) == (8, 1, 8, 7 * 256 // 2)
    assert pl.workspace_bytes == 3 * 8 * 32 * 128 * 128 * 4 + 7 * 256 * 32 * 64 * 128 * 2
    final = tab[20:20 + 13 * 8].reshape(8, 13)
    assert sorted(final[:, 6]) == list(range(0, 2048, 256)) and set(final[:, 1]) == {256}   # first chunk, count
    assert sorted(final[:, 7].tolist()) == [1] * 7 + [4]   # pieces 2..8 run from zero; piece 1 hands over its end
    lens1 = [4011, 4318, 6249, 7799, 532, 1400, 6787, 7785]   # configuration 1: 256 chains on 256 CUs
    pl, tab = _plan(lens1, 32, 256)
    # 611 chunks x 32 heads = 77 per CU at balance, but the longest chain has 122 chunks: the long sequences are cut
    # into pieces (a cut may be T chunks followed by the remainder), and no piece is longer than the balanced load
    # plus a quarter of it
    counts = _check_pieces(pl, tab, lens1, 32)[:, 1]
    assert pl.num_split >= 2 and pl.num_pieces > pl.num_split and counts.max() <= 77 * 5 // 4
    assert list(counts) == sorted(counts, reverse=True)                         # longest first
    pl, _ = _plan(lens1, 32, 64)                         # a quarter of the CUs: 306 chunks per CU, nothing is split
    assert pl.num_pieces == 0
    pl, _ = _plan([64, 100], 2, 256)                     # 1 + 2 chunks: too short to split
    assert pl.num_pieces == 0
    for lens in ([2048, 500], [1000, 900], [8192]):      # few chains on an idle chip: cut into short pieces
        pl, tab = _plan(lens, 2, 256)
        _check_pieces(pl, tab, lens, 2)
        assert pl.num_split == len([x for x in lens if x > 256]) and pl.num_pieces >= 2 * pl.num_split
    # the plan is made on the host for every serving step: a large batch with one long outlier stays cheap
    import time
    rng = np.random.default_rng(0)
    lens = list(rng.integers(64, 2048, size=255)) + [65536]
    t0 = time.perf_counter()
    pl, _ = _plan(lens, 32, 256)
    assert pl.num_split == 1 and time.perf_counter() - t0 < 0.05


def test_prefill_plan_one_chunk_pieces_and_engine_rounds():
    """Short sequences on an idle chip are cut down to one-chunk pieces; and the schedule the plan is costed with
    sends workgroup i to one shader engine of 8 CUs (the same for every i of one residue mod 32), where a workgroup
    that finds no free CU waits for one of that engine's, even with CUs idle elsewhere.  So a cut whose extra
    workgroups would wait behind long pieces loses to one that starts every workgroup at once (the reference eval's
    p12_loaded8k_0: 18 pieces, 228 workgroups, 141 us against 21 pieces, 264 workgroups, 164 us on MI355X), and
    one-chunk remainders that would wait are not made (p12_loaded16k_0)."""
    pl, tab = _plan([1024], 12, 256)                     # 16 chunks x 12 heads: 16 pieces of one chunk, 192 workgroups
    _check_pieces(pl, tab, [1024], 12)
    assert (pl.num_pieces, pl.num_split) == (16, 1)
    pl, tab = _plan([1600], 12, 256)                     # 25 chunks: twelve pieces of 2 and one of 1
    counts = _check_pieces(pl, tab, [1600], 12)[:, 1]
    assert sorted(counts.tolist()) == [1] + [2] * 12
    lens = [7808, 128]                                   # p12_loaded8k_0: 122 + 2 chunks
    pl, tab = _plan(lens, 12, 256)
    _check_pieces(pl, tab, lens, 12)
    assert pl.num_pieces == 18 and pl.num_chains * 12 <= 256
    lens = [5440, 1920, 8768]                            # p12_loaded16k_0
    pl, tab = _plan(lens, 12, 256)
    counts = _check_pieces(pl, tab, lens, 12)[:, 1]
    assert counts.min() >= 2 and pl.num_chains * 12 <= 256


# the reference eval's host gate layouts (kda/mi350x/benchmark/eval_kda_mi350x.py:98-112: (new tokens, has initial
# state, checkpoint offset) per sequence)
_GATE_LAYOUTS = {
    "p12_loaded16k_1": (12, [(3008, 1, 3008), (1536, 1, 1536), (256, 1, 64), (128, 0, 0), (1600, 1, 832), (640, 1, 0),
                             (576, 1, 0), (512, 1, 0), (448, 1, 0), (2560, 1, 2560), (320, 1, 256), (4288, 1, 3712)]),
    "p96_loaded8k_1": (96, [(384, 1, 0), (1344, 1, 896), (3008, 0, 2048), (2176, 1, 2048), (320, 1, 0), (832, 0, 0)]),
}


def test_prepare_time_gate():
    """prefill_prepare runs once per serving step on a new layout: the reference eval's bound is 1 ms + 5 us per
    sequence, median over 5 fresh layouts (the lengths jittered by up to 64 tokens between neighbours, checkpoints at
    multiples of 1024; eval_kda_mi350x.py:669-712).  The host plan alone is timed here (no device)."""
    import statistics
    import time
    import kda355
    for name, (H, seqs) in _GATE_LAYOUTS.items():
        times = []
        for j in range(5):
            lens = [s[0] for s in seqs]
            if len(lens) > 1:
                a, b = j % len(lens), (j + 1) % len(lens)
                d = min(64, lens[a] - 1)
                lens[a] -= d
                lens[b] += d
            cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
            offs = np.array([(x // 1024) * 1024 if x >= 1024 else 0 for x in lens], np.int32)
            t0 = time.perf_counter()
            kda355.plan(cu, H, checkpoint_offsets=offs)
            times.append((time.perf_counter() - t0) * 1e3)
        limit = 1.0 + 0.005 * len(seqs)
        assert statistics.median(times) <= limit, f"{name}: plan median {statistics.median(times):.3f} ms > {limit}"


def test_prefill_plan_schedules_both_checkpoint_kinds():
    """Later pieces get compose tasks for the single checkpoint and for every-n rows alike (the launch's mode picks
    one; a plan made without flags must still cover both): 8192 tokens (128 chunks) on an idle chip, single
    checkpoint at chunk 40, every-n rows every 8 chunks (row j is the state after 8 j chunks; rows inside the first
    piece are written by that piece itself)."""
    pl, tab = _plan([8192], 2, 256, every=8 * 64, ck=[40 * 64])
    ch = _check_pieces(pl, tab, [8192], 2, every=8, ck_chunk=[40])
    assert pl.num_split == 1
    off_ckc, nck = tab[13], tab[14]                      # header: compose list offset and length
    tasks = tab[off_ckc:off_ckc + 4 * nck].reshape(nck, 4)
    kinds = tasks[:, 3].tolist()
    first_len = int(ch[ch[:, 6] == 0, 1][0])             # chunks of the first piece
    inside = [j for j in range(1, 16) if 8 * j > first_len]
    assert kinds.count(1) == (1 if 40 > first_len else 0) and kinds.count(2) == len(inside)
    assert tasks[tasks[:, 3] == 1, 0].tolist() == ([0] if 40 > first_len else [])   # the single checkpoint of seq 0
    assert sorted(tasks[tasks[:, 3] == 2, 0].tolist()) == inside                      # every-n rows in later pieces


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


def test_unsupported_forms_raise_before_any_device_work():
    """Forms the kernels do not implement raise ValueError up front (no fallback): the K-major state layout of fla's
    chunk_kda (state_v_first=False) and the non-in-place final state of fused_recurrent_kda."""
    import pytest
    import torch
    import kda355
    x = torch.zeros(1, 4, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="value-first"):
        kda355.chunk_kda(x, x, x, torch.zeros(1, 4, 2, 128), torch.zeros(1, 4, 2), state_v_first=False)
    with pytest.raises(ValueError, match="in-place"):
        kda355.fused_recurrent_kda(x, x, x, torch.zeros(1, 4, 2, 128), torch.zeros(1, 4, 2), inplace_final_state=False)


def test_operator_helpers_report_the_design():
    """The reference serving module's operator helpers (kernel.py:113-209) exist with its return shapes and report
    what this build's design implies: no relay faults, no decode workspaces to heal, no range-guard switch, no
    co-tenant launch forms."""
    import warnings
    import kda355
    h = kda355.prefill_health()
    assert h["ok"] is True and h["faults"] == [] and set(h) == {"ok", "relay", "relay_state", "serial", "faults"}
    d = kda355.decode_health(heal=True)
    assert d["ok"] is True and d["ghost_events"] == 0
    assert kda355.decode_warmup()["library"].endswith("libkda355.so")
    assert kda355.decode_cotenant_mode() == ""
    assert kda355.prefill_range_guard() is False
    for call in (lambda: kda355.prefill_range_guard(True), lambda: kda355.decode_cotenant_mode("lds_free")):
        with warnings.catch_warnings(record=True) as w:   # a request the design cannot honour says so
            warnings.simplefilter("always")
            assert call() in (False, "")
        assert any(issubclass(x.category, RuntimeWarning) for x in w)
