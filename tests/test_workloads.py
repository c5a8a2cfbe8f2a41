"""The workload tables this build measures and tests against, checked on the CPU against the reference evaluation's
own tables (tests/golden/reference_workloads.json, written by tests/golden/make_workloads.py from
kda/mi350x/workloads/*.json): the 13 serving prefill steps and 10 decode steps, the phase-1 prefill layouts and decode
shapes with their recorded baselines, the 17 held-out decode shapes, the 7 numerics probes and the eval's constants."""
import json
from pathlib import Path

import pytest

GOLD = json.loads((Path(__file__).resolve().parent / "golden" / "reference_workloads.json").read_text())
T = GOLD["tables"]


def _plain(x):
    """Tuples to lists, recursively (the JSON form of a table)."""
    return json.loads(json.dumps(x))


def test_serving_prefill_steps():
    import bench
    assert set(bench.SERVING_PREFILL) == set(T["PREFILL_WORKLOADS"])
    for name, (H, seqs, _ref) in bench.SERVING_PREFILL.items():
        assert _plain([H, seqs]) == T["PREFILL_WORKLOADS"][name], name


def test_serving_decode_steps():
    import bench
    assert set(bench.SERVING_DECODE) == set(T["DECODE_WORKLOADS"])
    for name, (H, B, S, _ref) in bench.SERVING_DECODE.items():
        assert [H, B, S] == T["DECODE_WORKLOADS"][name], name


def test_phase1_prefill_layouts_and_baselines():
    import bench
    assert set(bench.PLAIN_PREFILL) == set(T["LEGACY_PREFILL"]) == set(bench.LEGACY_PREFILL_BASE_MS)
    for name, (lens, _ref) in bench.PLAIN_PREFILL.items():
        assert list(lens) == T["LEGACY_PREFILL"][name], name
        assert bench.LEGACY_PREFILL_BASE_MS[name] == pytest.approx(GOLD["legacy_prefill_baseline_ms"][name], rel=1e-4)


def test_phase1_decode_shapes_and_baselines():
    import bench
    assert set(bench.LEGACY_DECODE) == set(T["LEGACY_DECODE"])
    for name, (H, B, S, base) in bench.LEGACY_DECODE.items():
        assert [H, B, S] == T["LEGACY_DECODE"][name], name
        assert base == pytest.approx(GOLD["legacy_decode_baseline_us"][name], rel=1e-4), name


def test_heldout_decode_shapes():
    from test_gpu_decode import _HELDOUT
    assert {k: list(v) for k, v in _HELDOUT.items()} == T["DECODE_HELDOUT"]


def test_numerics_probes():
    from test_gpu_contract import _PROBES
    assert _plain(_PROBES) == T["NUMERIC_PROBES"]


def test_cotenant_step_is_the_eval_step():
    from test_gpu_cotenant import P12_LOADED16K_1
    assert _plain(P12_LOADED16K_1) == T["PREFILL_WORKLOADS"]["p12_loaded16k_1"][1]


def test_constants():
    import test_gpu_contract as c
    import test_gpu_decode as d
    k = GOLD["constants"]
    assert c.LB == d.LB == k["LB"]
    assert d.NORM_EPS == k["NORM_EPS"]
    assert c.P_RTOL == k["P_RTOL"]
    assert d.W == k["W"] and c.D == k["D"]
    assert d.PAGE_PAD == k["PAGE_PAD"]
    assert c.LEAD == k["DEC_TOKENS_FIRST"]
