"""CPU tests of the contest trace-set reader (kachua_mlsys_amd.contest): the
directory layout, shape resolution against const / workload axes, dtypes,
safetensors inputs, scalars, missing inputs and seeded random inputs.  No
kernel runs here (tests/test_gpu_contest.py runs the workloads)."""

import json

import pytest
import torch

from contest_sets import DECODE_DEF, PREFILL_DEF, write_trace_set
from kachua_mlsys_amd import contest, decode, prefill


def test_resolve_root_and_one_level_below(tmp_path):
    base, _ = write_trace_set(tmp_path)
    assert contest.resolve_trace_set(base) == base
    assert contest.resolve_trace_set(tmp_path) == base
    with pytest.raises(FileNotFoundError):
        contest.resolve_trace_set(tmp_path / "missing")
    (tmp_path / "empty").mkdir()
    with pytest.raises(FileNotFoundError):
        contest.resolve_trace_set(tmp_path / "empty")


def test_definitions_and_workloads(tmp_path):
    base, _ = write_trace_set(tmp_path)
    assert contest.load_definition(base, contest.PREFILL)["inputs"].keys() == PREFILL_DEF["inputs"].keys()
    assert len(contest.load_workloads(base, contest.DECODE)) == 2
    assert len(contest.load_workloads(base, contest.PREFILL)) == 2
    with pytest.raises(FileNotFoundError):
        contest.load_definition(base, "gdn_unknown")


def test_resolve_shape():
    axes = PREFILL_DEF["axes"]
    assert contest.resolve_shape(None, axes, {}) is None
    assert contest.resolve_shape(["total_seq_len", "num_qk_heads", 128], axes, {"total_seq_len": 5}) == [5, 4, 128]
    with pytest.raises(KeyError):
        contest.resolve_shape(["total_seq_len"], axes, {})          # variable axis the workload leaves out
    with pytest.raises(KeyError):
        contest.resolve_shape(["no_such_axis"], axes, {})


def test_safetensors_inputs_round_trip(tmp_path):
    base, bundles = write_trace_set(tmp_path)
    p = bundles[contest.PREFILL][0]
    w = contest.load_workloads(base, contest.PREFILL)
    got = contest.workload_inputs(contest.load_definition(base, contest.PREFILL), w[0], base)
    assert list(got) == list(PREFILL_DEF["inputs"])
    for n in ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b", "cu_seqlens"):
        assert got[n].dtype == getattr(p, n).dtype, n
        assert torch.equal(got[n], getattr(p, n)), n
    assert got["scale"] == 0.25
    none = contest.workload_inputs(contest.load_definition(base, contest.PREFILL), w[1], base)
    assert none["state"] is None


def test_random_inputs_follow_the_definition(tmp_path):
    base, _ = write_trace_set(tmp_path)
    d = contest.load_definition(base, contest.DECODE)
    w = contest.load_workloads(base, contest.DECODE)[1]
    a = contest.workload_inputs(d, w, base, seed=5)
    b = contest.workload_inputs(d, w, base, seed=5)
    c = contest.workload_inputs(d, w, base, seed=6)
    assert a["q"].shape == (2, 1, 4, 128) and a["q"].dtype == torch.bfloat16
    assert a["state"].shape == (2, 8, 128, 128) and a["state"].dtype == torch.float32
    assert a["scale"] is None                        # the workload gives no scale
    assert all(torch.equal(a[n], b[n]) for n in ("q", "state", "a"))
    assert not torch.equal(a["q"], c["q"])


def test_random_integer_and_bool_ranges():
    g = torch.Generator("cpu").manual_seed(0)
    x = contest._random([4096], torch.int32, g)
    assert x.dtype == torch.int32 and int(x.min()) >= -16 and int(x.max()) <= 15
    m = contest._random([256], torch.bool, g)
    assert m.dtype == torch.bool and 0 < int(m.sum()) < 256


def test_mismatched_file_shape_and_bad_inputs(tmp_path):
    base, _ = write_trace_set(tmp_path)
    d = contest.load_definition(base, contest.PREFILL)
    w = json.loads(json.dumps(contest.load_workloads(base, contest.PREFILL)[0]))
    w["axes"]["total_seq_len"] = 104                  # the files hold 103 tokens
    with pytest.raises(ValueError):
        contest.workload_inputs(d, w, base)
    w = json.loads(json.dumps(contest.load_workloads(base, contest.PREFILL)[0]))
    w["inputs"]["scale"] = {"type": "random"}
    with pytest.raises(ValueError):
        contest.workload_inputs(d, w, base)
    w["inputs"]["scale"] = {"type": "url", "value": "x"}
    with pytest.raises(ValueError):
        contest.workload_inputs(d, w, base)
    bad = json.loads(json.dumps(DECODE_DEF))
    bad["inputs"]["q"]["dtype"] = "float8"
    with pytest.raises(ValueError):
        contest.workload_inputs(bad, contest.load_workloads(base, contest.DECODE)[0], base)


def test_entry_points():
    assert contest.entry_point(contest.DECODE) is decode.launch_gdn
    assert contest.entry_point(contest.PREFILL) is prefill.launch_gdn
    with pytest.raises(KeyError):
        contest.entry_point("gdn_other")


def test_contest_check_tolerance_rule():
    # the reference harness's per-output rule: allclose(atol=rtol=1e-2), max abs
    # and max rel (denominator clamped at 1e-12)
    import contest_check

    ref = torch.tensor([1.0, 2.0, 0.0])
    e = contest_check._errors(ref, torch.tensor([1.005, 2.0, 0.0]))
    assert e["within_tolerance"] and abs(e["max_abs_error"] - 0.005) < 1e-6 and abs(e["max_rel_error"] - 0.005) < 1e-5
    e = contest_check._errors(ref, torch.tensor([1.05, 2.0, 0.0]))
    assert not e["within_tolerance"] and abs(e["max_abs_error"] - 0.05) < 1e-6
    e = contest_check._errors(ref, torch.tensor([1.0, 2.0, 0.005]))   # |x| <= atol near zero: within
    assert e["within_tolerance"] and e["max_rel_error"] > 1e6
    e = contest_check._errors(torch.empty(0), torch.empty(0))
    assert e["within_tolerance"]
