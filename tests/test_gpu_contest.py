"""Contest trace sets through the HIP path: workloads read by
kachua_mlsys_amd.contest (safetensors inputs, a scalar scale, a missing
state) run through launch_gdn on the GPU and match the fp32 oracle; every
workload of a trace set is checked under the reference harness's rule
(contest_check)."""

import os

import pytest
import torch

import contest_check
from contest_sets import write_trace_set
from gpu_util import assert_parity
from kachua_mlsys_amd import contest
from oracle.gdn_oracle import decode_ref, prefill_ref

pytestmark = pytest.mark.gpu


def test_contest_decode_workload(gpu, tmp_path):
    base, bundles = write_trace_set(tmp_path)
    d = bundles[contest.DECODE][0]
    w = contest.load_workloads(base, contest.DECODE)[0]
    inputs = contest.workload_inputs(contest.load_definition(base, contest.DECODE), w, base, device=gpu)
    print("[case] contest decode B=3 (safetensors, scale 0 -> default)", flush=True)
    out, ns = contest.call(contest.DECODE, inputs)
    torch.cuda.synchronize()
    o_ref, s_ref = decode_ref(*d.args())
    assert_parity(out, ns, o_ref, s_ref, "contest decode B=3")


@pytest.mark.parametrize("idx", [0, 1])
def test_contest_prefill_workloads(gpu, tmp_path, idx):
    base, bundles = write_trace_set(tmp_path)
    p = bundles[contest.PREFILL][idx]
    w = contest.load_workloads(base, contest.PREFILL)[idx]
    inputs = contest.workload_inputs(contest.load_definition(base, contest.PREFILL), w, base, device=gpu)
    print(f"[case] contest prefill workload {idx} (lengths [70, 0, 33], state {'given' if idx == 0 else 'None'})",
          flush=True)
    out, ns = contest.call(contest.PREFILL, inputs)
    torch.cuda.synchronize()
    p.scale = 0.25
    if idx == 1:
        p.state = None
    o_ref, s_ref, o32 = prefill_ref(*p.args(), return_fp32_out=True)
    assert_parity(out, ns, o32, s_ref, f"contest prefill workload {idx}")


def test_contest_every_workload_checked(gpu, tmp_path):
    # the per-workload check that precedes timing, over every workload of both
    # definitions of the synthetic trace set
    base, bundles = write_trace_set(tmp_path)
    for name in (contest.DECODE, contest.PREFILL):
        print(f"[case] contest check, every {name} workload", flush=True)
        results = contest_check.check_trace_set(base, name)
        assert len(results) == len(bundles[name])
        for r in results:
            print(f"[check] {name} #{r['workload_idx']}: max_abs {r['max_abs_error']:.3e} "
                  f"state_rel {r['state_rel_error']:.3e}", flush=True)
            assert r["within_tolerance"], r


@pytest.mark.skipif(not os.environ.get("FIB_DATASET_PATH"),
                    reason="contest dataset not present (FIB_DATASET_PATH unset); it is not available offline")
def test_contest_dataset_every_workload(gpu):
    bad = []
    for name in (contest.DECODE, contest.PREFILL):
        for r in contest_check.check_trace_set(os.environ["FIB_DATASET_PATH"], name):
            if not r["within_tolerance"]:
                bad.append((name, r["workload_idx"], r["max_abs_error"], r["state_rel_error"]))
    assert not bad, bad
