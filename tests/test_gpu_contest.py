"""Contest trace sets through the HIP path: workloads read by
kachua_mlsys_amd.contest (safetensors inputs, a scalar scale, a missing
state) run through launch_gdn on the GPU and match the fp32 oracle."""

import pytest
import torch

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
