"""Correctness of every workload of a contest trace set, checked before it is
timed.  Each workload runs through the HIP ``launch_gdn`` (read by
kachua_mlsys_amd.contest) and through the fp32 oracle on the CPU, and every
output is compared under the reference harness's rule
(``scripts/bench_fi_timing.py:241-312`` of both reference paths):
``torch.allclose`` with atol = rtol = 1e-2, with the max abs / max rel error
(denominator clamped at 1e-12) reported per output.  It also applies this
build's state bound: max |S - S_ref| / max |S_ref| <= 2e-3.

This is test infrastructure (it imports the oracle), so it lives with the
tests:

    python tests/contest_check.py --trace-set PATH [--definition NAME] [--workload-idx I]

prints one JSON line per workload and exits with status 1 if any workload is
outside tolerance.
"""

import argparse
import json
import os
import sys
from pathlib import Path

import torch

_ROOT = Path(__file__).resolve().parent.parent
if str(_ROOT) not in sys.path:
    sys.path.insert(0, str(_ROOT))

from kachua_mlsys_amd import contest  # noqa: E402
from oracle.gdn_oracle import decode_ref, prefill_ref  # noqa: E402

ATOL = 1e-2
RTOL = 1e-2
STATE_REL = 2e-3


def _errors(ref: torch.Tensor, got: torch.Tensor) -> dict:
    """The reference harness's per-output figures (``_tensor_errors`` and the
    allclose test of ``check_correctness``)."""
    ref_f = ref.detach().float().cpu()
    got_f = got.detach().float().cpu().reshape(ref_f.shape)
    if ref_f.numel() == 0:
        return {"max_abs_error": 0.0, "max_rel_error": 0.0, "within_tolerance": True}
    err = (got_f - ref_f).abs()
    return {
        "max_abs_error": float(err.max()),
        "max_rel_error": float((err / ref_f.abs().clamp_min(1e-12)).max()),
        "within_tolerance": bool(torch.allclose(got_f, ref_f, atol=ATOL, rtol=RTOL)),
    }


def _oracle(definition_name: str, inputs: dict):
    cpu = {k: (v.detach().cpu() if isinstance(v, torch.Tensor) else v) for k, v in inputs.items()}
    if isinstance(cpu.get("scale"), torch.Tensor):
        cpu["scale"] = float(cpu["scale"])
    if definition_name == contest.DECODE:
        return decode_ref(**cpu)
    o, s, _ = prefill_ref(**cpu, return_fp32_out=True)
    return o, s


def check_workload(definition_name: str, inputs: dict) -> dict:
    """One workload: the kernel once, the oracle once, the errors per output."""
    out, new_state = contest.call(definition_name, dict(inputs))
    torch.cuda.synchronize()
    o_ref, s_ref = _oracle(definition_name, inputs)
    per = {"output": _errors(o_ref, out), "new_state": _errors(s_ref, new_state)}
    s_ref_f = s_ref.detach().float()
    den = float(s_ref_f.abs().max()) if s_ref_f.numel() else 0.0
    num = float((new_state.detach().float().cpu() - s_ref_f).abs().max()) if s_ref_f.numel() else 0.0
    state_rel = num / den if den > 0.0 else num
    finite = bool(torch.isfinite(out.float()).all()) and bool(torch.isfinite(new_state).all())
    return {
        "max_abs_error": max(p["max_abs_error"] for p in per.values()),
        "max_rel_error": max(p["max_rel_error"] for p in per.values()),
        "state_rel_error": state_rel,
        "within_tolerance": finite and all(p["within_tolerance"] for p in per.values()) and state_rel <= STATE_REL,
        "atol": ATOL,
        "rtol": RTOL,
        "per_output": per,
    }


def check_trace_set(root, definition_name: str, idxs=None, device: str = "cuda") -> list:
    """Every workload (or those in ``idxs``) of one definition of a trace set."""
    root = contest.resolve_trace_set(root)
    definition = contest.load_definition(root, definition_name)
    workloads = contest.load_workloads(root, definition_name)
    results = []
    for i in (range(len(workloads)) if idxs is None else idxs):
        inputs = contest.workload_inputs(definition, workloads[i], root, device=device, seed=i)
        r = check_workload(definition_name, inputs)
        r.update({"definition": definition_name, "workload_idx": i, "axes": workloads[i].get("axes", {})})
        results.append(r)
    return results


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="check every contest workload against the oracle")
    ap.add_argument("--trace-set", default=os.environ.get("FIB_DATASET_PATH"),
                    help="trace-set directory (default: $FIB_DATASET_PATH)")
    ap.add_argument("--definition", default=None, choices=[contest.DECODE, contest.PREFILL],
                    help="one definition (default: both)")
    ap.add_argument("--workload-idx", type=int, default=-1, help="-1 checks every workload")
    args = ap.parse_args(argv)
    if not args.trace_set:
        ap.error("no trace set: pass --trace-set or set FIB_DATASET_PATH")
    if not torch.cuda.is_available():
        raise SystemExit("a GPU is required")
    ok = True
    for name in ([args.definition] if args.definition else [contest.DECODE, contest.PREFILL]):
        idxs = None if args.workload_idx < 0 else [args.workload_idx]
        for r in check_trace_set(args.trace_set, name, idxs):
            ok = ok and r["within_tolerance"]
            print(json.dumps(r), flush=True)
    return 0 if ok else 1


if __name__ == "__main__":
    raise SystemExit(main())
