"""Tolerance checks shared by the GPU parity tests.

Tolerances (fixed here, from the north-star contract and the reference harness
rule scripts/bench_fi_timing.py:241-242,295):
  outputs : torch.allclose(out.float(), ref_fp32, atol=1e-2, rtol=1e-2)
  states  : max|S - S_ref| / max|S_ref| <= 2e-3
"""

import torch

OUT_ATOL = 1e-2
OUT_RTOL = 1e-2
STATE_REL = 2e-3


def state_rel(got: torch.Tensor, ref: torch.Tensor) -> float:
    got = got.detach().float().cpu()
    ref = ref.detach().float().cpu()
    den = float(ref.abs().max())
    num = float((got - ref).abs().max())
    if den == 0.0:
        return num
    return num / den


def assert_parity(out, new_state, ref_out32, ref_state, label=""):
    out = out.detach().float().cpu().reshape(ref_out32.shape)
    ref_out32 = ref_out32.float()
    assert torch.isfinite(out).all(), f"{label}: non-finite output"
    assert torch.isfinite(new_state.cpu()).all(), f"{label}: non-finite state"
    max_abs = float((out - ref_out32).abs().max()) if out.numel() else 0.0
    ok = torch.allclose(out, ref_out32, atol=OUT_ATOL, rtol=OUT_RTOL)
    srel = state_rel(new_state, ref_state)
    print(f"[parity] {label}: out max_abs={max_abs:.3e} state_rel={srel:.3e}", flush=True)
    assert ok, f"{label}: output outside atol/rtol 1e-2 (max_abs {max_abs:.3e})"
    assert srel <= STATE_REL, f"{label}: state rel error {srel:.3e} > {STATE_REL}"
    return max_abs, srel
