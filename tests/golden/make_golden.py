"""Write golden vectors from the reference oracles (run in the build container only).

The closed forms and the fp64 recurrence in tests/test_oracle.py pin the math
of oracle/gdn_oracle.py, but not its bit-level conventions: operation order,
torch's softplus threshold, the per-token bf16 rounding of the prefill output
and the fp32 decode output.  This script imports the reference's own
``reference_torch_impl.run`` (decode and prefill) from /root/reference and
stores seeded inputs with its outputs as .npz fixtures next to this file.
Only the fixtures travel; the reference never does.

    python tests/golden/make_golden.py
"""

import importlib.util
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
sys.path.insert(0, str(REPO))
from kachua_mlsys_amd.inputs import decode_inputs, prefill_inputs_from_lengths  # noqa: E402

REF = Path("/root/reference")


def _load(path, name):
    spec = importlib.util.spec_from_file_location(name, str(path))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _np(t):
    if t is None:
        return None
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)   # raw bf16 bits
    return t.numpy()


def main():
    dec = _load(REF / "gdn_decode_qk4_v8_d128_k_last/solution/reference_torch_impl.py", "ref_decode")
    pre = _load(REF / "gdn_prefill_qk4_v8_d128_k_last/solution/reference_torch_impl.py", "ref_prefill")

    # decode: configuration 0 exactly (B=1, seed 0), and B=2 with scale 0.3
    for name, d in (("decode_c0", decode_inputs(1, seed=0)), ("decode_b2_scale", decode_inputs(2, seed=5))):
        scale = d.scale if name == "decode_c0" else 0.3
        o, s = dec.run(d.q, d.k, d.v, d.state, d.A_log, d.a, d.dt_bias, d.b, scale)
        np.savez_compressed(HERE / f"{name}.npz", q=_np(d.q), k=_np(d.k), v=_np(d.v), state=_np(d.state),
                            A_log=_np(d.A_log), a=_np(d.a), dt_bias=_np(d.dt_bias), b=_np(d.b),
                            scale=np.float64(scale), out=_np(o), new_state=_np(s))

    # prefill: lengths {0, 1, 71, 128} with a nonzero state (bf16-valued to keep the file small)
    p = prefill_inputs_from_lengths([0, 1, 71, 128], seed=11)
    state = p.state.to(torch.bfloat16).float()
    o, s = pre.run(p.q, p.k, p.v, state, p.A_log, p.a, p.dt_bias, p.b, p.cu_seqlens, None)
    np.savez_compressed(HERE / "prefill_ragged.npz", q=_np(p.q), k=_np(p.k), v=_np(p.v),
                        state_bf16=_np(state.to(torch.bfloat16)), A_log=_np(p.A_log), a=_np(p.a),
                        dt_bias=_np(p.dt_bias), b=_np(p.b), cu_seqlens=p.cu_seqlens.numpy(),
                        out=_np(o), new_state=_np(s))
    # prefill: one 256-token sequence, zero state given as None
    p = prefill_inputs_from_lengths([256], seed=12, zero_state=True)
    o, s = pre.run(p.q, p.k, p.v, None, p.A_log, p.a, p.dt_bias, p.b, p.cu_seqlens, 0.0)
    np.savez_compressed(HERE / "prefill_t256_nostate.npz", q=_np(p.q), k=_np(p.k), v=_np(p.v),
                        A_log=_np(p.A_log), a=_np(p.a), dt_bias=_np(p.dt_bias), b=_np(p.b),
                        cu_seqlens=p.cu_seqlens.numpy(), out=_np(o), new_state=_np(s))
    for f in sorted(HERE.glob("*.npz")):
        print(f.name, f.stat().st_size)


if __name__ == "__main__":
    main()
