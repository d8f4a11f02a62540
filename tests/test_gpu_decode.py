"""GPU parity of the HIP decode kernel (through the C ABI) against the oracle."""

from pathlib import Path

import numpy as np
import pytest
import torch

from gpu_util import assert_parity
from kachua_mlsys_amd import decode
from kachua_mlsys_amd.inputs import decode_config, decode_inputs
from oracle.gdn_oracle import decode_ref

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


def _run(d, dev, **kw):
    out, ns = decode.launch_gdn(*d.to(dev).args(), **kw)
    torch.cuda.synchronize()
    return out, ns


@pytest.mark.parametrize("cfg", [0, 1])
@pytest.mark.parametrize("rows", [0, 16, 32])
def test_decode_configs(gpu, cfg, rows):
    d = decode_config(cfg)
    o_ref, s_ref = decode_ref(*d.args())
    out, ns = _run(d, gpu, rows_per_wave=rows)
    assert out.dtype == torch.bfloat16 and tuple(out.shape) == tuple(o_ref.shape)
    assert_parity(out, ns, o_ref, s_ref, f"decode c{cfg} rows={rows}")


@pytest.mark.parametrize("B", [2, 3, 7, 33])
def test_decode_batch_sizes(gpu, B):
    d = decode_inputs(B, seed=100 + B)
    o_ref, s_ref = decode_ref(*d.args())
    out, ns = _run(d, gpu)
    assert_parity(out, ns, o_ref, s_ref, f"decode B={B}")


def test_decode_golden_c0(gpu):
    z = np.load(GOLDEN / "decode_c0.npz")

    def bf(x):
        return torch.from_numpy(x.view(np.int16).copy()).view(torch.bfloat16).to(gpu)

    def f(x):
        return torch.from_numpy(np.asarray(x).copy()).to(gpu)

    out, ns = decode.launch_gdn(bf(z["q"]), bf(z["k"]), bf(z["v"]), f(z["state"]), f(z["A_log"]),
                                bf(z["a"]), f(z["dt_bias"]), bf(z["b"]), float(z["scale"]))
    torch.cuda.synchronize()
    assert_parity(out, ns, torch.from_numpy(z["out"]), torch.from_numpy(z["new_state"]),
                  "decode golden c0")


@pytest.mark.parametrize("scale", [None, 0.0, 0.3, -1.5])
def test_decode_scale(gpu, scale):
    d = decode_inputs(4, seed=1)
    d.scale = scale
    o_ref, s_ref = decode_ref(*d.args())
    out, ns = _run(d, gpu)
    assert_parity(out, ns, o_ref, s_ref, f"decode scale={scale}")


@pytest.mark.parametrize("case", ["g0", "beta0", "beta1", "big_state"])
def test_decode_gate_extremes(gpu, case):
    d = decode_inputs(4, seed=2)
    if case == "g0":          # g underflows to 0: S' = beta v k^T
        d.A_log.fill_(3.0)
        d.a.fill_(30.0)
    elif case == "beta0":     # beta -> 0: S' = g S
        d.b.fill_(-30.0)
    elif case == "beta1":
        d.b.fill_(30.0)
    else:
        d.state.mul_(50.0)
    o_ref, s_ref = decode_ref(*d.args())
    out, ns = _run(d, gpu)
    assert_parity(out, ns, o_ref, s_ref, f"decode {case}")


def test_decode_out_4d_and_side_stream(gpu):
    d = decode_inputs(5, seed=3).to(gpu)
    out = torch.empty((5, 1, 8, 128), dtype=torch.bfloat16, device=gpu)
    ns = torch.empty_like(d.state)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        decode.launch_gdn(*d.args(), out, ns)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    o_ref, s_ref = decode_ref(*decode_inputs(5, seed=3).args())
    assert_parity(out.reshape(5, 8, 128), ns, o_ref, s_ref, "decode 4-D out on a side stream")


def test_decode_state_untouched_and_deterministic(gpu):
    d = decode_inputs(8, seed=4).to(gpu)
    before = d.state.clone()
    o1, s1 = decode.launch_gdn(*d.args())
    o2, s2 = decode.launch_gdn(*d.args())
    torch.cuda.synchronize()
    assert torch.equal(d.state, before)
    assert torch.equal(o1, o2) and torch.equal(s1, s2)


def test_decode_chain_matches_oracle_chain(gpu):
    # several steps with new_state fed back as state
    d = decode_inputs(3, seed=5)
    st_ref = d.state.clone()
    st = d.state.to(gpu)
    for step in range(4):
        dd = decode_inputs(3, seed=50 + step)
        o_ref, st_ref = decode_ref(dd.q, dd.k, dd.v, st_ref, d.A_log, dd.a, d.dt_bias, dd.b, None)
        g = dd.to(gpu)
        o, st = decode.launch_gdn(g.q, g.k, g.v, st, d.A_log.to(gpu), g.a, d.dt_bias.to(gpu), g.b, None)
    torch.cuda.synchronize()
    assert_parity(o, st, o_ref, st_ref, "decode 4-step chain")


def test_decode_torch_binding_path(gpu):
    # outputs given: the C++ binding checks and launches; without them the
    # Python checks run and ctypes launches.  Both give the same bytes.
    from kachua_mlsys_amd import _lib
    assert _lib.load_binding() is not None, "torch binding not built"
    d = decode_inputs(5, seed=17).to(gpu)
    o_slow, s_slow = decode.launch_gdn(*d.args())
    out = torch.empty((5, 8, 128), dtype=torch.bfloat16, device=gpu)
    ns = torch.empty_like(d.state)
    o_fast, s_fast = decode.launch_gdn(*d.args(), out, ns)
    torch.cuda.synchronize()
    assert o_fast is out and s_fast is ns
    assert torch.equal(o_fast.view(torch.int16), o_slow.view(torch.int16)) and torch.equal(s_fast, s_slow)
    # an argument outside the common case still gets the descriptive error
    with pytest.raises(TypeError, match="q: expected dtype"):
        decode.launch_gdn(d.q.float(), *d.args()[1:], out, ns)


# Seeded random decode steps: batch size, wave shape, gate regime (default,
# near-1 decay, strong decay with beta near 0 or 1), state magnitude, value
# range and scale, all drawn from the seed; each step is compared with the
# oracle at the usual bar.
def _random_decode(seed):
    gen = torch.Generator("cpu").manual_seed(20_000 + seed)
    B = int(torch.randint(1, 97, (1,), generator=gen))
    d = decode_inputs(B, seed=30_000 + seed)
    regime = int(torch.randint(0, 4, (1,), generator=gen))
    if regime == 1:     # near-1 decay
        d.A_log = torch.empty(8).uniform_(-8.0, -5.0, generator=gen)
    elif regime == 2:   # strong decay, beta close to 1
        d.A_log = torch.empty(8).uniform_(1.0, 2.5, generator=gen)
        d.b = d.b.float().add(6.0).to(torch.bfloat16)
    elif regime == 3:   # beta close to 0
        d.b = d.b.float().sub(8.0).to(torch.bfloat16)
    d.state = d.state * float(10.0 ** torch.empty(1).uniform_(-2.0, 2.0, generator=gen))
    d.v = (d.v.float() * float(10.0 ** torch.empty(1).uniform_(-1.0, 1.0, generator=gen))).to(torch.bfloat16)
    d.scale = float(torch.empty(1).uniform_(0.05, 0.2, generator=gen))
    rows = (0, 16, 32)[int(torch.randint(0, 3, (1,), generator=gen))]
    return d, rows, f"random decode seed={seed}: B={B} regime={regime} rows={rows}"


@pytest.mark.parametrize("seed", range(12))
def test_decode_random_steps(gpu, seed):
    d, rows, label = _random_decode(seed)
    print(f"[case] {label}", flush=True)
    o_ref, s_ref = decode_ref(*d.args())
    out, ns = _run(d, gpu, rows_per_wave=rows)
    assert_parity(out, ns, o_ref, s_ref, label)
