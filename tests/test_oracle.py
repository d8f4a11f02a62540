"""CPU tests that pin the oracle (oracle/gdn_oracle.py) before it judges the GPU.

* golden vectors written from the reference's own reference_torch_impl.run
  (tests/golden/make_golden.py) pin the fp32 restatements to ~1e-6;
* closed forms pin both the fp32 restatement and the fp64 statement
  (one-hot k, q so |k| = 1 exactly; b = +/-30 so beta rounds to 1 / 0;
  A_log = 3, a = 30 so g underflows to 0);
* the chunked y-space algebra that the HIP prefill implements is pinned to the
  fp64 token recurrence for several chunk sizes, ragged batches and empty
  sequences; resume and prefill->decode continuation are checked as well.
"""

from pathlib import Path

import numpy as np
import pytest
import torch

from kachua_mlsys_amd.inputs import (decode_inputs, loguniform_lengths, prefill_config,
                                     prefill_inputs_from_lengths)
from oracle.gdn_oracle import (chunk_step_f64, chunk_terms_f64, decode_f64, decode_ref,
                               gates_f64, gates_fp32, prefill_chunked_f64, prefill_f64,
                               prefill_ref)

GOLDEN = Path(__file__).resolve().parent / "golden"


def _bf(a):
    return torch.from_numpy(np.asarray(a).view(np.int16).copy()).view(torch.bfloat16)


def _f(a):
    return torch.from_numpy(np.asarray(a).copy())


# ---------------------------------------------------------------- goldens ----

@pytest.mark.parametrize("name", ["decode_c0", "decode_b2_scale"])
def test_decode_golden(name):
    z = np.load(GOLDEN / f"{name}.npz")
    o, s = decode_ref(_bf(z["q"]), _bf(z["k"]), _bf(z["v"]), _f(z["state"]), _f(z["A_log"]),
                      _bf(z["a"]), _f(z["dt_bias"]), _bf(z["b"]), float(z["scale"]))
    assert o.dtype == torch.float32 and tuple(o.shape) == z["out"].shape
    np.testing.assert_allclose(o.numpy(), z["out"], rtol=0, atol=2e-6)
    np.testing.assert_allclose(s.numpy(), z["new_state"], rtol=0, atol=2e-6)


def test_decode_golden_matches_config0_generator():
    # the committed c0 inputs are exactly what inputs.decode_config(0) draws
    z = np.load(GOLDEN / "decode_c0.npz")
    d = decode_inputs(1, seed=0)
    assert torch.equal(d.q, _bf(z["q"])) and torch.equal(d.state, _f(z["state"]))
    assert torch.equal(d.b, _bf(z["b"])) and torch.equal(d.A_log, _f(z["A_log"]))


def test_prefill_golden_ragged():
    z = np.load(GOLDEN / "prefill_ragged.npz")
    state = _bf(z["state_bf16"]).float()
    o, s = prefill_ref(_bf(z["q"]), _bf(z["k"]), _bf(z["v"]), state, _f(z["A_log"]), _bf(z["a"]),
                       _f(z["dt_bias"]), _bf(z["b"]), _f(z["cu_seqlens"]), None)
    ref_o = _bf(z["out"]).float()
    # per-token bf16 rounding: allow one bf16 ulp where fp32 op order differs
    assert (o.float() - ref_o).abs().max() <= 2e-3 * ref_o.abs().max()
    assert (o.float() != ref_o).float().mean() < 1e-3
    np.testing.assert_allclose(s.numpy(), z["new_state"], rtol=0, atol=2e-6)
    assert np.all(z["new_state"][0] == 0)        # empty first sequence -> zero state


def test_prefill_golden_no_state():
    z = np.load(GOLDEN / "prefill_t256_nostate.npz")
    o, s = prefill_ref(_bf(z["q"]), _bf(z["k"]), _bf(z["v"]), None, _f(z["A_log"]), _bf(z["a"]),
                       _f(z["dt_bias"]), _bf(z["b"]), _f(z["cu_seqlens"]), 0.0)
    ref_o = _bf(z["out"]).float()
    assert (o.float() - ref_o).abs().max() <= 2e-3 * ref_o.abs().max()
    np.testing.assert_allclose(s.numpy(), z["new_state"], rtol=0, atol=2e-6)


# ----------------------------------------------------------- closed forms ----

def _onehot_bf16(shape_lead, idx):
    x = torch.zeros(shape_lead + (128,), dtype=torch.bfloat16)
    x[..., idx] = 1.0
    return x


def _decode_case(B=2, b_val=30.0, A_log_val=0.0, a_val=0.0, seed=0):
    gen = torch.Generator().manual_seed(seed)
    k = _onehot_bf16((B, 1, 4), 5)
    q = k.clone()
    v = torch.randn((B, 1, 8, 128), generator=gen).to(torch.bfloat16)
    state = torch.randn((B, 8, 128, 128), generator=gen) * 0.1
    A_log = torch.full((8,), A_log_val)
    dt_bias = torch.zeros(8)
    a = torch.full((B, 1, 8), a_val).to(torch.bfloat16)
    b = torch.full((B, 1, 8), b_val).to(torch.bfloat16)
    return q, k, v, state, A_log, a, dt_bias, b


@pytest.mark.parametrize("impl", ["fp32", "fp64"])
def test_closed_form_beta1_unit_k_equals_q(impl):
    # beta = 1, q = k, |k| = 1  =>  S' k = v  =>  o = scale v (any S, g)
    q, k, v, state, A_log, a, dt_bias, b = _decode_case(b_val=30.0, A_log_val=0.5, a_val=0.7)
    fn = decode_ref if impl == "fp32" else decode_f64
    o, s = fn(q, k, v, state, A_log, a, dt_bias, b, 0.25)
    o = np.asarray(o, np.float64)
    np.testing.assert_allclose(o, 0.25 * v[:, 0].double().numpy(), atol=1e-6)


@pytest.mark.parametrize("impl", ["fp32", "fp64"])
def test_closed_form_g0(impl):
    # g -> 0 (A_log = 3, a = 30)  =>  S' = beta v k^T, o = scale beta (k.q) v
    q, k, v, state, A_log, a, dt_bias, b = _decode_case(b_val=0.0, A_log_val=3.0, a_val=30.0)
    fn = decode_ref if impl == "fp32" else decode_f64
    o, s = fn(q, k, v, state, A_log, a, dt_bias, b, None)
    beta = 0.5
    vv = v[:, 0].double().numpy()
    kk = np.repeat(k[:, 0].double().numpy(), 2, axis=1)
    np.testing.assert_allclose(np.asarray(s, np.float64), beta * vv[..., :, None] * kk[..., None, :], atol=1e-7)
    np.testing.assert_allclose(np.asarray(o, np.float64), (128 ** -0.5) * beta * vv, atol=1e-7)


@pytest.mark.parametrize("impl", ["fp32", "fp64"])
def test_closed_form_beta0(impl):
    # beta -> 0 (b = -30)  =>  S' = g S, o = scale g S q
    q, k, v, state, A_log, a, dt_bias, b = _decode_case(b_val=-30.0, A_log_val=-0.3, a_val=0.2)
    fn = decode_ref if impl == "fp32" else decode_f64
    o, s = fn(q, k, v, state, A_log, a, dt_bias, b, 1.0)
    g = np.exp(-np.exp(-0.3) * np.log1p(np.exp(np.float64(torch.tensor(0.2).to(torch.bfloat16).item()))))
    S = state.double().numpy()
    np.testing.assert_allclose(np.asarray(s, np.float64), g * S, rtol=2e-6, atol=1e-9)
    np.testing.assert_allclose(np.asarray(o, np.float64), g * S[..., :, 5], rtol=2e-6, atol=1e-9)


def test_closed_form_gva_permutation():
    # permuting q/k heads permutes the corresponding v-head pairs
    d = decode_inputs(1, seed=3)
    perm = [2, 0, 3, 1]
    vperm = [2 * p + j for p in perm for j in range(2)]
    o, s = decode_f64(d.q, d.k, d.v, d.state, d.A_log, d.a, d.dt_bias, d.b)
    o2, s2 = decode_f64(d.q[:, :, perm], d.k[:, :, perm], d.v[:, :, vperm], d.state[:, vperm],
                        d.A_log[vperm], d.a[:, :, vperm], d.dt_bias[vperm], d.b[:, :, vperm])
    np.testing.assert_allclose(o2, o[:, vperm], atol=1e-12)
    np.testing.assert_allclose(s2, s[:, vperm], atol=1e-12)


def test_softplus_threshold_semantics():
    # torch's softplus is the identity above 20; the fp64 statement agrees
    x = torch.tensor([-30.0, -1.0, 0.0, 5.0, 19.9, 20.0, 20.5, 40.0])
    g32, _ = gates_fp32(torch.zeros(1), x[:, None], torch.zeros(1), torch.zeros(len(x), 1))
    g64, _ = gates_f64(np.zeros(1), x[:, None].numpy(), np.zeros(1), np.zeros((len(x), 1)))
    np.testing.assert_allclose(g32.numpy(), g64, rtol=1e-6)
    np.testing.assert_allclose(g64[-1, 0], np.exp(-40.0), rtol=1e-12)


# ----------------------------------------------------- fp32 vs fp64 forms ----

def test_decode_fp32_matches_fp64():
    d = decode_inputs(4, seed=9)
    o, s = decode_ref(*d.args())
    o64, s64 = decode_f64(*d.args())
    np.testing.assert_allclose(o.numpy(), o64, atol=1e-6)
    np.testing.assert_allclose(s.numpy(), s64, atol=1e-6)


def test_prefill_fp32_matches_fp64():
    p = prefill_inputs_from_lengths([0, 3, 70, 1], seed=4)
    o, s, o32 = prefill_ref(*p.args(), return_fp32_out=True)
    o64, s64 = prefill_f64(*p.args())
    np.testing.assert_allclose(o32.numpy(), o64, atol=1e-6)
    np.testing.assert_allclose(s.numpy(), s64, atol=1e-6)
    # the bf16 output is the rounded fp32 output
    assert torch.equal(o, o32.to(torch.bfloat16))


def test_prefill_one_token_equals_decode():
    p = prefill_inputs_from_lengths([1, 1, 1], seed=2)
    o64, s64 = prefill_f64(*p.args())
    od, sd = decode_f64(p.q[:, None], p.k[:, None], p.v[:, None], p.state, p.A_log,
                        p.a[:, None], p.dt_bias, p.b[:, None])
    np.testing.assert_allclose(o64, od, atol=1e-12)
    np.testing.assert_allclose(s64, sd, atol=1e-12)


# ---------------------------------------------- chunked algebra invariants ----

@pytest.mark.parametrize("chunk", [1, 7, 16, 64])
def test_chunked_equals_token_recurrence(chunk):
    p = prefill_inputs_from_lengths([0, 1, 65, 130, 17], seed=chunk)
    o64, s64 = prefill_f64(*p.args())
    oc, sc = prefill_chunked_f64(*p.args(), chunk=chunk)
    np.testing.assert_allclose(oc, o64, atol=1e-10)
    np.testing.assert_allclose(sc, s64, atol=1e-10)


def test_chunked_strong_decay_is_finite():
    # gates that drive the cumulative decay far below fp32's range stay finite
    p = prefill_inputs_from_lengths([128], seed=1)
    p.A_log.fill_(2.0)
    p.a.fill_(15.0)
    o64, s64 = prefill_f64(*p.args())
    oc, sc = prefill_chunked_f64(*p.args(), chunk=64)
    assert np.isfinite(oc).all() and np.isfinite(sc).all()
    np.testing.assert_allclose(oc, o64, atol=1e-10)
    np.testing.assert_allclose(sc, s64, atol=1e-10)


def test_chunk_terms_brute_force():
    # Tb solves (I + N) Tb = diag(beta): check A Tb = diag(beta) on a tiny chunk
    rng = np.random.default_rng(0)
    c = 5
    kc = rng.standard_normal((c, 8))
    kc /= np.linalg.norm(kc, axis=1, keepdims=True)
    qc = rng.standard_normal((c, 8))
    gc = rng.uniform(0.2, 0.99, c)
    bc = rng.uniform(0.1, 0.9, c)
    Tb, Aqk, gam, tail = chunk_terms_f64(kc, qc, gc, bc)
    for t in range(c):
        for i in range(c):
            rho = np.prod(gc[i + 1:t + 1]) if i <= t else 0.0
            expect_aqk = rho * qc[t] @ kc[i] if i <= t else 0.0
            assert abs(Aqk[t, i] - expect_aqk) < 1e-12
    A = np.eye(c)
    for t in range(c):
        for i in range(t):
            A[t, i] = bc[t] * np.prod(gc[i + 1:t + 1]) * (kc[t] @ kc[i])
    np.testing.assert_allclose(A @ Tb, np.diag(bc), atol=1e-12)
    np.testing.assert_allclose(gam, np.cumprod(gc), rtol=1e-12)
    np.testing.assert_allclose(tail, np.cumprod(gc)[-1] / np.cumprod(gc), rtol=1e-12)


def test_resume_invariant():
    # prefill(A) then prefill(B, state) == prefill(A || B)
    p = prefill_inputs_from_lengths([150], seed=8)
    sl_a, sl_b = slice(0, 61), slice(61, 150)

    def part(sl, state):
        return prefill_f64(p.q[sl], p.k[sl], p.v[sl], state, p.A_log, p.a[sl], p.dt_bias, p.b[sl],
                           [0, sl.stop - sl.start], p.scale)

    o_all, s_all = prefill_f64(*p.args())
    o_a, s_a = part(sl_a, p.state)
    o_b, s_b = part(sl_b, s_a)
    np.testing.assert_allclose(np.concatenate([o_a, o_b]), o_all, atol=1e-12)
    np.testing.assert_allclose(s_b, s_all, atol=1e-12)


def test_chunk_step_linear_in_state():
    # one chunk step is affine in the incoming state: f(S1 + S2) = f(S1) + f(S2) - f(0)
    rng = np.random.default_rng(1)
    c = 64
    kc = rng.standard_normal((c, 128)); kc /= np.linalg.norm(kc, axis=1, keepdims=True)
    qc = rng.standard_normal((c, 128)); vc = rng.standard_normal((c, 128))
    terms = chunk_terms_f64(kc, qc, rng.uniform(0.3, 0.99, c), rng.uniform(0.1, 0.9, c))
    S1, S2 = rng.standard_normal((2, 128, 128)) * 0.1
    Z = np.zeros((128, 128))
    o1, s1 = chunk_step_f64(S1, kc, qc, vc, *terms, 0.1)
    o2, s2 = chunk_step_f64(S2, kc, qc, vc, *terms, 0.1)
    o0, s0 = chunk_step_f64(Z, kc, qc, vc, *terms, 0.1)
    o12, s12 = chunk_step_f64(S1 + S2, kc, qc, vc, *terms, 0.1)
    np.testing.assert_allclose(o12, o1 + o2 - o0, atol=1e-12)
    np.testing.assert_allclose(s12, s1 + s2 - s0, atol=1e-12)


# ------------------------------------------------------------ input recipes ----

def test_config_recipes():
    p3 = prefill_config(3)
    L = p3.lengths
    assert len(L) == 16 and sum(L) == 16384 and min(L) >= 1
    assert p3.cu_seqlens.dtype == torch.int32 and p3.state.shape == (16, 8, 128, 128)
    p4 = prefill_config(4)
    assert len(p4.lengths) == 512 and min(p4.lengths) >= 4 and max(p4.lengths) <= 64
    p2 = prefill_config(2)
    assert p2.lengths == [1024] and float(p2.state.abs().max()) == 0.0
    qn = p3.q.float().norm(dim=-1)
    assert float((qn - 1).abs().max()) < 1e-2


def test_loguniform_lengths_exact_sum():
    gen = torch.Generator().manual_seed(5)
    for total in (16, 100, 16384):
        L = loguniform_lengths(16, total, 128, 4096, gen)
        assert sum(L) == total and min(L) >= 1
