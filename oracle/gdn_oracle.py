"""CPU restatement of the reference GDN oracles (TEST INFRASTRUCTURE ONLY).

This module is the checker for the HIP product path and the CPU baseline that
``bench.py`` times.  It is never imported by ``kachua_mlsys_amd``.

Three families of functions live here:

* ``decode_ref`` / ``prefill_ref`` — fp32 torch restatements of the reference
  oracles, keeping their loop structure and operation order:
  ``gdn_decode_qk4_v8_d128_k_last/solution/reference_torch_impl.py:11-72`` and
  ``gdn_prefill_qk4_v8_d128_k_last/solution/reference_torch_impl.py:16-92``.
  Pinned by the golden vectors under ``tests/golden`` (written from the real
  reference) and by the closed forms / fp64 recurrence in ``tests/``.
* ``decode_f64`` / ``prefill_f64`` — an independent fp64 numpy statement of the
  same recurrence in rank-1 form ``S' = g S + beta (v - g S k) k^T``.  Pinned by
  the closed-form special cases in ``tests/test_oracle.py``.
* ``prefill_chunked_f64`` — the chunked "y-space" WY algebra that the HIP
  prefill kernels implement, in fp64.  It is not a reference function; the
  tests pin it to ``prefill_f64`` (equality to ~1e-10 for every chunk size).

Conventions shared with the reference: 4 q/k heads, 8 v heads, v-head ``h``
reads q/k head ``h // 2`` (``repeat_interleave``, decode ``:46-47``, prefill
``:38-39``); state is k-last ``[N, 8, V=128, K=128]`` fp32; ``scale`` of None or
0 means ``1/sqrt(128)`` (decode ``:32-33``, prefill ``:31-32``).
"""

from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

NUM_QK_HEADS = 4
NUM_V_HEADS = 8
HEAD_DIM = 128
GVA = NUM_V_HEADS // NUM_QK_HEADS


def _default_scale(scale, head_dim=HEAD_DIM):
    if scale is None or scale == 0.0:
        return 1.0 / math.sqrt(head_dim)
    return float(scale)


def gates_fp32(A_log, a, dt_bias, b):
    """Per-(token, v-head) decay g and write strength beta in fp32.

    g = exp(-exp(A_log) * softplus(a + dt_bias)), beta = sigmoid(b), with torch's
    softplus (threshold 20).  Reference: decode ``reference_torch_impl.py:36-38``,
    prefill ``reference_torch_impl.py:34-36``.
    """
    x = a.float() + dt_bias.float()
    g = torch.exp(-torch.exp(A_log.float()) * F.softplus(x))
    beta = torch.sigmoid(b.float())
    return g, beta


@torch.no_grad()
def decode_ref(q, k, v, state, A_log, a, dt_bias, b, scale=None):
    """fp32 restatement of the decode oracle (``reference_torch_impl.py:11-72``).

    q, k: [B,1,4,128] bf16; v: [B,1,8,128] bf16; state: [B,8,128,128] fp32 (k-last);
    A_log, dt_bias: [8] fp32; a, b: [B,1,8] bf16.
    Returns (out [B,8,128] fp32, new_state [B,8,128,128] fp32).  The reference
    returns the fp32 output (its bf16 cast is commented out, ``:71``).
    """
    B = q.shape[0]
    scale = _default_scale(scale, q.shape[-1])
    g, beta = gates_fp32(A_log, a, dt_bias, b)
    g = g[:, 0]        # [B, 8]
    beta = beta[:, 0]  # [B, 8]
    # GVA expansion: v-head h reads q/k head h // 2
    qh = q[:, 0].float().repeat_interleave(GVA, dim=1)   # [B, 8, K]
    kh = k[:, 0].float().repeat_interleave(GVA, dim=1)
    vh = v[:, 0].float()                                 # [B, 8, V]
    out = torch.empty(B, NUM_V_HEADS, v.shape[-1], dtype=torch.float32)
    new_state = torch.empty_like(state, dtype=torch.float32)
    for n in range(B):
        for h in range(NUM_V_HEADS):
            # [V,K] -> [K,V] view of this head's state, as the reference does
            hkv = state[n, h].float().clone().t()
            decayed = g[n, h] * hkv
            pred = kh[n, h] @ decayed                      # k^T (g S^T): [V]
            blended = beta[n, h] * vh[n, h] + (1 - beta[n, h]) * pred
            hkv = decayed - torch.outer(kh[n, h], pred) + torch.outer(kh[n, h], blended)
            out[n, h] = scale * (qh[n, h] @ hkv)
            new_state[n, h] = hkv.t()
    return out, new_state


@torch.no_grad()
def prefill_ref(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale=None,
                return_fp32_out=False):
    """fp32 restatement of the prefill oracle (``reference_torch_impl.py:16-92``).

    q, k: [T,4,128] bf16; v: [T,8,128] bf16; a, b: [T,8] bf16; state: [N,8,128,128]
    fp32 or None (zeros); cu_seqlens: [N+1] integer.  Token loop per sequence,
    vectorised over the 8 heads like the reference.  The output row of every
    token is rounded to bf16 (``:88``).  An empty sequence is skipped and its
    ``new_state`` stays zero (``:45-55``).

    With ``return_fp32_out`` the fp32 output before the bf16 rounding is
    returned as a third value (the tolerance check compares against it).
    """
    T = q.shape[0]
    assert q.shape[1] == NUM_QK_HEADS and k.shape[1] == NUM_QK_HEADS
    assert v.shape[1] == NUM_V_HEADS and q.shape[2] == HEAD_DIM
    cu = [int(x) for x in cu_seqlens.tolist()]
    N = len(cu) - 1
    scale = _default_scale(scale, q.shape[-1])
    g, beta = gates_fp32(A_log, a, dt_bias, b)               # [T, 8]
    qh = q.repeat_interleave(GVA, dim=1)                     # [T, 8, K] bf16
    kh = k.repeat_interleave(GVA, dim=1)
    out = torch.zeros(T, NUM_V_HEADS, HEAD_DIM, dtype=torch.bfloat16)
    out32 = torch.zeros(T, NUM_V_HEADS, HEAD_DIM, dtype=torch.float32) if return_fp32_out else None
    new_state = torch.zeros(N, NUM_V_HEADS, HEAD_DIM, HEAD_DIM, dtype=torch.float32)
    for s in range(N):
        t0, t1 = cu[s], cu[s + 1]
        if t1 <= t0:
            continue
        if state is not None:
            hkv = state[s].float().clone().transpose(-1, -2)   # [8, K, V]
        else:
            hkv = torch.zeros(NUM_V_HEADS, HEAD_DIM, HEAD_DIM, dtype=torch.float32)
        for t in range(t0, t1):
            k_row = kh[t].unsqueeze(1).float()          # [8, 1, K]
            q_row = qh[t].unsqueeze(1).float()
            v_row = v[t].unsqueeze(1).float()           # [8, 1, V]
            g_t = g[t].view(NUM_V_HEADS, 1, 1)
            b_t = beta[t].view(NUM_V_HEADS, 1, 1)
            decayed = g_t * hkv
            pred = k_row @ decayed                      # [8, 1, V]
            blended = b_t * v_row + (1.0 - b_t) * pred
            k_col = k_row.transpose(-1, -2)             # [8, K, 1]
            hkv = decayed - torch.bmm(k_col, pred) + torch.bmm(k_col, blended)
            o = (scale * (q_row @ hkv)).squeeze(1)      # [8, V]
            out[t] = o.to(torch.bfloat16)
            if out32 is not None:
                out32[t] = o
        new_state[s] = hkv.transpose(-1, -2)
    if return_fp32_out:
        return out, new_state, out32
    return out, new_state


# ----------------------------------------------------------------------------
# fp64 numpy statement of the same recurrence (rank-1 form)
# ----------------------------------------------------------------------------

def _softplus64(x):
    # torch semantics: identity above the threshold 20
    return np.where(x > 20.0, x, np.log1p(np.exp(np.minimum(x, 20.0))))


def gates_f64(A_log, a, dt_bias, b):
    x = np.asarray(a, np.float64) + np.asarray(dt_bias, np.float64)
    g = np.exp(-np.exp(np.asarray(A_log, np.float64)) * _softplus64(x))
    beta = 1.0 / (1.0 + np.exp(-np.asarray(b, np.float64)))
    return g, beta


def _np64(t):
    if isinstance(t, torch.Tensor):
        return t.detach().cpu().double().numpy()
    return np.asarray(t, np.float64)


def decode_f64(q, k, v, state, A_log, a, dt_bias, b, scale=None):
    """fp64: S' = g S + beta (v - g S k) k^T ; o = scale S' q (per batch, v-head)."""
    q, k, v, S = _np64(q)[:, 0], _np64(k)[:, 0], _np64(v)[:, 0], _np64(state)
    g, beta = gates_f64(_np64(A_log), _np64(a)[:, 0], _np64(dt_bias), _np64(b)[:, 0])
    scale = _default_scale(scale, q.shape[-1])
    kh = np.repeat(k, GVA, axis=1)          # [B, 8, K]
    qh = np.repeat(q, GVA, axis=1)
    Sd = g[:, :, None, None] * S            # [B, 8, V, K]
    pred = np.einsum("bhvk,bhk->bhv", Sd, kh)
    delta = beta[:, :, None] * (v - pred)
    Snew = Sd + delta[:, :, :, None] * kh[:, :, None, :]
    out = scale * np.einsum("bhvk,bhk->bhv", Snew, qh)
    return out, Snew


def prefill_f64(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale=None):
    """fp64 token recurrence over a cu_seqlens ragged batch.

    Returns (out [T,8,V] fp64, new_state [N,8,V,K] fp64); empty sequences give a
    zero state, matching the reference oracle.
    """
    q, k, v = _np64(q), _np64(k), _np64(v)
    cu = [int(x) for x in np.asarray(cu_seqlens).tolist()]
    N = len(cu) - 1
    g, beta = gates_f64(_np64(A_log), _np64(a), _np64(dt_bias), _np64(b))
    scale = _default_scale(scale, q.shape[-1])
    kh = np.repeat(k, GVA, axis=1)
    qh = np.repeat(q, GVA, axis=1)
    T = q.shape[0]
    out = np.zeros((T, NUM_V_HEADS, HEAD_DIM))
    new_state = np.zeros((N, NUM_V_HEADS, HEAD_DIM, HEAD_DIM))
    S_in = None if state is None else _np64(state)
    for s in range(N):
        t0, t1 = cu[s], cu[s + 1]
        if t1 <= t0:
            continue
        S = np.zeros((NUM_V_HEADS, HEAD_DIM, HEAD_DIM)) if S_in is None else S_in[s].copy()
        for t in range(t0, t1):
            S *= g[t][:, None, None]
            pred = np.einsum("hvk,hk->hv", S, kh[t])
            delta = beta[t][:, None] * (v[t] - pred)
            S += delta[:, :, None] * kh[t][:, None, :]
            out[t] = scale * np.einsum("hvk,hk->hv", S, qh[t])
        new_state[s] = S
    return out, new_state


# ----------------------------------------------------------------------------
# fp64 model of the chunked y-space WY algebra used by the HIP prefill kernels
# ----------------------------------------------------------------------------

def chunk_terms_f64(kc, qc, gc, bc):
    """State-independent terms of one chunk for one v-head (fp64).

    kc, qc: [c, K]; gc, bc: [c] (decay, beta).  With Gam_t = sum_{i<=t} log g_i:
      rho[t, i]  = exp(Gam_t - Gam_i)                      (bounded, <= 1 for i <= t)
      A          = I + strict_lower(beta_t rho[t,i] (k_t . k_i))
      Tb         = A^{-1} diag(beta)
      Aqk        = lower(rho[t,i] (q_t . k_i))              (diagonal included)
      gam        = exp(Gam), tail = exp(Gam_c - Gam)
    """
    c = kc.shape[0]
    Gam = np.cumsum(np.log(gc))
    strict = np.tril(np.ones((c, c)), -1)
    lower = np.tril(np.ones((c, c)))
    # only i <= t is ever used; exp is taken on the masked (<= 0) exponent so
    # the unused upper triangle cannot overflow
    rho = lower * np.exp(np.minimum(Gam[:, None] - Gam[None, :], 0.0))
    A = np.eye(c) + strict * (bc[:, None] * rho * (kc @ kc.T))
    Tb = np.linalg.solve(A, np.eye(c)) * bc[None, :]
    Aqk = lower * rho * (qc @ kc.T)
    gam = np.exp(Gam)
    tail = np.exp(Gam[-1] - Gam)
    return Tb, Aqk, gam, tail


def chunk_step_f64(S, kc, qc, vc, Tb, Aqk, gam, tail, scale):
    """Advance one v-head state S [V, K] over one chunk; returns (out [c,V], S').

      Delta = Tb (V_c - diag(gam) K S^T)
      O     = scale (diag(gam) Q S^T + Aqk Delta)
      S'    = gam_c S + (diag(tail) Delta)^T K
    """
    X = kc @ S.T
    Y = qc @ S.T
    Delta = Tb @ (vc - gam[:, None] * X)
    O = scale * (gam[:, None] * Y + Aqk @ Delta)
    S_new = gam[-1] * S + (tail[:, None] * Delta).T @ kc
    return O, S_new


def prefill_chunked_f64(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale=None,
                        chunk=64):
    """Chunked (y-space WY) evaluation of the prefill recurrence in fp64."""
    q, k, v = _np64(q), _np64(k), _np64(v)
    cu = [int(x) for x in np.asarray(cu_seqlens).tolist()]
    N = len(cu) - 1
    g, beta = gates_f64(_np64(A_log), _np64(a), _np64(dt_bias), _np64(b))
    scale = _default_scale(scale, q.shape[-1])
    T = q.shape[0]
    out = np.zeros((T, NUM_V_HEADS, HEAD_DIM))
    new_state = np.zeros((N, NUM_V_HEADS, HEAD_DIM, HEAD_DIM))
    S_in = None if state is None else _np64(state)
    for s in range(N):
        t0, t1 = cu[s], cu[s + 1]
        if t1 <= t0:
            continue
        for h in range(NUM_V_HEADS):
            hq = h // GVA
            S = np.zeros((HEAD_DIM, HEAD_DIM)) if S_in is None else S_in[s, h].copy()
            for c0 in range(t0, t1, chunk):
                c1 = min(c0 + chunk, t1)
                kc, qc, vc = k[c0:c1, hq], q[c0:c1, hq], v[c0:c1, h]
                Tb, Aqk, gam, tail = chunk_terms_f64(kc, qc, g[c0:c1, h], beta[c0:c1, h])
                O, S = chunk_step_f64(S, kc, qc, vc, Tb, Aqk, gam, tail, scale)
                out[c0:c1, h] = O
            new_state[s, h] = S
    return out, new_state
