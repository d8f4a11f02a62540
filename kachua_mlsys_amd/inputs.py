"""Seeded synthetic inputs for the five benchmark configurations.

Everything is drawn on the CPU with ``torch.Generator("cpu").manual_seed(seed)``
so the CPU baseline and the GPU see identical bytes; callers move the tensors
to the device.  Draw order is fixed: lengths (varlen only) -> q -> k -> v ->
state -> A_log -> dt_bias -> a -> b.

* q, k: randn fp32, L2-normalised over the head dim, then bf16
* v, a, b: randn -> bf16
* state: 0.02 * randn fp32 (zeros where a config says so)
* A_log: U(-1, 1); dt_bias: 0.1 * randn
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

NUM_QK_HEADS = 4
NUM_V_HEADS = 8
HEAD_DIM = 128


def _unit_rows_bf16(shape, gen):
    x = torch.randn(shape, generator=gen, dtype=torch.float32)
    x = x / x.norm(dim=-1, keepdim=True)
    return x.to(torch.bfloat16)


def _params(gen, lead):
    A_log = torch.rand(NUM_V_HEADS, generator=gen) * 2.0 - 1.0
    dt_bias = torch.randn(NUM_V_HEADS, generator=gen) * 0.1
    a = torch.randn(lead + (NUM_V_HEADS,), generator=gen).to(torch.bfloat16)
    b = torch.randn(lead + (NUM_V_HEADS,), generator=gen).to(torch.bfloat16)
    return A_log, dt_bias, a, b


@dataclass
class DecodeInputs:
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    state: torch.Tensor
    A_log: torch.Tensor
    a: torch.Tensor
    dt_bias: torch.Tensor
    b: torch.Tensor
    scale: float

    def args(self):
        return (self.q, self.k, self.v, self.state, self.A_log, self.a, self.dt_bias, self.b,
                self.scale)

    def to(self, device):
        return DecodeInputs(*(t.to(device) if isinstance(t, torch.Tensor) else t
                              for t in self.args()))


@dataclass
class PrefillInputs:
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    state: torch.Tensor | None
    A_log: torch.Tensor
    a: torch.Tensor
    dt_bias: torch.Tensor
    b: torch.Tensor
    cu_seqlens: torch.Tensor
    scale: float

    def args(self):
        return (self.q, self.k, self.v, self.state, self.A_log, self.a, self.dt_bias, self.b,
                self.cu_seqlens, self.scale)

    def to(self, device):
        return PrefillInputs(*(t.to(device) if isinstance(t, torch.Tensor) else t
                               for t in self.args()))

    @property
    def lengths(self):
        cu = self.cu_seqlens.cpu().long()
        return (cu[1:] - cu[:-1]).tolist()


def decode_inputs(batch: int, seed: int = 0, zero_state: bool = False) -> DecodeInputs:
    """Decode config: q,k [B,1,4,128], v [B,1,8,128], state [B,8,128,128]."""
    gen = torch.Generator("cpu").manual_seed(seed)
    q = _unit_rows_bf16((batch, 1, NUM_QK_HEADS, HEAD_DIM), gen)
    k = _unit_rows_bf16((batch, 1, NUM_QK_HEADS, HEAD_DIM), gen)
    v = torch.randn((batch, 1, NUM_V_HEADS, HEAD_DIM), generator=gen).to(torch.bfloat16)
    state = torch.randn((batch, NUM_V_HEADS, HEAD_DIM, HEAD_DIM), generator=gen) * 0.02
    if zero_state:
        state.zero_()
    A_log, dt_bias, a, b = _params(gen, (batch, 1))
    return DecodeInputs(q, k, v, state, A_log, a, dt_bias, b, 1.0 / math.sqrt(HEAD_DIM))


def prefill_inputs_from_lengths(lengths, seed: int = 0, zero_state: bool = False,
                                gen: torch.Generator | None = None,
                                cu_dtype=torch.int32) -> PrefillInputs:
    """Prefill inputs for explicit per-sequence lengths (zero-length allowed)."""
    if gen is None:
        gen = torch.Generator("cpu").manual_seed(seed)
    lengths = [int(x) for x in lengths]
    T = sum(lengths)
    N = len(lengths)
    cu = torch.zeros(N + 1, dtype=torch.int64)
    if N:
        cu[1:] = torch.cumsum(torch.tensor(lengths, dtype=torch.int64), 0)
    q = _unit_rows_bf16((T, NUM_QK_HEADS, HEAD_DIM), gen)
    k = _unit_rows_bf16((T, NUM_QK_HEADS, HEAD_DIM), gen)
    v = torch.randn((T, NUM_V_HEADS, HEAD_DIM), generator=gen).to(torch.bfloat16)
    if zero_state:
        state = torch.zeros((N, NUM_V_HEADS, HEAD_DIM, HEAD_DIM))
    else:
        state = torch.randn((N, NUM_V_HEADS, HEAD_DIM, HEAD_DIM), generator=gen) * 0.02
    A_log, dt_bias, a, b = _params(gen, (T,))
    return PrefillInputs(q, k, v, state, A_log, a, dt_bias, b, cu.to(cu_dtype),
                         1.0 / math.sqrt(HEAD_DIM))


def loguniform_lengths(n: int, total: int, lo: int, hi: int, gen: torch.Generator):
    """n lengths ~ exp(U(ln lo, ln hi)), rescaled to sum exactly to ``total``.

    L' = floor(L * total / sum L); the remainder goes +1 to the largest
    fractional parts; every length is clamped to >= 1 (the excess is then taken
    back from the longest sequences so the sum stays ``total``).
    """
    u = torch.rand(n, generator=gen, dtype=torch.float64)
    L = torch.exp(math.log(lo) + u * (math.log(hi) - math.log(lo)))
    scaled = L * (total / L.sum())
    base = torch.floor(scaled).long()
    frac = scaled - base.double()
    rem = int(total - base.sum().item())
    if rem > 0:
        order = torch.argsort(frac, descending=True)
        base[order[:rem]] += 1
    base = base.clamp_min(1)
    excess = int(base.sum().item()) - total
    while excess > 0:
        i = int(torch.argmax(base).item())
        base[i] -= 1
        excess -= 1
    return base.tolist()


def prefill_config(cfg: int, seed: int = 0) -> PrefillInputs:
    """The three prefill configurations (2: T=1024 N=1; 3: 16-seq varlen 16k; 4: 512 short)."""
    gen = torch.Generator("cpu").manual_seed(seed)
    if cfg == 2:
        return prefill_inputs_from_lengths([1024], gen=gen, zero_state=True)
    if cfg == 3:
        lengths = loguniform_lengths(16, 16384, 128, 4096, gen)
        return prefill_inputs_from_lengths(lengths, gen=gen)
    if cfg == 4:
        lengths = torch.randint(4, 65, (512,), generator=gen).tolist()
        return prefill_inputs_from_lengths(lengths, gen=gen)
    raise ValueError(f"unknown prefill config {cfg}")


def decode_config(cfg: int, seed: int = 0) -> DecodeInputs:
    """Decode configurations 0 (B=1) and 1 (B=64)."""
    if cfg == 0:
        return decode_inputs(1, seed)
    if cfg == 1:
        return decode_inputs(64, seed)
    raise ValueError(f"unknown decode config {cfg}")
