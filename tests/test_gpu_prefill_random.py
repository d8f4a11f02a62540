"""GPU parity of the prefill path on seeded random batches.

Each case draws one batch from its seed: the number of sequences, a mix of
lengths (empty, one token, both sides of the 16-token block and 64-token
chunk boundaries, a few hundred, a few thousand tokens), the decay regime
(the default gate distribution, near-1 decay, or strong decay on half the
heads), the initial state (random, zero, or None), int32 or int64
cu_seqlens, and the output scale.  Between them the cases reach the direct
path, the short-sequence consumer, warm-up and M-run segments and the finish
in combinations that the hand-written cases do not list one by one.  Every
case is compared with the fp32 oracle at the same bar as the other prefill
tests (outputs allclose 1e-2 / 1e-2, states 2e-3 relative); the per-token
oracle keeps each batch below ~8k tokens so that all cases run in seconds.
"""

import pytest
import torch

from gpu_util import assert_parity
from kachua_mlsys_amd import prefill
from kachua_mlsys_amd.inputs import prefill_inputs_from_lengths
from oracle.gdn_oracle import prefill_ref

BOUNDARY = [15, 16, 17, 31, 32, 33, 63, 64, 65, 127, 128, 129, 191, 192, 193]
MAX_TOKENS = 8000


def _draw_lengths(gen: torch.Generator, tiny: bool):
    def pick(lo, hi):
        return int(torch.randint(lo, hi + 1, (1,), generator=gen))

    if tiny:   # T <= 128 with at most 64 sequences: the single-launch direct path
        n = pick(1, 40)
        lengths = [pick(0, 6) for _ in range(n)]
        while sum(lengths) > 128:
            lengths[lengths.index(max(lengths))] -= 1
        return lengths
    n = pick(1, 24)
    lengths = []
    for _ in range(n):
        u = float(torch.rand(1, generator=gen))
        if u < 0.05:
            lengths.append(0)
        elif u < 0.10:
            lengths.append(1)
        elif u < 0.35:
            lengths.append(BOUNDARY[pick(0, len(BOUNDARY) - 1)])
        elif u < 0.65:
            lengths.append(pick(2, 200))
        elif u < 0.90:
            lengths.append(pick(200, 1500))
        else:
            lengths.append(pick(1500, 4000))
    while sum(lengths) > MAX_TOKENS:   # keep the oracle fast: trim the longest
        i = lengths.index(max(lengths))
        lengths[i] = max(lengths[i] // 2, 1)
    return lengths


def _draw_case(seed: int):
    gen = torch.Generator("cpu").manual_seed(10_000 + seed)
    tiny = seed % 5 == 4
    lengths = _draw_lengths(gen, tiny)
    cu64 = bool(torch.randint(0, 2, (1,), generator=gen))
    state_kind = ("random", "zero", "none")[int(torch.randint(0, 3, (1,), generator=gen))]
    decay = ("default", "near-1", "strong")[int(torch.randint(0, 3, (1,), generator=gen))]
    p = prefill_inputs_from_lengths(lengths, gen=gen, zero_state=state_kind == "zero",
                                    cu_dtype=torch.int64 if cu64 else torch.int32)
    if state_kind == "none":
        p.state = None
    if decay == "near-1":
        p.A_log = torch.empty(8).uniform_(-8.0, -5.0, generator=gen)
    elif decay == "strong":
        p.A_log[:4] = 2.0
        p.a[:, :4] = p.a[:, :4].float().add(6.0).to(torch.bfloat16)
    p.scale = float(torch.empty(1).uniform_(0.05, 0.2, generator=gen))
    label = (f"random seed={seed}: N={len(lengths)} T={sum(lengths)} state={state_kind} "
             f"decay={decay} cu64={cu64}")
    return p, label


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(15))
def test_prefill_random_batches(gpu, seed):
    p, label = _draw_case(seed)
    print(f"[case] {label}: lengths={p.lengths[:10]}{'...' if len(p.lengths) > 10 else ''}", flush=True)
    _, s_ref, o32 = prefill_ref(*p.args(), return_fp32_out=True)
    out, ns = prefill.launch_gdn(*p.to(gpu).args())
    torch.cuda.synchronize()
    assert_parity(out, ns, o32, s_ref, label)


def test_random_cases_reach_every_regime():
    """The seeds above cover the direct path, multi-chunk sequences, every
    decay regime and state kind, and both cu_seqlens widths (a CPU check of
    the draws themselves, so that a change to the generator cannot silently
    narrow the coverage)."""
    labels = [_draw_case(s)[1] for s in range(15)]
    cases = [_draw_case(s)[0] for s in range(15)]
    assert any(sum(c.lengths) <= 128 and len(c.lengths) <= 64 for c in cases)
    assert any(max(c.lengths) > 20 * 64 for c in cases)
    for word in ("state=random", "state=zero", "state=none", "decay=default", "decay=near-1",
                 "decay=strong", "cu64=True", "cu64=False"):
        assert any(word in lab for lab in labels), word
