"""HIP-graph capture of the drop-in calls.  A decode or prefill call captured
into a graph and replayed several times, with other eager calls and
synchronisations between the replays, gives the eager result bit for bit on
every replay.  The calls record no memset nodes: the planner clears its own
queue counters in-kernel, and the Python entry points only allocate."""

import pytest
import torch

from kachua_mlsys_amd import decode, prefill
from kachua_mlsys_amd.inputs import decode_inputs, prefill_inputs_from_lengths

pytestmark = pytest.mark.gpu

REPLAYS = 3


def _short_batch():
    g = torch.Generator().manual_seed(12)
    return [int(x) for x in torch.randint(1, 65, (70,), generator=g)]


@pytest.mark.parametrize("name,lengths,state_none", [
    ("segmented", [700, 64, 1300, 0, 200], False),   # plan in the prepass, split consumer, finish
    ("short", _short_batch(), False),                  # full-head consumer over the short list
    ("direct", [100, 28], False),                      # one launch, terms in LDS
    ("segmented state=None", [900, 300], True),
])
def test_prefill_graph_replays(gpu, name, lengths, state_none):
    p = prefill_inputs_from_lengths(lengths, seed=sum(lengths) % 101).to(gpu)
    state = None if state_none else p.state
    args = (p.q, p.k, p.v, state, p.A_log, p.a, p.dt_bias, p.b, p.cu_seqlens, p.scale)
    T, N = p.q.shape[0], p.cu_seqlens.numel() - 1
    print(f"[case] prefill graph replays: {name}, T={T}, N={N}", flush=True)
    o_ref, s_ref = prefill.launch_gdn(*args)
    torch.cuda.synchronize()

    out = torch.empty_like(o_ref)
    ns = torch.empty_like(s_ref)
    ws = torch.empty(prefill.workspace_bytes(N, T), dtype=torch.uint8, device=gpu)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        prefill.launch_gdn(*args, out, ns, workspace=ws)

    other = prefill_inputs_from_lengths([300, 5, 70], seed=5).to(gpu)
    for r in range(REPLAYS):
        out.fill_(7.0)
        ns.fill_(7.0)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, o_ref), f"{name}: replay {r} output differs from the eager call"
        assert torch.equal(ns, s_ref), f"{name}: replay {r} state differs from the eager call"
        prefill.launch_gdn(*other.args())   # eager work between the replays, its own workspace
        torch.cuda.synchronize()
    del graph


@pytest.mark.parametrize("B", [1, 64])
def test_decode_graph_replays(gpu, B):
    d = decode_inputs(B, seed=40 + B).to(gpu)
    print(f"[case] decode graph replays: B={B}", flush=True)
    o_ref, s_ref = decode.launch_gdn(*d.args())
    torch.cuda.synchronize()
    out = torch.empty_like(o_ref)
    ns = torch.empty_like(s_ref)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        decode.launch_gdn(*d.args(), out, ns)
    other = decode_inputs(3, seed=9).to(gpu)
    for r in range(REPLAYS):
        out.fill_(7.0)
        ns.fill_(7.0)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, o_ref), f"decode B={B}: replay {r} output differs from the eager call"
        assert torch.equal(ns, s_ref), f"decode B={B}: replay {r} state differs from the eager call"
        decode.launch_gdn(*other.args())
        torch.cuda.synchronize()
    del graph
