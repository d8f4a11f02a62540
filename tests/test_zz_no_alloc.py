"""GPU tests of gdn_prefill_fwd_noalloc (workspace from the library's static
device array) through the C ABI: two calls in a row, the second on a smaller
batch, each bit-identical to gdn_prefill_fwd with a default workspace and within
the oracle tolerance; and the call captured into a HIP graph after one eager
call on the device, every replay bit-identical to the eager result."""

import ctypes

import pytest
import torch

from gpu_util import assert_parity
from kachua_mlsys_amd import _lib, prefill
from kachua_mlsys_amd.inputs import prefill_inputs_from_lengths
from oracle.gdn_oracle import prefill_ref

pytestmark = pytest.mark.gpu


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _noalloc(lib, g, out, ns):
    T, N = g.q.shape[0], g.cu_seqlens.numel() - 1
    stream = torch.cuda.current_stream().cuda_stream
    return lib.gdn_prefill_fwd_noalloc(
        _ptr(g.q), _ptr(g.k), _ptr(g.v), _ptr(g.state), _ptr(g.A_log), _ptr(g.a), _ptr(g.dt_bias), _ptr(g.b),
        _ptr(g.cu_seqlens), int(g.cu_seqlens.dtype == torch.int64), N, T, float(g.scale), _ptr(out), _ptr(ns),
        ctypes.c_void_p(stream))


@pytest.mark.parametrize("run", [0])
def test_prefill_noalloc_two_calls(gpu, run):
    lib = _lib.load()
    for lengths, seed in (([3000, 1500, 700, 40], 61), ([300, 65, 1], 62)):
        print(f"[case] noalloc lengths={lengths}", flush=True)
        p = prefill_inputs_from_lengths(lengths, seed=seed)
        T, N = p.q.shape[0], len(lengths)
        assert prefill.workspace_bytes(N, T) <= (128 << 20)
        g = p.to(gpu)
        out = torch.full((T, 8, 128), float("nan"), dtype=torch.bfloat16, device=gpu)
        ns = torch.full((N, 8, 128, 128), float("nan"), device=gpu)
        st = _noalloc(lib, g, out, ns)
        assert st == 0, lib.gdn_status_string(st)
        ref_out, ref_ns = prefill.launch_gdn(*g.args())
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref_out.view(torch.int16)), "output differs from gdn_prefill_fwd"
        assert torch.equal(ns, ref_ns), "new_state differs from gdn_prefill_fwd"
        o_ref, s_ref, o32 = prefill_ref(*p.args(), return_fp32_out=True)
        assert_parity(out, ns, o32, s_ref, f"noalloc {lengths}")


def test_prefill_noalloc_graph_capture(gpu):
    # The first call on a device resolves the array's address (which can load
    # its code object), so it is made eagerly; the captured call then records
    # kernels only, and replays with other eager work in between match.
    lib = _lib.load()
    lengths = [900, 64, 1300, 0, 33]
    print(f"[case] noalloc graph capture lengths={lengths}", flush=True)
    p = prefill_inputs_from_lengths(lengths, seed=63)
    T, N = p.q.shape[0], len(lengths)
    g = p.to(gpu)
    ref_out = torch.empty((T, 8, 128), dtype=torch.bfloat16, device=gpu)
    ref_ns = torch.empty((N, 8, 128, 128), device=gpu)
    st = _noalloc(lib, g, ref_out, ref_ns)
    assert st == 0, lib.gdn_status_string(st)
    torch.cuda.synchronize()
    out = torch.empty_like(ref_out)
    ns = torch.empty_like(ref_ns)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        st = _noalloc(lib, g, out, ns)
    assert st == 0, lib.gdn_status_string(st)
    other = prefill_inputs_from_lengths([300, 5, 70], seed=5).to(gpu)
    oo = torch.empty((other.q.shape[0], 8, 128), dtype=torch.bfloat16, device=gpu)
    on = torch.empty((3, 8, 128, 128), device=gpu)
    for r in range(3):
        out.fill_(7.0)
        ns.fill_(7.0)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref_out.view(torch.int16)), f"replay {r}: output differs"
        assert torch.equal(ns, ref_ns), f"replay {r}: new_state differs"
        # eager work between replays, through the same device array
        assert _noalloc(lib, other, oo, on) == 0
        torch.cuda.synchronize()
    del graph
