"""Prefill entry point: drop-in for gdn_prefill_qk4_v8_d128_k_last's launch_gdn.

Same signature, argument order and None-handling as the reference
(``solution/triton/kernel.py:56-91``): ``output`` / ``new_state`` of None are
allocated, ``state`` of None means zeros, ``scale`` of None or 0 means
1/sqrt(128); ``(output, new_state)`` is returned.  Like the reference it reads
only shapes on the host (no ``.item()``, no synchronisation); the record plan is
built on the device from ``cu_seqlens``.  An empty sequence gets
``new_state = 0`` as in the oracle (``reference_torch_impl.py:45-55``).
"""

from __future__ import annotations

import torch

from . import _lib
from ._checks import as_tensor, check_device, check_tensor, ptr, resolve_scale

NUM_QK_HEADS = 4
NUM_V_HEADS = 8
HEAD_DIM = 128


def workspace_bytes(num_seqs: int, total_tokens: int) -> int:
    """Default workspace size (what launch_gdn allocates when none is given)."""
    return int(_lib.load().gdn_prefill_workspace_bytes(int(num_seqs), int(total_tokens)))


def workspace_min_bytes(num_seqs: int, total_tokens: int) -> int:
    """Smallest accepted workspace: no segment slots (long sequences then run
    their chunks one after the other); results are the same."""
    return int(_lib.load().gdn_prefill_workspace_min_bytes(int(num_seqs), int(total_tokens)))


def launch_gdn(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale=None, output=None,
               new_state=None, *, workspace=None):
    """Chunked prefill over a cu_seqlens ragged batch on the current stream.

    q, k [T,4,128] bf16; v [T,8,128] bf16; state [N,8,128,128] fp32 or None;
    A_log, dt_bias [8] fp32; a, b [T,8] bf16; cu_seqlens [N+1] int32/int64.
    ``workspace`` (optional) is a uint8 GPU tensor of at least
    ``workspace_min_bytes(N, T)`` bytes (``workspace_bytes(N, T)`` gives the
    default number of segment slots); by default one is taken from torch's
    caching allocator per call, as the reference does with torch.empty.
    """
    # common case first: tensors only, on the current GPU, outputs given ->
    # checks and launch in the C++ binding (no launch when anything differs;
    # then the checks below raise the descriptive error)
    if output is not None and new_state is not None and (scale is None or type(scale) in (float, int)):
        fast = _lib.load_binding()
        if fast is not None and type(q) is torch.Tensor:
            di = q.get_device()
            if di >= 0 and di == torch._C._cuda_getDevice():
                try:
                    st = fast.prefill(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens,
                                      0.0 if scale is None else float(scale), output, new_state, workspace,
                                      torch._C._cuda_getCurrentRawStream(di), di)
                except TypeError:   # an argument that is not a tensor (DLPack producers)
                    st = fast.NOT_FAST
                if st != fast.NOT_FAST:
                    _lib.check(st, "gdn_prefill_fwd")
                    return output, new_state
    q, k, v = as_tensor(q, "q"), as_tensor(k, "k"), as_tensor(v, "v")
    state = as_tensor(state, "state")
    A_log, a, dt_bias, b = (as_tensor(x, n) for x, n in
                            ((A_log, "A_log"), (a, "a"), (dt_bias, "dt_bias"), (b, "b")))
    cu_seqlens = as_tensor(cu_seqlens, "cu_seqlens")
    output, new_state = as_tensor(output, "output"), as_tensor(new_state, "new_state")
    if not isinstance(q, torch.Tensor):
        raise TypeError(f"q: expected a torch.Tensor, got {type(q).__name__}")
    dev = q.device
    if q.dim() != 3:
        raise ValueError(f"q: expected [T,4,128], got {tuple(q.shape)}")
    T = q.shape[0]
    check_tensor(q, "q", torch.bfloat16, (T, NUM_QK_HEADS, HEAD_DIM), dev)
    check_tensor(k, "k", torch.bfloat16, (T, NUM_QK_HEADS, HEAD_DIM), dev)
    check_tensor(v, "v", torch.bfloat16, (T, NUM_V_HEADS, HEAD_DIM), dev)
    check_tensor(A_log, "A_log", torch.float32, (NUM_V_HEADS,), dev)
    check_tensor(dt_bias, "dt_bias", torch.float32, (NUM_V_HEADS,), dev)
    check_tensor(a, "a", torch.bfloat16, (T, NUM_V_HEADS), dev)
    check_tensor(b, "b", torch.bfloat16, (T, NUM_V_HEADS), dev)
    if not isinstance(cu_seqlens, torch.Tensor) or cu_seqlens.dim() != 1 or cu_seqlens.numel() < 1:
        raise ValueError("cu_seqlens: expected a 1-D tensor [N+1]")
    if cu_seqlens.dtype not in (torch.int32, torch.int64):
        raise TypeError(f"cu_seqlens: expected int32 or int64, got {cu_seqlens.dtype}")
    check_tensor(cu_seqlens, "cu_seqlens", cu_seqlens.dtype, cu_seqlens.shape, dev)
    N = cu_seqlens.numel() - 1
    if output is None:
        output = torch.empty((T, NUM_V_HEADS, HEAD_DIM), dtype=torch.bfloat16, device=dev)
    check_tensor(output, "output", torch.bfloat16, (T, NUM_V_HEADS, HEAD_DIM), dev)
    if new_state is None:
        new_state = torch.empty((N, NUM_V_HEADS, HEAD_DIM, HEAD_DIM), dtype=torch.float32,
                                device=dev)
    check_tensor(new_state, "new_state", torch.float32, (N, NUM_V_HEADS, HEAD_DIM, HEAD_DIM), dev)
    if state is not None:
        check_tensor(state, "state", torch.float32, (N, NUM_V_HEADS, HEAD_DIM, HEAD_DIM), dev)
        if N > 0 and state.data_ptr() == new_state.data_ptr():
            raise ValueError("new_state must not alias state (in-place update is not supported)")
    scale = resolve_scale(scale, HEAD_DIM)
    check_device(q, "q")
    if N == 0:
        return output, new_state
    lib = _lib.load()
    if workspace is None:
        workspace = torch.empty(int(lib.gdn_prefill_workspace_bytes(N, T)), dtype=torch.uint8, device=dev)
    else:
        check_device(workspace, "workspace")
        need = int(lib.gdn_prefill_workspace_min_bytes(N, T))
        if workspace.dtype != torch.uint8 or not workspace.is_contiguous() or workspace.numel() < need:
            raise ValueError(f"workspace: need a contiguous uint8 tensor of >= {need} bytes")
    with torch.cuda.device(dev):
        stream = torch.cuda.current_stream(dev).cuda_stream
        status = lib.gdn_prefill_fwd(
            ptr(q), ptr(k), ptr(v), ptr(state), ptr(A_log), ptr(a), ptr(dt_bias), ptr(b),
            ptr(cu_seqlens), int(cu_seqlens.dtype == torch.int64), N, T, scale, ptr(output),
            ptr(new_state), ptr(workspace), workspace.numel(), stream)
    _lib.check(status, "gdn_prefill_fwd")
    return output, new_state
