"""Decode entry point: drop-in for gdn_decode_qk4_v8_d128_k_last's launch_gdn.

Same argument order and destination-passing convention as the reference
(``solution/cuda/kernel.cu:982-994``; the harness wrapper ``binding.py:33-52``
allocates ``out [B, 8, 128] bf16`` and ``new_state = empty_like(state)``).
Differences, all compatible: ``out`` / ``new_state`` may be omitted and are
then allocated, both are returned, and ``scale`` is honoured (the reference
kernel multiplies by a hard-coded 1/sqrt(128), ``kernel.cu:25,457-460``).
"""

from __future__ import annotations

import torch

from . import _lib
from ._checks import as_tensor, check_device, check_tensor, ptr, resolve_scale

NUM_QK_HEADS = 4
NUM_V_HEADS = 8
HEAD_DIM = 128


def launch_gdn(q, k, v, state, A_log, a, dt_bias, b, scale=None, out=None, new_state=None,
               *, rows_per_wave: int = 0):
    """One decode step for B sequences on the current stream.

    q, k [B,1,4,128] bf16; v [B,1,8,128] bf16; state [B,8,128,128] fp32 (k-last);
    A_log, dt_bias [8] fp32; a, b [B,1,8] bf16.  Writes out [B,8,128] (or
    [B,1,8,128]) bf16 and new_state [B,8,128,128] fp32; returns (out, new_state).
    ``state`` is only read; in-place update (new_state is state) is rejected.
    """
    # common case first: tensors only, on the current GPU, outputs given ->
    # checks and launch in the C++ binding (no launch when anything differs;
    # then the checks below raise the descriptive error)
    if out is not None and new_state is not None and (scale is None or type(scale) in (float, int)):
        fast = _lib.load_binding()
        if fast is not None and type(q) is torch.Tensor:
            di = q.get_device()
            if di >= 0 and di == torch._C._cuda_getDevice():
                try:
                    st = fast.decode(q, k, v, state, A_log, a, dt_bias, b, 0.0 if scale is None else float(scale),
                                     out, new_state, rows_per_wave, torch._C._cuda_getCurrentRawStream(di), di)
                except TypeError:   # an argument that is not a tensor (DLPack producers)
                    st = fast.NOT_FAST
                if st != fast.NOT_FAST:
                    _lib.check(st, "gdn_decode_fwd")
                    return out, new_state
    q, k, v, state = (as_tensor(x, n) for x, n in ((q, "q"), (k, "k"), (v, "v"), (state, "state")))
    A_log, a, dt_bias, b = (as_tensor(x, n) for x, n in
                            ((A_log, "A_log"), (a, "a"), (dt_bias, "dt_bias"), (b, "b")))
    out, new_state = as_tensor(out, "out"), as_tensor(new_state, "new_state")
    if not isinstance(q, torch.Tensor):
        raise TypeError(f"q: expected a torch.Tensor, got {type(q).__name__}")
    dev = q.device
    if q.dim() != 4:
        raise ValueError(f"q: expected [B,1,4,128], got {tuple(q.shape)}")
    B = q.shape[0]
    check_tensor(q, "q", torch.bfloat16, (B, 1, NUM_QK_HEADS, HEAD_DIM), dev)
    check_tensor(k, "k", torch.bfloat16, (B, 1, NUM_QK_HEADS, HEAD_DIM), dev)
    check_tensor(v, "v", torch.bfloat16, (B, 1, NUM_V_HEADS, HEAD_DIM), dev)
    check_tensor(state, "state", torch.float32, (B, NUM_V_HEADS, HEAD_DIM, HEAD_DIM), dev)
    check_tensor(A_log, "A_log", torch.float32, (NUM_V_HEADS,), dev)
    check_tensor(dt_bias, "dt_bias", torch.float32, (NUM_V_HEADS,), dev)
    check_tensor(a, "a", torch.bfloat16, (B, 1, NUM_V_HEADS), dev)
    check_tensor(b, "b", torch.bfloat16, (B, 1, NUM_V_HEADS), dev)
    if out is None:
        out = torch.empty((B, NUM_V_HEADS, HEAD_DIM), dtype=torch.bfloat16, device=dev)
    elif tuple(out.shape) == (B, 1, NUM_V_HEADS, HEAD_DIM):
        check_tensor(out, "out", torch.bfloat16, (B, 1, NUM_V_HEADS, HEAD_DIM), dev)
    else:
        check_tensor(out, "out", torch.bfloat16, (B, NUM_V_HEADS, HEAD_DIM), dev)
    if new_state is None:
        new_state = torch.empty_like(state)
    check_tensor(new_state, "new_state", torch.float32, (B, NUM_V_HEADS, HEAD_DIM, HEAD_DIM), dev)
    if new_state.data_ptr() == state.data_ptr() and B > 0:
        raise ValueError("new_state must not alias state (in-place update is not supported)")
    if rows_per_wave not in (0, 16, 32):
        raise ValueError("rows_per_wave must be 0, 16 or 32")
    scale = resolve_scale(scale, HEAD_DIM)
    check_device(q, "q")
    if B == 0:
        return out, new_state
    lib = _lib.load()
    with torch.cuda.device(dev):
        stream = torch.cuda.current_stream(dev).cuda_stream
        status = lib.gdn_decode_fwd(ptr(q), ptr(k), ptr(v), ptr(state), ptr(A_log), ptr(a),
                                    ptr(dt_bias), ptr(b), scale, ptr(out), ptr(new_state), B,
                                    rows_per_wave, stream)
    _lib.check(status, "gdn_decode_fwd")
    return out, new_state
