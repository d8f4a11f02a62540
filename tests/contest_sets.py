"""Synthetic contest trace sets (definitions, workload lines, safetensors files)
in the layout kachua_mlsys_amd.contest reads, for the loader and parity tests.
The contest datasets themselves are not available offline; these definitions
name the same inputs, dtypes and axes as the reference's launch_gdn signatures."""

import json
from pathlib import Path

import torch
from safetensors.torch import save_file

from kachua_mlsys_amd.contest import DECODE, PREFILL
from kachua_mlsys_amd.inputs import decode_inputs, prefill_inputs_from_lengths

CONST = {"num_qk_heads": {"type": "const", "value": 4}, "num_v_heads": {"type": "const", "value": 8},
         "head_size": {"type": "const", "value": 128}}

DECODE_DEF = {
    "name": DECODE,
    "axes": dict(CONST, batch_size={"type": "var"}, seq_len={"type": "const", "value": 1}),
    "inputs": {
        "q": {"shape": ["batch_size", "seq_len", "num_qk_heads", "head_size"], "dtype": "bfloat16"},
        "k": {"shape": ["batch_size", "seq_len", "num_qk_heads", "head_size"], "dtype": "bfloat16"},
        "v": {"shape": ["batch_size", "seq_len", "num_v_heads", "head_size"], "dtype": "bfloat16"},
        "state": {"shape": ["batch_size", "num_v_heads", "head_size", "head_size"], "dtype": "float32"},
        "A_log": {"shape": ["num_v_heads"], "dtype": "float32"},
        "a": {"shape": ["batch_size", "seq_len", "num_v_heads"], "dtype": "bfloat16"},
        "dt_bias": {"shape": ["num_v_heads"], "dtype": "float32"},
        "b": {"shape": ["batch_size", "seq_len", "num_v_heads"], "dtype": "bfloat16"},
        "scale": {"shape": None, "dtype": "float32"},
    },
}

PREFILL_DEF = {
    "name": PREFILL,
    "axes": dict(CONST, total_seq_len={"type": "var"}, num_seqs={"type": "var"}, len_cu_seqlens={"type": "var"}),
    "inputs": {
        "q": {"shape": ["total_seq_len", "num_qk_heads", "head_size"], "dtype": "bfloat16"},
        "k": {"shape": ["total_seq_len", "num_qk_heads", "head_size"], "dtype": "bfloat16"},
        "v": {"shape": ["total_seq_len", "num_v_heads", "head_size"], "dtype": "bfloat16"},
        "state": {"shape": ["num_seqs", "num_v_heads", "head_size", "head_size"], "dtype": "float32"},
        "A_log": {"shape": ["num_v_heads"], "dtype": "float32"},
        "a": {"shape": ["total_seq_len", "num_v_heads"], "dtype": "bfloat16"},
        "dt_bias": {"shape": ["num_v_heads"], "dtype": "float32"},
        "b": {"shape": ["total_seq_len", "num_v_heads"], "dtype": "bfloat16"},
        "cu_seqlens": {"shape": ["len_cu_seqlens"], "dtype": "int64"},
        "scale": {"shape": None, "dtype": "float32"},
    },
}

TENSORS = ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b")


def _file_inputs(fname, tensors, keys, scale):
    inputs = {n: {"type": "safetensors", "path": f"blobs/{fname}", "tensor_key": n} for n in keys}
    inputs["scale"] = {"type": "scalar", "value": scale}
    return inputs


def write_trace_set(root: Path, nest: bool = True):
    """Definitions and two workloads per definition under ``root`` (under
    ``root/trace`` when nest).  Returns (trace-set root, {definition: [the
    input bundles behind each workload line, None for a random workload]})."""
    base = root / "trace" if nest else root
    (base / "blobs").mkdir(parents=True, exist_ok=True)
    for sub in ("definitions/gdn", "workloads/gdn"):
        (base / sub).mkdir(parents=True, exist_ok=True)
    (base / "definitions/gdn" / f"{DECODE}.json").write_text(json.dumps(DECODE_DEF))
    (base / "definitions/gdn" / f"{PREFILL}.json").write_text(json.dumps(PREFILL_DEF))

    d = decode_inputs(3, seed=41)
    save_file({n: getattr(d, n).contiguous() for n in TENSORS}, str(base / "blobs/decode_b3.safetensors"))
    dec_lines = [
        {"workload": {"axes": {"batch_size": 3}, "inputs": _file_inputs("decode_b3.safetensors", d, TENSORS, 0.0)}},
        {"workload": {"axes": {"batch_size": 2}, "inputs": {n: {"type": "random"} for n in TENSORS}}},
    ]
    p = prefill_inputs_from_lengths([70, 0, 33], seed=42, cu_dtype=torch.int64)
    blobs = {n: getattr(p, n).contiguous() for n in TENSORS}
    blobs["cu_seqlens"] = p.cu_seqlens.contiguous()
    save_file(blobs, str(base / "blobs/prefill_3seq.safetensors"))
    pre_inputs = _file_inputs("prefill_3seq.safetensors", p, TENSORS + ("cu_seqlens",), 0.25)
    pre_none = dict(pre_inputs)
    del pre_none["state"]            # a workload that leaves state out: state=None
    pre_lines = [
        {"workload": {"axes": {"total_seq_len": 103, "num_seqs": 3, "len_cu_seqlens": 4}, "inputs": pre_inputs}},
        {"workload": {"axes": {"total_seq_len": 103, "num_seqs": 3, "len_cu_seqlens": 4}, "inputs": pre_none}},
    ]
    with open(base / "workloads/gdn" / f"{DECODE}.jsonl", "w") as f:
        f.write("\n".join(json.dumps(x) for x in dec_lines) + "\n")
    with open(base / "workloads/gdn" / f"{PREFILL}.jsonl", "w") as f:
        f.write("\n".join(json.dumps(x) for x in pre_lines) + "\n")
    return base, {DECODE: [d, None], PREFILL: [p, p]}
