"""Contest trace sets -> ``launch_gdn`` calls.

A trace set is a directory holding ``definitions/**/<name>.json`` and
``workloads/**/<name>.jsonl`` (or one level above such a directory).  A
definition names its inputs with a dtype and a shape over named axes; a const
axis carries its value in the definition, a variable axis takes it from the
workload.  Each workload line is ``{"workload": {"axes": {...}, "inputs":
{...}}}`` with, per input, one of ``{"type": "scalar", "value": v}``,
``{"type": "safetensors", "path": p, "tensor_key": key}`` (``p`` relative to
the trace-set root unless absolute) or ``{"type": "random"}``; an input the
workload leaves out is passed as None.  This follows the loader of the
reference's timing scripts
(``gdn_prefill_qk4_v8_d128_k_last/scripts/bench_fi_timing.py:49-211``, the
decode copy is the same): the same directory resolution, shape resolution,
dtype names and random distributions (randn for floating point, integers in
[-16, 16), booleans in {0, 1}).  Random inputs here come from a seeded
generator so a workload can be rerun.

Inputs reach the entry point by name (the definition's input names are the
``launch_gdn`` parameter names), so the order of a definition's inputs does
not matter.  Timing follows bench.py's protocol in miniature (HIP events
around each call, the caches flushed before it).  The parity check against
the reference's semantics lives in the tests (tests/test_gpu_contest.py); the
datasets themselves are not available offline.

Command line::

    python -m kachua_mlsys_amd.contest --trace-set PATH \\
        --definition gdn_prefill_qk4_v8_d128_k_last --workload-idx -1
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
from pathlib import Path

import torch

DTYPES = {
    "float32": torch.float32,
    "float16": torch.float16,
    "bfloat16": torch.bfloat16,
    "int8": torch.int8,
    "int16": torch.int16,
    "int32": torch.int32,
    "int64": torch.int64,
    "bool": torch.bool,
}

DECODE = "gdn_decode_qk4_v8_d128_k_last"
PREFILL = "gdn_prefill_qk4_v8_d128_k_last"


def _is_root(path: Path) -> bool:
    return (path / "definitions").is_dir() and (path / "workloads").is_dir()


def resolve_trace_set(path) -> Path:
    """The trace-set root: ``path`` itself or its first child holding
    definitions/ and workloads/."""
    root = Path(path).expanduser()
    if not root.exists():
        raise FileNotFoundError(f"trace set path does not exist: {root}")
    if _is_root(root):
        return root
    for child in sorted(root.iterdir()):
        if child.is_dir() and _is_root(child):
            return child
    raise FileNotFoundError(f"no definitions/ and workloads/ under {root} or one level below")


def _find(root: Path, sub: str, filename: str) -> Path:
    hits = sorted((root / sub).rglob(filename))
    if not hits:
        raise FileNotFoundError(f"{filename} not found under {root / sub}")
    return hits[0]


def load_definition(root: Path, name: str) -> dict:
    return json.loads(_find(root, "definitions", f"{name}.json").read_text())


def load_workloads(root: Path, name: str) -> list:
    """Every workload of ``name`` in file order (the ``workload`` objects)."""
    path = _find(root, "workloads", f"{name}.jsonl")
    out = []
    with open(path, encoding="utf-8") as f:
        for line in f:
            if line.strip():
                out.append(json.loads(line)["workload"])
    return out


def resolve_shape(spec, axes_def: dict, workload_axes: dict):
    """Concrete shape of one input (None for a scalar)."""
    if spec is None:
        return None
    shape = []
    for dim in spec:
        if isinstance(dim, int):
            shape.append(dim)
        elif dim in workload_axes:
            shape.append(int(workload_axes[dim]))
        else:
            ax = axes_def.get(dim)
            if not ax or ax.get("type") != "const":
                raise KeyError(f"cannot resolve axis {dim!r}: not in the workload and not a const axis")
            shape.append(int(ax["value"]))
    return shape


def _random(shape, dtype, generator):
    if dtype in (torch.float32, torch.float16, torch.bfloat16):
        return torch.randn(shape, generator=generator, dtype=torch.float32).to(dtype)
    if dtype is torch.bool:
        return torch.randint(0, 2, shape, generator=generator).to(torch.bool)
    return torch.randint(-16, 16, shape, generator=generator, dtype=torch.int64).to(dtype)


def workload_inputs(definition: dict, workload: dict, root: Path, device="cpu", seed: int = 0):
    """{input name: tensor, scalar or None} for one workload, in definition order."""
    from safetensors.torch import load_file   # plain tensor files: nothing in them executes

    gen = torch.Generator("cpu").manual_seed(seed)
    axes_def = definition.get("axes", {})
    waxes = workload.get("axes", {})
    winputs = workload.get("inputs", {})
    files = {}
    out = {}
    for name, idef in definition["inputs"].items():
        if idef["dtype"] not in DTYPES:
            raise ValueError(f"input {name!r}: unsupported dtype {idef['dtype']!r}")
        dtype = DTYPES[idef["dtype"]]
        shape = resolve_shape(idef.get("shape"), axes_def, waxes)
        src = winputs.get(name)
        if src is None:
            out[name] = None
        elif src["type"] == "scalar":
            out[name] = src["value"]
        elif src["type"] == "safetensors":
            path = Path(src["path"])
            if not path.is_absolute():
                path = root / path
            if path not in files:
                files[path] = load_file(str(path))
            t = files[path][src["tensor_key"]]
            if shape is not None and list(t.shape) != shape:
                raise ValueError(f"input {name!r}: file holds shape {list(t.shape)}, definition says {shape}")
            out[name] = t.to(device=device, dtype=dtype)
        elif src["type"] == "random":
            if shape is None:
                raise ValueError(f"input {name!r}: a random scalar is not supported")
            out[name] = _random(shape, dtype, gen).to(device)
        else:
            raise ValueError(f"input {name!r}: unsupported workload input type {src['type']!r}")
    return out


def entry_point(definition_name: str):
    """The ``launch_gdn`` that implements a definition."""
    from . import decode, prefill

    if definition_name == DECODE:
        return decode.launch_gdn
    if definition_name == PREFILL:
        return prefill.launch_gdn
    raise KeyError(f"no entry point for definition {definition_name!r}")


def call(definition_name: str, inputs: dict):
    """Run one workload; returns (output, new_state)."""
    return entry_point(definition_name)(**inputs)


def time_call(definition_name: str, inputs: dict, iters: int = 20, warmup: int = 3):
    """Median / min µs per call: HIP events around each call on the current
    stream, a 512 MiB buffer written before each call (cold L2 and MALL)."""
    fn = entry_point(definition_name)
    flush = torch.empty(512 << 20, dtype=torch.uint8, device="cuda")
    for _ in range(warmup):
        fn(**inputs)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    times = []
    for i in range(iters):
        flush.fill_(i & 0xff)
        start.record()
        fn(**inputs)
        end.record()
        torch.cuda.synchronize()
        times.append(start.elapsed_time(end) * 1e3)
    del flush
    return statistics.median(times), min(times)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="run contest trace-set workloads through launch_gdn")
    ap.add_argument("--trace-set", default=os.environ.get("FIB_DATASET_PATH"),
                    help="trace-set directory (default: $FIB_DATASET_PATH)")
    ap.add_argument("--definition", default=PREFILL, choices=[DECODE, PREFILL])
    ap.add_argument("--workload-idx", type=int, default=0, help="-1 runs every workload")
    ap.add_argument("--iters", type=int, default=20)
    args = ap.parse_args(argv)
    if not args.trace_set:
        ap.error("no trace set: pass --trace-set or set FIB_DATASET_PATH")
    if not torch.cuda.is_available():
        raise SystemExit("a GPU is required")
    root = resolve_trace_set(args.trace_set)
    definition = load_definition(root, args.definition)
    workloads = load_workloads(root, args.definition)
    idxs = range(len(workloads)) if args.workload_idx < 0 else [args.workload_idx]
    for i in idxs:
        inputs = workload_inputs(definition, workloads[i], root, device="cuda", seed=i)
        med, mn = time_call(args.definition, inputs, iters=args.iters)
        print(json.dumps({"definition": args.definition, "workload_idx": i, "axes": workloads[i].get("axes", {}),
                          "median_us": round(med, 3), "min_us": round(mn, 3)}), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
