"""Build and load ``libgdn_mi355x.so`` (the C ABI declared in include/gdn_mi355x.h).

The library is compiled in-tree with ``hipcc --offload-arch=gfx950`` and loaded
with ctypes.  Loaded after ``import torch`` it binds to the HIP runtime torch
already mapped (same soname), so torch's stream handles are valid in it.
There is no fallback: a missing library raises, it is never replaced by a CPU
or PyTorch path.
"""

from __future__ import annotations

import ctypes
import os
import shutil
import subprocess
import tempfile
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC_DIR = PKG_DIR / "csrc"
INCLUDE_DIR = REPO_DIR / "include"
LIB_DIR = PKG_DIR / "_lib"
LIB_PATH = LIB_DIR / "libgdn_mi355x.so"
SOURCES = ("gdn_decode.hip", "gdn_prefill.hip", "gdn_noalloc.hip", "gdn_capi.hip")
# bandwidth probe for bench.py (measurement only, not an entry point of the path)
PROBE_PATH = LIB_DIR / "libhbm_probe.so"
PROBE_SOURCES = ("hbm_stream.hip",)
ARCH = "gfx950"

# Every HIP translation unit is built with packed-fp32 instructions disabled.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-shared", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]

# exported symbol -> (restype, argtypes)
_VP = ctypes.c_void_p
SIGNATURES = {
    "gdn_abi_version": (ctypes.c_int, []),
    "gdn_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "gdn_decode_fwd": (ctypes.c_int, [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, ctypes.c_float,
                                      _VP, _VP, ctypes.c_int, ctypes.c_int, _VP]),
    "gdn_prefill_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int, ctypes.c_longlong]),
    "gdn_prefill_workspace_min_bytes": (ctypes.c_size_t, [ctypes.c_int, ctypes.c_longlong]),
    "gdn_prefill_fwd": (ctypes.c_int, [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, ctypes.c_int,
                                       ctypes.c_int, ctypes.c_longlong, ctypes.c_float, _VP, _VP,
                                       _VP, ctypes.c_size_t, _VP]),
    "gdn_prefill_fwd_noalloc": (ctypes.c_int, [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, ctypes.c_int,
                                               ctypes.c_int, ctypes.c_longlong, ctypes.c_float, _VP, _VP,
                                               _VP]),
}
ABI_VERSION = 2


def hipcc_path() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; the gfx950 library cannot be built")


def _compile(sources, target: Path, verbose: bool) -> Path:
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    fd, tmp = tempfile.mkstemp(prefix=target.stem + ".", suffix=".so.tmp", dir=LIB_DIR)
    os.close(fd)
    cmd = [hipcc_path(), *HIPCC_FLAGS, f"-I{INCLUDE_DIR}", "-o", tmp,
           *[str(CSRC_DIR / s) for s in sources]]
    try:
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stderr}")
        if verbose:
            print(" ".join(cmd))
        os.chmod(tmp, 0o755)   # readable by whoever runs it (the GPU box's user)
        os.replace(tmp, target)
    finally:
        if os.path.exists(tmp):
            os.unlink(tmp)
    return target


def binding_path() -> Path:
    import sysconfig

    return LIB_DIR / ("_gdn_torch" + sysconfig.get_config_var("EXT_SUFFIX"))


def build_binding(verbose: bool = False) -> Path:
    """Compile the torch binding (csrc/gdn_torch_binding.cpp) with the host
    compiler against torch's headers and LIB_PATH (found next to it at run time)."""
    import sysconfig

    import torch
    from torch.utils import cpp_extension

    target = binding_path()
    # a binding left from an earlier build must not outlive a failed rebuild
    # against a newer library
    target.unlink(missing_ok=True)
    fd, tmp = tempfile.mkstemp(prefix="_gdn_torch.", suffix=".so.tmp", dir=LIB_DIR)
    os.close(fd)
    cxx = shutil.which("c++") or shutil.which("g++")
    if cxx is None:
        raise RuntimeError("no host C++ compiler for the torch binding")
    cmd = [cxx, "-O2", "-std=c++17", "-shared", "-fPIC",
           "-DTORCH_EXTENSION_NAME=_gdn_torch", "-DTORCH_API_INCLUDE_EXTENSION_H",
           f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
           *[f"-isystem{d}" for d in cpp_extension.include_paths()],
           f"-isystem{sysconfig.get_paths()['include']}", f"-I{INCLUDE_DIR}",
           str(CSRC_DIR / "gdn_torch_binding.cpp"), "-o", tmp,
           *[f"-L{d}" for d in cpp_extension.library_paths()],
           "-lc10", "-ltorch_cpu", "-ltorch", "-ltorch_python",
           f"-L{LIB_DIR}", "-l:" + LIB_PATH.name, "-Wl,-rpath,$ORIGIN"]
    try:
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"torch binding build failed ({res.returncode}):\n{res.stderr}")
        if verbose:
            print(" ".join(cmd))
        os.chmod(tmp, 0o755)   # readable by whoever runs it (the GPU box's user)
        os.replace(tmp, target)
    finally:
        if os.path.exists(tmp):
            os.unlink(tmp)
    return target


def build(verbose: bool = False) -> Path:
    """Compile the HIP sources into LIB_PATH, the bandwidth probe into
    PROBE_PATH and the torch binding next to them (atomic replace of each)."""
    _compile(PROBE_SOURCES, PROBE_PATH, verbose)
    path = _compile(SOURCES, LIB_PATH, verbose)
    build_binding(verbose)
    return path


_LIB = None


def load() -> ctypes.CDLL:
    """Load the built library (raises if it was never built)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it first with "
            "`python -c 'import __graft_entry__ as g; g.build()'`")
    import torch  # noqa: F401  (map torch's HIP runtime before ours resolves it)
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    ver = lib.gdn_abi_version()
    if ver != ABI_VERSION:
        raise RuntimeError(f"{LIB_PATH} has ABI version {ver}, expected {ABI_VERSION}; rebuild it")
    _LIB = lib
    return lib


_BINDING = None


def load_binding():
    """The torch binding module (built by build()); None when it is not built
    or was built against another ABI version than the loaded library's, in
    which case the Python entry points validate and call the C ABI through
    ctypes themselves."""
    global _BINDING
    if _BINDING is None:
        path = binding_path()
        if not path.exists():
            _BINDING = False
        else:
            import importlib.util

            lib = load()   # the C library first: the binding resolves its symbols there
            spec = importlib.util.spec_from_file_location("_gdn_torch", path)
            mod = importlib.util.module_from_spec(spec)
            spec.loader.exec_module(mod)
            _BINDING = mod if getattr(mod, "ABI", None) == lib.gdn_abi_version() else False
    return _BINDING or None


_PROBE = None


def load_probe() -> ctypes.CDLL:
    """The bandwidth probe library (bench.py only)."""
    global _PROBE
    if _PROBE is None:
        if not PROBE_PATH.exists():
            raise RuntimeError(f"{PROBE_PATH} is missing: run build() first")
        import torch  # noqa: F401
        lib = ctypes.CDLL(str(PROBE_PATH))
        lib.hbm_stream_copy.restype = ctypes.c_int
        lib.hbm_stream_copy.argtypes = [_VP, _VP, ctypes.c_longlong, ctypes.c_int, ctypes.c_int, _VP]
        _PROBE = lib
    return _PROBE


def check(status: int, what: str) -> None:
    if status != 0:
        msg = load().gdn_status_string(status).decode()
        raise RuntimeError(f"{what} failed with status {status}: {msg}")


# ---- per-kernel resource report (compiler metadata of the built sources) ----

# gfx950 per-CU limits used to turn a kernel's resources into waves per SIMD
GFX950_VGPRS_PER_LANE = 512      # unified VGPR + AGPR file of a SIMD, per lane
GFX950_VGPR_GRANULE = 8
GFX950_LDS_BYTES = 160 * 1024
GFX950_MAX_WAVES_PER_SIMD = 8
GFX950_SIMDS_PER_CU = 4


def kernel_resources(sources=SOURCES) -> list[dict]:
    """Per kernel of the HIP sources: VGPRs (the unified count, AGPRs
    included), AGPRs, SGPRs, spills, LDS and scratch bytes per work-group, the
    launch bound on the block size, and the resident waves per SIMD that
    registers and LDS allow.  Read from the AMDGPU metadata hipcc emits for a
    device-only assembly build of each source (the same flags as the library)."""
    import re

    rows = []
    with tempfile.TemporaryDirectory() as td:
        for src in sources:
            out = Path(td) / (Path(src).stem + ".s")
            flags = [f for f in HIPCC_FLAGS if f not in ("-shared", "-fPIC")]
            cmd = [hipcc_path(), *flags, f"-I{INCLUDE_DIR}", "--cuda-device-only", "-S", "-o", str(out),
                   str(CSRC_DIR / src)]
            res = subprocess.run(cmd, capture_output=True, text=True)
            if res.returncode != 0:
                raise RuntimeError(f"hipcc failed on {src}:\n{res.stderr}")
            text = out.read_text()
            if "amdhsa.kernels:" not in text:
                continue
            meta = text[text.index("amdhsa.kernels:"):]
            for blk in meta.split("\n  - ")[1:]:
                def get(key, cast=str, default=None):
                    m = re.search(r"(?:^|\n)\s*" + re.escape(key) + r":\s*(\S+)", blk)
                    return cast(m.group(1)) if m else default
                name = get(".name")
                if name is None or name.startswith("__"):
                    continue
                vgpr = get(".vgpr_count", int, 0)
                agpr = get(".agpr_count", int, 0)
                lds = get(".group_segment_fixed_size", int, 0)
                block = get(".max_flat_workgroup_size", int, 1024)
                granted = -(-vgpr // GFX950_VGPR_GRANULE) * GFX950_VGPR_GRANULE
                by_vgpr = GFX950_VGPRS_PER_LANE // max(granted, GFX950_VGPR_GRANULE)
                waves_per_group = -(-block // 64)
                groups_by_lds = GFX950_LDS_BYTES // lds if lds else 1 << 30
                by_lds = groups_by_lds * waves_per_group / GFX950_SIMDS_PER_CU
                rows.append({
                    "source": src, "kernel": name, "vgpr": vgpr, "agpr": agpr,
                    "sgpr": get(".sgpr_count", int, 0),
                    "vgpr_spill": get(".vgpr_spill_count", int, 0),
                    "sgpr_spill": get(".sgpr_spill_count", int, 0),
                    "lds_bytes": lds, "scratch_bytes": get(".private_segment_fixed_size", int, 0),
                    "max_block": block,
                    "waves_per_simd": min(GFX950_MAX_WAVES_PER_SIMD, by_vgpr, int(by_lds)),
                    "waves_per_simd_by_vgpr": by_vgpr, "waves_per_simd_by_lds": by_lds,
                })
    return rows
