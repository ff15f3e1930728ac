"""Build recipe for the gfx950 kernel library ``libmi355_fused.so``.

Compiles every ``csrc/*.hip`` translation unit for gfx950 with hipcc (in
parallel, objects under ``_build/``) and links them into one shared library
next to this file, which ``_lib.py`` loads with ctypes.  Then builds the
host-side launchers (``csrc/torch_launchers.cpp``, a torch extension that
calls that library's C ABI) into ``_mi355_torch*.so`` beside it, and the
measurement-only probe library (``csrc/probe/*.hip``) that bench.py uses.
Cross-compiles on a machine without a GPU.

    python llm-inference-optimizer_amd/build.py
    python llm-inference-optimizer_amd/build.py --out /tmp/libmi355_fused.so   # the library alone, elsewhere
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
LIB_NAME = "libmi355_fused.so"
PROBE_NAME = "libmi355_probe.so"  # measurement-only probe kernels used by bench.py
EXT_NAME = "_mi355_torch"  # host-side launchers (torch extension over the C ABI)
ARCH = "gfx950"

# -packed-fp32-ops: keep hipcc from forming v_pk_{add,mul,fma}_f32, which
# have produced intermittent wrong results on the target pool.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _compile(src: Path, obj: Path, extra: list[str]) -> None:
    cmd = [hipcc(), *HIPCC_FLAGS, *extra, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{' '.join(cmd)}\n{res.stdout}{res.stderr}")


def build(out: Path | None = None, jobs: int | None = None) -> Path:
    """Compile and link the library; returns its path.  Always rebuilds.
    The default output also rebuilds the probe library and the torch
    launchers beside it."""
    out = Path(out) if out is not None else PKG_DIR / LIB_NAME
    objdir = PKG_DIR / "_build" / "default"
    objdir.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    objs = [objdir / (s.stem + ".o") for s in sources]
    jobs = jobs or min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda so: _compile(so[0], so[1], []), zip(sources, objs)))
    tmp = out.with_name(out.name + ".tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{res.stdout}{res.stderr}")
    os.replace(tmp, out)
    if out == PKG_DIR / LIB_NAME:
        build_probe()
        build_torch_ext()
    return out


def ext_path() -> Path:
    import sysconfig
    return PKG_DIR / (EXT_NAME + sysconfig.get_config_var("EXT_SUFFIX"))


def build_torch_ext() -> Path:
    """Build the host-side launchers: a CPython extension module that takes
    torch tensors and calls libmi355_fused.so's C ABI (linked beside it,
    found through an $ORIGIN rpath).  Host code only, compiled with g++."""
    import sysconfig

    import torch
    from torch.utils import cpp_extension

    out = ext_path()
    tmp = out.with_name(out.name + ".tmp")
    incs = [*cpp_extension.include_paths(device_type="cuda"), sysconfig.get_paths()["include"]]
    libdirs = cpp_extension.library_paths(device_type="cuda")
    cmd = [shutil.which("g++") or "g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-fvisibility=hidden",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-DTORCH_EXTENSION_NAME={EXT_NAME}",
           f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
           *[f"-I{i}" for i in incs], str(CSRC / "torch_launchers.cpp"), "-o", str(tmp),
           f"-L{PKG_DIR}", "-lmi355_fused", *[f"-L{d}" for d in libdirs],
           "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python", "-lc10_hip", "-ltorch_hip",
           "-Wl,-rpath,$ORIGIN", *[f"-Wl,-rpath,{d}" for d in libdirs]]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"torch launcher build failed:\n{' '.join(cmd)}\n{res.stdout}{res.stderr}")
    os.replace(tmp, out)
    return out


def build_probe() -> Path:
    """Build the measurement-only probes bench.py uses (csrc/probe/*.hip: the
    streaming copy and read ceilings, the empty kernel, the int8 weight-stream
    probes of the decode decomposition)."""
    out = PKG_DIR / PROBE_NAME
    tmp = out.with_name(out.name + ".tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, "-shared", *map(str, sorted((CSRC / "probe").glob("*.hip"))), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"probe build failed:\n{' '.join(cmd)}\n{res.stdout}{res.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    args = sys.argv[1:]
    out = None
    if "--out" in args:
        i = args.index("--out")
        out = Path(args[i + 1])
        del args[i : i + 2]
    if args:
        sys.exit(f"unknown arguments {args}; usage: build.py [--out PATH]")
    print(build(out))
