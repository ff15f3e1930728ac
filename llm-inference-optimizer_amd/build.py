"""Build recipe for the gfx950 kernel library ``libmi355_fused.so``.

Compiles every ``csrc/*.hip`` translation unit for gfx950 with hipcc (in
parallel, objects under ``_build/``) and links them into one shared library
next to this file, which ``_lib.py`` loads with ctypes.  Then builds the
host-side launchers (``csrc/torch_launchers.cpp``, a torch extension that
calls that library's C ABI) into ``_mi355_torch*.so`` beside it.
Cross-compiles on a machine without a GPU.

    python llm-inference-optimizer_amd/build.py            # default build
    python llm-inference-optimizer_amd/build.py -DMI355_SILU_UNROLL=2 --out /tmp/x.so
    python llm-inference-optimizer_amd/build.py --variant rms_block_rows2 [...]
    python llm-inference-optimizer_amd/build.py --variant all

A *variant* (``VARIANTS`` below) is the library with one translation unit
rebuilt under other launch-shape switches, written to
``_variants/libmi355_fused_<name>.so``; ``bench.py --sweep <name>...`` times
its kernels beside the default build's.  The switches change how rows and
chunks are spread over waves and workgroups; the arithmetic is the same, and
the outputs are bit-identical to the default library's except where a
variant changes the order of a row's fp32 sum of squares
(``REORDERING_VARIANTS``).
"""
from __future__ import annotations

import concurrent.futures as cf
import hashlib
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
LIB_NAME = "libmi355_fused.so"
PROBE_NAME = "libmi355_probe.so"  # measurement-only copy kernel used by bench.py
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


def build(extra_flags: list[str] | None = None, out: Path | None = None, jobs: int | None = None) -> Path:
    """Compile and link the library; returns its path.  Always rebuilds."""
    extra = list(extra_flags or [])
    out = Path(out) if out is not None else PKG_DIR / LIB_NAME
    tag = hashlib.sha1(" ".join(extra).encode()).hexdigest()[:10] if extra else "default"
    objdir = PKG_DIR / "_build" / tag
    objdir.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    objs = [objdir / (s.stem + ".o") for s in sources]
    jobs = jobs or min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda so: _compile(so[0], so[1], extra), zip(sources, objs)))
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


# name -> (translation unit, -D switches).  The alternatives to the shipped
# launch shapes that the design measured, kept buildable so every A/B can be
# rerun from the repository.
VARIANTS = {
    # RMSNorm: rows held per wave / per workgroup iteration (loads of all of
    # them in flight before the first reduction)
    "rms_wave_rows2": ("rmsnorm", ["-DMI355_RMS_WAVE_ROWS=2"]),
    "rms_wave_rows4": ("rmsnorm", ["-DMI355_RMS_WAVE_ROWS=4"]),
    "rms_add_wave_rows1": ("rmsnorm", ["-DMI355_RMS_WAVE_ROWS_ADD=1"]),
    "rms_add_wave_rows4": ("rmsnorm", ["-DMI355_RMS_WAVE_ROWS_ADD=4"]),
    "rms_block_rows2": ("rmsnorm", ["-DMI355_RMS_BLOCK_ROWS=2"]),
    "rms_block_rows4": ("rmsnorm", ["-DMI355_RMS_BLOCK_ROWS=4"]),
    # RMSNorm: rows up to 8 packets per lane as one wave (C4: one wave x 7
    # packets instead of 4 waves x 2), with 1 or 2 rows per wave
    "rms_one_wave": ("rmsnorm", ["-DMI355_RMS_WAVE_MAX_VPL=8"]),
    "rms_one_wave_rows2": ("rmsnorm", ["-DMI355_RMS_WAVE_MAX_VPL=8", "-DMI355_RMS_WAVE_ROWS=2"]),
    # RMSNorm: the weight row staged in LDS and broadcast to the waves of a
    # workgroup (instead of each wave loading its packets from L2)
    "rms_weight_lds": ("rmsnorm", ["-DMI355_RMS_WEIGHT_LDS=1"]),
    "rms_weight_lds_block1024": ("rmsnorm", ["-DMI355_RMS_WEIGHT_LDS=1", "-DMI355_RMS_WAVE_BLOCK=1024"]),
    # RMSNorm: persistent grids (waves per CU), rows striding over them
    "rms_persistent8": ("rmsnorm", ["-DMI355_RMS_WAVES_PER_CU=8"]),
    "rms_persistent16": ("rmsnorm", ["-DMI355_RMS_WAVES_PER_CU=16"]),
    "rms_block_persistent4": ("rmsnorm", ["-DMI355_RMS_BLOCKS_PER_CU=4"]),
    "rms_block_persistent8": ("rmsnorm", ["-DMI355_RMS_BLOCKS_PER_CU=8"]),
    # RMSNorm: wide rows streamed through a persistent grid, S rows in flight
    # per workgroup (rmsnorm_block_stream), workgroups per CU
    "rms_stream2": ("rmsnorm", ["-DMI355_RMS_STREAM_ROWS=2"]),
    "rms_stream4": ("rmsnorm", ["-DMI355_RMS_STREAM_ROWS=4"]),
    "rms_stream4_wg2": ("rmsnorm", ["-DMI355_RMS_STREAM_ROWS=4", "-DMI355_RMS_STREAM_BLOCKS_PER_CU=2"]),
    "rms_stream4_wg8": ("rmsnorm", ["-DMI355_RMS_STREAM_ROWS=4", "-DMI355_RMS_STREAM_BLOCKS_PER_CU=8"]),
    "rms_stream4_vpl1": ("rmsnorm", ["-DMI355_RMS_STREAM_ROWS=4", "-DMI355_RMS_TARGET_VPL=1"]),
    "rms_stream8_vpl1_wg2": ("rmsnorm", ["-DMI355_RMS_STREAM_ROWS=8", "-DMI355_RMS_TARGET_VPL=1",
                                         "-DMI355_RMS_STREAM_BLOCKS_PER_CU=2"]),
    # RMSNorm: packets per lane of the workgroup-per-row kernel (C4: 7 waves x
    # 1 packet, 2 waves x 4, against the shipped 4 x 2)
    "rms_target_vpl1": ("rmsnorm", ["-DMI355_RMS_TARGET_VPL=1"]),
    "rms_target_vpl4": ("rmsnorm", ["-DMI355_RMS_TARGET_VPL=4"]),
    # RMSNorm: workgroup size of the wave-per-row kernel
    "rms_wave_block64": ("rmsnorm", ["-DMI355_RMS_WAVE_BLOCK=64"]),
    "rms_wave_block512": ("rmsnorm", ["-DMI355_RMS_WAVE_BLOCK=512"]),
    # SiLU-and-mul below 2^27 elements (C2): packets per lane, workgroup size
    "silu_unroll1": ("silu_mul", ["-DMI355_SILU_UNROLL=1"]),
    "silu_unroll3": ("silu_mul", ["-DMI355_SILU_UNROLL=3"]),
    "silu_unroll4_block256": ("silu_mul", ["-DMI355_SILU_UNROLL=4", "-DMI355_SILU_BLOCK=256"]),
    "silu_block1024": ("silu_mul", ["-DMI355_SILU_BLOCK=1024"]),
    # SiLU-and-mul from 2^27 elements (C4): the small-size shape, other chunks
    "silu_large_block512_unroll2": ("silu_mul", ["-DMI355_SILU_LARGE_BLOCK=512", "-DMI355_SILU_LARGE_UNROLL=2"]),
    "silu_large_block256_unroll8": ("silu_mul", ["-DMI355_SILU_LARGE_UNROLL=8"]),
    "silu_large_block128_unroll8": ("silu_mul", ["-DMI355_SILU_LARGE_BLOCK=128", "-DMI355_SILU_LARGE_UNROLL=8"]),
    # SiLU-and-mul: every size on one shape, and the load order
    "silu_large_shape_everywhere": ("silu_mul", ["-DMI355_SILU_LARGE_MIN_NUMEL=0"]),
    "silu_load_order1": ("silu_mul", ["-DMI355_SILU_LOAD_ORDER=1"]),
    # W8A16 tiled GEMM (prefill rows): widen each sub-step's int8 weights right
    # before its own MFMAs instead of one sub-step ahead
    "tiled_widen_in_place": ("w8a16", ["-DMI355_TILED_WIDEN_AHEAD=0"]),
    # W8A16 tiled GEMMs (single and gate/up + SiLU-and-mul): tile counts that
    # are not a multiple of 8 keep the dispatch order instead of XCD ranges
    "w8_xcd_dispatch_order": ("w8a16", ["-DMI355_TILED_XCD_RAGGED=0"]),
    "gate_up_xcd_dispatch_order": ("gate_up_silu", ["-DMI355_TILED_XCD_RAGGED=0"]),
    # 16-bit gate/up + SiLU-and-mul: the column split's whole rounds cut at
    # 128-column blocks of every row block
    "gate_up_rounds_by_columns": ("gate_up_silu", ["-DMI355_GU_ROUNDS_BY_COLUMNS=1"]),
    # 16-bit gate/up + SiLU-and-mul: the column split's rest in one shape
    # (4: 256 x 64; 5: 128 x 128 of 8 waves) whenever it fits one round
    **{f"gate_up_rest_shape{f}": ("gate_up_silu", [f"-DMI355_GU_REST_SHAPE={f}"]) for f in (4, 5)},
    # 16-bit gate/up + SiLU-and-mul: m-blocks per group of the tile order (default 4)
    **{f"gate_up_group_m{g}": ("gate_up_silu", [f"-DMI355_GU_GROUP_M={g}"]) for g in (2, 8, 64)},
    # W8A16 tiled GEMM, wide outputs from 1024 rows: the column split (whole
    # rounds of 128 x 128, the rest in 128 x 64) when the last round is more
    # than half full (1) or whenever the rest fits one round (2)
    **{f"w8_colsplit{m}": ("w8a16", [f"-DMI355_W8_COLSPLIT={m}"]) for m in (1, 2)},
    # W8A16 tiled GEMM: tiles ordered in 2 / 4 / 8 column bands before the
    # XCD ranges (every single-matrix launch)
    **{f"w8_bands{b}": ("w8a16", [f"-DMI355_W8_BANDS={b}"]) for b in (2, 4, 8)},
    # W8A16 tiled GEMM: m-blocks per group of the tile order (default 4)
    **{f"w8_group_m{g}": ("w8a16", [f"-DMI355_W8_GROUP_M={g}"]) for g in (1, 2, 8, 16, 64)},
    # W8A16 tiled GEMM: an L2 prefetch wave per workgroup, 2 / 4 / 8 K steps
    # past the LDS ring
    "tiled_prefetch2": ("w8a16", ["-DMI355_TILED_PREFETCH=2"]),
    "tiled_prefetch4": ("w8a16", ["-DMI355_TILED_PREFETCH=4"]),
    "tiled_prefetch8": ("w8a16", ["-DMI355_TILED_PREFETCH=8"]),
    # W8A16 decode (skinny) kernels: the launch-shape sweep build, whose
    # mi355_w8_sweep_config / mi355_w8_sweep_ks force G x waves x U and a
    # split of K over workgroups (bench.py --w8-skinny-sweep), with the
    # main loop as shipped and with U blocks kept in flight throughout
    "w8_skinny_sweep": ("w8a16", ["-DMI355_W8_SWEEP"]),
    "w8_skinny_sweep_pipe": ("w8a16", ["-DMI355_W8_SWEEP", "-DMI355_W8_PIPE=1"]),
    # W8A16 tiled GEMM: one tile configuration for every prefill launch
    # (MI355_W8_FORCE in w8a16.hip lists them)
    **{f"w8_tile_cfg{i}": ("w8a16", [f"-DMI355_W8_FORCE={i}"]) for i in range(1, 43)},
    # 192 x 128 tiles of 8 waves squeezed to 4 waves per SIMD (two
    # workgroups per CU; a few VGPRs spill)
    "w8_tile_cfg37_wpe4": ("w8a16", ["-DMI355_W8_FORCE=37", "-DMI355_TILED_MIN_WAVES_PER_SIMD=4"]),
    # W8A16 gate/up + SiLU-and-mul tiled GEMM above 256 rows: one tile
    # configuration for every launch (MI355_W8_DUAL_FORCE in w8a16.hip)
    **{f"w8_dual_cfg{i}": ("w8a16", [f"-DMI355_W8_DUAL_FORCE={i}"]) for i in range(1, 12)},
    # RMSNorm: keep the row's fp32 widening live between the two passes
    # instead of re-widening the packed row (more VGPRs, fewer conversions),
    # per kernel: the shipped choice is the wave kernel re-widening and the
    # workgroup kernel keeping fp32
    "rms_wave_keep_f32": ("rmsnorm", ["-DMI355_RMS_KEEP_F32_WAVE=1"]),
    "rms_block_rewiden": ("rmsnorm", ["-DMI355_RMS_KEEP_F32_BLOCK=0"]),
}
# Built with every default build (``__graft_entry__.build``), so the GPU tests
# of tests/test_launch_variants.py run on them: one variant per distinct code
# path of the kernels (several rows per wave and per workgroup, a row over
# one wave, the LDS weight, a persistent grid, another SiLU-and-mul chunk,
# the W8A16 widening order, the W8A16 decode kernel's sweep builds with their
# split of K over workgroups and pipelined loop, the 256 x 128 and 256 x 256
# W8A16 tiles that the launch plan now picks only for k > 4096).
CORE_VARIANTS = ("rms_wave_rows2", "rms_block_rows2", "rms_one_wave", "rms_weight_lds", "rms_persistent8",
                 "rms_block_persistent4", "silu_unroll1", "silu_large_block512_unroll2", "tiled_widen_in_place",
                 "w8_skinny_sweep", "w8_skinny_sweep_pipe", "w8_tile_cfg2", "w8_tile_cfg3",
                 "gate_up_xcd_dispatch_order")
VARIANT_DIR = PKG_DIR / "_variants"
# Variants that spread a row over waves differently from the default build
# (one wave per wide row; one packet per lane over more waves): the fp32 sum
# of squares then adds in another order, so an output may differ
# from the default library's in its last bit (both stay within one ulp of the
# exactly rounded result).  Every other variant is bit-identical to the
# default library.
REORDERING_VARIANTS = frozenset({"rms_one_wave", "rms_one_wave_rows2", "rms_stream4_vpl1", "rms_stream8_vpl1_wg2",
                                 "rms_target_vpl1", "rms_target_vpl4"})


def variant_path(name: str) -> Path:
    return VARIANT_DIR / f"libmi355_fused_{name}.so"


def build_variants(names=CORE_VARIANTS) -> list[Path]:
    """Builds the named variants in parallel (the default objects must be
    current: call after build())."""
    with cf.ThreadPoolExecutor(max_workers=min(8, len(names))) as ex:
        return list(ex.map(build_variant, names))


def build_variant(name: str) -> Path:
    """The library with VARIANTS[name]'s translation unit recompiled under its
    switches and every other unit from the default build's objects."""
    unit, flags = VARIANTS[name]
    default_dir = PKG_DIR / "_build" / "default"
    objdir = PKG_DIR / "_build" / f"variant_{name}"
    objdir.mkdir(parents=True, exist_ok=True)
    objs = []
    for src in sorted(CSRC.glob("*.hip")):
        if src.stem == unit:
            obj = objdir / (src.stem + ".o")
            _compile(src, obj, flags)
        else:
            obj = default_dir / (src.stem + ".o")
            if not obj.exists():
                default_dir.mkdir(parents=True, exist_ok=True)
                _compile(src, obj, [])
        objs.append(obj)
    out = variant_path(name)
    out.parent.mkdir(parents=True, exist_ok=True)
    tmp = out.with_name(out.name + ".tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{res.stdout}{res.stderr}")
    os.replace(tmp, out)
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
    """Build the stand-alone copy kernel bench.py uses for the copy ceiling."""
    out = PKG_DIR / PROBE_NAME
    tmp = out.with_name(out.name + ".tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, "-shared", str(CSRC / "probe" / "stream_copy.hip"), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"probe build failed:\n{' '.join(cmd)}\n{res.stdout}{res.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    args = sys.argv[1:]
    if args[:1] == ["--variant"]:
        names = list(VARIANTS) if args[1:] == ["all"] else args[1:]
        unknown = [n for n in names if n not in VARIANTS]
        if unknown or not names:
            sys.exit(f"unknown variant(s) {unknown}; known: {', '.join(VARIANTS)}")
        with cf.ThreadPoolExecutor(max_workers=min(8, len(names))) as ex:
            for path in ex.map(build_variant, names):
                print(path)
        sys.exit(0)
    out = None
    if "--out" in args:
        i = args.index("--out")
        out = Path(args[i + 1])
        del args[i : i + 2]
    print(build(args, out))
