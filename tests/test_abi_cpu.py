"""Host-side checks of the C ABI and the Python boundary that need no GPU:
the library loads, exports every symbol include/*.h declares, reports its
ABI version, and rejects bad arguments (or no-ops on empty work) before any
HIP call.  Also: the product package never imports the oracle, and the
Python launchers raise the reference's AssertionError for host tensors."""
import ctypes
import importlib
import re
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
PKG_DIR = ROOT / "llm-inference-optimizer_amd"


def _declared_symbols():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(mi355_[a-z0-9_]+)\s*\(", text))
    return names


@pytest.fixture(scope="module")
def L():
    return importlib.import_module("llm-inference-optimizer_amd._lib")


@pytest.fixture(scope="module")
def lib(L):
    return L.load()


def test_header_declares_expected_entry_points(L):
    declared = _declared_symbols()
    assert declared == set(L.EXPORTED_SYMBOLS), declared


def test_library_exports_every_declared_symbol(lib):
    raw = ctypes.CDLL(str(PKG_DIR / "libmi355_fused.so"))
    for name in _declared_symbols():
        assert hasattr(raw, name), f"{name} declared in include/ but not exported"


def test_abi_version(L, lib):
    assert lib.mi355_abi_version() == L.ABI_VERSION == 1
    hdr = (ROOT / "include" / "mi355_fused.h").read_text()
    assert re.search(r"#define MI355_ABI_VERSION 1\b", hdr)


def test_dtype_codes_match_header(L):
    hdr = (ROOT / "include" / "mi355_fused.h").read_text()
    assert re.search(r"MI355_F32 = 0", hdr) and re.search(r"MI355_F16 = 1", hdr) and re.search(r"MI355_BF16 = 2", hdr)
    assert (L.F32, L.F16, L.BF16) == (0, 1, 2)


# Argument validation happens before any HIP call, so these run without a GPU.
P = 0x10000  # a fake, never-dereferenced device address


@pytest.mark.parametrize("args,code,msg", [
    ((P, P, P, 4, 64, 64, 64, 1e-6, 7, 1, 1), -1, "unknown dtype"),
    ((P, P, P, 4, 64, 64, 64, 1e-6, 1, 1, 2), -2, "y dtype"),
    ((P, P, P, -1, 64, 64, 64, 1e-6, 1, 1, 1), -1, "rows"),
    ((P, P, P, 4, 0, 64, 64, 1e-6, 1, 1, 1), -1, "n must be"),
    ((P, P, P, 4, 2**31, 2**31, 2**31, 1e-6, 1, 1, 1), -1, "n must be"),
    ((0, P, P, 4, 64, 64, 64, 1e-6, 1, 1, 1), -1, "null pointer"),
    ((P, P, P, 4, 64, 32, 64, 1e-6, 1, 1, 1), -1, "row strides"),
    ((P, P, P, 2**40, 64, 2**40, 64, 1e-6, 1, 1, 1), -1, "overflows"),
])
def test_rmsnorm_abi_rejects(lib, args, code, msg):
    st = lib.mi355_rmsnorm_fwd(*args, None)
    assert st == code
    assert msg in lib.mi355_last_error().decode()


def test_rmsnorm_abi_zero_rows_is_noop(lib):
    assert lib.mi355_rmsnorm_fwd(0, 0, 0, 0, 64, 64, 64, 1e-6, 1, 1, 1, None) == 0
    assert lib.mi355_last_error().decode() == ""


@pytest.mark.parametrize("args,code,msg", [
    ((P, P, P, 16, 9, 1), -1, "unknown dtype"),
    ((P, P, P, 16, 1, 2), -2, "out dtype"),
    ((P, P, P, -5, 1, 1), -1, "numel"),
    ((P, 0, P, 16, 1, 1), -1, "null pointer"),
])
def test_silu_mul_abi_rejects(lib, args, code, msg):
    st = lib.mi355_silu_mul_fwd(*args, None)
    assert st == code
    assert msg in lib.mi355_last_error().decode()


def test_silu_mul_abi_zero_numel_is_noop(lib):
    assert lib.mi355_silu_mul_fwd(0, 0, 0, 0, 1, 1, None) == 0


# (x, w_gate, w_up, out, rows, k, n_out, x_row_stride, w_row_stride, out_row_stride, dtype, out_dtype)
@pytest.mark.parametrize("args,code,msg", [
    ((P, P, P, P, 8, 64, 32, 64, 64, 32, 7, 1), -1, "unknown dtype"),
    ((P, P, P, P, 8, 64, 32, 64, 64, 32, 0, 0), -2, "fp16 or bf16"),
    ((P, P, P, P, 8, 64, 32, 64, 64, 32, 1, 2), -2, "out dtype"),
    ((P, P, P, P, -1, 64, 32, 64, 64, 32, 1, 1), -1, "need rows"),
    ((P, P, P, P, 8, 0, 32, 64, 64, 32, 1, 1), -1, "need rows"),
    ((P, P, P, P, 8, 64, 32, 56, 64, 32, 1, 1), -1, "row strides"),
    ((P, P, P, P, 8, 64, 32, 64, 64, 16, 1, 1), -1, "row strides"),
    ((P, P, 0, P, 8, 64, 32, 64, 64, 32, 2, 2), -1, "null pointer"),
    ((P, P, P, P, 8, 60, 32, 64, 64, 32, 1, 1), -2, "multiples of 8"),
    ((P, P, P, P, 8, 64, 32, 68, 64, 32, 1, 1), -2, "multiples of 8"),
    ((P + 2, P, P, P, 8, 64, 32, 64, 64, 32, 1, 1), -2, "16-byte aligned"),
    ((P, P, P, P, 8, 64, 32, 64, 2**24, 32, 1, 1), -2, "limits"),
    ((P, P, P, P, 8, 64, 32, 2**24, 64, 32, 1, 1), -2, "limits"),
    ((P, P, P, P, 65535 * 32 + 1, 64, 32, 64, 64, 32, 1, 1), -2, "limits"),
    ((P, P, P, P, 2**40, 64, 32, 64, 64, 2**40, 1, 1), -2, "limits"),
])
def test_gate_up_silu_abi_rejects(lib, args, code, msg):
    st = lib.mi355_gate_up_silu_fwd(*args, None)
    assert st == code
    assert msg in lib.mi355_last_error().decode()


def test_gate_up_silu_abi_empty_is_noop(lib):
    assert lib.mi355_gate_up_silu_fwd(0, 0, 0, 0, 0, 64, 32, 64, 64, 32, 1, 1, None) == 0
    assert lib.mi355_gate_up_silu_fwd(0, 0, 0, 0, 8, 64, 0, 64, 64, 0, 2, 0, None) == 0
    assert lib.mi355_last_error().decode() == ""


def test_python_check_raises_with_message(L, lib):
    st = lib.mi355_silu_mul_fwd(P, P, P, -5, 1, 1, None)
    with pytest.raises(L.KernelError, match="numel must be >= 0"):
        L.check("mi355_silu_mul_fwd", st)


def test_missing_library_fails_loudly(L, monkeypatch, tmp_path):
    monkeypatch.setattr(L, "LIB_PATH", tmp_path / "nope.so")
    monkeypatch.setattr(L, "_lib", None)
    with pytest.raises(L.KernelLibraryMissing):
        L.load()


def test_launchers_assert_on_host_tensors(pkg):
    """Same precondition as the reference (assert x.is_cuda ...): host tensors
    are rejected with AssertionError, never computed on the CPU."""
    x = torch.randn(4, 64, dtype=torch.float16)
    with pytest.raises(AssertionError):
        pkg.fused_rmsnorm(x, torch.ones(64, dtype=torch.float16))
    with pytest.raises(AssertionError):
        pkg.fused_silu_mul(x, x)
    with pytest.raises(AssertionError):
        pkg.fused_gate_up_silu(x, torch.ones(16, 64, dtype=torch.float16), torch.ones(16, 64, dtype=torch.float16))
    with pytest.raises(AssertionError):
        pkg.fused_silu_mul(x, torch.randn(4, 65, dtype=torch.float16))


def test_product_package_never_touches_the_oracle():
    for f in PKG_DIR.rglob("*"):
        if f.suffix in (".py", ".hip", ".h", ".cpp"):
            text = f.read_text()
            assert not re.search(r"\boracle\b", text), f"{f} mentions the oracle"


def test_bench_refuses_multi_gpu():
    import subprocess
    import sys
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr


@pytest.mark.parametrize("args,code,msg", [
    ((P, P, P, P, P, 4, 64, 64, 64, 64, 64, 1e-6, 1, 1, 7), -1, "unknown dtype"),
    ((P, P, P, P, P, 4, 64, 64, 64, 64, 64, 1e-6, 2, 2, 1), -2, "y dtype"),
    ((P, 0, P, P, P, 4, 64, 64, 64, 64, 64, 1e-6, 1, 1, 1), -1, "null pointer"),
    ((P, P, P, P, 0, 4, 64, 64, 64, 64, 64, 1e-6, 1, 1, 1), -1, "null pointer"),
    ((P, P, P, P, P, 4, 64, 64, 63, 64, 64, 1e-6, 1, 1, 1), -1, "row strides"),
    ((P, P, P, P, P, 4, 64, 64, 64, 64, 8, 1e-6, 1, 1, 1), -1, "row strides"),
    ((P, P, P, P, P, -2, 64, 64, 64, 64, 64, 1e-6, 1, 1, 1), -1, "rows"),
])
def test_add_rmsnorm_abi_rejects(lib, args, code, msg):
    st = lib.mi355_add_rmsnorm_fwd(*args, None)
    assert st == code
    assert msg in lib.mi355_last_error().decode()


def test_add_rmsnorm_abi_zero_rows_is_noop(lib):
    assert lib.mi355_add_rmsnorm_fwd(0, 0, 0, 0, 0, 0, 64, 64, 64, 64, 64, 1e-6, 1, 1, 1, None) == 0


def test_fused_add_rmsnorm_asserts_on_host_tensors(pkg):
    x = torch.randn(4, 64, dtype=torch.float16)
    with pytest.raises(AssertionError):
        pkg.fused_add_rmsnorm(x, x, torch.ones(64, dtype=torch.float16))


# (x, w_q, scale, bias, out, rows, k, n, x_row_stride, w_row_stride, out_row_stride,
#  x_dtype, scale_dtype, bias_dtype, out_dtype)
@pytest.mark.parametrize("args,code,msg", [
    ((P, P, P, 0, P, 8, 64, 32, 64, 64, 32, 5, 0, 0, 1), -1, "unknown dtype"),
    ((P, P, P, P, P, 8, 64, 32, 64, 64, 32, 1, 0, 9, 1), -1, "unknown dtype"),
    ((P, P, P, 0, P, 8, 64, 32, 64, 64, 32, 0, 0, 0, 0), -2, "fp16 or bf16"),
    ((P, P, P, 0, P, 8, 64, 32, 64, 64, 32, 1, 0, 0, 2), -2, "out dtype"),
    ((P, P, P, 0, P, -1, 64, 32, 64, 64, 32, 1, 0, 0, 1), -1, "need rows"),
    ((P, P, P, 0, P, 8, 0, 32, 64, 64, 32, 1, 0, 0, 1), -1, "need rows"),
    ((P, P, P, 0, P, 8, 64, 32, 63, 64, 32, 1, 0, 0, 1), -1, "row strides"),
    ((P, P, P, 0, P, 8, 64, 32, 64, 32, 32, 1, 0, 0, 1), -1, "row strides"),
    ((P, P, P, 0, P, 8, 64, 32, 64, 64, 31, 1, 0, 0, 1), -1, "row strides"),
    ((P, P, 0, 0, P, 8, 64, 32, 64, 64, 32, 1, 0, 0, 1), -1, "null pointer"),
    ((P, P, P, 0, P, 8, 64, 32, 2**23, 64, 32, 1, 0, 0, 1), -2, "limits"),
    ((P, P, P, 0, P, 8, 64, 32, 64, 2**24, 32, 1, 0, 0, 1), -2, "limits"),
    ((P, P, P, 0, P, 65535 * 64 + 1, 64, 32, 64, 64, 32, 1, 0, 0, 1), -2, "limits"),
])
def test_w8a16_abi_rejects(lib, args, code, msg):
    st = lib.mi355_w8a16_linear_fwd(*args, None)
    assert st == code
    assert msg in lib.mi355_last_error().decode()


def test_w8a16_abi_empty_is_noop(lib):
    assert lib.mi355_w8a16_linear_fwd(0, 0, 0, 0, 0, 0, 64, 32, 64, 64, 32, 1, 0, 0, 1, None) == 0
    assert lib.mi355_w8a16_linear_fwd(0, 0, 0, 0, 0, 8, 64, 0, 64, 64, 0, 2, 0, 0, 2, None) == 0
    assert lib.mi355_last_error().decode() == ""


# (w, w_q, scale, n, k, w_row_stride, q_row_stride, w_dtype)
@pytest.mark.parametrize("args,code,msg", [
    ((P, P, P, 4, 64, 64, 64, 3), -1, "unknown dtype"),
    ((P, P, P, -1, 64, 64, 64, 1), -1, "need n"),
    ((P, P, P, 4, 0, 64, 64, 1), -1, "need n"),
    ((P, P, P, 4, 64, 32, 64, 1), -1, "row strides"),
    ((P, P, P, 4, 64, 64, 60, 1), -1, "row strides"),
    ((P, 0, P, 4, 64, 64, 64, 0), -1, "null pointer"),
])
def test_quantize_int8_abi_rejects(lib, args, code, msg):
    st = lib.mi355_quantize_int8_fwd(*args, None)
    assert st == code
    assert msg in lib.mi355_last_error().decode()


def test_quantize_int8_abi_empty_is_noop(lib):
    assert lib.mi355_quantize_int8_fwd(0, 0, 0, 0, 64, 64, 64, 1, None) == 0


def test_w8a16_launchers_assert_on_host_tensors(pkg):
    x = torch.randn(4, 64, dtype=torch.float16)
    q = torch.zeros(16, 64, dtype=torch.int8)
    with pytest.raises(AssertionError):
        pkg.w8a16_linear(x, q, torch.ones(16))
    with pytest.raises(AssertionError):
        pkg.quantize_int8_weight(torch.randn(16, 64))
    with pytest.raises(AssertionError):
        pkg.QuantizedLinearInt8.from_linear(torch.nn.Linear(64, 16))


# (x, wq_gate, wq_up, scale_gate, scale_up, out, rows, k, n_out, x_row_stride, w_row_stride,
#  out_row_stride, x_dtype, scale_dtype, out_dtype)
@pytest.mark.parametrize("args,code,msg", [
    ((P, P, P, P, P, P, 8, 64, 32, 64, 64, 32, 3, 0, 1), -1, "unknown dtype"),
    ((P, P, P, P, P, P, 8, 64, 32, 64, 64, 32, 0, 0, 0), -2, "fp16 or bf16"),
    ((P, P, P, P, P, P, 8, 64, 32, 64, 64, 32, 1, 0, 2), -2, "out dtype"),
    ((P, P, P, P, P, P, -1, 64, 32, 64, 64, 32, 1, 0, 1), -1, "need rows"),
    ((P, P, P, P, P, P, 8, 0, 32, 64, 64, 32, 1, 0, 1), -1, "need rows"),
    ((P, P, P, P, P, P, 8, 64, 32, 32, 64, 32, 1, 0, 1), -1, "row strides"),
    ((P, P, P, P, P, P, 8, 64, 32, 64, 64, 16, 1, 0, 1), -1, "row strides"),
    ((P, P, 0, P, P, P, 8, 64, 32, 64, 64, 32, 1, 0, 1), -1, "null pointer"),
    ((P, P, P, P, 0, P, 8, 64, 32, 64, 64, 32, 1, 0, 1), -1, "null pointer"),
    ((P, P, P, P, P, P, 8, 64, 32, 2**23, 64, 32, 1, 0, 1), -2, "limits"),
    ((P, P, P, P, P, P, 65535 * 64 + 1, 64, 32, 64, 64, 32, 1, 0, 1), -2, "limits"),
])
def test_gate_up_w8a16_abi_rejects(lib, args, code, msg):
    st = lib.mi355_gate_up_silu_w8a16_fwd(*args, None)
    assert st == code
    assert msg in lib.mi355_last_error().decode()


def test_gate_up_w8a16_abi_empty_is_noop(lib):
    assert lib.mi355_gate_up_silu_w8a16_fwd(0, 0, 0, 0, 0, 0, 0, 64, 32, 64, 64, 32, 1, 0, 1, None) == 0
    assert lib.mi355_gate_up_silu_w8a16_fwd(0, 0, 0, 0, 0, 0, 8, 64, 0, 64, 64, 0, 2, 0, 2, None) == 0
    assert lib.mi355_last_error().decode() == ""


def test_gate_up_w8a16_launcher_asserts_on_host_tensors(pkg):
    x = torch.randn(4, 64, dtype=torch.float16)
    q = torch.zeros(16, 64, dtype=torch.int8)
    with pytest.raises(AssertionError):
        pkg.fused_gate_up_silu_w8a16(x, q, torch.ones(16), q, torch.ones(16))


def test_torch_launchers_load_and_match_the_abi(L):
    """The launchers' host side (the _mi355_torch extension over the C ABI)
    is built beside the library and reports the same ABI version."""
    ext = L.ext()
    assert ext.abi_version() == L.ABI_VERSION
    for name in ("rmsnorm", "add_rmsnorm", "silu_mul", "gate_up_silu", "linear16", "w8a16_linear",
                 "gate_up_silu_w8a16"):
        assert callable(getattr(ext, name))


def test_torch_launchers_keep_the_reference_messages(pkg):
    x = torch.randn(4, 64, dtype=torch.float16)
    with pytest.raises(AssertionError, match="x and weight must be ROCm GPU tensors"):
        pkg.fused_rmsnorm(x, torch.ones(64, dtype=torch.float16))
    with pytest.raises(AssertionError, match=r"shape mismatch \(4, 64\) vs \(4, 65\)"):
        pkg.fused_silu_mul(x, torch.randn(4, 65, dtype=torch.float16))
    with pytest.raises(AssertionError, match="out_dtype must be torch.float16 or float32"):
        pkg.linear16(x, x, out_dtype=torch.float64)


def test_header_is_plain_c_and_links(tmp_path):
    """A C99 caller (the INTEGRATION guide's route for a compiled host):
    include/mi355_fused.h compiles as strict C, every entry point's
    prototype type-checks, and a program linked against the library reads
    the ABI version and gets the argument-check status back -- no GPU call."""
    import shutil
    import subprocess

    gcc = shutil.which("gcc")
    so = PKG_DIR / "libmi355_fused.so"
    if gcc is None or not so.exists():
        pytest.skip("gcc or the built library missing")
    src = tmp_path / "caller.c"
    src.write_text(r'''
#include <stdio.h>
#include "mi355_fused.h"
int main(void) {
  if (mi355_abi_version() != MI355_ABI_VERSION) return 2;
  /* n = 0 is rejected before any HIP call */
  int st = mi355_rmsnorm_fwd((const void*)0, (const void*)0, (void*)0, 1, 0, 0, 0, 1e-6f,
                             MI355_F16, MI355_F16, MI355_F16, (void*)0);
  if (st != MI355_ERR_INVALID) return 3;
  printf("%s\n", mi355_last_error());
  return 0;
}
''')
    exe = tmp_path / "caller"
    cmd = [gcc, "-std=c99", "-Wall", "-Werror", "-pedantic", f"-I{ROOT / 'include'}", str(src), str(so),
           f"-Wl,-rpath,{PKG_DIR}", "-o", str(exe)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stdout + res.stderr
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert run.returncode == 0, (run.returncode, run.stdout, run.stderr)
    assert "mi355_rmsnorm_fwd" in run.stdout
