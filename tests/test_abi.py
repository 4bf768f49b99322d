"""The C ABI: every symbol ``include/kx355.h`` declares is exported and bound, and argument
validation rejects bad calls before any GPU work. CPU only (no kernel is launched)."""

import ctypes
import re
from pathlib import Path

import pytest

from kinomlx_amd import _lib

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "kx355.h"


def _declared() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(kx_\w+)\s*\(", text, flags=re.M)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = _declared()
    assert len(names) >= 15
    for name in names:
        assert hasattr(lib, name), name


def test_binding_covers_every_declared_entry_point():
    declared = {n for n in _declared() if n not in ("kx_abi_version", "kx_last_error")}
    assert declared == set(_lib.SIGNATURES)


def test_binding_argument_counts_match_header():
    text = HEADER.read_text()
    for name, args in _lib.SIGNATURES.items():
        m = re.search(rf"{name}\s*\(([^;]*)\);", text, flags=re.S)
        assert m, name
        assert len([a for a in m.group(1).split(",") if a.strip()]) == len(args), name


def test_abi_version():
    assert _lib.load().kx_abi_version() == 1


def _null_call(name):
    args = []
    for t in _lib.SIGNATURES[name]:
        if t is ctypes.c_void_p:
            args.append(None)
        elif t is ctypes.c_float:
            args.append(1.0)
        else:
            args.append(1)
    return getattr(_lib.load(), name)(*args)


@pytest.mark.parametrize("name", sorted(_lib.SIGNATURES))
def test_null_tensors_are_rejected_without_touching_the_gpu(name):
    assert _null_call(name) == _lib.KX_ERR_INVALID
    assert name in _lib.load().kx_last_error().decode()


def test_shape_and_format_checks():
    lib = _lib.load()
    fake = 1 << 20  # never dereferenced: validation fails first
    # head_dim other than 64/128
    assert lib.kx_attention_fwd_bf16(fake, 96, fake, 96, fake, 96, fake, 96, 1, 1, 1, 1, 96, 1.0, None, 0, None) == -1
    # k not a multiple of 8
    assert lib.kx_gemm_bf16(fake, 16, fake, 16, None, fake, 8, 4, 4, 12, 0, None, 0, None, 1, 0, None) == -1
    # bits 3, group 32
    assert lib.kx_qgemm_affine_bf16(fake, 64, fake, fake, fake, None, fake, 8, 1, 8, 64, 64, 3, 0, None, 0, None, 1, 0,
                                    None) == -1
    assert lib.kx_qgemm_affine_bf16(fake, 64, fake, fake, fake, None, fake, 8, 1, 8, 64, 32, 4, 0, None, 0, None, 1, 0,
                                    None) == -1
    # bias flag without a bias
    assert lib.kx_gemm_bf16(fake, 16, fake, 16, None, fake, 8, 4, 8, 16, 1, None, 0, None, 1, 0, None) == -1
    assert "bias" in lib.kx_last_error().decode()
    # unknown epilogue bits
    assert lib.kx_gemm_bf16(fake, 16, fake, 16, None, fake, 8, 4, 8, 16, 1 << 12, None, 0, None, 1, 0, None) == -1
    # Q/K norm projection: heads must be whole 128-wide column blocks inside n, k a multiple of 64
    qk = lib.kx_gemm_qknorm_rope_bf16
    assert qk(fake, 64, fake, 64, None, fake, 512, 4, 512, 64, 192, 384, fake, fake, 0, 1e-6, 0.0, fake, fake, 128, 0,
              4, 0, None) == -1
    assert "128-wide heads" in lib.kx_last_error().decode()
    assert qk(fake, 64, fake, 64, None, fake, 512, 4, 512, 64, 256, 640, fake, fake, 0, 1e-6, 0.0, fake, fake, 128, 0,
              4, 0, None) == -1
    assert qk(fake, 48, fake, 48, None, fake, 512, 4, 512, 48, 256, 512, fake, fake, 0, 1e-6, 0.0, fake, fake, 128, 0,
              4, 0, None) == -1
    assert qk(fake, 96, fake, 96, None, fake, 512, 4, 512, 96, 256, 512, fake, fake, 0, 1e-6, 0.0, fake, fake, 128, 0,
              4, 0, None) == -1
    assert "k % 64" in lib.kx_last_error().decode()
    assert qk(fake, 64, fake, 64, None, fake, 512, 4, 512, 64, 256, 512, fake, fake, 0, 1e-6, 0.0, fake, fake, 130, 0,
              4, 0, None) == -1
    # fused RoPE on a width the fused kernel does not take is refused, not silently changed
    assert lib.kx_rmsnorm_rope_bf16(fake, 96, fake, 96, 1, 96, 96, fake, 0, 1e-6, 0.0, 1, fake, fake, 48, 24, 1, 0,
                                    48, None) == _lib.KX_ERR_UNSUPPORTED


def test_zero_sized_work_is_a_no_op():
    lib = _lib.load()
    fake = 1 << 20
    assert lib.kx_gemm_bf16(fake, 16, fake, 16, None, fake, 8, 0, 8, 16, 0, None, 0, None, 1, 0, None) == 0
    assert lib.kx_adaln_norm_bf16(fake, 512, fake, 512, 0, 512, None, None, 1, 0, 1e-6, 0, None) == 0


def test_product_package_never_imports_the_oracle():
    for path in (ROOT / "kinomlx_amd").rglob("*.py"):
        text = path.read_text()
        assert not re.search(r"^\s*(from|import)\s+oracle", text, flags=re.M), path
