"""CPU checks of the C ABI: the built library loads and exports every declared entry point."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADERS = sorted((ROOT / "include").glob("*.h"))


def _declared() -> list[str]:
    names: list[str] = []
    for h in HEADERS:
        text = h.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(qs_\w+)\s*\(", text, re.M):
            names.append(m.group(1))
    return sorted(set(names))


def test_header_declares_entry_points():
    names = _declared()
    assert "qs_qrow_matmul" in names and "qs_last_error" in names
    assert len(names) >= 6


def test_library_exports_every_declared_symbol():
    import mrun_pub_amd._native as nat

    if not nat.LIB_PATH.exists():
        pytest.skip("library not built (run __graft_entry__.build())")
    import torch  # noqa: F401  (HIP runtime first, as in production)

    lib = ctypes.CDLL(str(nat.LIB_PATH))
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"
    # every declared symbol has a ctypes signature in the binding and vice versa
    assert set(_declared()) == set(nat.SIGNATURES)


def test_version_and_error_string_without_gpu():
    import mrun_pub_amd._native as nat

    if not nat.LIB_PATH.exists():
        pytest.skip("library not built")
    lib = nat.load()
    assert lib.qs_version() >= 100
    # a validation failure is reported without touching the device
    st = lib.qs_qrow_matmul(None, 1, 16, None, None, None, 16, 1, 16, 16, None)
    assert st == nat.QS_ERR_INVALID
    assert b"null" in lib.qs_last_error()
    with pytest.raises(ValueError):
        nat.check(st, "qs_qrow_matmul")


def test_moe_entry_point_validation_without_gpu():
    """The MoE entry points added for the weight-only flow and the fused route reject bad
    arguments before any device work (status codes as documented in the header)."""
    import mrun_pub_amd._native as nat

    if not nat.LIB_PATH.exists():
        pytest.skip("library not built")
    lib = nat.load()
    fake = ctypes.c_void_p(4096)  # never dereferenced: validation fails first
    # weight-only grouped GEMM: null pointers, K not a multiple of 64, SwiGLU output dtype
    st = lib.qs_moe_grouped_gemm_w8a16(None, None, 0, fake, 0, fake, 0, fake, fake, None, 1, 64, 128, 0, 0, fake,
                                       nat.QS_BF16, None)
    assert st == nat.QS_ERR_INVALID and b"null" in lib.qs_last_error()
    st = lib.qs_moe_grouped_gemm_w8a16(fake, None, 0, fake, 0, fake, 0, fake, fake, None, 1, 64, 100, 0, 0, fake,
                                       nat.QS_BF16, None)
    assert st == nat.QS_ERR_UNSUPPORTED and b"multiple of 64" in lib.qs_last_error()
    st = lib.qs_moe_grouped_gemm_w8a16(fake, None, 0, fake, 0, fake, 0, fake, fake, None, 1, 64, 128, 0, 1, fake,
                                       nat.QS_F32, None)
    assert st == nat.QS_ERR_INVALID and b"SwiGLU" in lib.qs_last_error()
    # gathered int8 grouped GEMM: row_ids required
    st = lib.qs_moe_grouped_gemm_i8_rows(fake, fake, None, 4, fake, 0, fake, 0, fake, fake, None, 1, 64, 128, 0, 0,
                                         fake, nat.QS_BF16, None)
    assert st == nat.QS_ERR_INVALID and b"row_ids" in lib.qs_last_error()
    # fused route + quantization: dtype checks
    st = lib.qs_moe_route_quant(fake, nat.QS_I64, fake, nat.QS_F32, 4, 2, 8, fake, fake, fake, fake, None, fake,
                                nat.QS_F16, 64, 64, fake, fake, None)
    assert st == nat.QS_ERR_INVALID and b"F32 or BF16" in lib.qs_last_error()


def test_build_rejects_kernels_that_use_scratch():
    """The build fails on a kernel whose resource remarks report scratch memory."""
    import importlib.util

    spec = importlib.util.spec_from_file_location("qs_build", ROOT / "mrun-pub_amd" / "build.py")
    build = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(build)
    remarks = "\n".join([
        "a.hip:1:1: remark: Function Name: k_fine [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:1:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:9:1: remark: Function Name: k_stack [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:9:1: remark:     ScratchSize [bytes/lane]: 200 [-Rpass-analysis=kernel-resource-usage]",
    ])
    assert build._scratch_kernels(remarks) == ["k_stack (200 bytes/lane)"]
