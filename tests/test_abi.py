"""CPU-side checks of the C ABI: the library loads and exports every symbol the header declares."""
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def _declared():
    text = (ROOT / "include" / "mindpipe_amd.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char \*)\s*(mp_\w+)\s*\(", text, re.M)))


def test_header_declares_expected_entry_points():
    names = _declared()
    for n in ("mp_w4a16_gemm", "mp_quant_per_token_i8", "mp_w8a8_gemm", "mp_moe_permute_quant",
              "mp_i8_gemm_swiglu_requant", "mp_w8a8_grouped_gemm", "mp_moe_unpermute_combine"):
        assert n in names


def test_library_exports_every_declared_symbol():
    from mindpipe_amd import _lib
    if not _lib.LIB_PATH.exists():
        pytest.skip("library not built")
    lib = _lib.load()
    for name in _declared():
        assert hasattr(lib, name), name
    assert set(_declared()) == set(_lib.SIGNATURES)
    assert lib.mp_abi_version() == _lib.ABI_VERSION
    assert lib.mp_strerror(1).decode().startswith("mindpipe_amd")


def test_host_validation_without_gpu():
    """Argument checks run on the host before any launch (no GPU needed).  Every pointer argument is
    a real (host) buffer that no check reaches through: the calls are rejected before a launch."""
    import ctypes
    from mindpipe_amd import _lib
    if not _lib.LIB_PATH.exists():
        pytest.skip("library not built")
    lib = _lib.load()
    buf = ctypes.create_string_buffer(4096)
    p = ctypes.addressof(buf)
    assert lib.mp_w4a16_gemm(None, 1, 128, None, 16, None, None, 128, None, None, 0, None) == 5
    assert lib.mp_w8a8_gemm(p, p, p, p, None, 0, p, 9, 1, 16, 64, None) == 2      # bad out dtype
    assert lib.mp_w8a8_gemm(p, p, p, p, None, 0, p, 0, 1, 16, 1 << 18, None) == 1  # K too large for int32
    assert lib.mp_quant_per_token_i8(p, 4, 64, 7, p, p, 0, None) == 2
    assert lib.mp_i8_gemm_swiglu_requant(p, p, p, p, p, 8, 16, 64, 128, 0, 0, p, p, p, 0, None) == 6
    assert lib.mp_moe_unpermute_combine(p, p, p, 4, 2, 64, 1, p, 2, None) == 2   # fake rule needs fp16/bf16 out
