"""The C-ABI library loads and exports every symbol include/kanso_hip.h declares
(no compute calls: this runs without a GPU)."""
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "kanso_hip.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kanso_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared_functions()
    for required in ("kanso_paged_attention_v2", "kanso_ragged_paged_attention",
                     "kanso_pack_step", "kanso_kv_append", "kanso_gemv_q8_0", "kanso_gemv_q4_k"):
        assert required in names


def test_library_exports_every_declared_symbol():
    from kanso_infer_amd import _capi
    if not _capi.LIB_PATH.exists():
        pytest.fail("libkanso_hip.so is not built (python -m kanso_infer_amd.build)")
    lib = _capi.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
        assert name in _capi.SIGNATURES, f"{name} has no ctypes signature"


def test_no_fallback_when_library_missing(monkeypatch, tmp_path):
    from kanso_infer_amd import _capi
    monkeypatch.setattr(_capi, "_lib", None)
    monkeypatch.setenv("KANSO_HIP_LIB", str(tmp_path / "missing.so"))
    with pytest.raises(RuntimeError):
        _capi.load()
