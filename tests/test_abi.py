"""The C-ABI library loads and exports every entry point include/q35.h declares
(no compute calls: this runs without a GPU)."""
import ctypes
import re
from pathlib import Path

REPO = Path(__file__).resolve().parents[1]


def declared():
    txt = (REPO / "include" / "q35.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(q35_\w+)\s*\(", txt, re.M)))


def test_exports_every_declared_symbol():
    from qwen35 import load_library, lib_path
    assert lib_path().exists(), "build the library first (qwen3.5-0.8b_amd/build.py)"
    L = load_library()
    names = declared()
    assert len(names) >= 20
    for n in names:
        assert hasattr(L, n), n
    assert "q35_decode_step" in names and "q35_prefill" in names and "q35_mtp_round" in names


def test_bad_config_is_an_error_not_a_crash():
    from qwen35 import Engine, EngineError
    import pytest
    with pytest.raises(EngineError):
        Engine(max_rows=0, max_ctx=16, seed=None)
