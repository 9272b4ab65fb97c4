"""The C ABI: librfill.so loads without a GPU and exports every entry point include/rfill.h declares,
and the Python binding declares exactly those (no compute calls here)."""
import ctypes
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def declared():
    text = (ROOT / "include" / "rfill.h").read_text()
    return sorted(set(re.findall(r"^(?:int|const char\*)\s+(rf_\w+)\s*\(", text, re.M)))


def test_header_declares_the_entry_points():
    names = declared()
    assert "rf_map_apply" in names and "rf_norm_kv_write" in names and "rf_last_error" in names


def test_library_exports_every_declared_symbol():
    from rfill import _lib
    assert _lib.LIB_PATH.exists(), "librfill.so not built: run __graft_entry__.build()"
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing
    assert lib.rf_version() >= 1


def test_binding_covers_the_header():
    from rfill import _lib
    compute = [n for n in declared() if n not in ("rf_last_error", "rf_version")]
    assert sorted(_lib.SIGNATURES) == compute


def test_status_codes_match_the_header():
    from rfill import _lib
    text = (ROOT / "include" / "rfill.h").read_text()
    for name in ("RF_OK", "RF_EINVAL_SHAPE", "RF_EINVAL_ARG", "RF_EUNSUPPORTED", "RF_EHIP"):
        value = int(re.search(rf"#define {name} \(?(-?\d+)\)?", text).group(1))
        assert getattr(_lib, name) == value
    assert _lib.SSQ_COLS == int(re.search(r"#define RF_SSQ_COLS (\d+)", text).group(1))
