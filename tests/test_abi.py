"""The C ABI library loads and exports every entry point include/kvad_hip.h
declares, and the Python mirror binds exactly those.  No compute calls (no
GPU needed)."""
import ctypes
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "kvad_hip.h"


def declared() -> set[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(kh_[a-z0-9_]+)\s*\(", text))


def test_header_declares_the_boundary():
    names = declared()
    for must in ("kh_init", "kh_matvec", "kh_matvec_many", "kh_matmul", "kh_attend", "kh_kv_push",
                 "kh_weight_q8", "kh_weight_q4", "kh_weight_q4k", "kh_weight_row", "kh_debug_block_dots"):
        assert must in names


def test_library_exports_every_declared_symbol():
    import kvad_amd

    lib = ctypes.CDLL(str(kvad_amd.LIB_PATH))
    missing = [n for n in sorted(declared()) if not hasattr(lib, n)]
    assert not missing, missing


def test_python_mirror_binds_exactly_the_header():
    import kvad_amd

    assert set(kvad_amd.declared_symbols()) == declared()


def test_version_and_error_slot_work_without_a_device():
    import kvad_amd

    assert b"gfx950" in kvad_amd.lib.kh_version()
    assert kvad_amd.lib.kh_last_error() is not None
