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


GUIDE = ROOT / "INTEGRATION.md"  # the integration guide shipped beside the library


def _build_rs() -> str:
    """The build.rs step the integration guide hands a kvad maintainer."""
    text = GUIDE.read_text()
    m = re.search(r"```rust\n// crates/llm/build\.rs.*?```", text, flags=re.S)
    assert m, "the integration guide has no build.rs step"
    return m.group(0)


def _build_py():
    import importlib.util

    spec = importlib.util.spec_from_file_location("_kvad_build_check", ROOT / "kvad_amd" / "build.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_integration_build_compiles_every_source_build_py_does():
    rs = _build_rs()
    stems = {p.stem for p in (ROOT / "kvad_amd" / "csrc").glob("*.hip")}
    assert len(stems) >= 11
    # a fixed list of translation units, if the step names one, is the whole set
    for lst in re.findall(r"\[\s*(\"[a-z0-9_]+\"(?:\s*,\s*\"[a-z0-9_]+\")+)\s*\]", rs):
        names = set(re.findall(r"\"([a-z0-9_]+)\"", lst))
        if names & stems:
            assert names == stems, f"build.rs lists {sorted(names)}, csrc has {sorted(stems)}"
    # otherwise it globs the directory for .hip files, as build.py does
    assert 'join("hip/csrc")' in rs and "read_dir(&src)" in rs and 'x == "hip"' in rs
    build = _build_py()
    assert [p.stem for p in sorted(build.CSRC.glob("*.hip"))] == sorted(stems)
    # and compiles with build.py's flags (warnings aside)
    flags = [f for f in build.FLAGS if not f.startswith("-W") and not f.startswith("--offload-arch")]
    quoted = re.findall(r"\"(-[^\"]*)\"", rs)
    for f in flags:
        if f.startswith("-"):
            assert f in quoted, f"build.rs does not pass {f}"
    assert "--offload-arch=gfx950" in quoted


def test_built_library_leaves_no_internal_symbol_undefined():
    import shutil
    import subprocess

    import kvad_amd

    if shutil.which("nm") is None:
        import pytest

        pytest.skip("nm is not installed")
    out = subprocess.run(["nm", "-DC", "--undefined-only", str(kvad_amd.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    internal = [l for l in out.splitlines() if "kh::" in l or re.search(r"\bkh_[a-z0-9_]+\b", l)]
    assert not internal, internal
