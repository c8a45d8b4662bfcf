"""CPU checks of the C-ABI library: it loads, exports exactly what
include/wohper_hip.h declares, and its host-only entry points behave."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

import wohper_amd

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    text = (ROOT / "include" / "wohper_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(wh_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = wohper_amd.load_library()
    decl = declared_symbols()
    assert len(decl) >= 20
    for name in decl:
        assert hasattr(lib, name), name
    assert sorted(wohper_amd.EXPORTED) == decl


def test_status_strings_mirror_reference_error_enum():
    lib = wohper_amd.load_library()
    # DeepSeekV4KernelError order, E/deepseek_v4.rs:398-408
    ref = ["EmptyShape", "InvalidShape", "PackedWeightTooSmall", "ScaleTooSmall", "InputTooSmall",
           "OutputTooSmall", "ScratchTooSmall", "NonFiniteOutput"]
    for code, name in enumerate(ref, start=1):
        assert lib.wh_status_string(code).decode() == name
        assert wohper_amd.STATUS_NAMES[code] == name
    assert b"gfx950" in lib.wh_build_info()


def test_synthetic_generator_is_deterministic_and_in_range():
    lib = wohper_amd.load_library()
    from wohper_amd.workloads import synth_fp4_host

    a = synth_fp4_host(lib, 5, 3, 17, 2, 64, 256)
    b = synth_fp4_host(lib, 5, 3, 17, 2, 64, 256)
    c = synth_fp4_host(lib, 5, 3, 18, 2, 64, 256)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
    assert not np.array_equal(a[0], c[0])
    assert a[1].min() >= 119 and a[1].max() <= 127
    # packed bytes are close to uniform
    hist = np.bincount(a[0].reshape(-1), minlength=256)
    assert hist.min() > 0


def test_null_arguments_are_rejected_without_a_device():
    lib = wohper_amd.load_library()
    assert lib.wh_init(0, None) == 13
    assert lib.wh_synchronize(None) == 13
    assert lib.wh_shutdown(None) == 13


def test_oracle_is_not_imported_by_the_product():
    for p in (ROOT / "wohper_amd").rglob("*"):
        if p.suffix in (".py", ".hip", ".h", ".c", ".cpp"):
            assert "oracle" not in p.read_text().replace("test", ""), p


def _c_prototypes():
    text = (ROOT / "include" / "wohper_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    protos = {}
    for m in re.finditer(r"\n(?:int|void|const char\*)\s+(wh_\w+)\s*\(([^;]*)\);", text):
        params = m.group(2).strip()
        protos[m.group(1)] = 0 if params in ("", "void") else len(params.split(","))
    return protos


def test_rust_binding_matches_the_header():
    """ffi/rust (not compiled in this image) declares every non-debug entry
    point of the header with the same parameter count, and its Status enum
    follows the header's codes in order."""
    protos = _c_prototypes()
    sys_rs = (ROOT / "ffi" / "rust" / "src" / "sys.rs").read_text()
    decl = {}
    for m in re.finditer(r"pub fn (wh_\w+)\((.*?)\)(?: -> [^;]+)?;", sys_rs, flags=re.S):
        args = " ".join(m.group(2).split())
        decl[m.group(1)] = 0 if not args else len([a for a in args.split(",") if a.strip()])
    wanted = {k: v for k, v in protos.items() if not k.startswith("wh_debug_")}
    assert decl == wanted
    lib_rs = (ROOT / "ffi" / "rust" / "src" / "lib.rs").read_text()
    header = (ROOT / "include" / "wohper_hip.h").read_text()
    codes = {int(v): k for k, v in re.findall(r"\b(WH_[A-Z0-9_]+) = (\d+)", header.split("enum wh_status")[1].split("};")[0])}
    arms = dict((int(c), n) for c, n in re.findall(r"^\s+(\d+) => (\w+),$", lib_rs, flags=re.M))
    assert sorted(arms) == list(range(1, max(codes) + 1))
    for code, name in arms.items():
        assert codes[code].replace("WH_", "").replace("_", "").lower() == name.lower() or \
            (code == 22 and name == "Io"), (code, name, codes[code])
