"""CPU-side checks of the C ABI: the library loads and exports every entry point that
include/ckks_engine.h declares (no compute calls: there is no GPU here)."""
import os
import re
import subprocess

from conftest import REPO
from engine_loader import load_ckks


def declared_functions():
    names = []
    for fn in sorted(os.listdir(os.path.join(REPO, "include"))):
        if fn.endswith(".h"):
            text = open(os.path.join(REPO, "include", fn)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            names += re.findall(r"\b(ckks_\w+)\s*\(", text)
    return sorted(set(names))


def test_header_declares_entry_points():
    names = declared_functions()
    assert "ckks_ntt_forward" in names and "ckks_last_error" in names


def test_library_exports_every_declared_symbol():
    ckks = load_ckks()
    lib = ckks.load()
    for n in declared_functions():
        assert hasattr(lib, n), n
    out = subprocess.run(["nm", "-D", "--defined-only", ckks.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (ckks_\w+)", out))
    assert set(declared_functions()) <= exported
    assert set(ckks.SIGNATURES) <= exported


def test_python_front_end_covers_the_header():
    ckks = load_ckks()
    assert set(declared_functions()) == set(ckks.SIGNATURES)


def test_library_does_not_link_the_oracle():
    ckks = load_ckks()
    out = subprocess.run(["nm", "-D", ckks.LIB_PATH], capture_output=True, text=True).stdout
    assert "or_ntt_fwd" not in out and "liboracle" not in subprocess.run(
        ["ldd", ckks.LIB_PATH], capture_output=True, text=True).stdout
