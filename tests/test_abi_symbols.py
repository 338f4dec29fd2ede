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


# ---- the decode-step driver (libfhe_ssm_decode.so, include/fhe_ssm_decode.h): host code over the engine's ABI
def decoder_declared():
    text = open(os.path.join(REPO, "include", "fhe_ssm_decode.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fhe_ssm_\w+)\s*\(", text)))


def test_decoder_library_exports_its_header():
    from engine_loader import load_module
    ND = load_module("native_decode")
    ND.load()
    names = decoder_declared()
    assert "fhe_ssm_decoder_step" in names
    out = subprocess.run(["nm", "-D", "--defined-only", ND.LIB_PATH], capture_output=True, text=True).stdout
    assert set(names) <= set(re.findall(r"\bT (fhe_ssm_\w+)", out))
    assert set(names) == set(ND.SIGNATURES)


def test_decoder_is_host_code_over_the_engine_abi():
    """the driver links the engine library and nothing of the oracle, and carries no device code"""
    from engine_loader import load_module
    ND = load_module("native_decode")
    ldd = subprocess.run(["ldd", ND.LIB_PATH], capture_output=True, text=True).stdout
    assert "libckks_hip.so" in ldd and "liboracle" not in ldd
    undefined = subprocess.run(["nm", "-D", "--undefined-only", ND.LIB_PATH], capture_output=True, text=True).stdout
    assert not re.search(r"\bhip\w*", undefined), "the driver must reach the GPU only through ckks_* calls"
    assert re.search(r"\bckks_eval_bootstrap_many\b", undefined)


def test_decoder_rotation_steps_match_the_plan():
    """the native driver's rotation-step set (host logic, no device) equals the Python plan's"""
    from engine_loader import load_module
    ND = load_module("native_decode")
    M = load_module("rwkv_model")
    assert ND.rotation_steps() == M.rotation_steps()
