"""Loads the engine's Python modules (fhe-ssm_amd/*.py) by path: the package directory name is not a
Python identifier, so the directory goes on sys.path and its modules import each other by name."""
import importlib
import importlib.util
import os
import sys

_REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
_PKG = os.path.join(_REPO, "fhe-ssm_amd")
_PATH = os.path.join(_PKG, "ckks.py")


def load_ckks():
    spec = importlib.util.spec_from_file_location("fhe_ssm_amd_ckks", _PATH)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def load_module(name: str):
    if _PKG not in sys.path:
        sys.path.insert(0, _PKG)
    return importlib.import_module(name)
