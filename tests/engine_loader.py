"""Loads the engine's Python front end (fhe-ssm_amd/ckks.py) by path: the package directory name
is not a Python identifier."""
import importlib.util
import os

_REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
_PATH = os.path.join(_REPO, "fhe-ssm_amd", "ckks.py")


def load_ckks():
    spec = importlib.util.spec_from_file_location("fhe_ssm_amd_ckks", _PATH)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod
