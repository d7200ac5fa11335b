"""Loads the package module (its directory name is not a Python identifier)."""
import importlib.util
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "qwen3.8-27b-in-c_amd")


def _load():
    if "pyqwen" in sys.modules:
        return sys.modules["pyqwen"]
    spec = importlib.util.spec_from_file_location("pyqwen", os.path.join(PKG_DIR, "pyqwen.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules["pyqwen"] = mod
    spec.loader.exec_module(mod)
    return mod


pyqwen = _load()
host_lib = pyqwen.host_lib
