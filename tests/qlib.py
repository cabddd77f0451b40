"""Imports the library's Python host mirror (llm-project_amd/qllama.py) by path."""
import importlib.util
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "llm-project_amd")


def load():
    if "qllama" in sys.modules:
        return sys.modules["qllama"]
    spec = importlib.util.spec_from_file_location("qllama", os.path.join(PKG, "qllama.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules["qllama"] = mod
    spec.loader.exec_module(mod)
    return mod


def gpu_available():
    try:
        return load().lib().qllama_device_count() > 0
    except Exception:
        return False
