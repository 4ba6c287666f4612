"""Helpers shared by the tests: load the package (its directory name has a
hyphen) and its synthetic-input module by path."""
from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
PKG_DIR = ROOT / "streaming-attention_amd"


def _load(name: str, path: Path, package: bool = False):
    if name in sys.modules:
        return sys.modules[name]
    kw = {"submodule_search_locations": [str(path.parent)]} if package else {}
    spec = importlib.util.spec_from_file_location(name, path, **kw)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def load_pkg():
    return _load("streaming_attention_amd", PKG_DIR / "__init__.py", package=True)


def load_synth():
    return _load("streaming_attention_amd_synth", PKG_DIR / "synth.py")
