"""Test setup: the `gpu` marker, and the package and the oracle loaded by path.

The package directory is `xn-ptts_amd` (a hyphen), so it is loaded under the module name
`xn_ptts_amd`; the oracle (the CPU restatement used as the checker) under `oracle`.
"""
import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _load(name, path):
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, os.path.join(path, "__init__.py")
                                                  if os.path.isdir(path) else path,
                                                  submodule_search_locations=[path] if os.path.isdir(path) else None)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


xnp = _load("xn_ptts_amd", os.path.join(ROOT, "xn-ptts_amd"))
oracle = _load("oracle", os.path.join(ROOT, "oracle", "oracle.py"))
sys.path.insert(0, os.path.join(ROOT, "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def pytest_collection_modifyitems(config, items):
    # A GPU test on a machine without one fails loudly rather than skipping: the product path
    # has no CPU fallback.  Deselect them with -m "not gpu".
    pass
