"""Shared pytest setup.

* registers the ``gpu`` marker (tests that need an MI355X);
* puts the repository root on ``sys.path`` so ``oracle.oracle`` imports;
* loads the product package from the ``whisper.rs_amd/`` directory under the
  module name ``wrs_amd`` (the directory name is not a Python identifier).
"""
from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def load_wrs_amd():
    if "wrs_amd" in sys.modules:
        return sys.modules["wrs_amd"]
    pkg_dir = ROOT / "whisper.rs_amd"
    spec = importlib.util.spec_from_file_location(
        "wrs_amd", pkg_dir / "__init__.py", submodule_search_locations=[str(pkg_dir)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["wrs_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct MI355X (gfx950)")


@pytest.fixture(scope="session")
def wrs():
    mod = load_wrs_amd()
    # Name the library build this session calls (the in-tree one unless
    # WRS_ATTN_LIB points elsewhere).
    print(f"\n[wrs_amd] library: {mod._lib.LIB_PATH}", flush=True)
    return mod


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle as o
    o.lib()
    return o
