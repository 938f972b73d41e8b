import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import __graft_entry__  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def pytest_report_header(config):
    """Names the library the session tests and the sources it was built from."""
    try:
        pkg = __graft_entry__.load_package()
        from qwen_mlp_amd import _lib

        return [f"libqwen_mlp: {pkg.lib().qmlp_version().decode()} (tree src={_lib.tree_source_hash()})"]
    except Exception as e:  # a missing or stale library: the pkg fixture raises with the reason
        return [f"libqwen_mlp: not loadable ({e})"]


def _ensure_built():
    """Builds a missing library; a stale one (stamped with other sources) makes pkg.lib() raise."""
    from importlib import import_module

    lib_path = os.path.join(__graft_entry__.PKG_DIR, "libqwen_mlp.so")
    if not os.path.exists(lib_path):
        __graft_entry__.build()
    oracle_lib = os.path.join(ROOT, "oracle", "_build", "liboracle_bfp8.so")
    if not os.path.exists(oracle_lib):
        import_module("oracle.c_oracle").build()


@pytest.fixture(scope="session")
def pkg():
    _ensure_built()
    return __graft_entry__.load_package()


@pytest.fixture(scope="session")
def cuda(pkg):
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    return torch.device("cuda:0")
