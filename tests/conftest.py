"""Shared fixtures.  GPU tests are marked `gpu`; everything else runs on CPU."""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
TESTS = Path(__file__).resolve().parent
for p in (str(ROOT), str(ROOT / "oracle"), str(TESTS), str(TESTS / "golden")):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = TESTS / "golden" / "ref_vectors.npz"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def _ensure_oracle() -> None:
    so = ROOT / "oracle" / "liboracle.so"
    if not so.exists():
        subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], check=True)


def _ensure_lib() -> None:
    if not (ROOT / "yllm_amd" / "libyllm_hip.so").exists():
        from yllm_amd.build import build

        build(verbose=False)


@pytest.fixture(scope="session")
def oracle():
    _ensure_oracle()
    from oracle_lib import Oracle

    return Oracle()


@pytest.fixture(scope="session")
def ref():
    from oracle_lib import REF_SO, Ref

    if not REF_SO.exists():
        ref_tree = Path("/root/reference/inference/core/engine.c")
        if ref_tree.exists():
            subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), "ref"], check=True)
        else:
            pytest.skip("reference build oracle/_ref not available here; golden fixtures cover it")
    return Ref()


@pytest.fixture(scope="session")
def golden():
    return dict(np.load(GOLDEN))


@pytest.fixture(scope="session")
def hiplib():
    _ensure_lib()
    from yllm_amd._lib import lib

    return lib()


@pytest.fixture(scope="session")
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    name = torch.cuda.get_device_properties(0).gcnArchName
    assert "gfx950" in name, f"expected gfx950, got {name}"
    _ensure_lib()
    return torch.device("cuda:0")
