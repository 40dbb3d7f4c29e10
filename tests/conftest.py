"""Shared fixtures: repository on sys.path, the ``gpu`` marker, golden vectors."""

import gzip
import json
import sys
from functools import lru_cache
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden" / "lvsa_mask_golden.json.gz"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@lru_cache(maxsize=1)
def load_golden():
    with gzip.open(GOLDEN, "rt") as fh:
        return json.load(fh)


@pytest.fixture(scope="session")
def golden():
    return load_golden()


@pytest.fixture(scope="session")
def gpu():
    """The GPU device; GPU tests fail (not skip) when there is none."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("test marked gpu but no GPU is visible")
    from longvideosparseattention_amd import _capi

    _capi.lib()  # fail loudly when the HIP library is missing
    return torch.device("cuda", 0)
