import json
import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(Path(__file__).resolve().parent))

GOLDEN_DIR = Path(__file__).resolve().parent / "golden"

# Tolerance stated for fp16 attention outputs: max-abs difference.
ATOL = 2e-3


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def golden():
    """Reference-kernel outputs (tests/golden/make_golden.py) and their metadata."""
    arrays = np.load(GOLDEN_DIR / "attention_golden.npz", allow_pickle=False)
    meta = json.loads((GOLDEN_DIR / "attention_golden.json").read_text())
    return arrays, meta


@pytest.fixture(scope="session")
def hip():
    """The built HIP library on a real GPU; the test fails (not skips) without it."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("gpu test run without a GPU")
    from fast_infer_amd import _lib

    lib = _lib.load()
    name = torch.cuda.get_device_properties(0).gcnArchName
    print(f"[gpu] device={torch.cuda.get_device_name(0)} arch={name} lib={_lib.LIB_PATH}",
          flush=True)
    return lib


def banner(msg: str) -> None:
    """Name the case before a GPU step so a crash log shows what was running."""
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()
    os.sync() if hasattr(os, "sync") else None
