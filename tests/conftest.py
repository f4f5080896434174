"""Shared test fixtures.

`gpu` tests run the HIP library on an MI355X; everything else runs on the
CPU (oracle pins, loader, exported symbols, generator determinism).
"""
import os
import sys
import tempfile

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

from strasgpt_amd import synth  # noqa: E402

GOLDEN_DIR = os.path.join(REPO, "tests", "golden")
MODEL_SEED = 7
PROMPT_SEED = 3


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct MI355X (gfx950)")
    config.addinivalue_line("markers", "slow: full-size model shapes")


def _models_root():
    base = "/dev/shm" if os.path.isdir("/dev/shm") and os.access("/dev/shm", os.W_OK) else None
    return tempfile.mkdtemp(prefix="strasgpt_models_", dir=base)


@pytest.fixture(scope="session")
def models_root():
    root = _models_root()
    yield root
    import shutil
    shutil.rmtree(root, ignore_errors=True)


@pytest.fixture(scope="session")
def model_dir(models_root):
    """Factory: writes (once per session) the named synthetic model."""
    made = {}

    def make(name, shard_bytes=0, seed=MODEL_SEED):
        key = (name, shard_bytes, seed)
        if key not in made:
            d = os.path.join(models_root, f"{name}-{shard_bytes}-{seed}")
            synth.write_model(synth.shape(name), d, seed=seed, shard_bytes=shard_bytes)
            made[key] = d
        return made[key]

    return make
