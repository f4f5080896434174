"""The library driver's report flags (no device work): --show-safetensors
and --show-model print what the reference driver prints after its options
block (source/strasgpt.c:98-110), both drivers reading the model through the
library's safetensors reader."""
import os
import subprocess

import pytest

from conftest import REPO

REF_DRIVER = os.path.join(REPO, "oracle", "_ref", "ref_driver_hip")


@pytest.mark.skipif(not os.path.exists(REF_DRIVER),
                    reason="reference driver not built (needs the reference sources when building)")
@pytest.mark.parametrize("flag", ["--show-safetensors", "--show-model"])
def test_show_flags_match_reference_driver(flag, model_dir):
    from strasgpt_amd import _paths
    d = model_dir("tiny-qwen", shard_bytes=4096)
    out = {}
    for key, prog in (("ref", REF_DRIVER), ("lib", _paths.driver_exe())):
        r = subprocess.run([prog, "-m", d, flag], capture_output=True, text=True, timeout=60)
        assert r.returncode == 0, r.stderr[-2000:]
        out[key] = r.stderr
    assert out["lib"].strip()
    assert out["ref"].endswith(out["lib"])
