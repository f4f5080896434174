"""The C-ABI library loads and exports every function include/*.h declares
(no compute calls: these run without a GPU)."""
import ctypes
import os
import re

import pytest

from conftest import REPO
from strasgpt_amd import _paths

HEADERS = ["transformer.h", "transformer_hip.h", "safetensors.h", "sampler_hip.h", "strasgpt_kbench.h",
           "tokenizer.h"]


def declared_functions():
    names = set()
    for h in HEADERS:
        text = open(os.path.join(REPO, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w \*]*?\b([a-z_][a-z0-9_]*)\s*\(", text, re.M):
            name = m.group(1)
            if name not in ("if", "sizeof", "defined"):
                names.add(name)
    return sorted(names)


def test_headers_declare_the_reference_api():
    names = declared_functions()
    for ref in ["transformer_from_safetensors", "transformer_free", "transformer_print",
                "transformer_logits_malloc", "transformer_predict", "safetensors_read",
                "safetensors_free", "safetensors_aliased_out_weight"]:
        assert ref in names


@pytest.mark.skipif(not os.path.exists(_paths.hip_lib()), reason="library not built")
def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_paths.hip_lib())
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    assert hasattr(lib, "safetensors_type_str")


@pytest.mark.skipif(not os.path.exists(_paths.hip_lib()), reason="library not built")
def test_version_string_names_gfx950():
    from strasgpt_amd import runtime
    assert "gfx950" in runtime.version()


def test_config_struct_layout_matches_reference_prefix():
    """transformer_configuration_t keeps the reference field order
    (include/transformer.h:11-28): vocabulary_len at byte 48."""
    from strasgpt_amd.runtime import TransformerConfig
    assert TransformerConfig.vocabulary_len.offset == 48
    assert TransformerConfig.aliased_out_weight.offset == 112


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU; --gpus N > 1 exits with a message (the
    path has no multi-GPU form)."""
    import json
    import subprocess
    import sys
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "exactly one GPU" in json.loads(r.stdout.strip().splitlines()[-1])["error"]
