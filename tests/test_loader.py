"""The product's safetensors loader (strasgpt_amd/csrc/safetensors.c),
checked against Python's json reading of the same files, plus the error
paths of the reference's die-on-error convention (run in subprocesses)."""
import ctypes
import json
import os
import struct
import subprocess
import sys
import textwrap

import pytest

from conftest import REPO
from strasgpt_amd import _paths, synth

pytestmark = pytest.mark.skipif(not os.path.exists(_paths.hip_lib()), reason="library not built")


class Tensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("type", ctypes.c_int),
                ("dim_count", ctypes.c_size_t), ("dim", ctypes.c_size_t * 8),
                ("size", ctypes.c_size_t), ("file", ctypes.c_size_t),
                ("offset", ctypes.c_size_t)]


class Safetensors(ctypes.Structure):
    _fields_ = [("model_type", ctypes.c_char_p), ("embedding_dim", ctypes.c_size_t),
                ("head_dim", ctypes.c_size_t), ("hidden_dim", ctypes.c_size_t),
                ("layer_count", ctypes.c_size_t), ("q_head_count", ctypes.c_size_t),
                ("kv_head_count", ctypes.c_size_t), ("vocabulary_len", ctypes.c_size_t),
                ("context_len", ctypes.c_size_t), ("epsilon", ctypes.c_float),
                ("rope_theta", ctypes.c_float), ("rope_interleaved", ctypes.c_bool),
                ("mrope_section_count", ctypes.c_size_t),
                ("mrope_section", ctypes.c_size_t * 8), ("bos_token_id", ctypes.c_int),
                ("eos_token_id", ctypes.c_int), ("file_count", ctypes.c_size_t),
                ("file", ctypes.c_char_p * 64), ("tensor_count", ctypes.c_size_t),
                ("tensor", Tensor * 65536), ("expert_count", ctypes.c_size_t),
                ("expert_used_count", ctypes.c_size_t)]


def load(model_dir):
    lib = ctypes.CDLL(_paths.hip_lib())
    lib.safetensors_read_dir.restype = ctypes.POINTER(Safetensors)
    lib.safetensors_read_dir.argtypes = [ctypes.c_char_p]
    lib.safetensors_free.argtypes = [ctypes.c_void_p]
    p = lib.safetensors_read_dir(model_dir.encode())
    return lib, p


@pytest.mark.parametrize("name,shard", [("tiny-qwen", 0), ("tiny-qwen", 20000),
                                        ("tiny-moe", 0)])
def test_loader_matches_python(name, shard, model_dir):
    d = model_dir(name, shard_bytes=shard)
    lib, p = load(d)
    s = p.contents
    cfg = json.load(open(os.path.join(d, "config.json")))
    assert s.embedding_dim == cfg["hidden_size"]
    assert s.head_dim == cfg["head_dim"]
    assert s.hidden_dim == cfg["intermediate_size"]
    assert s.layer_count == cfg["num_hidden_layers"]
    assert s.q_head_count == cfg["num_attention_heads"]
    assert s.kv_head_count == cfg["num_key_value_heads"]
    assert s.vocabulary_len == cfg["vocab_size"]
    assert s.context_len == cfg["max_position_embeddings"]
    assert abs(s.epsilon - cfg["rms_norm_eps"]) <= 1e-12
    assert s.rope_theta == pytest.approx(cfg["rope_theta"])
    assert s.eos_token_id == cfg["eos_token_id"]
    assert s.expert_count == cfg.get("num_local_experts", 0)
    table = synth.tensor_table(d)
    assert s.tensor_count == len(table)
    files = []
    for t in table:
        if t[3] not in files:
            files.append(t[3])
    assert s.file_count == len(files) == (1 if shard == 0 else s.file_count)
    for i, (nm, dt, shp, path, off, size) in enumerate(table):
        t = s.tensor[i]
        assert t.name.decode() == nm
        assert ["F16", "BF16", "F32", "U8"][t.type] == dt
        assert list(t.dim[:t.dim_count]) == list(shp)
        assert (t.offset, t.size) == (off, size)
        assert s.file[t.file].decode() == path
    lib.safetensors_free(p)


def write_min_model(d, config, header_obj=None, dtype="BF16"):
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, "config.json"), "w") as f:
        f.write(config)
    hdr = header_obj or {"model.norm.weight": {"dtype": dtype, "shape": [4], "data_offsets": [0, 8]}}
    h = json.dumps(hdr).encode()
    end = max(v["data_offsets"][1] for k, v in hdr.items() if k != "__metadata__")
    with open(os.path.join(d, "model.safetensors"), "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h + b"\0" * end)


def run_loader(d):
    code = textwrap.dedent(f"""
        import ctypes
        lib = ctypes.CDLL({_paths.hip_lib()!r})
        lib.safetensors_read_dir.restype = ctypes.c_void_p
        lib.safetensors_read_dir.argtypes = [ctypes.c_char_p]
        lib.safetensors_read_dir({d!r}.encode())
        print("LOADED")
    """)
    return subprocess.run([sys.executable, "-c", code], capture_output=True, text=True)


def test_config_semantics(tmp_path):
    d = str(tmp_path / "m")
    write_min_model(d, '{"hidden_size": 64, "num_attention_heads": 4, "rms_norm_eps": 1e-06,'
                       ' "rope_theta": 1e6, "text_config": {"num_hidden_layers": 3},'
                       ' "rope_scaling": {"mrope_section": [2, 3], "mrope_interleaved": true},'
                       ' "eos_token_id": [7, 8], "unknown": {"model": [1, {"vocab": null}]}}',
                    header_obj={"__metadata__": {"format": "pt"},
                                "model.norm.weight": {"dtype": "BF16", "shape": [4],
                                                      "data_offsets": [24, 32]}})
    lib, p = load(d)
    s = p.contents
    assert s.head_dim == 16  # hidden_size / heads default (json_parser.y:616-619)
    assert s.layer_count == 3
    assert s.rope_interleaved
    assert list(s.mrope_section[:s.mrope_section_count]) == [2, 3]
    assert s.eos_token_id == 7
    # file offset of a tensor = 8 + header length + data_offsets begin
    hl, hdr = synth.read_header(os.path.join(d, "model.safetensors"))
    assert hdr["model.norm.weight"]["data_offsets"] == [24, 32]
    assert s.tensor_count == 1 and s.tensor[0].offset == 8 + hl + 24
    assert s.tensor[0].size == 8


@pytest.mark.parametrize("config,msg", [
    ('{"hidden_size": 64.5}', "non integer"),
    ('{"hidden_size": 64', "syntax error"),
])
def test_config_errors_exit(tmp_path, config, msg):
    d = str(tmp_path / "m")
    write_min_model(d, config)
    r = run_loader(d)
    assert r.returncode == 1 and "LOADED" not in r.stdout
    assert "[StrasGPT] Error" in r.stderr and msg in r.stderr


def test_missing_config_exits(tmp_path):
    r = run_loader(str(tmp_path))
    assert r.returncode == 1 and "failed to open file" in r.stderr


def test_unknown_dtype_exits(tmp_path):
    d = str(tmp_path / "m")
    write_min_model(d, '{"hidden_size": 64}', dtype="F8_E4M3")
    r = run_loader(d)
    assert r.returncode == 1 and "unknown data type" in r.stderr
