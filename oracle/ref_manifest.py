"""ORACLE — test infrastructure, not part of the product.

Manifest of a model directory for oracle/ref_harness.c (the StrasGPT
reference's own C sources, built into oracle/_ref/): the configuration the
reference parser would read (config.json keys, rope_scaling's
mrope_interleaved), the safetensors files and every tensor's
(file, absolute offset, size), the prompt and the step count. Used by
tests/golden/make_golden.py and by bench.py's CPU baseline.
"""
import json
import os
import struct
from typing import List, Sequence

_HERE = os.path.dirname(os.path.abspath(__file__))
HARNESS = os.path.join(_HERE, "_ref", "ref_harness")
BASELINE = os.path.join(_HERE, "_ref", "ref_baseline")


def _tensor_table(model_dir: str):
    idx = os.path.join(model_dir, "model.safetensors.index.json")
    if os.path.exists(idx):
        files: List[str] = []
        for f in json.load(open(idx))["weight_map"].values():
            if f not in files:
                files.append(f)
    else:
        files = ["model.safetensors"]
    out = []
    for f in files:
        path = os.path.join(model_dir, f)
        with open(path, "rb") as fh:
            (hl,) = struct.unpack("<Q", fh.read(8))
            hdr = json.loads(fh.read(hl))
        for name, t in hdr.items():
            if name in ("__metadata__", "metadata"):
                continue
            b, e = t["data_offsets"]
            out.append((name, path, 8 + hl + b, e - b))
    return out


def write(model_dir: str, prompt: Sequence[int], steps: int, path: str = None) -> str:
    cfg = json.load(open(os.path.join(model_dir, "config.json")))
    table = _tensor_table(model_dir)
    files: List[str] = []
    for t in table:
        if t[1] not in files:
            files.append(t[1])
    head_dim = cfg.get("head_dim") or cfg["hidden_size"] // cfg["num_attention_heads"]
    inter = int(bool((cfg.get("rope_scaling") or {}).get("mrope_interleaved", False)))
    lines = [" ".join(str(v) for v in (
        cfg["hidden_size"], head_dim, cfg["intermediate_size"],
        cfg["num_hidden_layers"], cfg["num_attention_heads"],
        cfg["num_key_value_heads"], cfg["vocab_size"],
        cfg["max_position_embeddings"], repr(cfg["rms_norm_eps"]),
        repr(cfg["rope_theta"]), inter))]
    lines.append(f"{len(files)} " + " ".join(files))
    lines.append(str(len(table)))
    lines += [f"{n} {files.index(p)} {o} {s}" for n, p, o, s in table]
    lines.append(f"{len(prompt)} " + " ".join(map(str, prompt)))
    lines.append(str(steps))
    path = path or os.path.join(model_dir, "manifest.txt")
    with open(path, "w") as f:
        f.write("\n".join(lines) + "\n")
    return path
