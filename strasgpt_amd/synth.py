"""Seeded synthetic model directories for StrasGPT-shaped decoders.

Model shapes are the benchmark configurations (dense Llama/Qwen/Mistral
shapes and one MXFP4 mixture-of-experts decoder) plus tiny shapes used by
the tests. Files are written by the native ``strasgpt-synth`` tool
(strasgpt_amd/csrc/synth_model.c): values are a pure function of (seed,
tensor name, index), so every host writes identical bytes.
"""
from __future__ import annotations

import dataclasses
import json
import os
import struct
import subprocess
from typing import Dict, List, Optional

import numpy as np

from . import _paths


@dataclasses.dataclass(frozen=True)
class ModelShape:
    name: str
    dim: int
    hidden: int
    layers: int
    heads: int
    kv_heads: int
    head_dim: int
    vocab: int
    theta: float
    eps: float
    prompt_len: int
    decode_len: int
    qk_norm: bool = False
    untied: bool = False
    experts: int = 0
    experts_per_tok: int = 0
    model_type: str = "llama"
    ctx: Optional[int] = None
    std: float = 0.02
    rope_interleaved: bool = False

    @property
    def context_len(self) -> int:
        return self.ctx if self.ctx is not None else self.prompt_len + self.decode_len

    def weight_bytes(self) -> int:
        d, hd, H = self.dim, self.head_dim, self.hidden
        attn = (self.heads + 2 * self.kv_heads) * hd * d * 2 + d * self.heads * hd * 2
        if self.experts:
            ffn = self.experts * d * 2 + self.experts * 3 * H * d * 17 // 32
        else:
            ffn = 3 * H * d * 2
        emb = self.vocab * d * 2 * (2 if self.untied else 1)
        return emb + self.layers * (attn + ffn)


# Benchmark shapes (random-init, bf16 N(0, 0.02), norms 1.0).
PRESETS: Dict[str, ModelShape] = {
    # Llama-3.2-1B-shaped: 8-token prompt, 16 decode tokens.
    "llama3.2-1b": ModelShape("llama3.2-1b", 2048, 8192, 16, 32, 8, 64, 128256,
                              500000.0, 1e-5, 8, 16),
    # Qwen3-4B-shaped with per-head QK RMSNorm: 512-token prompt, 128 decode.
    "qwen3-4b": ModelShape("qwen3-4b", 2560, 9728, 36, 32, 8, 128, 151936,
                           1000000.0, 1e-6, 512, 128, qk_norm=True,
                           model_type="qwen3"),
    # Llama-3.1-8B-shaped, untied: 8192-token prompt, 256 decode.
    "llama3.1-8b": ModelShape("llama3.1-8b", 4096, 14336, 32, 32, 8, 128, 128256,
                              500000.0, 1e-5, 8192, 256, untied=True),
    # MXFP4 MoE: 32 experts, top-4, expert FFN 2880: 256-token prompt, 128 decode.
    "moe-mxfp4": ModelShape("moe-mxfp4", 2880, 2880, 24, 64, 8, 64, 201088,
                            150000.0, 1e-5, 256, 128, untied=True, experts=32,
                            experts_per_tok=4, model_type="stras_moe"),
    # Mistral-Small-24B-shaped: 2048-token prompt, 128 decode.
    "mistral-small-24b": ModelShape("mistral-small-24b", 5120, 32768, 40, 32, 8, 128,
                                    131072, 100000000.0, 1e-5, 2048, 128,
                                    untied=True, model_type="mistral"),
}

# Tiny shapes for CPU golden fixtures and fast GPU parity cases. Their
# weights use std 0.25: at 0.02 such small models collapse into repeating
# one token, which would make greedy-token checks vacuous.
TINY: Dict[str, ModelShape] = {
    "tiny-llama": ModelShape("tiny-llama", 64, 128, 2, 4, 2, 16, 256, 10000.0, 1e-5,
                             8, 8, std=0.25),
    "tiny-qwen": ModelShape("tiny-qwen", 96, 192, 3, 6, 2, 32, 300, 1000000.0, 1e-6,
                            12, 8, qk_norm=True, untied=True, model_type="qwen3",
                            std=0.25),
    "tiny-chunk": ModelShape("tiny-chunk", 64, 96, 2, 4, 1, 32, 128, 500000.0, 1e-5,
                             520, 4, ctx=600, std=0.25),
    # Long context, 8 query heads on one kv head: decode attention over
    # 32 key chunks of more than one 64-key tile each.
    "tiny-long": ModelShape("tiny-long", 64, 96, 2, 8, 1, 32, 128, 500000.0, 1e-5,
                            2200, 6, ctx=2300, std=0.25),
    "tiny-moe": ModelShape("tiny-moe", 64, 64, 2, 4, 2, 16, 256, 150000.0, 1e-5, 8, 8,
                           untied=True, experts=8, experts_per_tok=2,
                           model_type="stras_moe", std=0.25),
    # Enough prompt tokens for several 32-slot tiles per expert in the
    # grouped prefill GEMMs.
    "tiny-moe-long": ModelShape("tiny-moe-long", 64, 96, 2, 4, 2, 16, 256, 150000.0, 1e-5,
                                200, 10, untied=True, experts=8, experts_per_tok=2,
                                model_type="stras_moe", std=0.25),
    # The MXFP4 MoE benchmark's expert shape (embedding and expert width
    # 2880, top-4) on two layers: decode kernels with full-length rows.
    # Weight std 0.02 as in the benchmark (at 0.25 and this width the
    # attention scores reach the hundreds and amplify rounding noise).
    "mid-moe": ModelShape("mid-moe", 2880, 2880, 2, 8, 2, 64, 512, 150000.0, 1e-5, 6, 10,
                          untied=True, experts=8, experts_per_tok=4, model_type="stras_moe",
                          std=0.02),
    # Prefill GEMM grids that the 256 x 256 kernel's XCD rectangles divide
    # (512 rows: 2 row tiles; QKV 12, O 4, gate/up 16, down 4 column tiles).
    "mid-dense": ModelShape("mid-dense", 1024, 2048, 1, 8, 8, 128, 512, 500000.0, 1e-5,
                            512, 4, ctx=600, untied=True, std=0.02),
    # A short prompt on wide rows: the QKV prefill GEMM takes the split-K
    # form with the separate epilogue (8 rows, 4 splits).
    "small-m": ModelShape("small-m", 1024, 2048, 2, 8, 2, 128, 512, 500000.0, 1e-5,
                          8, 6, ctx=64, untied=True, std=0.02),
    # FFN rows longer than one LDS stage of the decode GEMV (64 KiB of
    # fp32): the down projection takes the split-K form, in 3 ranges of
    # 14 steps (20480 = 40 steps of 512, the last range short) or 4 of 16.
    "tiny-wide": ModelShape("tiny-wide", 64, 20480, 2, 4, 2, 16, 256, 10000.0, 1e-5,
                            8, 6, std=0.05),
    "tiny-wide2": ModelShape("tiny-wide2", 64, 32768, 1, 4, 2, 16, 256, 10000.0, 1e-5,
                             8, 6, std=0.05),
    # Interleaved RoPE pairs (2j, 2j + 1), written as
    # rope_scaling.mrope_interleaved = true, with QK RMSNorm.
    "tiny-rope-il": ModelShape("tiny-rope-il", 96, 192, 3, 6, 2, 32, 300, 10000.0, 1e-5,
                               12, 8, qk_norm=True, model_type="qwen3", std=0.25,
                               rope_interleaved=True),
    # Interleaved RoPE with head_dim 128 and no QK-norm, over a prompt longer
    # than one 32-key decode attention tile (std 0.1: at 0.25 the attention
    # scores have a standard deviation near 16 at this head size).
    "tiny-rope-il128": ModelShape("tiny-rope-il128", 256, 256, 2, 4, 2, 128, 200, 500000.0,
                                  1e-5, 80, 6, untied=True, std=0.1, rope_interleaved=True),
}


# The benchmark shapes at full width and full prompt/decode length but only
# two layers: small enough for the CPU oracle to run the whole workload
# (every prefill chunk, every decode step) in seconds to minutes.
TRUNCATED: Dict[str, ModelShape] = {
    f"{n}-2l": dataclasses.replace(PRESETS[n], name=f"{n}-2l", layers=2)
    for n in ("llama3.1-8b", "moe-mxfp4", "mistral-small-24b")
}


def shape(name: str) -> ModelShape:
    for table in (PRESETS, TINY, TRUNCATED):
        if name in table:
            return table[name]
    raise KeyError(f"unknown model shape {name!r}")


def write_model(shp: ModelShape, out_dir: str, seed: int = 1234,
                shard_bytes: int = 0, threads: Optional[int] = None) -> str:
    """Writes the model directory (config.json, safetensors, tokenizer.json)."""
    exe = _paths.synth_exe()
    args = [exe, "--out", out_dir, "--seed", str(seed), "--dim", str(shp.dim),
            "--hidden", str(shp.hidden), "--layers", str(shp.layers),
            "--heads", str(shp.heads), "--kv-heads", str(shp.kv_heads),
            "--head-dim", str(shp.head_dim), "--vocab", str(shp.vocab),
            "--ctx", str(shp.context_len), "--theta", repr(shp.theta),
            "--eps", repr(shp.eps), "--model-type", shp.model_type,
            "--std", repr(shp.std)]
    if shp.qk_norm:
        args.append("--qk-norm")
    if shp.untied:
        args.append("--untied")
    if shp.rope_interleaved:
        args.append("--rope-interleaved")
    if shp.experts:
        args += ["--experts", str(shp.experts), "--experts-per-tok",
                 str(shp.experts_per_tok)]
    if shard_bytes:
        args += ["--shard-bytes", str(shard_bytes)]
    if threads:
        args += ["--threads", str(threads)]
    subprocess.run(args, check=True)
    return out_dir


def _mix64(z: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = z + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def prompt_tokens(vocab: int, count: int, seed: int = 42) -> List[int]:
    """Uniform-random token ids in [0, vocab): splitmix64 of (seed, i)."""
    i = np.arange(count, dtype=np.uint64)
    with np.errstate(over="ignore"):
        h = _mix64(np.uint64(seed) * np.uint64(0x100000001B3) + i)
    return [int(v) for v in (h % np.uint64(vocab))]


def read_header(path: str):
    """Returns (header_len, header dict) of one .safetensors file."""
    with open(path, "rb") as f:
        (n,) = struct.unpack("<Q", f.read(8))
        return n, json.loads(f.read(n))


def tensor_table(model_dir: str):
    """[(name, dtype, shape, file_path, absolute_offset, size)] in file order."""
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
        hl, hdr = read_header(path)
        for name, t in hdr.items():
            if name == "__metadata__":
                continue
            b, e = t["data_offsets"]
            out.append((name, t["dtype"], tuple(t["shape"]), path, 8 + hl + b, e - b))
    return out
