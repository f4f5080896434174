"""ORACLE — test infrastructure, not part of the product.

ctypes wrapper of liboracle.so. The model directory is read here with
Python's json module (independently of the product's C loader): config.json
keys as the reference reads them (json_scanner.l:27-50), tensor names
matched to weight classes like the reference's loading table
(source/transformer.c:513-625, including the Qwen3-VL
"model.language_model." aliases), tied output when no lm_head.weight
exists (source/safetensors.c:421-429).
"""
from __future__ import annotations

import ctypes
import json
import os
import re
import struct
from typing import List, Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

CLASSES = [
    "EMBEDDING", "MHA_NORM", "Q", "Q_NORM", "K", "K_NORM", "V", "O", "FFN_NORM",
    "GATE", "UP", "DOWN", "OUT_NORM", "OUT", "ROUTER", "GATE_BLOCKS",
    "GATE_SCALES", "UP_BLOCKS", "UP_SCALES", "DOWN_BLOCKS", "DOWN_SCALES",
]
CLS = {n: i for i, n in enumerate(CLASSES)}

_LAYER = {
    "input_layernorm.weight": "MHA_NORM",
    "self_attn.q_proj.weight": "Q",
    "self_attn.q_norm.weight": "Q_NORM",
    "self_attn.k_proj.weight": "K",
    "self_attn.k_norm.weight": "K_NORM",
    "self_attn.v_proj.weight": "V",
    "self_attn.o_proj.weight": "O",
    "post_attention_layernorm.weight": "FFN_NORM",
    "mlp.gate_proj.weight": "GATE",
    "mlp.up_proj.weight": "UP",
    "mlp.down_proj.weight": "DOWN",
    "mlp.router.weight": "ROUTER",
    "mlp.experts.gate_proj_blocks": "GATE_BLOCKS",
    "mlp.experts.gate_proj_scales": "GATE_SCALES",
    "mlp.experts.up_proj_blocks": "UP_BLOCKS",
    "mlp.experts.up_proj_scales": "UP_SCALES",
    "mlp.experts.down_proj_blocks": "DOWN_BLOCKS",
    "mlp.experts.down_proj_scales": "DOWN_SCALES",
}
_GLOBAL = {
    "model.embed_tokens.weight": "EMBEDDING",
    "model.language_model.embed_tokens.weight": "EMBEDDING",
    "model.norm.weight": "OUT_NORM",
    "model.language_model.norm.weight": "OUT_NORM",
    "lm_head.weight": "OUT",
}
_LAYER_RE = re.compile(r"^model\.(?:language_model\.)?layers\.(\d+)\.(.+)$")


class OracleConfig(ctypes.Structure):
    _fields_ = [
        ("embedding_dim", ctypes.c_size_t), ("head_dim", ctypes.c_size_t),
        ("hidden_dim", ctypes.c_size_t), ("layer_count", ctypes.c_size_t),
        ("q_head_count", ctypes.c_size_t), ("kv_head_count", ctypes.c_size_t),
        ("vocabulary_len", ctypes.c_size_t), ("context_len", ctypes.c_size_t),
        ("epsilon", ctypes.c_float), ("rope_theta", ctypes.c_float),
        ("rope_interleaved", ctypes.c_int), ("qk_norm", ctypes.c_int),
        ("tied", ctypes.c_int), ("expert_count", ctypes.c_size_t),
        ("expert_used_count", ctypes.c_size_t),
    ]


def _lib_path() -> str:
    return os.path.join(_HERE, "liboracle.so")


def oracle_available() -> bool:
    return os.path.exists(_lib_path())


def load_lib():
    global _LIB
    if _LIB is not None:
        return _LIB
    lib = ctypes.CDLL(_lib_path())
    P = ctypes.c_void_p
    sz = ctypes.c_size_t
    fp = ctypes.POINTER(ctypes.c_float)
    ip = ctypes.POINTER(ctypes.c_int)
    lib.oracle_create.restype = P
    lib.oracle_create.argtypes = [ctypes.POINTER(OracleConfig)]
    lib.oracle_load_tensor.argtypes = [P, ctypes.c_int, sz, ctypes.c_char_p, sz, sz]
    lib.oracle_finalize.argtypes = [P]
    lib.oracle_free.argtypes = [P]
    lib.oracle_reset.argtypes = [P]
    lib.oracle_cached_count.argtypes = [P]
    lib.oracle_cached_count.restype = sz
    lib.oracle_set_threads.argtypes = [ctypes.c_int]
    lib.oracle_predict.argtypes = [P, sz, ip, sz, fp]
    lib.oracle_capture_hidden.argtypes = [P, fp, fp]
    lib.oracle_capture_router_margin.argtypes = [P, fp]
    lib.oracle_argmax.argtypes = [fp, sz]
    lib.oracle_argmax.restype = sz
    lib.oracle_bf16_to_f32.argtypes = [ctypes.c_uint16]
    lib.oracle_bf16_to_f32.restype = ctypes.c_float
    lib.oracle_bf16_to_f32_array.argtypes = [P, sz, fp]
    lib.oracle_mxfp4_value.argtypes = [ctypes.c_uint8, ctypes.c_uint8]
    lib.oracle_mxfp4_value.restype = ctypes.c_float
    lib.oracle_mxfp4_dequant.argtypes = [P, P, sz, fp]
    lib.oracle_dot_bf16.argtypes = [sz, fp, P]
    lib.oracle_dot_bf16.restype = ctypes.c_float
    lib.oracle_rmsnorm.argtypes = [sz, fp, fp, P, ctypes.c_float]
    lib.oracle_rope_table.argtypes = [sz, sz, ctypes.c_float, ctypes.c_int, fp]
    lib.oracle_attention_row.argtypes = [sz, sz, fp, fp, fp, fp]
    lib.oracle_topk_softmax.argtypes = [sz, fp, sz, ip, fp]
    lib.oracle_set_kv_format.argtypes = [P, ctypes.c_int]
    lib.oracle_sample.argtypes = [ctypes.POINTER(SamplerState), fp, sz, P, ctypes.c_int,
                                  fp, ctypes.POINTER(ctypes.c_double)]
    lib.oracle_sample.restype = sz
    lib.oracle_round_bf16.argtypes = [ctypes.c_float]
    lib.oracle_round_bf16.restype = ctypes.c_float
    lib.oracle_round_fp8_e4m3.argtypes = [ctypes.c_float]
    lib.oracle_round_fp8_e4m3.restype = ctypes.c_float
    _LIB = lib
    return lib


def fptr(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def read_config(model_dir: str) -> dict:
    """config.json as the reference reads it; text_config members override."""
    cfg = json.load(open(os.path.join(model_dir, "config.json")))
    if isinstance(cfg.get("text_config"), dict):
        cfg = {**cfg, **cfg["text_config"]}
    return cfg


def tensor_table(model_dir: str):
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


def classify(name: str):
    if name in _GLOBAL:
        return _GLOBAL[name], 0
    m = _LAYER_RE.match(name)
    if m and m.group(2) in _LAYER:
        return _LAYER[m.group(2)], int(m.group(1))
    return None, None


class SamplerState(ctypes.Structure):
    """oracle_sampler_t (oracle.h)."""
    _fields_ = [("temperature", ctypes.c_float), ("top_k", ctypes.c_size_t),
                ("top_p", ctypes.c_float), ("presence_penalty", ctypes.c_float),
                ("rng_state", ctypes.c_ulonglong)]


class Sampler:
    """The reference sampler (source/sampler.c:234-337) on host logits."""

    def __init__(self, vocab: int, temperature: float, top_k: int, top_p: float, seed: int,
                 presence_penalty: float = 0.0):
        self.lib = load_lib()
        self.state = SamplerState(temperature, top_k, top_p, presence_penalty, seed)
        self.presence = np.zeros(vocab, np.uint8)
        self.vocab = vocab

    def sample(self, logits, prev: int, probabilities: bool = False):
        """(token, coin, margin) for one sampler_sample(logits, prev) call,
        and the final (renormalised) probabilities when asked."""
        x = np.array(logits, np.float32, copy=True)
        coin = ctypes.c_float()
        margin = ctypes.c_double()
        tok = self.lib.oracle_sample(ctypes.byref(self.state), fptr(x), self.vocab,
                                     self.presence.ctypes.data_as(ctypes.c_void_p), int(prev),
                                     ctypes.byref(coin), ctypes.byref(margin))
        if probabilities:
            return int(tok), coin.value, margin.value, x
        return int(tok), coin.value, margin.value

    @property
    def rng_state(self) -> int:
        return int(self.state.rng_state)


# KV-cache storage formats (oracle.h ORACLE_KV_*)
KV_F32, KV_BF16, KV_FP8_E4M3 = 0, 1, 2


class OracleModel:
    """The reference forward pass on the CPU, loaded from a model directory."""

    def __init__(self, model_dir: str, threads: Optional[int] = None, kv_format: int = KV_F32):
        self.lib = load_lib()
        if threads:
            self.lib.oracle_set_threads(int(threads))
        cfg = read_config(model_dir)
        table = tensor_table(model_dir)
        names = {t[0] for t in table}
        heads = int(cfg["num_attention_heads"])
        d = int(cfg["hidden_size"])
        hd = int(cfg.get("head_dim") or d // heads)
        qk = any(classify(n)[0] == "Q_NORM" for n in names)
        rs = cfg.get("rope_scaling") or {}
        c = OracleConfig(
            embedding_dim=d, head_dim=hd, hidden_dim=int(cfg["intermediate_size"]),
            layer_count=int(cfg["num_hidden_layers"]), q_head_count=heads,
            kv_head_count=int(cfg["num_key_value_heads"]),
            vocabulary_len=int(cfg["vocab_size"]),
            context_len=int(cfg["max_position_embeddings"]),
            epsilon=float(cfg.get("rms_norm_eps", 0.0)),
            rope_theta=float(cfg.get("rope_theta", 0.0)),
            rope_interleaved=int(bool(rs.get("mrope_interleaved", False))),
            qk_norm=int(qk), tied=int("lm_head.weight" not in names),
            expert_count=int(cfg.get("num_local_experts", 0) or 0),
            expert_used_count=int(cfg.get("num_experts_per_tok", 0) or 0),
        )
        self.config = c
        self.vocab = c.vocabulary_len
        self.dim = c.embedding_dim
        self.layers = c.layer_count
        self.handle = self.lib.oracle_create(ctypes.byref(c))
        if not self.handle:
            raise MemoryError("oracle_create failed")
        for name, path, off, size in table:
            cls, layer = classify(name)
            if cls is None:
                continue
            rc = self.lib.oracle_load_tensor(self.handle, CLS[cls], layer,
                                             path.encode(), off, size)
            if rc != 0:
                raise ValueError(f"oracle: bad tensor {name}")
        missing = self.lib.oracle_finalize(self.handle)
        if missing:
            raise ValueError(f"oracle: {missing} tensors missing")
        self.lib.oracle_set_kv_format(self.handle, int(kv_format))

    def close(self):
        if self.handle:
            self.lib.oracle_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reset(self):
        self.lib.oracle_reset(self.handle)

    @property
    def cached_count(self) -> int:
        return self.lib.oracle_cached_count(self.handle)

    def predict(self, tokens: Sequence[int], logits_count: int = 1,
                capture: bool = False):
        toks = (ctypes.c_int * len(tokens))(*tokens)
        lc = min(logits_count, len(tokens))
        logits = np.zeros((lc, self.vocab), np.float32)
        hid = fin = None
        if capture:
            hid = np.zeros((self.layers, len(tokens), self.dim), np.float32)
            fin = np.zeros((len(tokens), self.dim), np.float32)
            self.lib.oracle_capture_hidden(self.handle, fptr(hid), fptr(fin))
            # MoE: router tie margins of this call, [layers][tokens]
            self.router_margin = None
            if self.config.expert_count:
                self.router_margin = np.zeros((self.layers, len(tokens)), np.float32)
                self.lib.oracle_capture_router_margin(self.handle, fptr(self.router_margin))
        rc = self.lib.oracle_predict(self.handle, len(tokens), toks, logits_count,
                                     fptr(logits))
        if rc != 0:
            raise RuntimeError("context length exhausted")
        if capture:
            return logits, hid, fin
        return logits

    def generate(self, prompt: Sequence[int], steps: int):
        """Reference driver greedy loop: prefill, then steps-1 single steps."""
        out = []
        logits = self.predict(prompt)
        nxt = int(self.lib.oracle_argmax(fptr(logits[0]), self.vocab))
        out.append(nxt)
        while len(out) < steps:
            logits = self.predict([nxt])
            nxt = int(self.lib.oracle_argmax(fptr(logits[0]), self.vocab))
            out.append(nxt)
        return out
