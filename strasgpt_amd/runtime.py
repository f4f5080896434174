"""ctypes binding of libstrasgpt_hip.so: the StrasGPT C API on MI355X.

Mirrors the reference's C interface (include/transformer.h,
include/safetensors.h): a model directory is read into a safetensors
description, turned into a device-resident transformer, and driven with
predict (logits to the host) or the device-side greedy loop. There is no
CPU fallback: importing the binding without the built library raises.
"""
from __future__ import annotations

import ctypes
import os
from typing import List, Optional, Sequence, Tuple

import numpy as np

from . import _paths

_LIB = None


class TransformerConfig(ctypes.Structure):
    _fields_ = [
        ("embedding_dim", ctypes.c_size_t), ("head_dim", ctypes.c_size_t),
        ("hidden_dim", ctypes.c_size_t), ("layer_count", ctypes.c_size_t),
        ("q_head_count", ctypes.c_size_t), ("kv_head_count", ctypes.c_size_t),
        ("vocabulary_len", ctypes.c_size_t), ("context_len", ctypes.c_size_t),
        ("epsilon", ctypes.c_float), ("rope_theta", ctypes.c_float),
        ("rope_pair_bound", ctypes.c_size_t), ("rope_pair_offset", ctypes.c_size_t),
        ("rope_pair_stride", ctypes.c_size_t), ("mrope_section_count", ctypes.c_size_t),
        ("mrope_section", ctypes.POINTER(ctypes.c_size_t)),
        ("aliased_out_weight", ctypes.c_bool), ("qk_norm", ctypes.c_bool),
        ("expert_count", ctypes.c_size_t), ("expert_used_count", ctypes.c_size_t),
    ]


class TransformerState(ctypes.Structure):
    _fields_ = [
        ("embedding", ctypes.c_void_p), ("mha_q", ctypes.c_void_p),
        ("mha_att", ctypes.c_void_p), ("ffn_act", ctypes.c_void_p),
        ("logits", ctypes.c_void_p), ("cached_count", ctypes.c_size_t),
        ("k_cache", ctypes.c_void_p), ("v_cache", ctypes.c_void_p),
        ("rope_cos_sin", ctypes.c_void_p),
    ]


class TransformerT(ctypes.Structure):
    _fields_ = [
        ("config", ctypes.POINTER(TransformerConfig)), ("weights", ctypes.c_void_p),
        ("state", ctypes.POINTER(TransformerState)), ("device", ctypes.c_void_p),
    ]


class Timing(ctypes.Structure):
    _fields_ = [("prefill_s", ctypes.c_double), ("decode_s", ctypes.c_double),
                ("decode_count", ctypes.c_size_t)]


class KernelStat(ctypes.Structure):
    _fields_ = [("launches", ctypes.c_size_t), ("total_ms", ctypes.c_double),
                ("bytes", ctypes.c_double), ("flops", ctypes.c_double)]


def lib():
    """Loads the native library; raises if it has not been built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    path = _paths.hip_lib()
    if not os.path.exists(path):
        raise ImportError(f"{path} is missing: build it with __graft_entry__.build() "
                          "(there is no CPU fallback)")
    L = ctypes.CDLL(path)
    P = ctypes.c_void_p
    sz = ctypes.c_size_t
    TP = ctypes.POINTER(TransformerT)
    ip = ctypes.POINTER(ctypes.c_int)
    fp = ctypes.POINTER(ctypes.c_float)
    L.safetensors_read_dir.restype = P
    L.safetensors_read_dir.argtypes = [ctypes.c_char_p]
    L.safetensors_free.argtypes = [P]
    L.transformer_from_safetensors.restype = TP
    L.transformer_from_safetensors.argtypes = [P]
    L.transformer_free.argtypes = [TP]
    L.transformer_predict.argtypes = [TP, sz, ip, sz, fp]
    L.transformer_predict_argmax.restype = ctypes.c_int
    L.transformer_predict_argmax.argtypes = [TP, sz, ip]
    L.transformer_generate_greedy.restype = sz
    L.transformer_generate_greedy.argtypes = [TP, sz, ip, sz, ctypes.c_int, ip,
                                              ctypes.POINTER(Timing)]
    L.transformer_reset.argtypes = [TP]
    L.transformer_capture_hidden.argtypes = [TP, fp, fp]
    L.transformer_set_prefill_precision.restype = ctypes.c_int
    L.transformer_set_prefill_precision.argtypes = [TP, ctypes.c_int]
    L.transformer_set_decode_mode.restype = ctypes.c_int
    L.transformer_set_decode_mode.argtypes = [TP, ctypes.c_int]
    L.transformer_set_kv_cache_format.restype = ctypes.c_int
    L.transformer_set_kv_cache_format.argtypes = [TP, ctypes.c_int]
    dp = ctypes.POINTER(ctypes.c_double)
    L.transformer_hip_version.restype = ctypes.c_char_p
    L.transformer_profile.argtypes = [TP, ctypes.c_int]
    L.transformer_profile_read.restype = ctypes.c_int
    L.transformer_profile_read.argtypes = [TP, ctypes.c_int, ctypes.POINTER(KernelStat)]
    L.transformer_kernel_rate.restype = ctypes.c_int
    L.transformer_kernel_rate.argtypes = [TP, ctypes.c_int, ctypes.c_int, dp, dp]
    L.sampler_argmax.restype = sz
    L.sampler_argmax.argtypes = [fp, sz]
    VP = ctypes.c_void_p
    L.sampler_hip_build.restype = VP
    L.sampler_hip_build.argtypes = [sz, ctypes.c_float, sz, ctypes.c_float, ctypes.c_ulonglong]
    L.sampler_hip_free.argtypes = [VP]
    L.sampler_hip_set_presence_penalty.argtypes = [VP, ctypes.c_float]
    L.sampler_hip_sample.restype = sz
    L.sampler_hip_sample.argtypes = [VP, fp, ctypes.c_int]
    L.sampler_hip_rng_state.restype = ctypes.c_ulonglong
    L.sampler_hip_rng_state.argtypes = [VP]
    L.transformer_generate_sampled.restype = sz
    L.transformer_generate_sampled.argtypes = [TP, sz, ctypes.POINTER(ctypes.c_int), sz, ctypes.c_int, VP,
                                               ctypes.POINTER(ctypes.c_int), ctypes.POINTER(Timing)]
    TKP = ctypes.POINTER(TokenizerT)
    L.tokenizer_read_dir.restype = TKP
    L.tokenizer_read_dir.argtypes = [ctypes.c_char_p]
    L.tokenizer_free.argtypes = [TKP]
    L.tokenizer_decode.restype = ctypes.c_void_p
    L.tokenizer_decode.argtypes = [TKP, ctypes.c_int]
    L.tokenizer_tokenize.argtypes = [TKP, ctypes.c_char_p, ctypes.c_bool, ctypes.c_bool,
                                     ctypes.POINTER(sz), ctypes.POINTER(ip)]
    L.tokenizer_print.argtypes = [VP, TKP]
    L.tokenizer_print_tokens.argtypes = [TKP, VP, sz, ip, sz]
    L.tokenizer_print_token_string.argtypes = [VP, ctypes.c_char_p]
    _LIB = L
    return L


def _fp(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _ints(seq: Sequence[int]):
    return (ctypes.c_int * len(seq))(*[int(v) for v in seq])


# Kernel classes reported by transformer_profile_read (include/transformer_hip.h).
# transformer_set_decode_mode (include/transformer_hip.h)
DECODE_GRAPH, DECODE_EAGER = 1, 2
# transformer_set_kv_cache_format (include/transformer_hip.h)
KV_FP32, KV_BF16 = 0, 1

PROFILE_KERNELS = ["qkv_gemv", "attention_decode", "o_gemv", "gate_up_gemv", "down_gemv",
                   "logits_gemv", "argmax", "moe_route", "moe_gate_up", "moe_down",
                   "qkv_gemm", "attention_prefill", "o_gemm", "gate_up_gemm", "down_gemm",
                   "elementwise", "moe_route_prefill", "moe_gate_up_prefill", "moe_down_prefill"]


TOKENIZER_MAX_TOKEN_STRING = 262144


class TokenizerIndex(ctypes.Structure):
    _fields_ = [("token_string", ctypes.c_char_p), ("id", ctypes.c_int)]


class TokenizerT(ctypes.Structure):
    """tokenizer_t (include/tokenizer.h; the reference's field layout)."""
    _fields_ = [("token_string_count", ctypes.c_size_t),
                ("token_string", ctypes.c_void_p * TOKENIZER_MAX_TOKEN_STRING),
                ("score", ctypes.c_float * TOKENIZER_MAX_TOKEN_STRING),
                ("sorted_token_string", TokenizerIndex * TOKENIZER_MAX_TOKEN_STRING),
                ("max_token_string_len", ctypes.c_size_t),
                ("byte_string", ctypes.c_ubyte * 512),
                ("bos_token_id", ctypes.c_int), ("eos_token_id", ctypes.c_int)]


class Tokenizer:
    """tokenizer_t of a model directory's tokenizer.json: encode text to
    ids and ids to byte strings with the reference tokenizer's rules
    (source/tokenizer.c). Host code only."""

    def __init__(self, model_dir: str, bos: int = 0, eos: int = 0):
        self._lib = lib()
        self.handle = self._lib.tokenizer_read_dir(model_dir.encode())
        self.t = self.handle.contents
        self.t.bos_token_id = bos
        self.t.eos_token_id = eos

    def __len__(self) -> int:
        return int(self.t.token_string_count)

    def token_bytes(self, i: int) -> bytes:
        """Vocabulary entry i after the byte-level map is undone."""
        return ctypes.string_at(self.t.token_string[i])

    def encode(self, text: bytes, bos: bool = True, eos: bool = False) -> List[int]:
        n = ctypes.c_size_t(0)
        out = ctypes.POINTER(ctypes.c_int)()
        self._lib.tokenizer_tokenize(self.handle, text, bos, eos, ctypes.byref(n), ctypes.byref(out))
        ids = [out[i] for i in range(n.value)]
        _libc().free(ctypes.cast(out, ctypes.c_void_p))
        return ids

    def decode(self, token: int) -> bytes:
        return ctypes.string_at(self._lib.tokenizer_decode(self.handle, int(token)))

    def close(self):
        if getattr(self, "handle", None):
            self._lib.tokenizer_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


_LIBC = None


def _libc():
    global _LIBC
    if _LIBC is None:
        _LIBC = ctypes.CDLL(None)
        _LIBC.free.argtypes = [ctypes.c_void_p]
        _LIBC.fopen.restype = ctypes.c_void_p
        _LIBC.fopen.argtypes = [ctypes.c_char_p, ctypes.c_char_p]
        _LIBC.fclose.argtypes = [ctypes.c_void_p]
    return _LIBC


class Transformer:
    """A model loaded into HBM through the C API."""

    def __init__(self, model_dir: str):
        L = lib()
        self._lib = L
        self._st = L.safetensors_read_dir(model_dir.encode())
        self._t = L.transformer_from_safetensors(self._st)
        c = self._t.contents.config.contents
        self.vocab = c.vocabulary_len
        self.dim = c.embedding_dim
        self.layers = c.layer_count
        self.context_len = c.context_len
        self.config = c

    def close(self):
        if getattr(self, "_t", None):
            self._lib.transformer_free(self._t)
            self._t = None
        if getattr(self, "_st", None):
            self._lib.safetensors_free(self._st)
            self._st = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def cached_count(self) -> int:
        return self._t.contents.state.contents.cached_count

    def reset(self):
        self._lib.transformer_reset(self._t)

    def predict(self, tokens: Sequence[int], logits_count: int = 1,
                capture: bool = False):
        lc = min(logits_count, len(tokens))
        logits = np.zeros((lc, self.vocab), np.float32)
        hid = fin = None
        if capture:
            hid = np.zeros((self.layers, len(tokens), self.dim), np.float32)
            fin = np.zeros((len(tokens), self.dim), np.float32)
            self._lib.transformer_capture_hidden(self._t, _fp(hid), _fp(fin))
        self._lib.transformer_predict(self._t, len(tokens), _ints(tokens), logits_count,
                                      _fp(logits))
        if capture:
            return logits, hid, fin
        return logits

    def predict_argmax(self, tokens: Sequence[int]) -> int:
        return int(self._lib.transformer_predict_argmax(self._t, len(tokens), _ints(tokens)))

    def generate(self, prompt: Sequence[int], steps: int, eos: int = -1
                 ) -> Tuple[List[int], Timing]:
        out = (ctypes.c_int * max(steps, 1))()
        tm = Timing()
        n = self._lib.transformer_generate_greedy(self._t, len(prompt), _ints(prompt), steps,
                                                  eos, out, ctypes.byref(tm))
        return [int(out[i]) for i in range(n)], tm

    def generate_sampled(self, prompt: Sequence[int], steps: int, sampler: "Sampler", eos: int = -1
                         ) -> Tuple[List[int], Timing]:
        """transformer_generate_sampled: the decode loop with device sampling."""
        out = (ctypes.c_int * max(steps, 1))()
        tm = Timing()
        n = self._lib.transformer_generate_sampled(self._t, len(prompt), _ints(prompt), steps, eos,
                                                   sampler.handle, out, ctypes.byref(tm))
        return [int(out[i]) for i in range(n)], tm

    def set_prefill_precision(self, mode: int) -> int:
        return int(self._lib.transformer_set_prefill_precision(self._t, mode))

    def set_decode_mode(self, mode: int) -> int:
        """DECODE_GRAPH or DECODE_EAGER; returns the old mode."""
        return int(self._lib.transformer_set_decode_mode(self._t, mode))

    def set_kv_cache_format(self, fmt: int) -> int:
        """KV_FP32 or KV_BF16, while the cache is empty; returns the old format."""
        return int(self._lib.transformer_set_kv_cache_format(self._t, fmt))

    def profile(self, enable: bool):
        self._lib.transformer_profile(self._t, int(enable))

    def kernel_rate(self, name: str, reps: int = 4):
        """(avg_us, bytes_per_launch) of back-to-back launches of one decode
        kernel class over every layer, or None where unsupported."""
        us, by = ctypes.c_double(), ctypes.c_double()
        cls = PROFILE_KERNELS.index(name)
        if self._lib.transformer_kernel_rate(self._t, cls, reps, ctypes.byref(us), ctypes.byref(by)) != 0:
            return None
        return us.value, by.value

    def profile_read(self):
        out = {}
        for i, name in enumerate(PROFILE_KERNELS):
            st = KernelStat()
            if self._lib.transformer_profile_read(self._t, i, ctypes.byref(st)) == 0 and st.launches:
                out[name] = {"launches": st.launches, "total_ms": st.total_ms,
                             "bytes": st.bytes, "flops": st.flops}
        return out


def argmax(values: np.ndarray) -> int:
    """sampler_argmax: the reference's sample_argmax on the device."""
    v = np.ascontiguousarray(values, np.float32)
    return int(lib().sampler_argmax(_fp(v), v.size))


class Sampler:
    """sampler_hip_t: the reference's sampler with its state on the device."""

    def __init__(self, vocab: int, temperature: float, top_k: int, top_p: float, seed: int,
                 presence_penalty: float = 0.0):
        self._lib = lib()
        self.handle = self._lib.sampler_hip_build(vocab, temperature, top_k, top_p, seed)
        if presence_penalty:
            self._lib.sampler_hip_set_presence_penalty(self.handle, presence_penalty)

    def sample(self, logits: np.ndarray, prev: int) -> int:
        v = np.ascontiguousarray(logits, np.float32)
        return int(self._lib.sampler_hip_sample(self.handle, _fp(v), int(prev)))

    @property
    def rng_state(self) -> int:
        return int(self._lib.sampler_hip_rng_state(self.handle))

    def close(self):
        if getattr(self, "handle", None):
            self._lib.sampler_hip_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def version() -> str:
    return lib().transformer_hip_version().decode()
