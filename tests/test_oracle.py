"""Pins of the CPU oracle (oracle/): closed forms, float64 restatements,
planted mistakes, and the golden fixtures written by the reference C
sources (tests/golden/make_golden.py)."""
import ctypes
import hashlib
import os

import numpy as np
import pytest

from conftest import GOLDEN_DIR, MODEL_SEED, PROMPT_SEED

from oracle import oracle as orc
from strasgpt_amd import synth

pytestmark = pytest.mark.skipif(not orc.oracle_available(), reason="oracle not built")


def lib():
    return orc.load_lib()


def bf16_to_f32_np(u16):
    return (np.asarray(u16, np.uint32) << 16).view(np.float32)


def f32_to_bf16_np(x):
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def test_bf16_exhaustive():
    L = lib()
    codes = np.arange(65536, dtype=np.uint32)
    ref = (codes << 16).view(np.float32)
    # all 65,536 codes, compared as bit patterns in a C buffer (a float
    # returned through ctypes passes through a double, which quiets the 126
    # signaling-NaN codes)
    w = codes.astype(np.uint16)
    got = np.zeros(65536, np.float32)
    L.oracle_bf16_to_f32_array(w.ctypes.data, 65536, orc.fptr(got))
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))
    # the scalar entry point on the non-NaN codes
    finite = codes[~np.isnan(ref)][::97]
    sc = np.array([L.oracle_bf16_to_f32(int(c)) for c in finite], np.float32)
    np.testing.assert_array_equal(sc.view(np.uint32), (finite << 16).view(np.float32).view(np.uint32))


def test_mxfp4_exhaustive():
    """E2M1 x E8M0 against the OCP MX closed form, all 16 x 256 pairs."""
    L = lib()
    mag = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
    for s in range(256):
        for c in range(16):
            got = L.oracle_mxfp4_value(c, s)
            if s == 255:
                assert np.isnan(got)
                continue
            want = (-1.0 if c & 8 else 1.0) * mag[c & 7] * 2.0 ** (s - 127)
            assert np.float32(got) == np.float32(want), (c, s)


def test_mxfp4_dequant_layout():
    """Element 2i is the low nibble of byte i; one scale per 32 values."""
    L = lib()
    rng = np.random.default_rng(0)
    blocks = rng.integers(0, 256, 64, dtype=np.uint8)
    scales = np.array([120, 125, 119, 123], np.uint8)
    out = np.zeros(128, np.float32)
    L.oracle_mxfp4_dequant(blocks.ctypes.data, scales.ctypes.data, 128, orc.fptr(out))
    mag = np.array([0, .5, 1, 1.5, 2, 3, 4, 6])
    codes = np.empty(128, np.uint8)
    codes[0::2] = blocks & 15
    codes[1::2] = blocks >> 4
    want = np.where(codes & 8, -1.0, 1.0) * mag[codes & 7] * 2.0 ** (scales.repeat(32).astype(np.float64) - 127)
    np.testing.assert_array_equal(out, want.astype(np.float32))


def test_mxfp4_dequant_all_scales_bitwise():
    """The block dequantisation equals the closed form bit for bit for all
    16 codes in both nibble positions under every one of the 256 scales
    (scale 0 gives subnormal values, 255 NaN; code 8 is -0.0)."""
    L = lib()
    nblocks = 256
    codes = np.empty((nblocks, 16), np.uint8)
    for i in range(16):
        codes[:, i] = i | ((15 - i) << 4)
    scales = np.arange(256, dtype=np.uint8)
    out = np.zeros(nblocks * 32, np.float32)
    L.oracle_mxfp4_dequant(codes.ctypes.data, scales.ctypes.data, nblocks * 32, orc.fptr(out))
    mag = np.array([0, .5, 1, 1.5, 2, 3, 4, 6])
    c = np.empty((nblocks, 32), np.uint8)
    c[:, 0::2] = codes & 15
    c[:, 1::2] = codes >> 4
    want = (np.where(c & 8, -1.0, 1.0) * mag[c & 7] *
            2.0 ** (scales[:, None].astype(np.float64) - 127)).astype(np.float32)
    want[255] = np.nan
    got = out.reshape(nblocks, 32)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    np.testing.assert_array_equal(got[ok].view(np.uint32), want[ok].view(np.uint32))
    scalar = np.array([[L.oracle_mxfp4_value(int(c[b, i]), int(b)) for i in range(32)]
                       for b in range(0, 255, 17)], np.float32)
    np.testing.assert_array_equal(scalar.view(np.uint32), want[0:255:17].view(np.uint32))


def dot_model(a, w):
    """Reference AVX2 dot order (source/transformer.c:1095-1167) in float32."""
    a = np.asarray(a, np.float32)
    wf = bf16_to_f32_np(w)
    acc = np.zeros((4, 8), np.float32)
    for i in range(0, len(a), 32):
        blk = (a[i:i + 32].astype(np.float64) * wf[i:i + 32]).reshape(4, 8)
        # FMA: exact product, one rounding with the accumulator
        acc = (acc.astype(np.float64) + blk).astype(np.float32)
    v = (acc[0] + acc[1]) + (acc[2] + acc[3])
    s = v[:4] + v[4:]
    return (s[0] + s[1]) + (s[2] + s[3])


def test_dot_matches_fma_model_and_float64():
    L = lib()
    rng = np.random.default_rng(1)
    for n in (32, 64, 2048, 2880):
        a = rng.standard_normal(n).astype(np.float32)
        w = f32_to_bf16_np(rng.standard_normal(n) * 0.02)
        got = L.oracle_dot_bf16(n, orc.fptr(a), w.ctypes.data)
        exact = float(np.dot(a.astype(np.float64), bf16_to_f32_np(w).astype(np.float64)))
        assert np.float32(got) == dot_model(a, w)
        assert abs(got - exact) <= 1e-5 * (np.abs(a) @ np.abs(bf16_to_f32_np(w))) + 1e-30


def test_dot_planted_transpose_fails():
    """A transposed weight row (a plausible indexing mistake) is detected."""
    L = lib()
    rng = np.random.default_rng(2)
    a = rng.standard_normal(64).astype(np.float32)
    w = f32_to_bf16_np(rng.standard_normal(64))
    got = L.oracle_dot_bf16(64, orc.fptr(a), w.ctypes.data)
    wrong = float(np.dot(a, bf16_to_f32_np(w[::-1])))
    assert abs(got - wrong) > 1e-3


def test_rmsnorm_float64():
    L = lib()
    rng = np.random.default_rng(3)
    for n in (16, 128, 2560):
        x = rng.standard_normal(n).astype(np.float32)
        w = f32_to_bf16_np(1.0 + 0.1 * rng.standard_normal(n))
        y = np.zeros(n, np.float32)
        L.oracle_rmsnorm(n, orc.fptr(y), orc.fptr(x), w.ctypes.data, ctypes.c_float(1e-5))
        xd = x.astype(np.float64)
        want = xd / np.sqrt(np.mean(xd * xd) + 1e-5) * bf16_to_f32_np(w)
        np.testing.assert_allclose(y, want, rtol=2e-6, atol=1e-7)
        # planted mistake: forgetting the mean (sum instead) is far off
        assert np.abs(y - xd / np.sqrt(np.sum(xd * xd)) * bf16_to_f32_np(w)).max() > 1e-2


@pytest.mark.parametrize("interleaved", [0, 1])
def test_rope_table_float64(interleaved):
    L = lib()
    ctx, hd, theta = 40, 16, 10000.0
    out = np.zeros((ctx, hd), np.float32)
    L.oracle_rope_table(ctx, hd, ctypes.c_float(theta), interleaved, orc.fptr(out))
    pos = np.arange(ctx)[:, None].astype(np.float64)
    if interleaved:
        j = np.arange(0, hd, 2)
        ang = pos / theta ** (j / hd)
        np.testing.assert_allclose(out[:, 0::2], np.cos(ang), atol=2e-5)
        np.testing.assert_allclose(out[:, 1::2], np.sin(ang), atol=2e-5)
    else:
        j = np.arange(hd // 2)
        ang = pos / theta ** (2 * j / hd)
        np.testing.assert_allclose(out[:, :hd // 2], np.cos(ang), atol=2e-5)
        np.testing.assert_allclose(out[:, hd // 2:], np.sin(ang), atol=2e-5)


def test_attention_row_float64():
    L = lib()
    rng = np.random.default_rng(4)
    hd, n = 32, 17
    q = rng.standard_normal(hd).astype(np.float32)
    k = rng.standard_normal((n, hd)).astype(np.float32)
    v = rng.standard_normal((n, hd)).astype(np.float32)
    out = np.zeros(hd, np.float32)
    L.oracle_attention_row(hd, n, orc.fptr(q), orc.fptr(k), orc.fptr(v), orc.fptr(out))
    s = k.astype(np.float64) @ q / np.sqrt(hd)
    p = np.exp(s - s.max())
    p /= p.sum()
    np.testing.assert_allclose(out, p @ v, rtol=1e-5, atol=1e-6)
    # single key: output is that key's value exactly
    L.oracle_attention_row(hd, 1, orc.fptr(q), orc.fptr(k), orc.fptr(v), orc.fptr(out))
    np.testing.assert_allclose(out, v[0], rtol=0, atol=1e-7)


def test_argmax_semantics():
    L = lib()
    x = np.array([1.0, 3.0, 2.0, 3.0], np.float32)
    assert L.oracle_argmax(orc.fptr(x), 4) == 1  # first maximum
    x = np.array([np.nan, 5.0, 1.0], np.float32)
    assert L.oracle_argmax(orc.fptr(x), 3) == 0  # NaN at 0 is never replaced
    x = np.array([1.0, np.nan, 5.0], np.float32)
    assert L.oracle_argmax(orc.fptr(x), 3) == 2


def test_topk_softmax():
    L = lib()
    lg = np.array([0.5, 2.0, -1.0, 2.0, 1.5], np.float32)
    idx = (ctypes.c_int * 3)()
    w = np.zeros(3, np.float32)
    L.oracle_topk_softmax(5, orc.fptr(lg), 3, idx, orc.fptr(w))
    assert list(idx) == [1, 3, 4]  # ties to the lowest index, descending order
    e = np.exp(np.array([2.0, 2.0, 1.5]) - 2.0)
    np.testing.assert_allclose(w, e / e.sum(), rtol=1e-6)


@pytest.mark.parametrize("name", ["tiny-llama", "tiny-qwen", "tiny-chunk", "tiny-rope-il",
                                  "tiny-rope-il128"])
def test_oracle_matches_reference_golden(name, model_dir):
    """The oracle reproduces the reference C run of tests/golden/<name>.npz."""
    g = np.load(os.path.join(GOLDEN_DIR, f"{name}.npz"))
    d = model_dir(name)
    digest = hashlib.sha256(open(os.path.join(d, "model.safetensors"), "rb").read()).hexdigest()
    assert digest == str(g["sha256"]), "synthetic model generator drifted"
    prompt = [int(v) for v in g["prompt"]]
    assert prompt == synth.prompt_tokens(synth.shape(name).vocab, len(prompt), PROMPT_SEED)
    om = orc.OracleModel(d, threads=4)
    logits, hid, fin = om.predict(prompt, capture=True)
    np.testing.assert_allclose(logits[0], g["logits"], rtol=1e-4, atol=1e-4)
    last = g["hidden"].shape[1]
    np.testing.assert_allclose(fin[-last:], g["hidden"][-1], rtol=1e-4, atol=1e-4)
    # per-layer normalised residual stream (norm weights are 1.0)
    for l in range(om.layers - 1):
        xl = hid[l][-last:].astype(np.float64)
        xn = xl / np.sqrt(np.mean(xl * xl, axis=1, keepdims=True) + om.config.epsilon)
        np.testing.assert_allclose(xn, g["hidden"][l], rtol=1e-4, atol=1e-4)
    om.reset()
    assert om.generate(prompt, len(g["generated"])) == [int(v) for v in g["generated"]]


def test_oracle_chunk_invariance(model_dir):
    """Prefill in one call == prefill split across calls (reference chunk
    independence, source/transformer.c:1643-1726)."""
    d = model_dir("tiny-llama")
    om = orc.OracleModel(d, threads=2)
    prompt = synth.prompt_tokens(256, 8, 11)
    a = om.predict(prompt)
    om.reset()
    om.predict(prompt[:5])
    b = om.predict(prompt[5:])
    np.testing.assert_allclose(a, b, rtol=1e-5, atol=1e-6)


def _bf16_round_by_definition(x):
    """The nearer of the two bf16 values around x (same sign: the truncation
    toward zero and the next bf16 away from it), ties to the even pattern;
    values past the largest finite bf16 go to infinity as IEEE rounding does."""
    x = np.float32(x)
    u = int(np.array(x).view(np.uint32))
    lo_u = u & 0xFFFF0000
    hi_u = lo_u + 0x10000
    lo = float(np.array(lo_u, np.uint32).view(np.float32))
    # past the largest finite bf16 the next value would be 2^128 (IEEE
    # rounding overflows to infinity from halfway up)
    over = (hi_u & 0x7FFFFFFF) == 0x7F800000
    hi = (2.0 ** 128 if x > 0 else -2.0 ** 128) if over else float(np.array(hi_u, np.uint32).view(np.float32))
    dl, dh = abs(float(x) - lo), abs(hi - float(x))
    if dl < dh or (dl == dh and (lo_u >> 16) % 2 == 0):
        return np.float32(lo)
    return np.float32(np.copysign(np.inf, x)) if over else np.float32(hi)


def test_round_bf16_definition():
    """oracle_round_bf16 (the bf16 KV-cache format) against the definition
    of round-to-nearest-even on random patterns, exact ties, and the ends of
    the range."""
    L = lib()
    rng = np.random.default_rng(5)
    pats = rng.integers(0, 0x7F7F0000, 20000, dtype=np.uint64).astype(np.uint32)
    ties = (rng.integers(0, 0x7F7F, 2000).astype(np.uint32) << 16) | 0x8000
    for u in np.concatenate([pats, ties, np.array([0, 1, 0x7F7FFFFF, 0x7F7F7FFF, 0x00008000], np.uint32)]):
        for sign in (0, 0x80000000):
            x = float(np.array(int(u) | sign, np.uint32).view(np.float32))
            got = np.float32(L.oracle_round_bf16(x))
            want = _bf16_round_by_definition(x)
            assert got.view(np.uint32) == want.view(np.uint32), hex(int(u) | sign)
    assert np.isinf(L.oracle_round_bf16(float(np.float32(3.4e38))))
    assert np.isinf(L.oracle_round_bf16(float("inf")))
    assert np.isnan(L.oracle_round_bf16(float("nan")))


def _e4m3_values():
    """Every finite OCP FP8 E4M3 value by code (sign, 4-bit exponent with
    bias 7, 3-bit mantissa; exponent 0 is subnormal; S.1111.111 is NaN)."""
    out = {}
    for code in range(256):
        s, e, m = code >> 7, (code >> 3) & 15, code & 7
        if e == 15 and m == 7:
            continue
        v = (m / 8) * 2.0 ** -6 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7)
        out[code] = -v if s else v
    return out


def test_round_fp8_e4m3_definition():
    """oracle_round_fp8_e4m3 against a brute-force nearest search over the
    256 codes (ties to the even code, saturation at 448); the code table is
    pinned by the format's known points."""
    vals = _e4m3_values()
    assert vals[0x7E] == 448.0 and vals[0x08] == 2.0 ** -6 and vals[0x01] == 2.0 ** -9
    assert vals[0x38] == 1.0 and vals[0xB8] == -1.0 and len(vals) == 254
    codes = sorted(vals, key=lambda c: (vals[c], c))
    table = np.array([vals[c] for c in codes])
    L = lib()
    rng = np.random.default_rng(6)
    xs = np.concatenate([rng.uniform(-460, 460, 4000), rng.uniform(-0.03, 0.03, 4000),
                         np.array(table[:-1] + np.diff(table) / 2),  # exact midpoints
                         np.array([0.0, 1e-9, 447.9, 448.0, 463.9, 1000.0, -1000.0])])
    for x in xs.astype(np.float32):
        got = L.oracle_round_fp8_e4m3(float(x))
        if abs(x) >= 448:
            assert got == np.copysign(448.0, x)
            continue
        dist = np.abs(table - float(x))
        best = np.flatnonzero(dist == dist.min())
        cand = [codes[i] for i in best]
        even = [c for c in cand if c % 2 == 0 and (vals[c] != 0 or c == 0 or len(cand) == 1)]
        want = vals[(even or cand)[0]]
        assert got == want or (want == 0 and got == 0), (float(x), got, want)


def test_oracle_kv_formats(model_dir):
    """The oracle's KV-cache formats: bf16 moves the logits by a small
    amount and keeps the greedy tokens on tiny-qwen; every format stays
    chunk-invariant (rounding happens once per cached row)."""
    d = model_dir("tiny-qwen")
    prompt = synth.prompt_tokens(256, 12, 12)
    ref = orc.OracleModel(d, threads=2)
    want = ref.predict(prompt)
    ref.reset()
    want_tok = ref.generate(prompt, 8)
    for fmt, tol in ((orc.KV_BF16, 5e-2), (orc.KV_FP8_E4M3, None)):
        om = orc.OracleModel(d, threads=2, kv_format=fmt)
        a = om.predict(prompt)
        om.reset()
        om.predict(prompt[:5])
        b = om.predict(prompt[5:])
        np.testing.assert_array_equal(a, b)
        err = float(np.abs(a - want).max())
        print(f"kv format {fmt}: max |logit - fp32 cache| {err:.3g} (largest |logit| {float(np.abs(want).max()):.3g})")
        assert err > 0
        if tol is not None:
            assert err < tol
            om.reset()
            assert om.generate(prompt, 8) == want_tok
        om.close()


def test_oracle_moe_float64(model_dir):
    """MoE semantics (no reference counterpart) against a float64 numpy
    restatement on the tiny MoE model."""
    d = model_dir("tiny-moe")
    om = orc.OracleModel(d, threads=2)
    prompt = synth.prompt_tokens(256, 3, 5)
    got = om.predict(prompt)[0]
    want = numpy_forward(d, prompt)
    np.testing.assert_allclose(got, want, rtol=2e-4, atol=2e-4)


def test_oracle_router_margins(model_dir):
    """The router tie margins the oracle captures (k-th largest router logit
    minus the largest one left out, per layer and token) against the float64
    restatement's, on a prompt long enough to make some margins small; a
    planted swap of k-th and (k+1)-th in the restatement would change every
    margin's sign."""
    d = model_dir("tiny-moe")
    om = orc.OracleModel(d, threads=2)
    prompt = synth.prompt_tokens(256, 12, 9)
    om.predict(prompt, capture=True)
    got = om.router_margin
    want = []
    numpy_forward(d, prompt, margins=want)
    want = np.array(want)
    assert got.shape == want.shape == (2, 12)
    assert (want > 0).all()
    np.testing.assert_allclose(got, want, rtol=1e-3, atol=2e-5)
    om.close()


def numpy_forward(model_dir, prompt, margins=None):
    """float64 restatement of the forward pass (dense or MoE), last logits.
    With a list `margins`, MoE models append per layer the [T] router tie
    margins (k-th largest router logit minus the (k+1)-th)."""
    cfg = orc.read_config(model_dir)
    tab = {n: (p, o, s) for n, p, o, s in orc.tensor_table(model_dir)}
    meta = {n: (t, shp) for n, t, shp, *_ in synth.tensor_table(model_dir)}

    def get(name):
        p, o, s = tab[name]
        dt, shp = meta[name]
        raw = np.fromfile(p, np.uint8, s, offset=o)
        if dt == "BF16":
            return bf16_to_f32_np(raw.view(np.uint16)).astype(np.float64).reshape(shp)
        return raw.reshape(shp)

    d = cfg["hidden_size"]; hd = cfg["head_dim"]; L = cfg["num_hidden_layers"]
    qh = cfg["num_attention_heads"]; kvh = cfg["num_key_value_heads"]
    eps = cfg["rms_norm_eps"]; theta = cfg["rope_theta"]
    E = cfg.get("num_local_experts", 0); K = cfg.get("num_experts_per_tok", 0)
    T = len(prompt)

    def rms(x, w):
        return x / np.sqrt(np.mean(x * x, -1, keepdims=True) + eps) * w

    interleaved = bool((cfg.get("rope_scaling") or {}).get("mrope_interleaved", False))

    def rope(v, pos):
        # pair j rotates by pos / theta^(2j/hd): elements (j, j + hd/2), or
        # (2j, 2j + 1) in the interleaved layout
        half = hd // 2
        j = np.arange(half)
        ang = pos[:, None] / theta ** (2 * j / hd)
        c, s_ = np.cos(ang)[:, None], np.sin(ang)[:, None]
        i0 = 2 * j if interleaved else j
        i1 = i0 + 1 if interleaved else j + half
        v0, v1 = v[..., i0].copy(), v[..., i1].copy()
        out = v.copy()
        out[..., i0] = v0 * c - v1 * s_
        out[..., i1] = v0 * s_ + v1 * c
        return out

    def mx(blocks, scales):
        mag = np.array([0, .5, 1, 1.5, 2, 3, 4, 6])
        codes = np.stack([blocks & 15, blocks >> 4], -1).reshape(*blocks.shape[:-1], 32)
        val = np.where(codes & 8, -1.0, 1.0) * mag[codes & 7]
        val = val * 2.0 ** (scales[..., None].astype(np.float64) - 127)
        return val.reshape(*blocks.shape[:-2], -1)

    emb = get("model.embed_tokens.weight")
    x = emb[prompt]
    pos = np.arange(T, dtype=np.float64)
    for l in range(L):
        pre = f"model.layers.{l}."
        xn = rms(x, get(pre + "input_layernorm.weight"))
        q = (xn @ get(pre + "self_attn.q_proj.weight").T).reshape(T, qh, hd)
        k = (xn @ get(pre + "self_attn.k_proj.weight").T).reshape(T, kvh, hd)
        v = (xn @ get(pre + "self_attn.v_proj.weight").T).reshape(T, kvh, hd)
        if pre + "self_attn.q_norm.weight" in tab:  # per-head RMSNorm before RoPE
            q = rms(q, get(pre + "self_attn.q_norm.weight"))
            k = rms(k, get(pre + "self_attn.k_norm.weight"))
        q, k = rope(q, pos), rope(k, pos)
        att = np.zeros((T, qh, hd))
        for h in range(qh):
            kv = h // (qh // kvh)
            s = q[:, h] @ k[:, kv].T / np.sqrt(hd)
            s = np.where(np.tril(np.ones((T, T))) > 0, s, -np.inf)
            p = np.exp(s - s.max(1, keepdims=True))
            p /= p.sum(1, keepdims=True)
            att[:, h] = p @ v[:, kv]
        x = x + att.reshape(T, -1) @ get(pre + "self_attn.o_proj.weight").T
        xn = rms(x, get(pre + "post_attention_layernorm.weight"))
        if E:
            r = xn @ get(pre + "mlp.router.weight").T
            if margins is not None:
                srt = -np.sort(-r, axis=1)
                margins.append(srt[:, K - 1] - srt[:, K])
            G = mx(get(pre + "mlp.experts.gate_proj_blocks"), get(pre + "mlp.experts.gate_proj_scales"))
            U = mx(get(pre + "mlp.experts.up_proj_blocks"), get(pre + "mlp.experts.up_proj_scales"))
            D = mx(get(pre + "mlp.experts.down_proj_blocks"), get(pre + "mlp.experts.down_proj_scales"))
            out = np.zeros_like(x)
            for t in range(T):
                sel = np.argsort(-r[t], kind="stable")[:K]
                w = np.exp(r[t, sel] - r[t, sel].max())
                w /= w.sum()
                for j, e in enumerate(sel):
                    g = G[e] @ xn[t]
                    u = U[e] @ xn[t]
                    a = g / (1 + np.exp(-g)) * u
                    out[t] += w[j] * (D[e] @ a)
            x = x + out
        else:
            g = xn @ get(pre + "mlp.gate_proj.weight").T
            u = xn @ get(pre + "mlp.up_proj.weight").T
            x = x + (g / (1 + np.exp(-g)) * u) @ get(pre + "mlp.down_proj.weight").T
    xn = rms(x, get("model.norm.weight"))
    out_w = get("lm_head.weight") if "lm_head.weight" in tab else emb
    return xn[-1] @ out_w.T


@pytest.mark.parametrize("name", ["tiny-llama", "tiny-qwen", "tiny-rope-il", "tiny-rope-il128"])
def test_oracle_dense_float64(name, model_dir):
    """The oracle's dense forward against the float64 restatement: half-split
    RoPE (tiny-llama), per-head QK RMSNorm with untied output (tiny-qwen),
    interleaved RoPE pairs (tiny-rope-il)."""
    d = model_dir(name)
    shp = synth.shape(name)
    om = orc.OracleModel(d, threads=2)
    prompt = synth.prompt_tokens(shp.vocab, 5, 9)
    np.testing.assert_allclose(om.predict(prompt)[0], numpy_forward(d, prompt), rtol=2e-4, atol=2e-4)


def _xorshift_coins(seed, n):
    """Xorshift64* (the reference's random_u32, source/sampler.c:79-85) in
    Python integers, and the coin of source/sampler.c:87-90."""
    s, out = seed, []
    for _ in range(n):
        s ^= s >> 12
        s ^= (s << 25) & (2 ** 64 - 1)
        s ^= s >> 27
        u = ((s * 0x2545F4914F6CDD1D) & (2 ** 64 - 1)) >> 32
        out.append((u >> 8) / 16777216.0)
    return out, s


def test_sampler_coins():
    """The oracle sampler's coins are the xorshift64* stream (one draw per
    non-greedy call, none when greedy), uniform on [0, 1) in 2^-24 steps."""
    x = np.zeros(4, np.float32)
    s = orc.Sampler(4, 1.0, 0, 0.0, 12345)
    coins = [s.sample(x, -1)[1] for _ in range(2000)]
    want, state = _xorshift_coins(12345, 2000)
    assert coins == [np.float32(c) for c in want] and s.rng_state == state
    g = orc.Sampler(4, 0.0, 0, 0.0, 12345)
    assert g.sample(x, -1)[1] == -1 and g.rng_state == 12345
    big, _ = _xorshift_coins(7, 100000)
    hist = np.histogram(big, bins=10, range=(0, 1))[0]
    assert np.all(np.abs(hist - 10000) < 5 * 100)  # 5 sigma
    assert all(c * 16777216 == int(c * 16777216) for c in big[:1000])


def _filtered(logits, temp, top_k, top_p):
    """The sampling distribution of source/sampler.c:234-337 in float64:
    softmax at the temperature, the k most likely (index order among equal
    probabilities), then the shortest descending prefix reaching top_p,
    renormalized."""
    z = np.asarray(logits, np.float64) / temp
    p = np.exp(z - z.max())
    p /= p.sum()
    order = sorted(range(len(p)), key=lambda i: (-p[i], i))
    keep = order[:top_k] if top_k > 0 else order
    if 0 < top_p <= 1:
        cum, cut = 0.0, len(keep)
        for r, i in enumerate(keep):
            cum += p[i]
            if cum >= top_p:
                cut = r + 1
                break
        keep = keep[:cut]
    q = np.zeros_like(p)
    q[keep] = p[keep]
    return q / q.sum()


@pytest.mark.parametrize("temp,top_k,top_p", [(1.0, 0, 0.0), (0.7, 3, 0.0), (1.3, 0, 0.8),
                                               (1.0, 4, 0.9)])
def test_sampler_distribution(temp, top_k, top_p):
    """Sampled frequencies over 40000 calls match the float64 distribution
    the reference's steps define (within 5 sigma per token)."""
    logits = np.array([0.3, -1.2, 1.7, 0.9, 0.9, -0.4, 2.2, -3.0], np.float32)
    want = _filtered(logits, temp, top_k, top_p)
    s = orc.Sampler(len(logits), temp, top_k, top_p, 99)
    n = 40000
    got = np.bincount([s.sample(logits, -1)[0] for _ in range(n)], minlength=len(logits)) / n
    sigma = np.sqrt(want * (1 - want) / n) + 1e-9
    assert np.all(np.abs(got - want) <= 5 * sigma + 1e-12), (got, want)
    assert np.all(got[want == 0] == 0)


def test_sampler_special_cases():
    """Greedy and degenerate filters give the argmax (ties to the lower
    index); top-k 1 ignores the coin; a presence penalty removes a seen
    token."""
    tie = np.array([0.5, 2.0, -1.0, 2.0], np.float32)
    assert orc.Sampler(4, 0.0, 0, 0.0, 1).sample(tie, -1)[0] == 1
    s = orc.Sampler(4, 1.0, 1, 0.0, 3)
    assert {s.sample(tie, -1)[0] for _ in range(200)} == {1}
    s = orc.Sampler(4, 1.0, 0, 1e-7, 3)
    assert {s.sample(tie, -1)[0] for _ in range(200)} == {1}
    s = orc.Sampler(4, 0.0, 0, 0.0, 3, presence_penalty=100.0)
    assert s.sample(tie, 1)[0] == 3  # token 1 marked present and penalised
