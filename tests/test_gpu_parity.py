"""Parity of the HIP library (called through the C-ABI) with the golden
fixtures of the reference C sources and with the CPU oracle.

Bars: greedy token ids identical; logits and
per-layer hidden states within 2e-2 relative and 1e-3 absolute
(|gpu - ref| <= 1e-3 + 2e-2 |ref|), fp32 accumulation.
"""
import os
import subprocess
import sys
import textwrap
import time

import numpy as np
import pytest

from conftest import GOLDEN_DIR, PROMPT_SEED, REPO
from hidden_states import check_hidden
from strasgpt_amd import synth

pytestmark = pytest.mark.gpu

RTOL, ATOL = 2e-2, 1e-3


def log(msg):
    print(f"[parity] {msg}", flush=True)


def runtime():
    from strasgpt_amd import runtime as rt
    rt.lib()
    return rt


def oracle_model(d, threads=16):
    from oracle import oracle as orc
    return orc.OracleModel(d, threads=threads)


GOLDEN_SHAPES = ["tiny-llama", "tiny-qwen", "tiny-chunk", "tiny-rope-il", "tiny-rope-il128"]


@pytest.mark.parametrize("name", GOLDEN_SHAPES)
def test_tiny_golden(name, model_dir):
    """Tokens identical to the reference C run; logits within tolerance."""
    rt = runtime()
    g = np.load(os.path.join(GOLDEN_DIR, f"{name}.npz"))
    prompt = [int(v) for v in g["prompt"]]
    log(f"{name}: T={len(prompt)} steps={len(g['generated'])}")
    with rt.Transformer(model_dir(name)) as t:
        logits = t.predict(prompt)
        np.testing.assert_allclose(logits[0], g["logits"], rtol=RTOL, atol=ATOL)
        err = np.abs(logits[0] - g["logits"]).max()
        log(f"{name}: max |logit error| {err:.3g}")
        assert err < 5e-4  # fp32-accumulate agreement, far inside the bar
        t.reset()
        tokens, _ = t.generate(prompt, len(g["generated"]))
        assert tokens == [int(v) for v in g["generated"]]


@pytest.mark.parametrize("tile", ["256x256", "128x384", "128x256", "128x128", "64x128x64", "64x128x64s4", "64x128",
                                  "64x64", "64x64x64s6"])
@pytest.mark.parametrize("name", ["tiny-qwen", "tiny-chunk"])
def test_gemm_tile_shapes(name, tile, model_dir, monkeypatch):
    """Every prefill GEMM tile shape (forced with STRASGPT_GEMM_TILE; by
    default the shape follows the grid size, so small models never reach
    the large tiles) through every epilogue: fused QKV, residual, split-K
    partial sums and SwiGLU. The 64x128x64 shapes (64-deep K stages; a
    deeper ring for W, or a 4-stage ring) need K to be a multiple of 64: the
    two models reach them with every epilogue between them (tiny-chunk: QKV,
    O, gate/up; tiny-qwen: O, down) and fall back to 64x128 elsewhere. Logits and tokens as in test_tiny_golden."""
    rt = runtime()
    g = np.load(os.path.join(GOLDEN_DIR, f"{name}.npz"))
    prompt = [int(v) for v in g["prompt"]]
    monkeypatch.setenv("STRASGPT_GEMM_TILE", tile)
    with rt.Transformer(model_dir(name)) as t:
        logits = t.predict(prompt)
        err = np.abs(logits[0] - g["logits"]).max()
        log(f"{name} {tile}: max |logit error| {err:.3g}")
        np.testing.assert_allclose(logits[0], g["logits"], rtol=RTOL, atol=ATOL)
        assert err < 5e-4
        t.reset()
        tokens, _ = t.generate(prompt, len(g["generated"]))
        assert tokens == [int(v) for v in g["generated"]]


def test_gemm_tile_orders(model_dir, monkeypatch):
    """The 256 x 256 prefill GEMM under each tile order (STRASGPT_GEMM_ORDER
    0-3; 3 is the default) on grids its XCD rectangles divide: the order only
    changes which block computes a tile, so every order gives bit-identical
    logits, which agree with the oracle."""
    rt = runtime()
    d = model_dir("mid-dense")
    shp = synth.shape("mid-dense")
    prompt = synth.prompt_tokens(shp.vocab, shp.prompt_len, PROMPT_SEED)
    ol = oracle_model(d, 16).predict(prompt)
    monkeypatch.setenv("STRASGPT_GEMM_TILE", "256x256")
    got = {}
    for order in ("0", "1", "2", "3"):
        # the order is read once per process: each runs in a child
        code = textwrap.dedent(f"""
            import sys, numpy as np
            sys.path.insert(0, {REPO!r})
            from strasgpt_amd import runtime as rt
            with rt.Transformer({d!r}) as t:
                np.save(sys.argv[1], t.predict({list(prompt)!r}))
        """)
        out = os.path.join(d, f"order{order}.npy")
        env = dict(os.environ, STRASGPT_GEMM_ORDER=order)
        r = subprocess.run([sys.executable, "-c", code, out], env=env, capture_output=True, text=True,
                           timeout=300)
        assert r.returncode == 0, r.stderr[-2000:]
        got[order] = np.load(out)
        err = float(np.abs(got[order] - ol).max())
        log(f"mid-dense order {order}: max |logit error| {err:.3g}")
        np.testing.assert_allclose(got[order], ol, rtol=RTOL, atol=ATOL)
    for order in ("1", "2", "3"):
        assert np.array_equal(got[order], got["0"])


def test_small_prompt_split_gemms(model_dir, monkeypatch):
    """Prompts of at most 32 rows run the QKV GEMM split over K (partial
    sums, then an epilogue kernel that adds them in split order and writes
    q and the key / value cache rows): prefill logits and greedy tokens
    against the oracle, and a 40-row prompt (the fused epilogue) agrees
    too. (Dense prompts of at most 8 rows take the multi-row GEMVs unless
    STRASGPT_PREFILL_ROWS=0, which this test sets.)"""
    monkeypatch.setenv("STRASGPT_PREFILL_ROWS", "0")
    rt = runtime()
    d = model_dir("small-m")
    shp = synth.shape("small-m")
    om = oracle_model(d, 16)
    with rt.Transformer(d) as t:
        for T in (8, 40):
            prompt = synth.prompt_tokens(shp.vocab, T, 17)
            om.reset()
            ol = om.predict(prompt)
            om.reset()
            otok = om.generate(prompt, 6)
            t.reset()
            gl = t.predict(prompt)
            err = float(np.abs(gl - ol).max())
            log(f"small-m T={T}: max |logit error| {err:.3g}")
            np.testing.assert_allclose(gl, ol, rtol=RTOL, atol=ATOL)
            t.reset()
            gtok, _ = t.generate(prompt, 6)
            assert gtok == otok


@pytest.mark.parametrize("name,kv", [("small-m", "fp32"), ("tiny-wide", "fp32"), ("tiny-wide2", "fp32"),
                                     ("small-m", "bf16"), ("tiny-llama", "fp32")])
def test_prefill_rows_form(name, kv, model_dir, monkeypatch):
    """Dense prompts of 2 to 8 tokens take the multi-row GEMVs (each weight
    row read once for every prompt row, fp32 FMAs, RMSNorm fused in; down
    projections longer than one LDS stage split over K: tiny-wide's 20480
    and tiny-wide2's 32768; rows not a multiple of 512 elements: tiny-wide's
    64 and tiny-llama's): prefill logits and the hidden states of every
    layer against the oracle, and against the GEMM path
    (STRASGPT_PREFILL_ROWS=0) within 2e-3; greedy tokens from the prefill
    identical to the oracle's; with a bf16 cache against the oracle's bf16
    cache."""
    from oracle import oracle as orc
    rt = runtime()
    d = model_dir(name)
    shp = synth.shape(name)
    om = orc.OracleModel(d, threads=16, kv_format=orc.KV_BF16 if kv == "bf16" else orc.KV_F32)
    for T in (2, 3, 5, 8):
        prompt = synth.prompt_tokens(shp.vocab, T, 40 + T)
        om.reset()
        ol, oh, of = om.predict(prompt, capture=True)
        om.reset()
        otok = om.generate(prompt, 4)
        got = {}
        for form in ("1", "0"):
            monkeypatch.setenv("STRASGPT_PREFILL_ROWS", form)
            with rt.Transformer(d) as t:
                if kv == "bf16":
                    t.set_kv_cache_format(rt.KV_BF16)
                gl, gh, gf = t.predict(prompt, capture=True)
                t.reset()
                gtok, _ = t.generate(prompt, 4)
            got[form] = gl
            err = float(np.abs(gl - ol).max())
            log(f"{name} kv {kv} T={T} rows form {form}: max |logit error| {err:.3g}")
            np.testing.assert_allclose(gl, ol, rtol=RTOL, atol=ATOL)
            check_hidden(gh, gf, oh, of, f"{name} T={T} form {form}")
            assert gtok == otok
        assert float(np.abs(got["1"] - got["0"]).max()) <= 2e-3


_LONG_CUTS = [0, 7, 8, 16, 21, 29, 30, 36, 40]


@pytest.mark.parametrize("name,kv,cuts", [("tiny-chunk", "fp32", _LONG_CUTS), ("small-m", "bf16", _LONG_CUTS),
                                          ("tiny-rope-il128", "fp32", _LONG_CUTS),
                                          ("tiny-qwen", "bf16", [0, 5, 6, 11, 19])])
def test_prefill_rows_continued(name, kv, cuts, model_dir, monkeypatch):
    """A prompt fed in pieces of 1 to 8 tokens across calls, over position
    32 where the context allows: pieces of 2 to 8 tokens take the multi-row
    GEMVs, whose QK-norm / RoPE kernel writes the new key and value rows
    into the attention operand planes (rows before the piece come from
    earlier calls; single tokens take the decode step, which writes its own
    row). Logits after every call against the oracle fed the same pieces
    (head_dim 32 and 128, interleaved RoPE, QK-norm with the staged bf16
    keys on tiny-qwen, fp32 and bf16 caches), and the last logits against
    the same pieces through the GEMM path (STRASGPT_PREFILL_ROWS=0, planes
    by split_rows)."""
    from oracle import oracle as orc
    rt = runtime()
    d = model_dir(name)
    shp = synth.shape(name)
    prompt = synth.prompt_tokens(shp.vocab, cuts[-1], 77)
    pieces = [prompt[a:b] for a, b in zip(cuts[:-1], cuts[1:])]
    om = orc.OracleModel(d, threads=16, kv_format=orc.KV_BF16 if kv == "bf16" else orc.KV_F32)
    last = {}
    for form in ("1", "0"):
        monkeypatch.setenv("STRASGPT_PREFILL_ROWS", form)
        om.reset()
        with rt.Transformer(d) as t:
            if kv == "bf16":
                t.set_kv_cache_format(rt.KV_BF16)
            for i, piece in enumerate(pieces):
                gl = t.predict(piece)
                ol = om.predict(piece)
                err = float(np.abs(gl - ol).max())
                log(f"{name} kv {kv} form {form} piece {i} ({len(piece)} tokens at {cuts[i]}): "
                    f"max |logit error| {err:.3g}")
                np.testing.assert_allclose(gl, ol, rtol=RTOL, atol=ATOL)
            last[form] = gl
    assert float(np.abs(last["1"] - last["0"]).max()) <= 2e-3


@pytest.mark.parametrize("kernel", ["x3", "x3-16", "x3-32", "fp32"])
@pytest.mark.parametrize("name", ["tiny-llama", "tiny-qwen", "tiny-chunk"])
def test_prefill_attention_kernels(name, kernel, model_dir, monkeypatch):
    """Both prefill attention kernels (STRASGPT_PREFILL_ATTN): split-bf16
    matrix-core products (x3, the default, with 16 or 32 queries per
    wavefront by the grid size, x3-16 / x3-32 forcing one; head_dim 16 pads
    the 32-dim k-step with zeros) and fp32 matrix-core products, over
    head_dim 16 (tiny-llama) and 32 (tiny-qwen; tiny-chunk: 520 queries,
    several query blocks, a partial last one, and key tiles). Logits and
    tokens as in test_tiny_golden."""
    rt = runtime()
    g = np.load(os.path.join(GOLDEN_DIR, f"{name}.npz"))
    prompt = [int(v) for v in g["prompt"]]
    monkeypatch.setenv("STRASGPT_PREFILL_ATTN", kernel)
    with rt.Transformer(model_dir(name)) as t:
        logits = t.predict(prompt)
        err = np.abs(logits[0] - g["logits"]).max()
        log(f"{name} {kernel}: max |logit error| {err:.3g}")
        np.testing.assert_allclose(logits[0], g["logits"], rtol=RTOL, atol=ATOL)
        assert err < 5e-4
        t.reset()
        tokens, _ = t.generate(prompt, len(g["generated"]))
        assert tokens == [int(v) for v in g["generated"]]


@pytest.mark.parametrize("chunks", ["1", "8", "64"])
def test_decode_attention_chunk_counts(chunks, model_dir, monkeypatch):
    """Decode attention with at most 1, 8 or 64 blocks per kv head
    (STRASGPT_DECODE_ATTN_CHUNKS; the default is 256 / kv_heads): over the
    520-token prompt of tiny-chunk that is one block holding all 17 key
    tiles (its result written directly), 6 blocks of 3 tiles, and 9 blocks
    of 2; the greedy tokens are the reference run's either way."""
    rt = runtime()
    g = np.load(os.path.join(GOLDEN_DIR, "tiny-chunk.npz"))
    prompt = [int(v) for v in g["prompt"]]
    monkeypatch.setenv("STRASGPT_DECODE_ATTN_CHUNKS", chunks)
    with rt.Transformer(model_dir("tiny-chunk")) as t:
        tokens, _ = t.generate(prompt, len(g["generated"]))
    log(f"tiny-chunk attention chunks {chunks}: {tokens}")
    assert tokens == [int(v) for v in g["generated"]]


@pytest.mark.parametrize("kv", ["fp32", "bf16"])
@pytest.mark.parametrize("name", ["tiny-chunk", "tiny-long"])
def test_decode_attention_four_waves(name, kv, model_dir, monkeypatch):
    """Decode attention with four wavefronts per block
    (STRASGPT_DECODE_ATTN_WAVES=4: one per SIMD, two fp32 key tiles each;
    the default is eight): tiny-chunk (4 query heads per kv head, one per
    wave in the combine) and tiny-long (8 on one kv head, two per wave),
    with an fp32 and a bf16 cache. Greedy tokens (graph and eager decode)
    equal the oracle's run with the same cache format. The logits of
    single-token steps after the prompt meet the 2e-2 / 1e-3 bar against
    it with an fp32 cache; with a bf16 cache they stay within a quarter of
    the format's own effect (the bf16-cache oracle against the fp32-cache
    one), the bar of the bf16-cache tests."""
    from oracle import oracle as orc
    rt = runtime()
    d = model_dir(name)
    shp = synth.shape(name)
    prompt = synth.prompt_tokens(shp.vocab, shp.prompt_len, 31)
    steps = shp.decode_len + 1
    om = orc.OracleModel(d, threads=16, kv_format=orc.KV_BF16 if kv == "bf16" else orc.KV_F32)
    of = orc.OracleModel(d, threads=16) if kv == "bf16" else None
    otok = om.generate(prompt, steps)
    monkeypatch.setenv("STRASGPT_DECODE_ATTN_WAVES", "4")
    with rt.Transformer(d) as t:
        if kv == "bf16":
            t.set_kv_cache_format(rt.KV_BF16)
        got = {}
        for mode in (rt.DECODE_GRAPH, rt.DECODE_EAGER):
            t.set_decode_mode(mode)
            t.reset()
            got[mode], _ = t.generate(prompt, steps)
        t.reset()
        om.reset()
        t.predict(prompt)
        om.predict(prompt)
        if of is not None:
            of.predict(prompt)
        worst, fmt = 0.0, 0.0
        for tok in otok[:3]:
            g, o = t.predict([tok])[0], om.predict([tok])[0]
            if of is None:
                np.testing.assert_allclose(g, o, rtol=RTOL, atol=ATOL)
            else:
                fmt = max(fmt, float(np.abs(o - of.predict([tok])[0]).max()))
            worst = max(worst, float(np.abs(g - o).max()))
    log(f"{name} {kv} cache, four waves: oracle {otok}, graph {got[rt.DECODE_GRAPH]}, "
        f"eager {got[rt.DECODE_EAGER]}; decode steps max |logit difference| {worst:.3g}"
        + (f" (format effect {fmt:.3g})" if of is not None else ""))
    if of is not None:
        assert fmt > 0 and worst <= 0.25 * fmt
    assert got[rt.DECODE_GRAPH] == otok
    assert got[rt.DECODE_EAGER] == otok


@pytest.mark.parametrize("chunk", ["512", "600"])
def test_prefill_chunk_lengths(chunk, model_dir, monkeypatch):
    """The 520-token prompt of tiny-chunk in device chunks of 512 (two
    chunks, the API's chunk length) and of 600 rows (one chunk): tokens and
    logits as in the reference run either way."""
    rt = runtime()
    g = np.load(os.path.join(GOLDEN_DIR, "tiny-chunk.npz"))
    prompt = [int(v) for v in g["prompt"]]
    monkeypatch.setenv("STRASGPT_PREFILL_CHUNK", chunk)
    with rt.Transformer(model_dir("tiny-chunk")) as t:
        logits = t.predict(prompt)
        err = np.abs(logits[0] - g["logits"]).max()
        log(f"tiny-chunk, chunk {chunk}: max |logit error| {err:.3g}")
        assert err < 5e-4
        t.reset()
        tokens, _ = t.generate(prompt, len(g["generated"]))
        assert tokens == [int(v) for v in g["generated"]]


@pytest.mark.parametrize("name", ["tiny-llama", "tiny-qwen"])
def test_tiny_hidden_states(name, model_dir):
    """Residual stream after every layer and the final-norm output against
    the oracle (prefill path) and against the golden normalised states."""
    rt = runtime()
    d = model_dir(name)
    g = np.load(os.path.join(GOLDEN_DIR, f"{name}.npz"))
    prompt = [int(v) for v in g["prompt"]]
    om = oracle_model(d, 4)
    _, oh, of = om.predict(prompt, capture=True)
    with rt.Transformer(d) as t:
        _, gh, gf = t.predict(prompt, capture=True)
    np.testing.assert_allclose(gh, oh, rtol=RTOL, atol=ATOL)
    np.testing.assert_allclose(gf, of, rtol=RTOL, atol=ATOL)
    np.testing.assert_allclose(gf, g["hidden"][-1], rtol=RTOL, atol=ATOL)


def test_decode_path_hidden_states(model_dir):
    """Single-token (GEMV / split-K attention) path against the oracle."""
    rt = runtime()
    d = model_dir("tiny-qwen")
    prompt = synth.prompt_tokens(300, 6, 21)
    om = oracle_model(d, 4)
    with rt.Transformer(d) as t:
        t.predict(prompt[:5])
        om.predict(prompt[:5])
        gl, gh, gf = t.predict(prompt[5:], capture=True)
        ol, oh, of = om.predict(prompt[5:], capture=True)
    np.testing.assert_allclose(gh, oh, rtol=RTOL, atol=ATOL)
    np.testing.assert_allclose(gl, ol, rtol=RTOL, atol=ATOL)
    assert np.abs(gl - ol).max() < 1e-4


def test_predict_host_loop_equals_device_loop(model_dir):
    """transformer_predict + host argmax (reference driver loop) gives the
    same tokens as the device-resident greedy loop and predict_argmax."""
    rt = runtime()
    d = model_dir("tiny-qwen")
    prompt = synth.prompt_tokens(300, 7, 13)
    with rt.Transformer(d) as t:
        dev, _ = t.generate(prompt, 9)
        t.reset()
        host = []
        logits = t.predict(prompt)
        host.append(int(np.argmax(logits[0])))
        while len(host) < 9:
            host.append(int(np.argmax(t.predict([host[-1]])[0])))
        t.reset()
        assert t.predict_argmax(prompt) == dev[0]
    assert host == dev


@pytest.mark.parametrize("name", ["tiny-chunk", "tiny-long"])
def test_prefill_after_decode_steps(name, model_dir):
    """A prompt fed as one prefill, and as a prefill of its first 37 tokens,
    then 40 single-token steps (the decode path, which writes each row into
    the cache and into the attention kernels' bf16 planes), then one chunk
    of the rest: the second prefill converts its own rows from row 64 (a
    multiple of 32) and attends to rows 37-63 as the decode steps wrote
    them. Last-row logits agree within 2e-3 of their largest magnitude
    (different kernels and summation orders; a row missing from the planes
    moves the logits by orders of magnitude more)."""
    rt = runtime()
    prompt = synth.prompt_tokens(128, 300 if name == "tiny-chunk" else 600, 23)
    with rt.Transformer(model_dir(name)) as t:
        whole = t.predict(prompt)[0]
        t.reset()
        t.predict(prompt[:37])
        for tok in prompt[37:77]:
            t.predict([tok])
        parts = t.predict(prompt[77:])[0]
    err = np.abs(parts - whole).max()
    scale = max(1.0, float(np.abs(whole).max()))
    log(f"{name}: max |logit difference| {err:.3g} (largest |logit| {scale:.3g})")
    assert err <= 2e-3 * scale


@pytest.mark.parametrize("name", ["tiny-llama", "tiny-qwen", "tiny-chunk", "tiny-long",
                                  "tiny-rope-il", "tiny-rope-il128", "tiny-wide"])
def test_decode_modes_agree(name, model_dir):
    """The graph-replayed decode step and the same kernels launched eagerly
    give identical greedy tokens, equal to the oracle's; a second graph run
    after reset repeats the first."""
    rt = runtime()
    d = model_dir(name)
    shp = synth.shape(name)
    prompt = synth.prompt_tokens(shp.vocab, shp.prompt_len, 31)
    steps = shp.decode_len + 1
    om = oracle_model(d, 4)
    otok = om.generate(prompt, steps)
    with rt.Transformer(d) as t:
        got = {}
        for mode in (rt.DECODE_GRAPH, rt.DECODE_EAGER):
            t.set_decode_mode(mode)
            t.reset()
            got[mode], _ = t.generate(prompt, steps)
        t.set_decode_mode(rt.DECODE_GRAPH)
        t.reset()
        again, _ = t.generate(prompt, steps)
    log(f"{name}: oracle {otok}")
    log(f"{name}: graph {got[rt.DECODE_GRAPH]} eager {got[rt.DECODE_EAGER]}")
    assert got[rt.DECODE_GRAPH] == otok
    assert got[rt.DECODE_EAGER] == otok
    assert again == otok


@pytest.mark.parametrize("name", ["tiny-qwen", "tiny-rope-il128", "tiny-wide", "tiny-wide2"])
def test_decode_step_logits(name, model_dir):
    """Single-token transformer_predict calls (decode GEMVs, split-K
    attention over the cache, final norm): logits at each of several
    positions and the hidden states of the last step agree with the
    oracle's."""
    rt = runtime()
    d = model_dir(name)
    shp = synth.shape(name)
    prompt = synth.prompt_tokens(shp.vocab, shp.prompt_len, 5)
    nxt = synth.prompt_tokens(shp.vocab, 4, 6)
    om = oracle_model(d, 4)
    om.predict(prompt)
    with rt.Transformer(d) as t:
        t.predict(prompt)
        for i, tok in enumerate(nxt):
            if i == len(nxt) - 1:  # the residual stream after every layer too
                ol, oh, of = om.predict([tok], capture=True)
                gl, gh, gf = t.predict([tok], capture=True)
                np.testing.assert_allclose(gh, oh, rtol=RTOL, atol=ATOL)
                np.testing.assert_allclose(gf, of, rtol=RTOL, atol=ATOL)
            else:
                ol = om.predict([tok])
                gl = t.predict([tok])
            err = np.abs(gl - ol).max()
            log(f"{name}: decode step logits max |error| {err:.3g}")
            np.testing.assert_allclose(gl, ol, rtol=RTOL, atol=ATOL)
            assert err < 1e-3


def test_reset_starts_a_new_sequence(model_dir):
    """After transformer_reset, a new sequence that starts with 45
    single-token steps (their rows go into the cache and its bf16 planes)
    and then prefills the rest attends to its own rows, not to the previous
    sequence's (rows 0-31 are read as the decode steps wrote them): last-row
    logits agree with the oracle on the new sequence alone."""
    rt = runtime()
    d = model_dir("tiny-chunk")
    a = synth.prompt_tokens(128, 300, 41)
    b = synth.prompt_tokens(128, 120, 43)
    om = oracle_model(d, 4)
    ol = om.predict(b)
    with rt.Transformer(d) as t:
        t.predict(a)
        t.reset()
        for tok in b[:45]:
            t.predict([tok])
        gl = t.predict(b[45:])
    err = np.abs(gl - ol).max()
    log(f"reset: max |logit error| {err:.3g}")
    np.testing.assert_allclose(gl, ol, rtol=RTOL, atol=ATOL)
    assert err < 1e-3


def _ref_argmax(x):
    """sample_argmax (source/sampler.c:92-102), as a sequential scan."""
    best, bv = 0, x[0]
    for i in range(1, len(x)):
        if x[i] > bv:
            best, bv = i, x[i]
    return best


def test_device_argmax_planted():
    """sampler_argmax on the device against the reference's sequential scan
    on planted cases: ties across block boundaries (the device reduces 512
    blocks of 256-element slices), NaN at index 0 (never replaced), NaNs
    elsewhere (never win), infinities, all-equal and single-element inputs,
    the benchmark vocabulary sizes."""
    rt = runtime()
    rng = np.random.default_rng(5)
    cases = []
    for n in (1, 7, 256, 257, 131072, 151936, 201088):
        cases.append(("random", rng.standard_normal(n).astype(np.float32)))
    n = 201088
    base = rng.standard_normal(n).astype(np.float32)
    tie = base.copy(); tie[[300, 70000, 200000]] = 9.0  # ties in different blocks
    cases.append(("ties across blocks", tie))
    tie2 = base.copy(); tie2[[511, 512]] = 9.0  # adjacent, straddling a slice edge
    cases.append(("adjacent tie", tie2))
    late = base.copy(); late[n - 1] = 9.0
    cases.append(("max at the end", late))
    nan0 = base.copy(); nan0[0] = np.nan; nan0[1000] = 9.0
    cases.append(("NaN at 0", nan0))
    nans = base.copy(); nans[::7] = np.nan; nans[12345] = 9.0; nans[99999] = 9.0
    cases.append(("NaNs elsewhere", nans))
    allnan = np.full(1000, np.nan, np.float32); allnan[0] = 1.0
    cases.append(("all NaN but the first", allnan))
    inf = base.copy(); inf[[10, 150000]] = np.inf
    cases.append(("+inf ties", inf))
    ninf = np.full(70000, -np.inf, np.float32)
    cases.append(("all -inf", ninf))
    ninf2 = ninf.copy(); ninf2[[40000, 50000]] = -1.0
    cases.append(("-inf but two", ninf2))
    same = np.full(100000, 0.5, np.float32)
    cases.append(("all equal", same))
    zeros = np.zeros(3000, np.float32); zeros[0] = -0.0; zeros[2999] = 0.0
    cases.append(("signed zeros", zeros))
    for what, x in cases:
        got, want = rt.argmax(x), _ref_argmax(x.tolist())
        log(f"argmax {what} (n={x.size}): device {got} reference {want}")
        assert got == want, what


def test_strasgpt_host_loop_openmp_team(model_dir):
    """The reference's calling convention (source/strasgpt.c:206-252): the
    driver's --host-loop calls transformer_predict from every thread of an
    8-thread OpenMP team and samples on the host; the ids equal the
    reference run's golden ids, and equal the device loop's."""
    from strasgpt_amd import _paths
    g = np.load(os.path.join(GOLDEN_DIR, "tiny-qwen.npz"))
    prompt = " ".join(str(int(v)) for v in g["prompt"])
    want = [int(v) for v in g["generated"]]
    d = model_dir("tiny-qwen")
    exe = _paths.driver_exe()
    for extra in (["--host-loop", "-t", "8"], []):
        cmd = [exe, "-m", d, "-n", str(len(want)), "--temp", "0", "--pre-tokenized", "-p", prompt,
               "--ids"] + extra
        r = subprocess.run(cmd, capture_output=True, text=True, timeout=120)
        log(f"strasgpt {' '.join(extra) or '(device loop)'}: rc {r.returncode} out {r.stdout.strip()}")
        assert r.returncode == 0, r.stderr[-2000:]
        assert [int(v) for v in r.stdout.split()] == want
        assert "Prompt processing (prefill)" in r.stderr


def test_strasgpt_text_prompt_and_token_strings(model_dir):
    """Without --pre-tokenized the driver tokenizes the text with the
    model's tokenizer.json and prepends BOS (source/strasgpt.c:169-172),
    then prints the generated tokens' strings (source/strasgpt.c:217-247):
    the same ids as a --pre-tokenized run on the library tokenizer's
    encoding, and their strings on stdout."""
    import json
    from strasgpt_amd import _paths
    rt = runtime()
    d = model_dir("tiny-qwen")
    cfg = json.load(open(os.path.join(d, "config.json")))
    bos, eos = cfg["bos_token_id"], cfg["eos_token_id"]
    tk = rt.Tokenizer(d, bos, eos)
    text = "<5> a"
    prompt_ids = tk.encode(text.encode(), bos=True)
    exe = _paths.driver_exe()
    n = 10
    assert len(prompt_ids) + n - 1 <= cfg["max_position_embeddings"]
    ids_cmd = [exe, "-m", d, "-n", str(n), "--temp", "0", "--pre-tokenized", "-p",
               " ".join(map(str, prompt_ids)), "--ids"]
    r = subprocess.run(ids_cmd, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
    ids = [int(v) for v in r.stdout.split()]
    expect = tk.decode(ids[0])
    for i in ids[1:]:
        if i == eos:
            expect += b"<|end_of_text|>"
            break
        expect += tk.decode(i)
    txt_cmd = [exe, "-m", d, "-n", str(n), "--temp", "0", "-p", text]
    r = subprocess.run(txt_cmd, capture_output=True, timeout=120)
    out = r.stdout.decode("latin-1")
    log(f"strasgpt text prompt: {len(prompt_ids)} prompt ids, rc {r.returncode} out {out[:120]!r}")
    err = r.stderr.decode("latin-1")
    assert r.returncode == 0, err[-2000:]
    assert f"Tokens ({len(prompt_ids)}):" in err
    assert out.rstrip("\n") == expect.decode("latin-1")
    assert "Prompt processing (prefill): %4d tokens" % len(prompt_ids) in err
    tk.close()


def test_strasgpt_sampling_flags(model_dir):
    """--temp / --top-k / --top-p / -s select the device sampler in both
    loops: the reference loop (--host-loop, logits on the host) and the
    device loop draw the same tokens from the same seed; another seed
    draws a different sequence."""
    from strasgpt_amd import _paths
    g = np.load(os.path.join(GOLDEN_DIR, "tiny-qwen.npz"))
    prompt = " ".join(str(int(v)) for v in g["prompt"])
    d = model_dir("tiny-qwen")
    exe = _paths.driver_exe()
    runs = {}
    for key, extra in (("host", ["--host-loop", "-t", "4", "-s", "7"]), ("device", ["-s", "7"]),
                       ("other", ["-s", "8"])):
        cmd = [exe, "-m", d, "-n", "8", "--temp", "0.9", "--top-k", "20", "--top-p", "0.95",
               "--pre-tokenized", "-p", prompt, "--ids"] + extra
        r = subprocess.run(cmd, capture_output=True, text=True, timeout=120)
        assert r.returncode == 0, r.stderr[-2000:]
        runs[key] = [int(v) for v in r.stdout.split()]
        log(f"strasgpt sampled ({key}): {runs[key]}")
    assert len(runs["host"]) == 8 and runs["host"] == runs["device"]
    assert runs["other"] != runs["device"]


REF_DRIVER = os.path.join(REPO, "oracle", "_ref", "ref_driver_hip")


@pytest.mark.skipif(not os.path.exists(REF_DRIVER),
                    reason="reference driver not built (oracle/Makefile ref_driver_hip needs "
                           "the reference sources when building)")
def test_reference_driver_on_the_library(model_dir):
    """The reference's own driver (source/strasgpt.c, options.c, sampler.c,
    util.c) linked against libstrasgpt_hip in place of its transformer,
    safetensors, tokenizer and JSON front-end: its stdout matches the
    library driver's byte for byte on the golden prompt (greedy, and
    sampled with the reference's CPU sampler against the device sampler
    from the same seed) and on a text prompt the library tokenizes."""
    from strasgpt_amd import _paths
    g = np.load(os.path.join(GOLDEN_DIR, "tiny-qwen.npz"))
    prompt = " ".join(str(int(v)) for v in g["prompt"])
    d = model_dir("tiny-qwen")
    exe = _paths.driver_exe()
    n = str(len(g["generated"]))
    cases = {
        "greedy": ["-n", n, "--temp", "0", "--pre-tokenized", "-p", prompt],
        "sampled": ["-n", "8", "--temp", "0.9", "--top-k", "20", "--top-p", "0.95", "-s", "7",
                    "--pre-tokenized", "-p", prompt],
        "text": ["-n", "10", "--temp", "0", "-p", "<5> a"],
    }
    got = {}
    for key, args in cases.items():
        outs = []
        for prog in (REF_DRIVER, exe):
            r = subprocess.run([prog, "-m", d] + args, capture_output=True, timeout=120)
            err = r.stderr.decode("latin-1")
            assert r.returncode == 0, f"{prog} {key}: {err[-2000:]}"
            assert "Prompt processing (prefill):" in err
            outs.append(r.stdout)
        log(f"reference driver ({key}): {outs[0][:80]!r}")
        assert outs[0] == outs[1], (key, outs)
        got[key] = outs[0]
    assert got["greedy"].strip() and got["sampled"] != got["greedy"]


@pytest.mark.skipif(not os.path.exists(REF_DRIVER),
                    reason="reference driver not built (oracle/Makefile ref_driver_hip needs "
                           "the reference sources when building)")
@pytest.mark.parametrize("name", ["tiny-llama", "tiny-moe", "tiny-rope-il"])
def test_reference_driver_model_families(name, model_dir):
    """The reference driver on the library over a dense Llama-type model,
    an MXFP4 mixture of experts and interleaved RoPE: greedy output equal
    to the library driver's, byte for byte."""
    from strasgpt_amd import _paths
    shp = synth.shape(name)
    prompt = " ".join(str(v) for v in synth.prompt_tokens(shp.vocab, shp.prompt_len, PROMPT_SEED))
    d = model_dir(name)
    outs = []
    for prog in (REF_DRIVER, _paths.driver_exe()):
        r = subprocess.run([prog, "-m", d, "-n", str(shp.decode_len), "--temp", "0", "--pre-tokenized",
                            "-p", prompt], capture_output=True, timeout=120)
        assert r.returncode == 0, r.stderr.decode("latin-1")[-2000:]
        outs.append(r.stdout)
    log(f"reference driver {name}: {outs[0][:60]!r}")
    assert outs[0] == outs[1] and outs[0].strip()


def _prompt_tokens_block(err):
    """The driver's 'Tokens (n):' report of the prompt ids (stderr)."""
    i = err.index("Tokens (")
    return err[i:err.index("\033[1;34m", i)]


@pytest.mark.skipif(not os.path.exists(REF_DRIVER),
                    reason="reference driver not built (oracle/Makefile ref_driver_hip needs "
                           "the reference sources when building)")
def test_reference_driver_instruct(model_dir, tmp_path):
    """--instruct wraps the prompt ids in the model family's chat template
    (source/strasgpt.c:170-179, source/util.c:514-575): the reference
    driver and the library driver report the same prompt ids for qwen3,
    llama and mistral model types and, where the template's ids fit the
    vocabulary (mistral), generate the same text. The qwen3 and llama
    templates make the prompts longer than the tiny models' contexts: both
    drivers stop with the library's host-side context error before any
    device work."""
    import json
    import shutil
    from strasgpt_amd import _paths
    g = np.load(os.path.join(GOLDEN_DIR, "tiny-qwen.npz"))
    ids = " ".join(str(int(v)) for v in g["prompt"])
    exe = _paths.driver_exe()
    mistral = str(tmp_path / "tiny-qwen-as-mistral")
    shutil.copytree(model_dir("tiny-qwen"), mistral)
    cfg_path = os.path.join(mistral, "config.json")
    cfg = json.load(open(cfg_path))
    cfg["model_type"] = "mistral"
    json.dump(cfg, open(cfg_path, "w"))
    cases = [(model_dir("tiny-qwen"), ["--pre-tokenized", "-p", ids], False),
             (model_dir("tiny-llama"), ["--pre-tokenized", "-p", ids], False),
             (mistral, ["--pre-tokenized", "-p", ids], True),
             (mistral, ["-p", "<5> a"], True)]
    for d, extra, runs in cases:
        res = []
        for prog in (REF_DRIVER, exe):
            r = subprocess.run([prog, "-m", d, "-n", "4", "--temp", "0", "--instruct"] + extra,
                               capture_output=True, timeout=120)
            res.append((r.returncode, r.stdout, r.stderr.decode("latin-1")))
        log(f"instruct {os.path.basename(d)} {extra[0]}: rc {res[0][0]}/{res[1][0]}, "
            f"{_prompt_tokens_block(res[0][2]).splitlines()[0]}")
        assert _prompt_tokens_block(res[0][2]) == _prompt_tokens_block(res[1][2])
        if runs:
            assert res[0][0] == 0 and res[1][0] == 0, res[1][2][-2000:]
            assert res[0][1] == res[1][1]
        else:
            assert res[0][0] != 0 and res[1][0] != 0
            assert res[0][2].rstrip().endswith("context length exhausted")
            assert res[1][2].rstrip().endswith("context length exhausted")


def test_first_token_eos_does_not_stop(model_dir):
    """The reference tests only decode steps' tokens against EOS
    (source/strasgpt.c:217-248): an EOS predicted from the prompt is kept
    and generation goes on; a later EOS ends it after being written."""
    g = np.load(os.path.join(GOLDEN_DIR, "tiny-qwen.npz"))
    prompt = [int(v) for v in g["prompt"]]
    want = [int(v) for v in g["generated"]]
    rt = runtime()
    with rt.Transformer(model_dir("tiny-qwen")) as t:
        eos = want[0]
        later = [k for k in range(1, len(want)) if want[k] == eos]
        expect = want[:later[0] + 1] if later else want
        got, _ = t.generate(prompt, steps=len(want), eos=eos)
        log(f"eos {eos}: got {len(got)} ids, expected {len(expect)}")
        assert list(got) == expect
        t.reset()
        eos = want[3]
        k = min(i for i in range(1, len(want)) if want[i] == eos)
        got, _ = t.generate(prompt, steps=len(want), eos=eos)
        assert list(got) == want[:k + 1]


@pytest.mark.parametrize("hook", ["strasgpt_kbench_mxfp4_decode", "strasgpt_kbench_mxfp4_decode_bf16"])
def test_mxfp4_device_decode_exact(hook):
    """The expert kernels' device MXFP4 decode (hardware E2M1 conversion
    scaled by the E8M0 exponent: to fp32 pairs in the GEMVs, to packed bf16
    pairs in the grouped prefill GEMM's tiles) equals the oracle's
    dequantisation bit for bit on every (code, scale) pair: 16 codes in both
    nibble positions x 256 scales (scale 255 decodes to NaN in both)."""
    import ctypes
    from oracle import oracle as orc
    rt = runtime()
    L = rt.lib()
    ol = orc.load_lib()
    nblocks = 256
    codes = np.empty((nblocks, 16), np.uint8)
    for i in range(16):
        codes[:, i] = i | ((15 - i) << 4)
    scales = np.arange(256, dtype=np.uint8)
    got = np.zeros(nblocks * 32, np.float32)
    fn = getattr(L, hook)
    fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.POINTER(ctypes.c_float)]
    assert fn(codes.ctypes.data, scales.ctypes.data, nblocks, orc.fptr(got)) == 0
    want = np.zeros(nblocks * 32, np.float32)
    ol.oracle_mxfp4_dequant(codes.ctypes.data, scales.ctypes.data, nblocks * 32, orc.fptr(want))
    nan_w, nan_g = np.isnan(want), np.isnan(got)
    np.testing.assert_array_equal(nan_g, nan_w)
    np.testing.assert_array_equal(got[~nan_w].view(np.uint32), want[~nan_w].view(np.uint32))


def test_logits_window_and_chunking(model_dir):
    """logits_count > 1 returns the last rows; a prompt split across calls
    matches one call (chunk invariance)."""
    rt = runtime()
    d = model_dir("tiny-llama")
    prompt = synth.prompt_tokens(256, 8, 17)
    om = oracle_model(d, 4)
    ol = om.predict(prompt, logits_count=3)
    with rt.Transformer(d) as t:
        gl = t.predict(prompt, logits_count=3)
        t.reset()
        t.predict(prompt[:3])
        gl2 = t.predict(prompt[3:], logits_count=1)
    np.testing.assert_allclose(gl, ol, rtol=RTOL, atol=ATOL)
    np.testing.assert_allclose(gl2[0], ol[-1], rtol=RTOL, atol=ATOL)


def test_moe_grouped_gemm_slot_tiles(model_dir, monkeypatch):
    """The grouped prefill GEMM with 32- and with 64-slot tiles
    (STRASGPT_MOE_TILE; 64 is taken when the experts average 24 slots or
    more): the same logits to fp32 rounding, both against the oracle."""
    rt = runtime()
    d = model_dir("tiny-moe-long")
    shp = synth.shape("tiny-moe-long")
    prompt = synth.prompt_tokens(256, shp.prompt_len, PROMPT_SEED)
    ol = oracle_model(d, 4).predict(prompt)
    got = {}
    with rt.Transformer(d) as t:
        for tile in ("32", "64"):
            monkeypatch.setenv("STRASGPT_MOE_TILE", tile)
            t.reset()
            got[tile] = t.predict(prompt)
            err = float(np.abs(got[tile] - ol).max())
            log(f"tiny-moe-long, {tile}-slot tiles: max |logit error| {err:.3g}")
            np.testing.assert_allclose(got[tile], ol, rtol=RTOL, atol=ATOL)
    # the slot tiling does not change any product's K order
    np.testing.assert_array_equal(got["32"], got["64"])


@pytest.mark.parametrize("name", ["tiny-moe", "tiny-moe-long",
                                  pytest.param("mid-moe", marks=pytest.mark.slow)])
def test_moe_tiny_against_oracle(name, model_dir):
    """MXFP4 MoE decoder: tokens identical to the oracle (the build's own
    restatement; no reference counterpart exists). The long prompt runs the
    grouped prefill GEMMs with several 32-slot tiles per expert; mid-moe
    runs the decode kernels on 2880-wide rows (90 MXFP4 blocks) with top-4."""
    rt = runtime()
    d = model_dir(name)
    shp = synth.shape(name)
    prompt = synth.prompt_tokens(256, shp.prompt_len, PROMPT_SEED)
    om = oracle_model(d, 4 if shp.dim < 1024 else 16)
    ol = om.predict(prompt)
    om.reset()
    otok = om.generate(prompt, 9)
    with rt.Transformer(d) as t:
        gl = t.predict(prompt)
        t.reset()
        gtok, _ = t.generate(prompt, 9)
    np.testing.assert_allclose(gl, ol, rtol=RTOL, atol=ATOL)
    assert gtok == otok


@pytest.mark.parametrize("name", ["tiny-moe-long", "mid-moe"])
def test_moe_prefill_router_selections_agree(name, model_dir, monkeypatch):
    """The prefill router's two top-k selections (one expert per lane for at
    most 64 experts, the default here; the scan over groups of 64 experts
    that larger expert counts take, forced by STRASGPT_MOE_ROUTE_SCAN=1)
    route every token alike: prefill logits bit-identical, greedy tokens
    equal to the oracle's either way."""
    rt = runtime()
    d = model_dir(name)
    shp = synth.shape(name)
    prompt = synth.prompt_tokens(256, shp.prompt_len, PROMPT_SEED)
    om = oracle_model(d, 4 if shp.dim < 1024 else 16)
    otok = om.generate(prompt, 9)
    got = {}
    for scan in ("0", "1"):
        monkeypatch.setenv("STRASGPT_MOE_ROUTE_SCAN", scan)
        with rt.Transformer(d) as t:
            logits = t.predict(prompt)
            t.reset()
            tokens, _ = t.generate(prompt, 9)
        got[scan] = (logits, tokens)
    log(f"{name}: oracle {otok}, lane selection {got['0'][1]}, scan {got['1'][1]}")
    assert np.array_equal(got["0"][0], got["1"][0])
    assert got["0"][1] == otok and got["1"][1] == otok


@pytest.mark.parametrize("name,T", [("tiny-llama", 8), ("tiny-moe-long", 200)])
def test_prefill_precision_modes(name, T, model_dir):
    """bf16x2 (default) agrees with the oracle to fp32 noise; the single
    bf16 mode (documented as lossy) stays within a few percent RMS and is
    at least 50x further from the oracle than bf16x2. On the MoE model the
    grouped expert GEMMs keep both bf16 planes of their activations in
    either mode."""
    rt = runtime()
    d = model_dir(name)
    prompt = synth.prompt_tokens(256, T, 23)
    om = oracle_model(d, 4)
    ol = om.predict(prompt)
    with rt.Transformer(d) as t:
        g2 = t.predict(prompt)
        t.reset()
        assert t.set_prefill_precision(1) == 0
        g1 = t.predict(prompt)
    rms = lambda a: float(np.sqrt(np.mean(np.square(a, dtype=np.float64))))
    e2, e1 = rms(g2 - ol) / rms(ol), rms(g1 - ol) / rms(ol)
    log(f"{name}: relative RMS logit error: bf16x2 {e2:.2e}, bf16 {e1:.2e}")
    assert e2 < 1e-4
    assert e1 < 5e-2 and e1 > 50 * e2


def _alias_language_model(src, dst):
    """A copy of a model directory whose tensors carry the Qwen3-VL names
    "model.language_model.<rest>" for "model.<rest>" (lm_head.weight keeps
    its name: the reference's alias table, source/transformer.c:520-574,
    maps it to itself). The data bytes and their offsets are unchanged."""
    import json
    import shutil
    import struct
    os.makedirs(dst)
    for f in os.listdir(src):
        if not f.endswith(".safetensors"):
            shutil.copy(os.path.join(src, f), dst)
            continue
        hl, hdr = synth.read_header(os.path.join(src, f))
        out = {}
        for name, v in hdr.items():
            if name.startswith("model."):
                name = "model.language_model." + name[len("model."):]
            out[name] = v
        blob = json.dumps(out).encode()
        with open(os.path.join(src, f), "rb") as fi, open(os.path.join(dst, f), "wb") as fo:
            fo.write(struct.pack("<Q", len(blob)) + blob)
            fi.seek(8 + hl)
            shutil.copyfileobj(fi, fo)
    return dst


@pytest.mark.parametrize("name", ["tiny-qwen", "tiny-llama"])
def test_language_model_aliases(name, model_dir, tmp_path):
    """A model whose tensors use the "model.language_model." names loads as
    the same model: QK-norm detected from the aliased q_norm name, the
    output tied (tiny-llama) or read from lm_head.weight (tiny-qwen), and
    logits bit-identical to the base-named model's; tokens equal the
    oracle's on the aliased files."""
    rt = runtime()
    d = model_dir(name)
    a = _alias_language_model(d, str(tmp_path / "aliased"))
    _, hdr = synth.read_header(os.path.join(a, "model.safetensors"))
    assert any(k.startswith("model.language_model.layers.") for k in hdr)
    assert not any(k.startswith("model.layers.") for k in hdr)
    shp = synth.shape(name)
    prompt = synth.prompt_tokens(shp.vocab, shp.prompt_len, PROMPT_SEED)
    steps = shp.decode_len + 1
    with rt.Transformer(d) as t:
        base = t.predict(prompt)
        qk, tied = t.config.qk_norm, t.config.aliased_out_weight
    with rt.Transformer(a) as t:
        assert (t.config.qk_norm, t.config.aliased_out_weight) == (qk, tied)
        got = t.predict(prompt)
        t.reset()
        tokens, _ = t.generate(prompt, steps)
    assert bool(qk) == shp.qk_norm and bool(tied) == (not shp.untied)
    np.testing.assert_array_equal(got, base)
    om = oracle_model(a, 4)
    assert tokens == om.generate(prompt, steps)


def test_context_exhausted_exits(model_dir):
    d = model_dir("tiny-llama")
    code = textwrap.dedent(f"""
        import sys
        sys.path.insert(0, {REPO!r})
        from strasgpt_amd import runtime as rt
        t = rt.Transformer({d!r})
        t.predict(list(range(20)))
        print("NOT REACHED")
    """)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 1 and "NOT REACHED" not in r.stdout
    assert "context length exhausted" in r.stderr


def _full_size(name, model_dir, steps=None):
    """Full-size model: greedy tokens of the device loop identical to the
    oracle's; the prompt prefill's logits, the residual stream after every
    layer (reference source/transformer.c:1498-1504; at the scale the next
    layer reads it, each row divided by its RMS) and the final-norm output
    within 2e-2 rel / 1e-3 abs of the oracle's (the prompt is one chunk of
    at most 512 tokens, the capture's limit)."""
    rt = runtime()
    shp = synth.shape(name)
    t0 = time.time()
    d = model_dir(name)
    log(f"{name}: model written in {time.time() - t0:.1f}s")
    prompt = synth.prompt_tokens(shp.vocab, shp.prompt_len, 42)
    steps = steps or shp.decode_len + 1
    with rt.Transformer(d) as t:
        log(f"{name}: loaded on GPU")
        gtok, tm = t.generate(prompt, steps)
        log(f"{name}: GPU prefill {tm.prefill_s:.3f}s decode {tm.decode_s:.3f}s")
        t.reset()
        gl, gh, gf = t.predict(prompt, capture=True)
    om = oracle_model(d, 16)
    log(f"{name}: oracle loaded")
    t0 = time.time()
    ol, oh, of = om.predict(prompt, capture=True)
    log(f"{name}: oracle prefill {time.time() - t0:.1f}s")
    np.testing.assert_allclose(gl, ol, rtol=RTOL, atol=ATOL)
    log(f"{name}: max |logit error| {np.abs(gl - ol).max():.3g}")
    check_hidden(gh, gf, oh, of, f"{name} prefill, every layer")
    del gh, oh
    om.reset()
    otok = om.generate(prompt, steps)
    log(f"{name}: oracle generate done; tokens {otok[:8]}...")
    assert gtok == otok


@pytest.mark.slow
@pytest.mark.timeout(600)
def test_llama32_1b_shape_tokens(model_dir):
    _full_size("llama3.2-1b", model_dir)


@pytest.mark.slow
@pytest.mark.timeout(900)
def test_qwen3_4b_shape_tokens(model_dir):
    _full_size("qwen3-4b", model_dir)


@pytest.mark.parametrize("name,cls", [("tiny-qwen", "gate_up_gemv"), ("tiny-moe", "moe_gate_up")])
def test_kernel_rate_hook(name, cls, model_dir):
    """The sustained-rate hook (back-to-back launches of one decode kernel
    class over every layer) returns a positive duration and the class's
    algorithmic bytes, refuses other classes, and leaves the generation
    state alone: the next decode step's logits are bit-identical."""
    rt = runtime()
    d = model_dir(name)
    shp = synth.shape(name)
    prompt = synth.prompt_tokens(256, shp.prompt_len, PROMPT_SEED)
    with rt.Transformer(d) as t:
        t.predict(prompt)
        ref = t.predict([5])
        t.reset()
        t.predict(prompt)
        r = t.kernel_rate(cls, reps=2)
        after = t.predict([5])
        refused = t.kernel_rate("attention_decode", reps=1)
    assert r is not None and r[0] > 0
    if shp.experts:
        want = shp.experts_per_tok * 2 * shp.hidden * shp.dim * (0.5 + 1 / 32)
    else:
        want = 2 * shp.hidden * shp.dim * 2
    assert r[1] == pytest.approx(want)
    assert refused is None
    np.testing.assert_array_equal(after, ref)
