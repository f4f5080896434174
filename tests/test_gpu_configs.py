"""The benchmark configurations whose full workload is too large for the CPU
oracle, on the GPU through the C-ABI:

* Llama-3.1-8B-shaped, 8192-token prompt + 256 decode tokens (16 prefill
  chunks of the reference's 512, decode attention over 8.4K keys),
* the MXFP4 MoE decoder (32 experts, top-4, 64 q heads, vocab 201088),
  256-token prompt + 128 decode tokens,
* Mistral-Small-24B-shaped (d 5120, FFN 32768), 2048-token prompt + 128
  decode tokens.

Three checks per configuration:

1. Full width and full prompt/decode length on two layers, against the
   oracle: the prefill logits and the logits of every decode step within
   2e-2 relative / 1e-3 absolute, greedy tokens identical (host loop over
   transformer_predict, and the device-resident greedy loop); the residual
   stream after each layer and the final-norm output for the rows of the
   prompt's last 512-token chunk, within the same bar at the scale the
   next layer reads them (each row divided by its RMS).
2. Full depth (every layer) against the oracle on a 16-token prompt and 8
   decode steps: hidden states after every layer, logits and tokens, with
   the same bars.
3. Full depth at the full prompt/decode length, properties that need no CPU
   reference:
   graph-replayed and eager decode give identical tokens; after the same
   prompt prefill, single-token decode steps and one multi-token chunk of
   the same tokens give the same logits (different kernels: GEMV vs MFMA
   GEMM, split-K vs tiled attention, MoE expert GEMVs vs grouped GEMMs);
   the host argmax of each step's logits is the token the device loop
   chose; for dense models, the same logits as the last rows of one
   prefill over prompt + generated tokens; for prompts longer than 512
   tokens, device prefill chunks of 512 rows and of the whole prompt give
   the same last-row logits. These logits agree to within 2e-3 absolute
   (besides 2e-2 rel / 1e-3 abs), three times the largest difference
   measured between the paths.

   The MoE model is not compared across different prompt prefills: top-k
   routing is discontinuous, and over 24 layers x 256 tokens some router
   logits tie to within fp32 rounding. Two computations that differ only in
   summation order (a 256-row and a 264-row prefill choose different
   split-K counts) can then route such a token differently; that token's
   keys and values change and every later position moves by ~1e-3. (On the
   workload's seed, token 117 at layer 1: the oracle, a 256-row device
   prefill and a 260-row one pick two different expert sets.)
"""
import contextlib
import os
import shutil
import tempfile
import time

import numpy as np
import pytest

from hidden_states import check_hidden
from strasgpt_amd import synth

pytestmark = [pytest.mark.gpu, pytest.mark.slow]

RTOL, ATOL = 2e-2, 1e-3
# Full-depth GPU path against GPU path (two fp32-accumulating computations
# that differ in kernels and summation order): the largest logit difference
# measured over the three models is 6.9e-4 (largest |logit| about 7), so
# the bar is three times that; an error of 1% of a logit in one path (about
# 5e-2) fails it.
PROP_ATOL = 2e-3
MODEL_SEED = 7


def log(msg):
    print(f"[configs] {msg}", flush=True)


def runtime():
    from strasgpt_amd import runtime as rt
    rt.lib()
    return rt


def ref_argmax():
    """The reference sample_argmax (source/sampler.c:92-102) from the oracle."""
    from oracle import oracle as orc
    lib = orc.load_lib()
    return lambda row: int(lib.oracle_argmax(orc.fptr(np.ascontiguousarray(row, np.float32)),
                                             row.size))


@contextlib.contextmanager
def written_model(name):
    """A model directory written for one test and deleted after it (the
    full-depth models take 14-47 GB of host memory under /dev/shm)."""
    base = "/dev/shm" if os.access("/dev/shm", os.W_OK) else None
    d = tempfile.mkdtemp(prefix=f"strasgpt_{name}_", dir=base)
    try:
        t0 = time.time()
        synth.write_model(synth.shape(name), d, seed=MODEL_SEED)
        log(f"{name}: model written in {time.time() - t0:.1f}s")
        yield d
    finally:
        shutil.rmtree(d, ignore_errors=True)


def check_logits(got, want, what, bound=None):
    """Within 2e-2 rel / 1e-3 abs; with `bound`, also max |got - want| <= bound."""
    err = float(np.abs(got - want).max())
    log(f"{what}: max |logit error| {err:.3g} (largest |logit| {float(np.abs(want).max()):.3g})")
    np.testing.assert_allclose(got, want, rtol=RTOL, atol=ATOL, err_msg=what)
    if bound is not None:
        assert err <= bound, f"{what}: max |logit difference| {err:.3g} > {bound:.3g}"


@pytest.mark.timeout(1200)
@pytest.mark.parametrize("name", ["llama3.1-8b-2l", "moe-mxfp4-2l", "mistral-small-24b-2l"])
def test_truncated_config_against_oracle(name):
    rt = runtime()
    from oracle import oracle as orc
    amax = ref_argmax()
    shp = synth.shape(name)
    prompt = synth.prompt_tokens(shp.vocab, shp.prompt_len, 42)
    steps = shp.decode_len + 1
    n_last = len(prompt) % 512 or 512
    with written_model(name) as d:
        t0 = time.time()
        with rt.Transformer(d) as t:
            g_logits = [t.predict(prompt)[0]]
            g_tok = [amax(g_logits[0])]
            while len(g_tok) < steps:
                g_logits.append(t.predict([g_tok[-1]])[0])
                g_tok.append(amax(g_logits[-1]))
            t.reset()
            dev_tok, _ = t.generate(prompt, steps)
            # hidden states of the prompt's last 512-token chunk (the
            # capture's limit), after the rest of the prompt in the cache
            t.reset()
            if len(prompt) > n_last:
                t.predict(prompt[:-n_last])
            cl, ch, cf = t.predict(prompt[-n_last:], capture=True)
        log(f"{name}: GPU host loop and device loop done in {time.time() - t0:.1f}s")
        t0 = time.time()
        om = orc.OracleModel(d, threads=16)
        # the prompt in pieces of 1024 tokens, then the last chunk (the
        # oracle, like the reference, runs 512-token chunks either way), one
        # line per piece
        for c0 in range(0, len(prompt) - n_last, 1024):
            om.predict(prompt[c0:min(c0 + 1024, len(prompt) - n_last)])
            log(f"{name}: oracle prefill through token {min(len(prompt) - n_last, c0 + 1024)} "
                f"at {time.time() - t0:.1f}s")
        ol, oh, of = om.predict(prompt[-n_last:], capture=True)
        ol = ol[0]
        check_logits(g_logits[0], ol, f"{name} prefill")
        check_logits(cl[0], ol, f"{name} prefill with the last chunk captured")
        check_hidden(ch, cf, oh, of, f"{name} last prefill chunk", om.router_margin)
        del ch, oh
        o_tok = [amax(ol)]
        worst = 0.0
        t0 = time.time()
        while len(o_tok) < steps:
            if o_tok != g_tok[:len(o_tok)]:
                break  # inputs differ from here on: the token assertion reports it
            row = om.predict([o_tok[-1]])[0]
            np.testing.assert_allclose(g_logits[len(o_tok)], row, rtol=RTOL, atol=ATOL,
                                       err_msg=f"{name} decode step {len(o_tok)}")
            worst = max(worst, float(np.abs(g_logits[len(o_tok)] - row).max()))
            o_tok.append(amax(row))
        om.close()
        log(f"{name}: oracle decode of {len(o_tok) - 1} steps in {time.time() - t0:.1f}s; "
            f"max |logit error| over the steps {worst:.3g}")
    log(f"{name}: tokens {g_tok[:10]}...")
    assert g_tok == o_tok
    assert dev_tok == o_tok


@pytest.mark.timeout(1200)
@pytest.mark.parametrize("name", ["llama3.1-8b", "moe-mxfp4", "mistral-small-24b"])
def test_full_config_properties(name, monkeypatch):
    rt = runtime()
    amax = ref_argmax()
    shp = synth.shape(name)
    prompt = synth.prompt_tokens(shp.vocab, shp.prompt_len, 42)
    steps = shp.decode_len + 1
    n_chk = 8
    with written_model(name) as d:
        with rt.Transformer(d) as t:
            log(f"{name}: loaded ({shp.layers} layers)")
            gtok, tm = t.generate(prompt, steps)
            log(f"{name}: graph decode {tm.decode_count} tokens in {tm.decode_s * 1e3:.1f} ms, "
                f"prefill {tm.prefill_s * 1e3:.1f} ms")
            t.set_decode_mode(rt.DECODE_EAGER)
            t.reset()
            etok, _ = t.generate(prompt, steps)
            t.set_decode_mode(rt.DECODE_GRAPH)
            assert etok == gtok, "eager and graph-replayed decode differ"
            # single-token steps over the first generated tokens
            t.reset()
            first = t.predict(prompt)[0]
            assert amax(first) == gtok[0]
            step_logits = [t.predict([tok])[0] for tok in gtok[:n_chk]]
            for i, row in enumerate(step_logits):
                assert amax(row) == gtok[i + 1], f"step {i + 1}: host argmax != device loop"
            # the same tokens as one chunk after the same prompt prefill
            t.reset()
            t.predict(prompt)
            chunk = t.predict(gtok[:n_chk], logits_count=n_chk)
            for i in range(n_chk):
                check_logits(chunk[i], step_logits[i], f"{name} chunk row vs decode step {i + 1}",
                             PROP_ATOL)
            if not shp.experts:
                # and as the last rows of one prefill over prompt + tokens
                t.reset()
                rows = t.predict(prompt + gtok[:n_chk], logits_count=n_chk)
                for i in range(n_chk):
                    check_logits(rows[i], step_logits[i], f"{name} prefill row vs decode step {i + 1}",
                                 PROP_ATOL)
        if len(prompt) > 512:
            monkeypatch.setenv("STRASGPT_PREFILL_CHUNK", "512")
            with rt.Transformer(d) as t:
                small = t.predict(prompt)[0]
            check_logits(small, first, f"{name} prefill in 512-row chunks vs one chunk", PROP_ATOL)
            assert amax(small) == gtok[0]
    log(f"{name}: tokens {gtok[:10]}...")


@pytest.mark.timeout(1200)
@pytest.mark.parametrize("name", ["llama3.1-8b", "moe-mxfp4", "mistral-small-24b"])
def test_full_depth_against_oracle(name):
    """Every layer of the configuration against the oracle on the first 16
    tokens of the workload's prompt, then 8 greedy decode steps: the
    residual stream after every layer and the final-norm output of the
    prompt prefill, the prefill logits and every decode step's logits within
    2e-2 rel / 1e-3 abs; greedy tokens identical (host loop over
    transformer_predict, and the device-resident loop). The short prompt
    keeps the oracle's share of the test to seconds (the 40-layer model
    streams 47 GB per token on the CPU)."""
    rt = runtime()
    from oracle import oracle as orc
    amax = ref_argmax()
    shp = synth.shape(name)
    prompt = synth.prompt_tokens(shp.vocab, shp.prompt_len, 42)[:16]
    steps = 9
    with written_model(name) as d:
        with rt.Transformer(d) as t:
            gl, gh, gf = t.predict(prompt, capture=True)
            g_logits = [gl[0]]
            g_tok = [amax(gl[0])]
            while len(g_tok) < steps:
                g_logits.append(t.predict([g_tok[-1]])[0])
                g_tok.append(amax(g_logits[-1]))
            t.reset()
            dev_tok, _ = t.generate(prompt, steps)
        log(f"{name}: GPU done ({shp.layers} layers)")
        t0 = time.time()
        om = orc.OracleModel(d, threads=16)
        log(f"{name}: oracle loaded in {time.time() - t0:.1f}s")
        t0 = time.time()
        ol, oh, of = om.predict(prompt, capture=True)
        log(f"{name}: oracle prefill of {len(prompt)} tokens in {time.time() - t0:.1f}s")
        check_hidden(gh, gf, oh, of, f"{name} prefill, every layer", om.router_margin)
        check_logits(g_logits[0], ol[0], f"{name} prefill")
        o_tok = [amax(ol[0])]
        while len(o_tok) < steps:
            if o_tok != g_tok[:len(o_tok)]:
                break  # inputs differ from here on: the token assertion reports it
            row = om.predict([o_tok[-1]])[0]
            check_logits(g_logits[len(o_tok)], row, f"{name} decode step {len(o_tok)}")
            o_tok.append(amax(row))
        om.close()
    log(f"{name}: tokens {g_tok}")
    assert g_tok == o_tok
    assert dev_tok == o_tok
