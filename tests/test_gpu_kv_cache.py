"""The bf16 KV-cache format (transformer_set_kv_cache_format, no reference
counterpart: the reference cache is fp32, source/transformer.c:74 and
:1271-1291), on the GPU through the C-ABI.

Parity: against the oracle run with the same cache format (every key after
its norm and RoPE, and every value, rounded to the nearest bf16 when it is
written; oracle_set_kv_format): greedy tokens identical, and logits far
closer to that oracle than the format moves them. The bar is relative to
the format's own effect, not fp32 noise: the GPU's fp32 keys and values
differ from the oracle's by ~1e-5 relative (summation order, bf16x2
GEMM), so a fraction of them round to the other bf16 neighbour, a one-ulp
(2^-8) difference; on the tiny models (sharp attention) that leaves
~5-10% of the format's effect. A cache write that skipped the rounding, or
rounded a different value, would leave all of it.

Study: against the fp32-cache oracle the rounding itself moves the logits;
the tests print by how much, and the full-size shapes check that the moved
logits still meet the 2e-2 relative / 1e-3 absolute bar.
"""
import subprocess
import sys
import textwrap
import time

import numpy as np
import pytest

from conftest import REPO
from strasgpt_amd import synth

pytestmark = pytest.mark.gpu

RTOL, ATOL = 2e-2, 1e-3


def log(msg):
    print(f"[kv-bf16] {msg}", flush=True)


def runtime():
    from strasgpt_amd import runtime as rt
    rt.lib()
    return rt


def oracle(d, fmt, threads=4):
    from oracle import oracle as orc
    return orc.OracleModel(d, threads=threads, kv_format=fmt)


@pytest.mark.parametrize("name", ["tiny-llama", "tiny-qwen", "tiny-chunk", "tiny-long", "tiny-moe",
                                  "tiny-rope-il", "tiny-rope-il128"])
def test_bf16_cache_against_oracle(name, model_dir):
    """Prefill logits, greedy tokens (graph and eager decode) and the
    logits of single-token steps with a bf16 cache equal the bf16-cache
    oracle's; the fp32-cache oracle is further away (the format's own
    effect, printed)."""
    from oracle import oracle as orc
    rt = runtime()
    d = model_dir(name)
    shp = synth.shape(name)
    prompt = synth.prompt_tokens(shp.vocab, shp.prompt_len, 31)
    steps = shp.decode_len + 1
    ob = oracle(d, orc.KV_BF16)
    of = oracle(d, orc.KV_F32)
    ol_b, ol_f = ob.predict(prompt)[0], of.predict(prompt)[0]
    ob.reset()
    otok = ob.generate(prompt, steps)
    with rt.Transformer(d) as t:
        assert t.set_kv_cache_format(rt.KV_BF16) == rt.KV_FP32
        gl = t.predict(prompt)[0]
        t.reset()
        gtok, _ = t.generate(prompt, steps)
        t.set_decode_mode(rt.DECODE_EAGER)
        t.reset()
        etok, _ = t.generate(prompt, steps)
        t.set_decode_mode(rt.DECODE_GRAPH)
        # single-token steps after the prompt, both oracles alongside
        t.reset()
        ob.reset()
        of.reset()
        t.predict(prompt)
        ob.predict(prompt)
        of.predict(prompt)
        steps_gpu, steps_fmt = 0.0, 0.0
        for tok in otok[:3]:
            g, o, f = t.predict([tok])[0], ob.predict([tok])[0], of.predict([tok])[0]
            steps_gpu = max(steps_gpu, float(np.abs(g - o).max()))
            steps_fmt = max(steps_fmt, float(np.abs(o - f).max()))
    err = float(np.abs(gl - ol_b).max())
    fmt_err = float(np.abs(ol_b - ol_f).max())
    log(f"{name}: GPU vs bf16-cache oracle: prefill {err:.3g}, decode steps {steps_gpu:.3g}; "
        f"bf16 vs fp32 cache (oracle): prefill {fmt_err:.3g}, decode steps {steps_fmt:.3g} "
        f"(largest |logit| {float(np.abs(ol_f).max()):.3g})")
    assert fmt_err > 0 and steps_fmt > 0
    assert err <= 0.25 * fmt_err and steps_gpu <= 0.25 * steps_fmt
    assert gtok == otok
    assert etok == otok


def test_bf16_cache_prefill_after_decode_steps(model_dir):
    """Rows written by decode steps with a bf16 cache go into the attention
    kernels' planes as the prefill writes them: a prompt as one prefill, and
    as a prefill, 40 single-token steps and one chunk of the rest (which
    reads rows 37-63 from the decode steps), give the same last-row logits
    (within 2e-3 of their largest magnitude)."""
    rt = runtime()
    prompt = synth.prompt_tokens(128, 600, 23)
    with rt.Transformer(model_dir("tiny-long")) as t:
        t.set_kv_cache_format(rt.KV_BF16)
        whole = t.predict(prompt)[0]
        t.reset()
        t.predict(prompt[:37])
        for tok in prompt[37:77]:
            t.predict([tok])
        parts = t.predict(prompt[77:])[0]
    err = np.abs(parts - whole).max()
    scale = max(1.0, float(np.abs(whole).max()))
    log(f"tiny-long: max |logit difference| {err:.3g} (largest |logit| {scale:.3g})")
    assert err <= 2e-3 * scale


def test_format_switch_and_refusal(model_dir):
    """The format switches back and forth on an empty cache (fp32 results
    unchanged by a bf16 round trip), and a switch with tokens in the cache
    exits with the library's error."""
    rt = runtime()
    d = model_dir("tiny-qwen")
    prompt = synth.prompt_tokens(300, 12, 4)
    with rt.Transformer(d) as t:
        a = t.predict(prompt)
        t.reset()
        assert t.set_kv_cache_format(rt.KV_BF16) == rt.KV_FP32
        t.predict(prompt)
        t.reset()
        assert t.set_kv_cache_format(rt.KV_FP32) == rt.KV_BF16
        b = t.predict(prompt)
    np.testing.assert_array_equal(a, b)
    code = textwrap.dedent(f"""
        import sys
        sys.path.insert(0, {REPO!r})
        from strasgpt_amd import runtime as rt
        t = rt.Transformer({d!r})
        t.predict([1, 2, 3])
        t.set_kv_cache_format(rt.KV_BF16)
        print("NOT REACHED")
    """)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 1 and "NOT REACHED" not in r.stdout
    assert "KV-cache format can only change while the cache is empty" in r.stderr


@pytest.mark.slow
@pytest.mark.timeout(900)
@pytest.mark.parametrize("name", ["llama3.2-1b", "qwen3-4b"])
def test_bf16_cache_full_size(name, model_dir):
    """The Llama-3.2-1B and Qwen3-4B shapes at full size with the bf16 cache. The GPU's greedy
    tokens are replayed through the bf16-cache oracle (teacher forcing):
    every token is the oracle's argmax, or within 0.05 of it (a near tie
    that the ~5e-3 logit differences can flip; counted and printed). The
    prefill logits sit closer to the bf16-cache oracle than the format moves
    them (at most 35% of the bf16 - fp32 cache difference, rounding flips
    of the GPU's slightly different fp32 keys and values). The study: the
    prefill error against the fp32-cache oracle and the step where its own
    greedy tokens part from the GPU's, printed."""
    from oracle import oracle as orc
    rt = runtime()
    shp = synth.shape(name)
    t0 = time.time()
    d = model_dir(name)
    log(f"{name}: model written in {time.time() - t0:.1f}s")
    prompt = synth.prompt_tokens(shp.vocab, shp.prompt_len, 42)
    steps = shp.decode_len + 1
    with rt.Transformer(d) as t:
        t.set_kv_cache_format(rt.KV_BF16)
        gtok, tm = t.generate(prompt, steps)
        log(f"{name}: GPU prefill {tm.prefill_s:.3f}s decode {tm.decode_s:.3f}s")
        t.reset()
        gl = t.predict(prompt)[0]
    of = oracle(d, orc.KV_F32, threads=16)
    ol_f = of.predict(prompt)[0]
    of.reset()
    ftok = of.generate(prompt, steps)
    of.close()
    ob = oracle(d, orc.KV_BF16, threads=16)
    t0 = time.time()
    row = ob.predict(prompt)[0]
    ol_b = row
    near = []
    for i in range(steps):
        best = int(np.argmax(row))
        if best != gtok[i]:
            margin = float(row[best] - row[gtok[i]])
            near.append((i, margin))
            assert margin < 0.05, f"step {i}: GPU token {gtok[i]} is {margin:.3g} below the oracle's best"
        if i + 1 < steps:
            row = ob.predict([gtok[i]])[0]
    ob.close()
    err, fmt = float(np.abs(gl - ol_b).max()), float(np.abs(ol_b - ol_f).max())
    part = next((i for i, (a, b) in enumerate(zip(gtok, ftok)) if a != b), None)
    log(f"{name}: teacher-forced bf16-cache oracle over {steps} steps in {time.time() - t0:.1f}s: "
        f"{len(near)} near-tie choices {near}")
    log(f"{name}: prefill logits: GPU vs bf16-cache oracle {err:.3g}, bf16 vs fp32 cache {fmt:.3g}, "
        f"GPU vs fp32-cache oracle {float(np.abs(gl - ol_f).max()):.3g}; greedy tokens vs the "
        f"fp32-cache oracle: {'identical' if part is None else f'part at step {part}'} of {steps}")
    assert err <= 0.35 * fmt
    assert len(near) <= 2
