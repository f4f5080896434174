"""The device sampler (sampler_hip_t, transformer_generate_sampled) against
the reference's sampler_sample (source/sampler.c:234-337) restated by the
oracle (oracle_sample), on the GPU through the C-ABI.

The generator is integer arithmetic, so the state after every call must be
identical. The drawn token must be identical except where the device's
summation order can move a boundary across the coin: a different token is
accepted only when the coin lies within 4 sqrt(V) 2^-24 (four standard
deviations of the rounding walk of an fp32 running sum of V terms below 1:
7.5e-6 at V = 1000, 9.3e-5 at V = 151936) of the device token's interval in
the oracle's cumulative distribution (float64 sums of the oracle's final
probabilities), and top_p is that close to the oracle's cut. Sampling the
whole vocabulary of a flat distribution (intervals of ~7e-6 at V = 151936)
lands that close to a boundary often; filtered sampling rarely.
"""
import numpy as np
import pytest

from strasgpt_amd import synth

pytestmark = pytest.mark.gpu

def margin_bound(v):
    return 4 * np.sqrt(v) * 2.0 ** -24


def log(msg):
    print(f"[sampler] {msg}", flush=True)


def runtime():
    from strasgpt_amd import runtime as rt
    rt.lib()
    return rt


CASES = [  # temperature, top_k, top_p, presence penalty
    (1.0, 40, 0.9, 0.0),   # the reference driver's defaults (include/options.h:14-16)
    (1.0, 0, 0.0, 0.0),    # plain softmax sampling
    (0.7, 0, 0.95, 0.0),   # top-p only
    (1.3, 200, 0.0, 0.0),  # top-k only
    (1.0, 1, 0.0, 0.0),    # top-k 1: the argmax whatever the coin
    (0.0, 0, 0.0, 0.0),    # greedy: argmax, no coin drawn
    (0.0, 0, 0.0, 50.0),   # greedy with a presence penalty
    (0.9, 20, 0.8, 1.5),   # everything at once
]


@pytest.mark.parametrize("vocab", [1000, 151936])
@pytest.mark.parametrize("case", CASES, ids=[f"T{c[0]}-k{c[1]}-p{c[2]}-pen{c[3]}" for c in CASES])
def test_sampler_against_reference_steps(vocab, case):
    from oracle import oracle as orc
    rt = runtime()
    temp, k, p, pen = case
    rng = np.random.default_rng(vocab + int(100 * temp) + k)
    seed = 0x9E3779B97F4A7C15 + k
    dev = rt.Sampler(vocab, temp, k, p, seed, presence_penalty=pen)
    ref = orc.Sampler(vocab, temp, k, p, seed, presence_penalty=pen)
    close = 0
    prev = -1
    for i in range(24):
        logits = (rng.standard_normal(vocab) * rng.uniform(0.5, 4.0)).astype(np.float32)
        if i % 6 == 5:  # planted ties: the maximum repeated at a lower and a higher index
            j = int(np.argmax(logits))
            logits[(j + vocab // 3) % vocab] = logits[j]
            logits[(j + vocab // 2) % vocab] = logits[j]
        got = dev.sample(logits, prev)
        want, coin, margin, probs = ref.sample(logits, prev, probabilities=True)
        assert dev.rng_state == ref.rng_state, f"draw {i}: generator states differ"
        # every draw is a token of nonzero final probability: with top-k or
        # top-p, one of the kept set (the oracle zeroes the removed ones;
        # at temperature 0 it returns the argmax without probabilities)
        if temp > 0:
            assert probs[got] > 0, f"draw {i}: token {got} has probability 0 (removed)"
        if got != want:
            cdf = np.cumsum(probs.astype(np.float64))
            lo, hi = (cdf[got - 1] if got > 0 else 0.0), cdf[got]
            dist = max(lo - coin, coin - hi, 0.0)
            assert probs[got] > 0 and dist < margin_bound(vocab), \
                f"draw {i}: token {got} vs {want}, coin {coin}, device interval [{lo}, {hi}]"
            close += 1
        prev = want
    dev.close()
    log(f"V={vocab} {case}: 24 draws, {close} different (within {margin_bound(vocab):.2g} of the coin)")
    if k > 0 or 0 < p <= 1:
        assert close <= 1


@pytest.mark.parametrize("name", ["tiny-qwen", "tiny-moe"])
def test_generate_sampled_against_oracle(name, model_dir):
    """transformer_generate_sampled (device decode loop, one draw per
    token) replayed through the oracle forward pass and sampler (teacher
    forcing): every token is the oracle's draw with the same generator
    state, or a draw within 2e-3 of a boundary (the logits themselves differ
    by ~1e-4); the generator ends in the same state; temperature 0 gives the
    greedy tokens; graph and eager decode draw the same tokens."""
    from oracle import oracle as orc
    rt = runtime()
    d = model_dir(name)
    shp = synth.shape(name)
    prompt = synth.prompt_tokens(shp.vocab, shp.prompt_len, 8)
    steps = shp.decode_len + 1
    with rt.Transformer(d) as t:
        greedy, _ = t.generate(prompt, steps)
        t.reset()
        s0 = rt.Sampler(t.vocab, 0.0, 0, 0.0, 1)
        assert t.generate_sampled(prompt, steps, s0)[0] == greedy
        s0.close()
        toks = {}
        for mode in (rt.DECODE_GRAPH, rt.DECODE_EAGER):
            t.set_decode_mode(mode)
            t.reset()
            smp = rt.Sampler(t.vocab, 1.2, 10, 0.95, 4242)
            toks[mode], _ = t.generate_sampled(prompt, steps, smp)
            state = smp.rng_state
            smp.close()
        t.set_decode_mode(rt.DECODE_GRAPH)
    assert toks[rt.DECODE_GRAPH] == toks[rt.DECODE_EAGER]
    gtok = toks[rt.DECODE_GRAPH]
    om = orc.OracleModel(d, threads=4)
    ref = orc.Sampler(om.vocab, 1.2, 10, 0.95, 4242)
    row = om.predict(prompt)[0]
    prev = prompt[-1]
    near = 0
    for i in range(steps):
        want, coin, margin = ref.sample(row, prev)
        if want != gtok[i]:
            assert margin < 2e-3, f"step {i}: {gtok[i]} vs {want} (coin {coin}, margin {margin:.3g})"
            near += 1
        prev = gtok[i]
        if i + 1 < steps:
            row = om.predict([gtok[i]])[0]
    log(f"{name}: {steps} sampled tokens {gtok}; {near} near-boundary draws")
    assert ref.rng_state == state
    assert near <= 1


@pytest.mark.parametrize("n", [1, 63, 256, 1000, 151936, 262145])
@pytest.mark.parametrize("kind", ["probabilities", "full-range"])
def test_sort_desc_stable(n, kind):
    """The sampler's radix sort (hand-written, four 8-bit passes) through
    strasgpt_kbench_sort_desc: keys in descending order, equal keys in index
    order, bit for bit against numpy's stable argsort. Probability-like keys
    (fp32 bit patterns of values in [0, 1]: most of the high digits equal,
    many zeros and planted ties) and full-range 32-bit keys (every digit
    varies); sizes with ragged last tiles and chunks."""
    import ctypes
    rt = runtime()
    L = rt.lib()
    rng = np.random.default_rng(n + (7 if kind == "full-range" else 0))
    if kind == "probabilities":
        p = rng.exponential(1.0, n).astype(np.float32) ** 4
        p[rng.random(n) < 0.3] = 0.0  # many exact zeros
        p /= max(float(p.sum()), 1e-30)
        if n > 8:
            p[rng.integers(0, n, n // 8)] = p[rng.integers(0, n)]  # ties with one value
        keys = p.astype(np.float32).view(np.uint32)
    else:
        keys = rng.integers(0, 2 ** 32, n, dtype=np.uint64).astype(np.uint32)
        if n > 8:
            keys[rng.integers(0, n, n // 8)] = keys[rng.integers(0, n)]
    keys = np.ascontiguousarray(keys)
    got_k = np.zeros(n, np.uint32)
    got_i = np.zeros(n, np.int32)
    fn = L.strasgpt_kbench_sort_desc
    fn.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    assert fn(keys.ctypes.data, n, got_k.ctypes.data, got_i.ctypes.data) == 0
    order = np.argsort(-keys.astype(np.int64), kind="stable")
    np.testing.assert_array_equal(got_i, order.astype(np.int32))
    np.testing.assert_array_equal(got_k, keys[order])
    log(f"sort n={n} {kind}: order identical")
