"""Writes the golden fixtures of tests/golden/ from the StrasGPT reference.

Runs in the build container only (needs /root/reference): oracle/Makefile
compiles the reference's own C sources into oracle/_ref/ref_harness, which
runs the reference greedy loop (source/strasgpt.c:206-252, --temp 0) on
tiny seeded synthetic models. Each fixture (<shape>.npz) holds:
  prompt, generated  int32 token ids (prefill token + decode tokens)
  logits             float32 [vocab] after the prompt
  hidden             float32 [L][T'][d]: final-RMSNorm output of the last
                     prompt chunk when only layers < l+1 run (norm weights
                     are 1.0, so this is the normalised residual stream
                     after layer l; entry L-1 is the full model)
  sha256             digest of model.safetensors (generator drift check)

Usage: python tests/golden/make_golden.py [shape ...]
"""
import hashlib
import os
import subprocess
import sys
import tempfile

import numpy as np

REPO = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, REPO)
from oracle import ref_manifest  # noqa: E402
from strasgpt_amd import synth  # noqa: E402

HARNESS = ref_manifest.HARNESS
SHAPES = ["tiny-llama", "tiny-qwen", "tiny-chunk", "tiny-rope-il", "tiny-rope-il128"]
MODEL_SEED = 7
PROMPT_SEED = 3


def run(manifest_path, out, layers=None):
    cmd = [HARNESS, manifest_path, out, "4"] + ([str(layers)] if layers else [])
    subprocess.run(cmd, check=True)
    return open(out, "rb").read()


def make(name):
    shp = synth.shape(name)
    d = tempfile.mkdtemp(prefix="golden_")
    synth.write_model(shp, d, seed=MODEL_SEED)
    prompt = synth.prompt_tokens(shp.vocab, shp.prompt_len, PROMPT_SEED)
    steps = shp.decode_len + 1
    man = ref_manifest.write(d, prompt, steps)
    last = len(prompt) % 512 or 512
    hidden = []
    for layers in range(1, shp.layers + 1):
        raw = run(man, os.path.join(d, f"out{layers}.bin"),
                  layers if layers < shp.layers else None)
        gen = np.frombuffer(raw[:4 * steps], np.int32)
        logits = np.frombuffer(raw[4 * steps:4 * (steps + shp.vocab)], np.float32)
        hid = np.frombuffer(raw[4 * (steps + shp.vocab):], np.float32)
        hidden.append(hid.reshape(last, shp.dim))
    digest = hashlib.sha256(open(os.path.join(d, "model.safetensors"), "rb").read()).hexdigest()
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), f"{name}.npz")
    np.savez_compressed(out, prompt=np.array(prompt, np.int32), generated=gen,
                        logits=logits, hidden=np.stack(hidden),
                        sha256=np.array(digest), model_seed=np.array(MODEL_SEED),
                        prompt_seed=np.array(PROMPT_SEED))
    print(name, "generated", list(gen), "->", out)


if __name__ == "__main__":
    for n in sys.argv[1:] or SHAPES:
        make(n)
