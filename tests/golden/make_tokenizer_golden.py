"""Writes the tokenizer fixtures: two tokenizer.json vocabularies and, for
each, what the StrasGPT reference tokenizer produces on them.

The reference's tokenize / decode / report functions run compiled from
their own sources (oracle/_ref/ref_tokenizer, `make -C oracle ref`); the
harness restates only the post-parse steps of tokenizer_read (see
oracle/ref_tokenizer.c). Outputs, under tests/golden/:
  tokenizer/<case>/tokenizer.json   the vocabulary as a model directory holds it
  tokenizer-<case>.json             texts and ids fed in, and the outputs:
                                    unmapped vocabulary strings, token ids
                                    per text, decoded strings per id, and
                                    the report text (tokenizer_print and
                                    tokenizer_print_tokens)
Cases:
  bpe    ~700 entries: <unk> <s> </s>, the 256 "<0xHH>" byte entries,
         byte-level-BPE characters (Ġ = space, Ċ = newline, ...), raw
         UTF-8 characters of 2-4 bytes, strings that only a triple merge
         reaches, keys with JSON escapes kept verbatim, keys that unmap to
         the same bytes (duplicates), equal and non-integer scores, one
         score below -1e10; texts with stray continuation bytes, truncated
         sequences and one of 2500 characters.
  small  40 entries with BOS / EOS ids past the vocabulary and byte
         fallback ids past it too: such ids concatenate as "(null)" in the
         reference, and entries "(null)x" / "(null)(null)" make that
         observable.
Run from the repository root: python tests/golden/make_tokenizer_golden.py
"""
import json
import os
import random
import struct
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
HARNESS = os.path.join(ROOT, "oracle", "_ref", "ref_tokenizer")


def f32(x: float) -> float:
    return struct.unpack("<f", struct.pack("<f", x))[0]


def bpe_char(b: int) -> str:
    """Character standing for byte b in a byte-level vocabulary (the
    code points U+0100 + b that the reference maps back)."""
    return chr(0x100 + b)


def bpe_case(rng: random.Random):
    keys = ["<unk>", "<s>", "</s>"] + ["<0x%02X>" % b for b in range(256)]
    singles = [chr(c) for c in range(0x21, 0x7F) if chr(c) not in '"\\']
    keys += singles
    keys += [bpe_char(0x20), bpe_char(0x0A), bpe_char(0x09), " ", bpe_char(0x21)]
    keys += ["é", "€", "中", "😀", "éé", "中文"]
    alpha = "abcdeĠ"
    merged = {"abc"}  # scored below -1e10: never merged
    while len(merged) < 300:
        n = rng.randint(2, 6)
        merged.add("".join(rng.choice(alpha) for _ in range(n)))
    # reachable only by a triple merge: none of the pairs inside exists
    triples = ["qrs", "uvw", "QRS", "Ġxy"]
    for s in list(merged):
        for t in triples:
            if s in (t[:2], t[1:]):
                merged.discard(s)
    keys += sorted(merged) + triples
    keys += ['\\"q', "\\\\", "\\u0041", "Ā", "Āb", "ȀȀ", "Ġ\\n"]
    raw = [k.encode("utf-8") for k in keys]
    raw.append(b"\xc4A")          # lead byte 0xC4, next byte not a continuation
    raw.append(b"\xc5\x80z")      # U+0140 -> byte 0x40 '@', then 'z'
    scores = []
    for i in range(len(raw)):
        scores.append(str(i))
    for i in rng.sample(range(259, len(raw)), 80):   # shuffled merge priorities
        scores[i] = str(rng.randint(0, 2000))
    for i in rng.sample(range(300, len(raw)), 10):   # equal scores
        scores[i] = "777"
    for i in rng.sample(range(300, len(raw)), 6):    # non-integer numbers
        scores[i] = rng.choice(["12.5", "1e3", "-3", "2.5E+2", "0.125", "1500.75"])
    scores[raw.index(b"abc")] = "-1e11"
    texts = []
    for bos in (0, 1):
        for eos in (0, 1):
            texts.append((bos, eos, b""))
    pieces = ["a", "b", "c", "d", "e", " ", "\n", "\t", "qrs", "uvw", "xy", "é", "€",
              "中", "😀", "中文", '\\"q', "\\\\", "\\u0041", "@z", "!", "Z", "~"]
    for i in range(70):
        n = rng.randint(1, 60)
        s = "".join(rng.choice(pieces) for _ in range(n))
        texts.append((i % 2, (i // 2) % 2, s.encode("utf-8")))
    texts += [(1, 0, b"\x80\x80abc"), (0, 0, "é".encode() + b"\x80" * 5 + b"x"),
              (0, 1, b"ab\xe4"), (1, 1, b"\xf0\x9f\x98"), (0, 0, b"\xc4Aab"),
              (1, 0, b"\xff\xfe a"), (0, 0, b"abcabc abc")]
    long_text = "".join(rng.choice(pieces[:12]) for _ in range(1200)).encode("utf-8")[:2500]
    while long_text and (long_text[-1] & 0xC0) == 0x80:
        long_text = long_text[:-1]
    texts.append((1, 0, long_text))
    decode_ids = list(range(-2, len(raw) + 3))
    prints = [[1, 200, 300], [1] + [rng.randrange(len(raw)) for _ in range(20)] + [13, 4, -5, 9999],
              [16, 4, 263, 45]]
    return raw, scores, 1, 2, texts, decode_ids, prints


def small_case(rng: random.Random):
    keys = ["<unk>", "<s>", "</s>", "a", "b", "x", "ab", "(null)x", "(null)", "(null)(null)",
            "ba", "xa", "aba", "Ġ", "Ġa", "é"]
    while len(keys) < 40:
        keys.append("".join(rng.choice("abx") for _ in range(rng.randint(3, 5))))
        keys = list(dict.fromkeys(keys))
    raw = [k.encode("utf-8") for k in keys]
    scores = [str(i) for i in range(len(raw))]
    scores[raw.index(b"(null)x")] = "1000"
    scores[raw.index(b"(null)(null)")] = "900"
    texts = [(1, 1, b"xab"), (1, 0, b"xabba"), (0, 0, b"zz"), (1, 0, b"zzab"), (0, 1, b"a b"),
             (1, 1, b""), (0, 0, "é€".encode()), (1, 0, b"xxxx")]
    for i in range(20):
        texts.append((i % 2, 0, "".join(rng.choice("abxz é") for _ in range(rng.randint(1, 30))).encode()))
    decode_ids = list(range(-2, 45)) + [100, 101, 102]
    prints = [[100, 5, 3, 101], [7, 8, 9, 125, 100, 4, 4, 4, 4, 101]]
    return raw, scores, 100, 101, texts, decode_ids, prints


def hexs(b: bytes) -> str:
    return b.hex() if b else "-"


def write_vocab(path: str, raw, scores):
    body = b",".join(b'"' + k + b'":' + s.encode() for k, s in zip(raw, scores))
    with open(path, "wb") as f:
        f.write(b'{"version": "1.0", "added_tokens": [{"id": 0, "content": "<unk>"}],\n'
                b' "model": {"type": "BPE", "dropout": null, "vocab": {' + body +
                b'}, "merges": ["a b"]},\n "decoder": {"type": "ByteLevel"}}\n')


def run_reference(raw, scores, bos, eos, texts, decode_ids, prints):
    with tempfile.TemporaryDirectory() as d:
        man = os.path.join(d, "m.txt")
        with open(man, "w") as f:
            f.write("%d\n" % len(raw))
            for k, s in zip(raw, scores):
                f.write("%s %s\n" % (hexs(k), f32(float(s)).hex()))
            f.write("%d %d\n%d\n" % (bos, eos, len(texts)))
            for b, e, t in texts:
                f.write("%d %d %s\n" % (b, e, hexs(t)))
            f.write("%d %s\n" % (len(decode_ids), " ".join(map(str, decode_ids))))
            f.write("%d\n" % len(prints))
            for p in prints:
                f.write("%d %s\n" % (len(p), " ".join(map(str, p))))
        out, pout = os.path.join(d, "o.txt"), os.path.join(d, "p.txt")
        subprocess.run([HARNESS, man, out, pout], check=True, stderr=subprocess.DEVNULL)
        lines = open(out).read().split("\n")
        n = len(raw)
        unmapped = lines[:n]
        tokens = [[int(x) for x in ln.split()[1:]] for ln in lines[n:n + len(texts)]]
        decoded = lines[n + len(texts):n + len(texts) + len(decode_ids)]
        return unmapped, tokens, decoded, open(pout, "rb").read().decode("latin-1")


def main():
    if not os.path.exists(HARNESS):
        sys.exit("build the reference tokenizer first: make -C oracle ref")
    for name, make in (("bpe", bpe_case), ("small", small_case)):
        rng = random.Random(20251202 + len(name))
        raw, scores, bos, eos, texts, decode_ids, prints = make(rng)
        d = os.path.join(HERE, "tokenizer", name)
        os.makedirs(d, exist_ok=True)
        write_vocab(os.path.join(d, "tokenizer.json"), raw, scores)
        unmapped, tokens, decoded, report = run_reference(raw, scores, bos, eos, texts,
                                                          decode_ids, prints)
        doc = {"bos": bos, "eos": eos, "keys": [hexs(k) for k in raw],
               "unmapped": unmapped,
               "texts": [[b, e, hexs(t)] for b, e, t in texts], "tokens": tokens,
               "decode_ids": decode_ids, "decoded": decoded, "prints": prints,
               "report": report}
        with open(os.path.join(HERE, "tokenizer-%s.json" % name), "w") as f:
            json.dump(doc, f, indent=0)
        print(name, len(raw), "entries", len(texts), "texts")


if __name__ == "__main__":
    main()
