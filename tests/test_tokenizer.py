"""The tokenizer of libstrasgpt_hip (include/tokenizer.h) against the StrasGPT
reference tokenizer (source/tokenizer.c), on the CPU.

Fixtures (tests/golden/make_tokenizer_golden.py): two tokenizer.json
vocabularies and what the reference's own tokenize / decode / report
functions, compiled from its sources, produced on them. When the reference
build is present (oracle/_ref/ref_tokenizer, this container only), random
texts are also run through both.
"""
import ctypes
import json
import os
import random
import subprocess
import tempfile

import pytest

from conftest import GOLDEN_DIR
from strasgpt_amd import _paths

pytestmark = pytest.mark.skipif(not os.path.exists(_paths.hip_lib()), reason="library not built")

CASES = ["bpe", "small"]


def golden(case):
    with open(os.path.join(GOLDEN_DIR, "tokenizer-%s.json" % case)) as f:
        return json.load(f)


def unhex(s):
    return b"" if s == "-" else bytes.fromhex(s)


@pytest.fixture(scope="module", params=CASES)
def case(request):
    from strasgpt_amd.runtime import Tokenizer
    g = golden(request.param)
    tok = Tokenizer(os.path.join(GOLDEN_DIR, "tokenizer", request.param), g["bos"], g["eos"])
    yield request.param, g, tok
    tok.close()


def test_vocabulary_read_and_unmapped(case):
    """Entries in file order, the byte-level characters mapped back to bytes
    as the reference's tokenizer_read does (source/tokenizer.c:87-115,
    124-127)."""
    _, g, tok = case
    assert len(tok) == len(g["unmapped"])
    for i, u in enumerate(g["unmapped"]):
        assert tok.token_bytes(i) == unhex(u), i
    t = tok.t
    assert t.max_token_string_len == max(len(unhex(u)) for u in g["unmapped"])
    for b in range(256):
        assert t.byte_string[2 * b] == b and t.byte_string[2 * b + 1] == 0


def test_unmapping_known_answers():
    """Pins of the harness's restatement of the byte-level unmapping, from
    the definition of the map (code point U+0100 + b stands for byte b,
    only two-byte sequences with code points U+0100..U+01FF are mapped)."""
    g = golden("bpe")
    by_key = dict(zip((unhex(k) for k in g["keys"]), (unhex(u) for u in g["unmapped"])))
    assert by_key["Ġ".encode()] == b" "          # U+0120
    assert by_key["Ċ".encode()] == b"\n"         # U+010A
    assert by_key["ĉ".encode()] == b"\t"         # U+0109
    assert by_key["ġ".encode()] == b"!"          # U+0121: same bytes as "!"
    assert by_key["Ā".encode()] == b""           # U+0100 -> NUL ends the string
    assert by_key["Āb".encode()] == b""
    assert by_key["ȀȀ".encode()] == "ȀȀ".encode()  # U+0200: outside the map
    assert by_key["é".encode()] == "é".encode()  # U+00E9: outside the map
    assert by_key["中文".encode()] == "中文".encode()
    assert by_key[b"\xc4A"] == b"\x01"            # continuation bits not checked
    assert by_key[b"\xc5\x80z"] == b"@z"          # U+0140 -> 0x40
    assert by_key[b'\\"q'] == b'\\"q'            # JSON escapes kept as written
    assert by_key["Ġ\\n".encode()] == b" \\n"


def test_sorted_index(case):
    """The lookup index: strcmp order, equal strings in id order."""
    _, g, tok = case
    t = tok.t
    keys = [(t.sorted_token_string[i].token_string, t.sorted_token_string[i].id)
            for i in range(len(tok))]
    assert sorted(keys) == keys
    assert sorted(k[1] for k in keys) == list(range(len(tok)))


def test_tokenize_matches_reference(case):
    _, g, tok = case
    for (bos, eos, text), want in zip(g["texts"], g["tokens"]):
        assert tok.encode(unhex(text), bool(bos), bool(eos)) == want, (bos, eos, text[:80])


def test_decode_matches_reference(case):
    _, g, tok = case
    for i, want in zip(g["decode_ids"], g["decoded"]):
        assert tok.decode(i) == unhex(want), i


def test_report_lines_match_reference(case, capfd):
    """tokenizer_print and tokenizer_print_tokens write the reference's
    lines byte for byte."""
    from strasgpt_amd.runtime import _libc, _ints
    _, g, tok = case
    L, C = tok._lib, _libc()
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "r.txt").encode()
        f = C.fopen(path, b"w")
        L.tokenizer_print(f, tok.handle)
        for p in g["prints"]:
            L.tokenizer_print_tokens(tok.handle, f, len(p), _ints(p), 4)
        C.fclose(f)
        got = open(path, "rb").read().decode("latin-1")
    assert got == g["report"]


def test_tokenize_long_text_is_fast():
    """Cached pair / triple merges: 20000 characters in well under a second
    (the reference rebuilds every pair string per merge)."""
    import time
    from strasgpt_amd.runtime import Tokenizer
    g = golden("bpe")
    tok = Tokenizer(os.path.join(GOLDEN_DIR, "tokenizer", "bpe"), g["bos"], g["eos"])
    rng = random.Random(5)
    text = "".join(rng.choice(["a", "b", "c", "d", "e", " ", "qrs", "xy", "é"]) for _ in range(10000))
    t0 = time.perf_counter()
    ids = tok.encode(text.encode()[:20000])
    assert time.perf_counter() - t0 < 2.0
    assert ids[0] == g["bos"] and len(ids) > 100
    tok.close()


HARNESS = os.path.join(os.path.dirname(GOLDEN_DIR), "..", "oracle", "_ref", "ref_tokenizer")


@pytest.mark.skipif(not os.path.exists(HARNESS), reason="reference tokenizer not built here")
def test_random_texts_against_reference_build():
    """200 seeded random texts (vocabulary pieces, raw bytes, stray
    continuation bytes) through the reference's tokenize and the library's."""
    import importlib.util
    from strasgpt_amd.runtime import Tokenizer
    spec = importlib.util.spec_from_file_location(
        "mtg", os.path.join(GOLDEN_DIR, "make_tokenizer_golden.py"))
    mtg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mtg)
    rng = random.Random(11)
    for name, make in (("bpe", mtg.bpe_case), ("small", mtg.small_case)):
        raw, scores, bos, eos, _, _, _ = make(random.Random(20251202 + len(name)))
        pieces = [k for k in raw if k and b"\x00" not in k][:200] + [b"\x80", b"\xc3", b"\xe4\xb8", b" "]
        texts = []
        for i in range(100):
            s = b"".join(rng.choice(pieces) for _ in range(rng.randint(0, 40)))
            texts.append((rng.randint(0, 1), rng.randint(0, 1), s.replace(b"\x00", b"")))
        _, want, _, _ = mtg.run_reference(raw, scores, bos, eos, texts, [], [])
        tok = Tokenizer(os.path.join(GOLDEN_DIR, "tokenizer", name), bos, eos)
        for (b, e, s), w in zip(texts, want):
            assert tok.encode(s, bool(b), bool(e)) == w, (name, s[:60])
        tok.close()


def test_missing_tokenizer_file_dies(tmp_path):
    """Like the reference (source/json_parser.y:635-637): no tokenizer.json
    ends the process with an error line."""
    code = ("import ctypes,sys; L=ctypes.CDLL(sys.argv[1]); "
            "L.tokenizer_read_dir.restype=ctypes.c_void_p; L.tokenizer_read_dir(sys.argv[2].encode())")
    r = subprocess.run(["python3", "-c", code, _paths.hip_lib(), str(tmp_path)],
                       capture_output=True, text=True)
    assert r.returncode != 0
    assert "[StrasGPT] Error" in r.stderr and "tokenizer" in r.stderr


@pytest.mark.parametrize("body, what", [
    ('{"model": {"vocab": {}}}', "empty vocab"),
    ('{"model": 3}', "model is not an object"),
    ('{"model": {"vocab": {"a": "x"}}}', "expected a number"),
])
def test_malformed_tokenizer_file_dies(tmp_path, body, what):
    (tmp_path / "tokenizer.json").write_text(body)
    code = ("import ctypes,sys; L=ctypes.CDLL(sys.argv[1]); "
            "L.tokenizer_read_dir.restype=ctypes.c_void_p; L.tokenizer_read_dir(sys.argv[2].encode())")
    r = subprocess.run(["python3", "-c", code, _paths.hip_lib(), str(tmp_path)],
                       capture_output=True, text=True)
    assert r.returncode != 0 and what in r.stderr, r.stderr
