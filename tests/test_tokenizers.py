"""The hosts' tokenizers (host/qwen_tokenizer.c, host/llama_tokenizer.c) through host/tok_tool.

Qwen: the ids Hugging Face `tokenizers` gives the fixture texts (tests/golden/qwen_tok_cases.json, made by
make_tokenizers.py with the Qwen2 normalizer and pre-tokenizer) must come out exactly, and on the same data
file the reference's own tokenizer (qwen/tokenizer.c through its tok_test CLI, oracle/_ref/qwen_tok_test)
must agree id for id, with and without added tokens, also on seeded random texts that mix scripts,
combining marks in any order, Hangul jamo, white space of every kind, contractions and bytes that are not
UTF-8.  Decoding the ids gives back the NFC form of the text.

llama2.c (runq): the ids of runq.c's own encode (stored in llama_tok_cases.json, and live through
oracle/_ref/runq_tok when it is built) and the same printed pieces on decode."""
import json
import os
import random
import subprocess
import unicodedata

import pytest

from helpers import GOLDEN, PKG_DIR, REF_DIR, synth

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TOOL = os.path.join(PKG_DIR, "host", "tok_tool")
REF_QWEN = os.path.join(REPO, "oracle", "_ref", "qwen_tok_test")
REF_LLAMA = os.path.join(REPO, "oracle", "_ref", "runq_tok")
QTOK = os.path.join(GOLDEN, "qwen_tok_synth.bin")
LTOK = os.path.join(GOLDEN, "llama_tok_synth.bin")
QCASES = json.load(open(os.path.join(GOLDEN, "qwen_tok_cases.json")))
LCASES = json.load(open(os.path.join(GOLDEN, "llama_tok_cases.json")))


def tool():
    if not os.path.exists(TOOL):
        pytest.fail(f"{TOOL} is not built (make -C local-llama-pynq-z2_amd host/tok_tool)")
    return TOOL


def run(cmd, data):
    return subprocess.run(cmd, input=data, capture_output=True, check=True, timeout=120).stdout


def enc_lines(cmd, texts):
    """one list of ids per case (cases NUL-separated on input)"""
    out = run(cmd, b"\0".join(texts)).decode().split("\n")
    return [[int(v) for v in line.split()] for line in out[:len(texts)]]


def fuzz_texts(seed, count):
    rng = random.Random(seed)
    pieces = ["a", "Z", "q", "\u00e9", "e\u0301", "\u0327", "\u0301", "\u0308", "\u0323", "\u0300", "\u1100",
              "\u1161", "\u11a8", "\ud55c", "\u212b", "\u2126", "\u4e2d", "\u0416", "\u03a9", "\u0939", "\u094d",
              "1", "7", "\u0663", "\u00bd", " ", "  ", "\t", "\n", "\r\n", "\r", "\u00a0", "\u3000", "\u2003",
              "\x0b", "'", "'s", "'LL", "'re", "\u017f", "!", "...", "\U0001F600", "\U0001F3FD", "_", "-",
              "<|im_end|>", "<|im_start|>", "<|endoftext|>", "<|im", "the", "token", "prefill"]
    raw = [b"\xff", b"\xc3", b"\x80", b"\xed\xa0\x80", b"\xf4\x90\x80\x80", b"\xe2\x82", b"\xc0\xaf"]
    out = []
    for _ in range(count):
        parts = []
        for _ in range(rng.randint(0, 40)):
            if rng.random() < 0.06:
                parts.append(rng.choice(raw))
            else:
                parts.append(rng.choice(pieces).encode())
        out.append(b"".join(parts))
    return out


def test_qwen_matches_hugging_face_ids():
    texts = [c["text"].encode() for c in QCASES["cases"]]
    got = enc_lines([tool(), "qwen", QTOK, "enc", "-s"], texts)
    for c, g in zip(QCASES["cases"], got):
        assert g == c["ids"], repr(c["text"][:80])


@pytest.mark.parametrize("special", [True, False])
def test_qwen_matches_reference_tokenizer(special):
    if not os.path.exists(REF_QWEN):
        pytest.skip("oracle/_ref/qwen_tok_test is not built (make -C oracle ref)")
    texts = [c["text"].encode() for c in QCASES["cases"]] + fuzz_texts(1234 + special, 400)
    flag = ["-s"] if special else []
    mine = enc_lines([tool(), "qwen", QTOK, "enc", *flag], texts)
    ref = enc_lines([REF_QWEN, QTOK, "enc", *flag], texts)
    for t, a, b in zip(texts, mine, ref):
        assert a == b, t
    # decoding every id the cases produced, and every id of the vocabulary
    lines = [" ".join(map(str, ids)).encode() for ids in mine] + [" ".join(map(str, range(QCASES["n_ids"]))).encode()]
    assert run([tool(), "qwen", QTOK, "dec"], b"\n".join(lines)) == run([REF_QWEN, QTOK, "dec"], b"\n".join(lines))


def test_qwen_decode_gives_back_the_normalized_text():
    texts = [c["text"] for c in QCASES["cases"]]
    ids = enc_lines([tool(), "qwen", QTOK, "enc", "-s"], [t.encode() for t in texts])
    out = run([tool(), "qwen", QTOK, "dec"], b"\n".join(" ".join(map(str, i)).encode() for i in ids)).split(b"\0")
    for t, o in zip(texts, out):
        assert o.decode() == unicodedata.normalize("NFC", t), repr(t[:60])


def test_qwen_added_tokens_only_when_allowed():
    t = b"<|im_start|>user\nhi<|im_end|>"
    with_special = enc_lines([tool(), "qwen", QTOK, "enc", "-s"], [t])[0]
    plain = enc_lines([tool(), "qwen", QTOK, "enc"], [t])[0]
    n_base = QCASES["n_ids"] - 3
    assert with_special[0] >= n_base and with_special[-1] >= n_base
    assert max(plain) < n_base  # spelled out byte by byte when not allowed


def test_llama_matches_reference_ids():
    texts = [c["text"].encode() for c in LCASES["cases"]]
    got = enc_lines([tool(), "llama", LTOK, str(LCASES["vocab"]), "enc"], texts)
    for c, g in zip(LCASES["cases"], got):
        assert g == c["ids"], repr(c["text"])


def test_llama_matches_reference_live():
    if not os.path.exists(REF_LLAMA):
        pytest.skip("oracle/_ref/runq_tok is not built (make -C oracle ref)")
    v = str(LCASES["vocab"])
    texts = [c["text"].encode() for c in LCASES["cases"]] + [t for t in fuzz_texts(99, 200) if b"\0" not in t]
    mine = enc_lines([tool(), "llama", LTOK, v, "enc"], texts)
    ref = enc_lines([REF_LLAMA, LTOK, v, "enc"], texts)
    for t, a, b in zip(texts, mine, ref):
        assert a == b, t
    lines = b"\n".join(" ".join(map(str, ids)).encode() for ids in mine)
    lines += b"\n" + " ".join(map(str, range(int(v)))).encode()
    assert run([tool(), "llama", LTOK, v, "dec"], lines) == run([REF_LLAMA, LTOK, v, "dec"], lines)


def test_reference_qwen_links_this_tokenizer(tmp_path):
    """the reference's qwen.c built unchanged with host/qwen_tokenizer.c in place of its tokenizer.c
    (oracle/Makefile: _ref/qwen_ourtok) prints the same text as with its own, chat template and raw, greedy and
    sampled, on a synthetic model (CPU forward of the reference)"""
    ours, theirs = os.path.join(REF_DIR, "qwen_ourtok"), os.path.join(REF_DIR, "qwen")
    if not (os.path.exists(ours) and os.path.exists(theirs)):
        pytest.skip("oracle/_ref/qwen_ourtok or qwen is not built (make -C oracle ref)")
    model = synth("qwb", str(tmp_path / "m.qwb"), "tiny", 5, "max_seq=256")
    for args in (["-i", "Write a short poem about the sea.", "-m", "chat", "-t", "0"],
                 ["-i", "café <|im_end|> 12345\n\tend", "-m", "raw", "-t", "0.9", "-p", "0.9", "-s", "3"]):
        cmd = [model, *args, "-n", "24", "-c", "256", "-z", QTOK]
        a = subprocess.run([ours, *cmd], capture_output=True, timeout=300)
        b = subprocess.run([theirs, *cmd], capture_output=True, timeout=300)
        assert a.returncode == 0 and b.returncode == 0, (a.stderr, b.stderr)
        assert a.stdout == b.stdout and len(a.stdout) > 1
