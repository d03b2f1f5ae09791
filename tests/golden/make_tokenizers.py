"""Synthetic tokenizer fixtures for the hosts' text I/O (run from the repository root; CPU only).

  python tests/golden/make_tokenizers.py

Writes into tests/golden/:
  qwen_tok_synth.bin   a Qwen2-style byte-level BPE in the QWTOK001 layout that qwen/tokenizer.c reads
                       (tools/qwen_tok_export.py:21-41): 509 base tokens (the 256 bytes + merges learned by
                       Hugging Face `tokenizers` on a seeded multilingual corpus, with the Qwen2 NFC
                       normalizer and pre-tokenizer) and 3 added tokens, 512 ids in all (the tiny .qwb
                       vocabulary)
  qwen_tok_cases.json  test texts and the ids Hugging Face `tokenizers` gives them (added tokens split)
  llama_tok_synth.bin  a llama2.c tokenizer.bin (runq.c:638-662): <unk> <s> </s>, <0x00>..<0xFF>, then pieces
                       learned by a seeded greedy pair count, scores falling with the order learned; 512 ids
  llama_tok_cases.json test texts for it and the ids of runq.c's own encode (oracle/_ref/runq_tok, built
                       from the reference sources by `make -C oracle ref`, which has to run first)
  text_ref.json        the reference programs' text-prompt runs (oracle/_ref/qwen: -i, chat template or raw;
                       oracle/_ref/runq: runq.c's own CLI) on seeded synthetic models made by host/synth,
                       with these tokenizers: their arguments and stdout bytes

The Unicode table of the QWTOK001 file comes from Python's unicodedata (classes letter / number / white space,
canonical combining classes, canonical decompositions and compositions); test texts avoid code points whose
properties changed in later Unicode versions, where `tokenizers` may use newer tables."""
import json
import os
import random
import struct
import subprocess
import sys
import unicodedata

from tokenizers import Regex, Tokenizer, decoders, models, normalizers, pre_tokenizers, trainers

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
REF_TOK = os.path.join(REPO, "oracle", "_ref", "runq_tok")
SYNTH = os.path.join(REPO, "local-llama-pynq-z2_amd", "host", "synth")
# text runs: (name, model format, synth overrides, reference program, arguments after the model)
TEXT_RUNS = [
    ("qwen_chat", "qwb", ["max_seq=256"], "qwen",  # seed 5: a greedy loop that is not a single token
     ["-i", "Write a short poem about the sea.", "-m", "chat", "-t", "0", "-n", "24", "-c", "256"]),
    ("qwen_raw_sampled", "qwb", ["max_seq=256"], "qwen",
     ["-i", "the quick brown fox", "-m", "raw", "-t", "0.9", "-p", "0.9", "-s", "3", "-n", "24", "-c", "256"]),
    ("runq_greedy", "bin", ["vocab=512"], "runq", ["-i", "Once upon a time", "-n", "48", "-t", "0"]),
    ("runq_sampled", "bin", ["vocab=512"], "runq", ["-i", "The quick brown fox", "-n", "40", "-t", "0.8", "-p", "0.9",
                                                   "-s", "5"]),
    # runq.c's chat loop, turns from stdin.  Seed 1 at t 1.0 ends two replies with EOS; 155 positions stop
    # inside the third turn's prompt.  (A sampled run of hundreds of coins over 512 near-uniform rows is likely
    # to meet a coin within fp32 rounding of a cdf boundary somewhere: the sampler's bar, test_gpu_sample.py.)
    ("runq_chat_sampled", "bin", ["vocab=512", "max_seq=512"], "runq",
     ["-m", "chat", "-y", "Be brief.", "-i", "Hello there", "-n", "155", "-t", "1.0", "-p", "0.95", "-s", "1"],
     "How are you?\nTell me more\nBye\n"),
    ("runq_chat_greedy", "bin", ["vocab=512", "max_seq=512"], "runq", ["-m", "chat", "-n", "200", "-t", "0"],
     "Be brief.\nHello there\nHow are you?\n"),
]
QWEN_SPLIT = (r"(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}| ?[^\s\p{L}\p{N}]+[\r\n]*|"
              r"\s*[\r\n]+|\s+(?!\S)|\s+")
ADDED = ["<|endoftext|>", "<|im_start|>", "<|im_end|>"]
N_IDS = 512
# Unicode White_Space (what \s matches in the regex engine of `tokenizers`)
WHITE_SPACE = set(list(range(0x09, 0x0E)) + [0x20, 0x85, 0xA0, 0x1680] + list(range(0x2000, 0x200B)) +
                  [0x2028, 0x2029, 0x202F, 0x205F, 0x3000])


def corpus(seed=7):
    rng = random.Random(seed)
    words = ("the quick brown fox jumps over lazy dog token model layer weight scale group matrix vector "
             "prefill decode attention cache value key query head norm residual quantize integer float "
             "kernel memory bandwidth graph stream device host tensor batch sample greedy").split()
    extra = ["café", "naïve", "résumé", "Straße", "über", "mañana", "façade", "déjà", "Ελληνικά", "русский",
             "中文", "测试", "日本語", "한국어", "हिन्दी", "😀", "don't", "I'll", "we're", "it's", "THEY'VE", "x**2",
             "def", "return", "{}", "[]", "();", "==", "->", "//", "#include", "3.14", "2024", "1e-6"]
    lines = []
    for _ in range(3000):
        k = rng.randint(3, 12)
        ws = [rng.choice(words) if rng.random() < 0.8 else rng.choice(extra) for _ in range(k)]
        if rng.random() < 0.2:
            ws[0] = ws[0].capitalize()
        sep = rng.choice([" ", " ", " ", "  ", "\t", "\n", " \n"])
        lines.append(sep.join(ws) + rng.choice([".", "!", "?", "", ":\n", ",", "\n\n"]))
    return lines


def bytes_to_unicode():
    """GPT-2's byte <-> printable-character table of the byte-level pre-tokenizer"""
    bs = list(range(ord("!"), ord("~") + 1)) + list(range(ord("¡"), ord("¬") + 1)) + list(range(ord("®"), ord("ÿ") + 1))
    cs = bs[:]
    n = 0
    for b in range(256):
        if b not in bs:
            bs.append(b)
            cs.append(256 + n)
            n += 1
    return {b: chr(c) for b, c in zip(bs, cs)}


def train_qwen():
    tok = Tokenizer(models.BPE())
    tok.normalizer = normalizers.NFC()
    tok.pre_tokenizer = pre_tokenizers.Sequence([
        pre_tokenizers.Split(Regex(QWEN_SPLIT), behavior="isolated", invert=False),
        pre_tokenizers.ByteLevel(add_prefix_space=False, trim_offsets=False, use_regex=False)])
    tok.decoder = decoders.ByteLevel()
    trainer = trainers.BpeTrainer(vocab_size=N_IDS - len(ADDED), min_frequency=2, show_progress=False,
                                  initial_alphabet=pre_tokenizers.ByteLevel.alphabet())
    tok.train_from_iterator(corpus(), trainer=trainer)
    tok.add_special_tokens(ADDED)
    return tok


def unicode_tables():
    """run-length class/NFC table, NFD decompositions, NFC composition pairs"""
    pairs = []
    dec = {}
    second = set()
    for cp in range(0x110000):
        if 0xD800 <= cp < 0xE000 or 0xAC00 <= cp < 0xAC00 + 11172:
            continue
        ch = chr(cp)
        d = unicodedata.decomposition(ch)
        if not d or d.startswith("<"):
            continue
        nfd = unicodedata.normalize("NFD", ch)
        dec[cp] = [ord(c) for c in nfd]
        parts = [int(x, 16) for x in d.split()]
        if len(parts) == 2 and unicodedata.normalize("NFC", chr(parts[0]) + chr(parts[1])) == ch:
            pairs.append((parts[0], parts[1], cp))
            second.add(parts[1])
    runs = []
    prev = None
    for cp in range(0x110000):
        if 0xD800 <= cp < 0xE000:
            pay = 0
        else:
            ch = chr(cp)
            cat = unicodedata.category(ch)
            cls = 3 if cp in WHITE_SPACE else 1 if cat[0] == "L" else 2 if cat[0] == "N" else 0
            ccc = unicodedata.combining(ch)
            dirty = int(ccc != 0 or cp in dec or cp in second or unicodedata.normalize("NFC", ch) != ch
                        or (0x1100 <= cp < 0x1200))  # Hangul jamo compose arithmetically
            pay = cls | dirty << 2 | ccc << 3
        if pay != prev:
            runs.append(cp | pay << 21)
            prev = pay
    dec_cp = sorted(dec)
    off, pool = [0], []
    for cp in dec_cp:
        pool += dec[cp]
        off.append(len(pool))
    pairs.sort()
    return runs, dec_cp, off, pool, pairs


def pad4(b):
    return b + b"\0" * (-len(b) % 4)


def export_qwen(tok, path):
    j = json.loads(tok.to_str())
    vocab = j["model"]["vocab"]
    merges = j["model"]["merges"]
    inv = {c: b for b, c in bytes_to_unicode().items()}
    n_vocab = len(vocab)
    assert sorted(vocab.values()) == list(range(n_vocab))
    tok_bytes = [b""] * n_vocab
    for s, i in vocab.items():
        tok_bytes[i] = bytes(inv[c] for c in s)
    assert max(len(b) for b in tok_bytes) <= 255
    trip = []
    for m in merges:
        a, b = m.split(" ") if isinstance(m, str) else m
        trip += [vocab[a], vocab[b], vocab[a + b]]
    added = sorted((t.content, tok.token_to_id(t.content)) for t in tok.get_added_tokens_decoder().values())
    runs, dec_cp, dec_off, pool, comp = unicode_tables()
    blob = b"".join(tok_bytes)
    hdr = [n_vocab, len(added), len(merges), len(blob), len(runs), len(dec_cp), len(pool), len(comp), 0, 0, 0, 0]
    out = b"QWTOK001" + struct.pack("<12I", *hdr)
    out += pad4(bytes(len(b) for b in tok_bytes)) + pad4(blob) + struct.pack(f"<{len(trip)}I", *trip)
    for text, i in sorted(added, key=lambda x: x[1]):
        t = text.encode()
        out += struct.pack("<2I", i, len(t)) + pad4(t)
    out += struct.pack(f"<{len(runs)}I", *runs) + struct.pack(f"<{len(dec_cp)}I", *dec_cp)
    out += struct.pack(f"<{len(dec_off)}I", *dec_off) + struct.pack(f"<{len(pool)}I", *pool)
    out += struct.pack(f"<{3 * len(comp)}I", *[x for p in comp for x in p])
    with open(path, "wb") as f:
        f.write(out)
    return n_vocab, len(added)


QWEN_CASES = [
    "", "Hello world", "The quick brown fox jumps over the lazy dog.", "  leading and trailing spaces   ",
    "don't I'll we're THEY'VE it's you'D SHE'S o'clock 'twas", "can\u017ft", "x = 12345 + 3.14159e-6",
    "def f(x):\n\treturn x**2\n\n\n# end", "a\n\n\nb\r\nc\r\r\n   d", "tabs\t\tand\t \tmixed \t", "   ", "\n",
    "\t\n \n  ", "caf\u00e9 na\u00efve r\u00e9sum\u00e9 Stra\u00dfe", "cafe\u0301 nai\u0308ve (decomposed)",
    "e\u0327\u0301 a\u0301\u0327 o\u0328\u0304 (marks out of order)", "\u1100\u1161\u11a8 \ud55c\uad6d\uc5b4 \u1112\u1161\u11ab",
    "\u212b \u2126 A\u030a \u00c5 (singletons)", "\u4e2d\u6587\u6d4b\u8bd5\uff0c\u65e5\u672c\u8a9e\u3002",
    "\u0395\u03bb\u03bb\u03b7\u03bd\u03b9\u03ba\u03ac \u0440\u0443\u0441\u0441\u043a\u0438\u0439 \u0939\u093f\u0928\u094d\u0926\u0940",
    "emoji \U0001F600\U0001F44D\U0001F3FD! ...!!! ???", "<<<>>> [[1,2],{3:4}] a->b // c == d",
    "<|im_start|>system\nYou are a helpful assistant.<|im_end|>\n<|im_start|>user\nhi<|im_end|>\n<|im_start|>assistant\n",
    "text<|endoftext|>more<|im_end|><|im_end|>", "<|im_start", "a" * 700, "ab" * 300 + " " + "xyz" * 100,
    "1234567890" * 5, " non\u00a0breaking\u3000spaces\u2003line", "mixed \u2028\n space \x0b\x0c end",
    "snake_case CamelCase kebab-case UPPER_CASE", "quote's end'", "'s's's", "$100.00 (approx) 50% off!",
    "\u1e9b\u0323 \u0041\u030a\u0301 \u0f73 \u0958 compositions and exclusions",
]

LLAMA_CASES = [
    "", "Hello world", "Once upon a time, there was a little girl.", "  two leading spaces", "tabs\tand\nnew lines",
    "café über 中文 \U0001F600", "numbers 12345 and 3.14", "aaaaaaaaaaaaaaaaaaaa",
    "the the the the", "x", " ", "éé", "punctuation!?.,;:", "The quick brown fox jumps over the lazy dog",
]


def llama_vocab(seed=11):
    """<unk> <s> </s>, the 256 byte pieces, then pieces from greedy pair merges over a corpus in which spaces
    start words (as in llama2.c's export of SentencePiece, which writes the meta space as ' ')"""
    text = " " + " ".join(corpus(seed))
    seqs = [list(" " + w) for w in text.split(" ") if w]
    pieces, scores = ["<unk>", "<s>", "</s>"], [0.0, 0.0, 0.0]
    pieces += [f"<0x{b:02X}>" for b in range(256)]
    scores += [0.0] * 256
    seen = set(pieces)
    for ch in sorted({c for s in seqs for c in s}):  # single characters first
        if len(pieces) >= N_IDS:
            break
        if ch not in seen:
            pieces.append(ch)
            scores.append(-1000.0 - len(pieces))
            seen.add(ch)
    rank = 0
    while len(pieces) < N_IDS:
        counts = {}
        for s in seqs:
            for a, b in zip(s, s[1:]):
                counts[(a, b)] = counts.get((a, b), 0) + 1
        if not counts:
            break
        (a, b), _ = max(counts.items(), key=lambda kv: (kv[1], kv[0]))
        m = a + b
        if m not in seen:
            pieces.append(m)
            scores.append(-float(rank))
            seen.add(m)
        rank += 1
        for s in seqs:
            i = 0
            while i + 1 < len(s):
                if s[i] == a and s[i + 1] == b:
                    s[i:i + 2] = [m]
                i += 1
    return pieces, scores


def write_llama(path):
    pieces, scores = llama_vocab()
    enc = [p.encode() for p in pieces]
    with open(path, "wb") as f:
        f.write(struct.pack("<i", max(len(e) for e in enc)))
        for e, s in zip(enc, scores):
            f.write(struct.pack("<fi", s, len(e)) + e)
    return len(pieces)


def text_runs():
    import tempfile
    out = {}
    d = tempfile.mkdtemp()
    for name, fmt, over, prog, args, *stdin in TEXT_RUNS:
        model = os.path.join(d, f"{name}.{fmt}")
        seed = "5" if name == "qwen_chat" else "1"
        subprocess.run([SYNTH, fmt, model, "tiny", seed, *over], check=True, capture_output=True)
        tok = os.path.join(HERE, "qwen_tok_synth.bin" if fmt == "qwb" else "llama_tok_synth.bin")
        feed = stdin[0].encode() if stdin else b""
        r = subprocess.run([os.path.join(REPO, "oracle", "_ref", prog), model, *args, "-z", tok], capture_output=True,
                           check=True, timeout=300, input=feed)
        out[name] = {"format": fmt, "synth": ["tiny", seed, *over], "args": args, "stdin": feed.decode(),
                     "stdout_hex": r.stdout.hex()}
    json.dump(out, open(os.path.join(HERE, "text_ref.json"), "w"), indent=1)


def main():
    tok = train_qwen()
    n_vocab, n_added = export_qwen(tok, os.path.join(HERE, "qwen_tok_synth.bin"))
    assert n_vocab + n_added == N_IDS, (n_vocab, n_added)
    cases = [{"text": t, "ids": tok.encode(t, add_special_tokens=False).ids} for t in QWEN_CASES]
    json.dump({"n_ids": N_IDS, "cases": cases}, open(os.path.join(HERE, "qwen_tok_cases.json"), "w"), indent=0)
    path = os.path.join(HERE, "llama_tok_synth.bin")
    n = write_llama(path)
    assert n == N_IDS, n
    r = subprocess.run([REF_TOK, path, str(n), "enc"], input=b"\0".join(t.encode() for t in LLAMA_CASES),
                       capture_output=True, check=True)
    ids = [[int(v) for v in line.split()] for line in r.stdout.decode().split("\n")[:len(LLAMA_CASES)]]
    cases = [{"text": t, "ids": i} for t, i in zip(LLAMA_CASES, ids)]
    json.dump({"vocab": n, "cases": cases}, open(os.path.join(HERE, "llama_tok_cases.json"), "w"), indent=0)
    text_runs()
    print(f"qwen: {n_vocab} base + {n_added} added; llama: {n} pieces", file=sys.stderr)


if __name__ == "__main__":
    main()
