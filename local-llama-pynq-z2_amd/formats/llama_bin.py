"""llama2.c checkpoints for runq: walk and validate the int8 version-2 file, and quantize a float
version-0 checkpoint to it.

  python llama_bin.py check model_q80.bin                   walk the file as runq.c's loader does
  python llama_bin.py from-float model.bin model_q80.bin    the role of tools/bin2q80.py

Version 2 (runq.c:273-357, bin2q80.py:48-59): a 256-byte header "<Ii7iBi" = magic 0x616b3432, version 2, dim,
hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len, u8 shared_classifier, group_size, zero padding;
then, unpadded, f32 rms_att[L][dim], rms_ffn[L][dim], rms_final[dim], and the tensors, each int8 q[n]
followed by f32 s[n / group_size]: tok_embeddings (vocab x dim), wq[L], wk[L], wv[L], wo[L], w1[L], w2[L],
w3[L], and wcls (vocab x dim) when the classifier is not shared.

Version 0 (llama2.c's legacy export): i32 dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size (negative:
a separate classifier follows), seq_len, then f32 token_embedding (vocab x dim), rms_att[L][dim], wq, wk, wv,
wo, rms_ffn[L][dim], w1, w2, w3, rms_final[dim], freq_cis_real and _imag (seq_len x head_size/2 each) and the
classifier when present.  Quantization per group of gs values (the largest of 64, 32, ... dividing dim):
s = max|w| / 127 in float32, q = round(w / s) to nearest, ties to even (numpy's rounding), q = 0 for s = 0."""
import os
import struct
import sys

import numpy as np

HEADER = struct.Struct("<Ii7iBi")
MAGIC = 0x616B3432


class BinError(ValueError):
    pass


class Q80:
    """A walked version-2 file: cfg, rms_att [L, dim], rms_ffn [L, dim], rms_final [dim], and per tensor
    name ("tok_embeddings", ("wq", l), ...) the int8 values [rows, n] and scales [rows, n / gs]."""

    def __init__(self, path):
        mm = np.memmap(path, dtype=np.uint8, mode="r")
        if mm.size < 256:
            raise BinError(f"{path}: shorter than the 256-byte header")
        magic, ver, dim, hid, L, heads, kvh, vocab, seq, shared, gs = HEADER.unpack(bytes(mm[:HEADER.size]))
        if magic != MAGIC or ver != 2:
            raise BinError(f"{path}: not a version-2 int8 llama2.c file (magic {magic:#x}, version {ver})")
        self.cfg = dict(dim=dim, hidden_dim=hid, n_layers=L, n_heads=heads, n_kv_heads=kvh, vocab_size=vocab,
                        seq_len=seq, shared_classifier=bool(shared), group_size=gs)
        if min(dim, hid, L, heads, kvh, vocab, seq, gs) <= 0 or dim % heads or heads % kvh:
            raise BinError(f"{path}: inconsistent header {self.cfg}")
        if dim % gs or hid % gs:
            raise BinError(f"{path}: group size {gs} does not divide dim {dim} and hidden {hid}")
        self.path, self.mm, self.off = path, mm, 256
        kv = dim // heads * kvh
        f32 = lambda n: self._take(n * 4).view("<f4")
        self.rms_att = f32(L * dim).reshape(L, dim)
        self.rms_ffn = f32(L * dim).reshape(L, dim)
        self.rms_final = f32(dim)
        self.tensors = {"tok_embeddings": self._tensor(vocab, dim)}
        for name, (rows, n) in (("wq", (dim, dim)), ("wk", (kv, dim)), ("wv", (kv, dim)), ("wo", (dim, dim)),
                                ("w1", (hid, dim)), ("w2", (dim, hid)), ("w3", (hid, dim))):
            for l in range(L):
                self.tensors[(name, l)] = self._tensor(rows, n)
        if not shared:
            self.tensors["wcls"] = self._tensor(vocab, dim)
        if self.off != mm.size:
            raise BinError(f"{path}: the layout ends at byte {self.off}, the file has {mm.size}")

    def _take(self, nbytes):
        if self.off + nbytes > self.mm.size:
            raise BinError(f"{self.path}: truncated (an array of {nbytes} bytes at {self.off})")
        a = self.mm[self.off:self.off + nbytes]
        self.off += nbytes
        return a

    def _tensor(self, rows, n):
        q = self._take(rows * n).view(np.int8).reshape(rows, n)
        s = self._take(rows * n // self.cfg["group_size"] * 4).view("<f4").reshape(rows, -1)
        if not np.all(np.isfinite(s)) or np.any(s < 0):
            raise BinError(f"{self.path}: negative or non-finite scales")
        return q, s


def check(path):
    return Q80(path)


def quantize_q80(w, gs):
    """int8 values, float32 scales and the largest reconstruction error of float32 w, per group of gs"""
    g = np.asarray(w, np.float32).reshape(-1, gs)
    s = (np.abs(g).max(axis=1) / np.float32(127.0)).astype(np.float32)
    safe = np.where(s == 0, np.float32(1.0), s)
    q = np.rint(g / safe[:, None]).astype(np.int8)  # to nearest, ties to even
    err = float(np.abs(q * s[:, None] - g).max()) if g.size else 0.0
    return q, s, err


def from_float(src, dst):
    """legacy float (version 0) checkpoint -> version 2 int8; returns (cfg, largest quantization error)"""
    head = np.fromfile(src, np.int32, 7)
    if head.size < 7:
        raise BinError(f"{src}: too short")
    dim, hid, L, heads, kvh, vocab, seq = (int(v) for v in head)
    shared, vocab = vocab > 0, abs(vocab)
    if min(dim, hid, L, heads, kvh, vocab, seq) <= 0 or dim % heads or heads % kvh:
        raise BinError(f"{src}: inconsistent header")
    data = np.fromfile(src, np.float32, offset=28)
    hs, kv = dim // heads, dim // heads * kvh
    sizes = [("emb", vocab * dim), ("rms_att", L * dim), ("wq", L * dim * dim), ("wk", L * kv * dim),
             ("wv", L * kv * dim), ("wo", L * dim * dim), ("rms_ffn", L * dim), ("w1", L * hid * dim),
             ("w2", L * dim * hid), ("w3", L * hid * dim), ("rms_final", dim), ("freq_cis", 2 * seq * (hs // 2))]
    if not shared:
        sizes.append(("wcls", vocab * dim))
    if sum(n for _, n in sizes) != data.size:
        raise BinError(f"{src}: {data.size} floats after the header, the layout needs {sum(n for _, n in sizes)}")
    part, at = {}, 0
    for name, n in sizes:
        part[name] = data[at:at + n]
        at += n
    gs = 64
    while dim % gs:
        gs //= 2
    per_layer = lambda name: np.split(part[name], L)
    worst = 0.0
    with open(dst, "wb") as f:
        h = HEADER.pack(MAGIC, 2, dim, hid, L, heads, kvh, vocab, seq, int(shared), gs)
        f.write(h + b"\0" * (256 - len(h)))
        for name in ("rms_att", "rms_ffn", "rms_final"):
            f.write(part[name].astype("<f4").tobytes())
        mats = [part["emb"]] + [m for k in ("wq", "wk", "wv", "wo", "w1", "w2", "w3") for m in per_layer(k)]
        if not shared:
            mats.append(part["wcls"])
        for m in mats:
            q, s, err = quantize_q80(m, gs)
            f.write(q.tobytes())
            f.write(s.astype("<f4").tobytes())
            worst = max(worst, err)
    return check(dst).cfg, worst


def main(argv):
    if len(argv) == 2 and argv[0] == "check":
        c = check(argv[1]).cfg
        print(f"OK: {argv[1]} (dim={c['dim']} hidden={c['hidden_dim']} layers={c['n_layers']} heads="
              f"{c['n_heads']}/{c['n_kv_heads']} vocab={c['vocab_size']} seq_len={c['seq_len']} "
              f"group={c['group_size']} shared classifier={c['shared_classifier']})")
        return 0
    if len(argv) == 3 and argv[0] == "from-float":
        c, err = from_float(argv[1], argv[2])
        print(f"wrote {argv[2]}: {os.path.getsize(argv[2]) / 2**20:.1f} MiB, dim={c['dim']} layers={c['n_layers']} "
              f"vocab={c['vocab_size']} group={c['group_size']} max quantization error={err:.5f}")
        return 0
    print(__doc__.split("\n\n")[1], file=sys.stderr)
    return 2


if __name__ == "__main__":
    try:
        sys.exit(main(sys.argv[1:]))
    except BinError as e:
        print(f"error: {e}", file=sys.stderr)
        sys.exit(1)
