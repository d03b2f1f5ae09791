""".qwb v1 weight files (the reference's qwen/qwen.c format): walk and validate, and convert a Qwen2 GGUF.

  python qwb.py check model.qwb [model.gguf]          walk the file as the loader does; with a GGUF, compare
                                                      every tensor (the role of tools/qwb_check.py)
  python qwb.py from-gguf model.gguf head_ids.npy out.qwb   convert (the role of tools/gguf2qwb.py)

Layout (tools/gguf2qwb.py:5-14, qwen.c:195-271), little-endian, every array starting on a 64-byte boundary:
  header of 256 bytes: "QWB1", u32 1, i32 dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, head_k,
      max_seq_len, group_size (32), emb_bits (4 or 8), f32 rope_theta, rms_eps, zero padding;
  f32 attn_norm[L][dim], ffn_norm[L][dim], bq[L][dim], bk[L][kv], bv[L][kv], output_norm[dim];
  i32 head_ids[head_k] (strictly ascending token ids of the output-head rows);
  matrices, each an integer plane then an fp16 scale plane (one per group of 32 along a row): wq, wk, wv, wo,
      w1 (gate), w2 (down), w3 (up), each for every layer, 4-bit; then head (the embedding's head_ids rows) and
      the embedding (vocab rows), emb_bits.  4-bit planes hold two's-complement nibbles, element 2i of a row
      in the low nibble of byte i.  The file ends at the last plane's padding."""
import os
import struct
import sys

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import gguf  # noqa: E402

HEADER = struct.Struct("<4sI10i2f")
KINDS = ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_down", "ffn_up")
SMALL = ("attn_norm.weight", "ffn_norm.weight", "attn_q.bias", "attn_k.bias", "attn_v.bias")


class QwbError(ValueError):
    pass


def pad64(n):
    return n + (-n % 64)


class Qwb:
    """A walked .qwb: cfg (dict), small [kind][layer] f32 arrays, output_norm, head_ids, and for every matrix
    (name, layer or None) the raw integer plane and fp16 scale plane (views of the file)."""

    def __init__(self, path):
        self.path = path
        self.mm = np.memmap(path, dtype=np.uint8, mode="r")
        if self.mm.size < 256:
            raise QwbError(f"{path}: shorter than the 256-byte header")
        magic, ver, *ints = HEADER.unpack(bytes(self.mm[:HEADER.size]))
        if magic != b"QWB1" or ver != 1:
            raise QwbError(f"{path}: not a .qwb v1 file (magic {magic!r}, version {ver})")
        keys = ("dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads", "vocab_size", "head_k", "max_seq_len",
                "group_size", "emb_bits")
        self.cfg = dict(zip(keys, ints[:10]))
        self.cfg["rope_theta"], self.cfg["rms_eps"] = ints[10], ints[11]
        c = self.cfg
        for k in keys:
            if c[k] <= 0:
                raise QwbError(f"{path}: {k} = {c[k]}")
        if c["group_size"] != 32 or c["emb_bits"] not in (4, 8):
            raise QwbError(f"{path}: group size {c['group_size']} / embedding bits {c['emb_bits']} (32 / 4 or 8)")
        if c["dim"] % c["n_heads"] or c["n_heads"] % c["n_kv_heads"] or c["dim"] % 32 or c["hidden_dim"] % 32:
            raise QwbError(f"{path}: inconsistent shape {c}")
        if c["head_k"] > c["vocab_size"]:
            raise QwbError(f"{path}: head_k {c['head_k']} > vocab {c['vocab_size']}")
        self.off = 256
        L, dim, hid = c["n_layers"], c["dim"], c["hidden_dim"]
        kv = dim // c["n_heads"] * c["n_kv_heads"]
        self.kv = kv
        widths = {"attn_norm.weight": dim, "ffn_norm.weight": dim, "attn_q.bias": dim, "attn_k.bias": kv,
                  "attn_v.bias": kv}
        self.small = {k: [self._take(widths[k] * 4).view("<f4") for _ in range(L)] for k in SMALL}
        self.output_norm = self._take(dim * 4).view("<f4")
        self.head_ids = self._take(c["head_k"] * 4).view("<i4")
        if np.any(np.diff(self.head_ids.astype(np.int64)) <= 0) or self.head_ids[0] < 0 or \
                self.head_ids[-1] >= c["vocab_size"]:
            raise QwbError(f"{path}: head_ids not strictly ascending within the vocabulary")
        shapes = {"attn_q": (dim, dim), "attn_k": (kv, dim), "attn_v": (kv, dim), "attn_output": (dim, dim),
                  "ffn_gate": (hid, dim), "ffn_down": (dim, hid), "ffn_up": (hid, dim)}
        self.shapes = shapes
        self.mats = {}
        self.offsets = {}  # (name, layer) -> byte offsets of the integer plane and the scale plane
        for k in KINDS:
            for l in range(L):
                self.mats[(k, l)] = self._matrix(*shapes[k], 4)
                self.offsets[(k, l)] = self._last
        self.mats[("head", None)] = self._matrix(c["head_k"], dim, c["emb_bits"])
        self.offsets[("head", None)] = self._last
        self.mats[("embedding", None)] = self._matrix(c["vocab_size"], dim, c["emb_bits"])
        self.offsets[("embedding", None)] = self._last
        self.head_ids_offset = 256 + sum(pad64(a.size * 4) for k in SMALL for a in self.small[k]) + pad64(dim * 4)
        if self.off != self.mm.size:
            raise QwbError(f"{path}: the layout ends at byte {self.off}, the file has {self.mm.size}")

    def _take(self, nbytes):
        if self.off + nbytes > self.mm.size:
            raise QwbError(f"{self.path}: truncated (an array of {nbytes} bytes at {self.off})")
        a = self.mm[self.off:self.off + nbytes]
        self.off = pad64(self.off + nbytes)
        return a

    def _matrix(self, rows, n, bits):
        at = self.off
        plane = self._take(rows * n * bits // 8)
        self._last = (at, self.off)
        return plane, self._take(rows * n // 32 * 2).view("<f2")

    def ints(self, name, layer=None):
        """int8 values [rows, n] of a matrix"""
        plane, _ = self.mats[(name, layer)]
        rows, n = self.shape_of(name)
        if self._bits(name) == 8:
            return plane.view(np.int8).reshape(rows, n)
        p = plane.reshape(rows, n // 2)
        q = np.empty((rows, n), np.int8)
        q[:, 0::2] = ((p & 0x0F) ^ 8).astype(np.int8) - 8
        q[:, 1::2] = ((p >> 4) ^ 8).astype(np.int8) - 8
        return q

    def scales(self, name, layer=None):
        rows, n = self.shape_of(name)
        return self.mats[(name, layer)][1].reshape(rows, n // 32)

    def dequant(self, name, layer=None):
        rows, n = self.shape_of(name)
        q, s = self.ints(name, layer), self.scales(name, layer).astype(np.float32)
        return (q.reshape(rows, n // 32, 32) * s[:, :, None]).reshape(rows, n)

    def shape_of(self, name):
        c = self.cfg
        if name == "head":
            return c["head_k"], c["dim"]
        if name == "embedding":
            return c["vocab_size"], c["dim"]
        return self.shapes[name]

    def _bits(self, name):
        return self.cfg["emb_bits"] if name in ("head", "embedding") else 4


def check(path, gguf_path=None):
    """walks the file (QwbError on any inconsistency); with a GGUF, every tensor must equal its source"""
    q = Qwb(path)
    if np.any(np.abs(q.dequant("head").astype(np.float64) - q.dequant("embedding")[q.head_ids]) > 0):
        raise QwbError(f"{path}: head rows are not the embedding's head_ids rows")
    if gguf_path:
        g = gguf.GGUF(gguf_path)
        t = g.tensors
        L = q.cfg["n_layers"]
        for k in SMALL:
            for l in range(L):
                if not np.array_equal(q.small[k][l], gguf.dequantize(t[f"blk.{l}.{k}"]).reshape(-1)):
                    raise QwbError(f"blk.{l}.{k} differs")
        if not np.array_equal(q.output_norm, gguf.dequantize(t["output_norm.weight"]).reshape(-1)):
            raise QwbError("output_norm differs")
        for k in KINDS:
            for l in range(L):
                if not np.array_equal(q.dequant(k, l), gguf.dequantize(t[f"blk.{l}.{k}.weight"])):
                    raise QwbError(f"blk.{l}.{k}.weight differs")
        emb = gguf.dequantize(t["token_embd.weight"])
        if not np.array_equal(q.dequant("embedding"), emb) or not np.array_equal(q.dequant("head"), emb[q.head_ids]):
            raise QwbError("embedding or head differs from token_embd.weight")
    return q


def _pack4(q):
    u = (q.astype(np.int16) & 0x0F).astype(np.uint8)
    return u[:, 0::2] | (u[:, 1::2] << 4)


def from_gguf(gguf_path, head_ids, out_path):
    """Qwen2 GGUF (Q4_0 layer matrices, Q4_0 or Q8_0 tied embedding, F32 norms and biases) -> .qwb; the
    written file is walked again and compared tensor by tensor with the GGUF before returning"""
    g = gguf.GGUF(gguf_path)
    f, t = g.fields, g.tensors
    if f.get("general.architecture") != "qwen2":
        raise QwbError(f"{gguf_path}: architecture {f.get('general.architecture')!r}, expected qwen2")
    head_ids = np.asarray(head_ids, np.int64)
    if head_ids.ndim != 1 or np.any(np.diff(head_ids) <= 0):
        raise QwbError("head ids must be strictly ascending")
    L = int(f["qwen2.block_count"])
    emb = t["token_embd.weight"]
    if emb.type not in (gguf.Q4_0, gguf.Q8_0):
        raise QwbError(f"token_embd.weight: {emb.type_name()}, expected Q4_0 or Q8_0")
    emb_bits = 4 if emb.type == gguf.Q4_0 else 8
    if head_ids[0] < 0 or head_ids[-1] >= emb.rows:
        raise QwbError("head ids outside the vocabulary")
    cfg = [int(f["qwen2.embedding_length"]), int(f["qwen2.feed_forward_length"]), L,
           int(f["qwen2.attention.head_count"]), int(f["qwen2.attention.head_count_kv"]), emb.rows, len(head_ids),
           int(f["qwen2.context_length"]), 32, emb_bits]

    def f32(name):
        x = t[name]
        if x.type != gguf.F32:
            raise QwbError(f"{name}: {x.type_name()}, expected F32")
        return gguf.dequantize(x).reshape(-1)

    with open(out_path, "wb") as o:
        def put(a):
            b = np.ascontiguousarray(a).tobytes()
            o.write(b + b"\0" * (-len(b) % 64))

        head = HEADER.pack(b"QWB1", 1, *cfg, float(f["qwen2.rope.freq_base"]),
                           float(f["qwen2.attention.layer_norm_rms_epsilon"]))
        o.write(head + b"\0" * (256 - len(head)))
        for k in SMALL:
            for l in range(L):
                put(f32(f"blk.{l}.{k}"))
        put(f32("output_norm.weight"))
        put(head_ids.astype("<i4"))
        for k in KINDS:
            for l in range(L):
                x = t[f"blk.{l}.{k}.weight"]
                if x.type != gguf.Q4_0:
                    raise QwbError(f"{x.name}: {x.type_name()}, expected Q4_0 (quantize with --pure)")
                q, d = gguf.ints_scales(x)
                put(_pack4(q))
                put(d)
        q, d = gguf.ints_scales(emb)
        for rows in (head_ids, slice(None)):
            put(_pack4(q[rows]) if emb_bits == 4 else q[rows])
            put(d[rows])
    return check(out_path, gguf_path)


def main(argv):
    if len(argv) >= 2 and argv[0] == "check":
        q = check(argv[1], argv[2] if len(argv) > 2 else None)
        c = q.cfg
        print(f"OK: {argv[1]} (dim={c['dim']} hidden={c['hidden_dim']} layers={c['n_layers']} heads="
              f"{c['n_heads']}/{c['n_kv_heads']} vocab={c['vocab_size']} head={c['head_k']} ctx={c['max_seq_len']}"
              f" emb={c['emb_bits']}-bit)" + (f", every tensor equal to {argv[2]}" if len(argv) > 2 else ""))
        return 0
    if len(argv) == 4 and argv[0] == "from-gguf":
        q = from_gguf(argv[1], np.load(argv[2], allow_pickle=False), argv[3])
        print(f"wrote {argv[3]}: {os.path.getsize(argv[3]) / 2**20:.1f} MiB, dim={q.cfg['dim']} "
              f"layers={q.cfg['n_layers']} head={q.cfg['head_k']}, every tensor checked against the GGUF")
        return 0
    print(__doc__.split("\n\n")[1], file=sys.stderr)
    return 2


if __name__ == "__main__":
    try:
        sys.exit(main(sys.argv[1:]))
    except (QwbError, gguf.GGUFError) as e:
        print(f"error: {e}", file=sys.stderr)
        sys.exit(1)
