"""The reference-order ("strict") mode against the reference's own C at every configuration's full workload.

Bar: bitwise.  Strict mode runs every float operation of qwen.c / runq.c in their order (group products summed
per row in group order, RMSNorm's sum of squares and softmax's sum as single running sums, attention
normalized before the weighted sum of V, and expf evaluated as the reference's C library evaluates it), so the
logits of every position, the greedy ids and every layer's K/V cache rows must equal the reference's bit for
bit.  The reference here is the reference's own qwen.c / runq.c compiled with strict IEEE flags into
oracle/_ref/libref_{qwen,runq}.so (its forward() per position, OpenMP as in the reference), so nothing is
restated on the checking side.  The workloads:
  C1  llama2.c 288/6L .bin, 8-token prompt, greedy to the full 256 positions (runq steps clamp to seq_len)
  C2  llama2.c 768/12L .bin, 8-token prompt, greedy to the full 1024 positions (the KV cache fills)
  C3  Qwen2 0.5B-shape .qwb (24 layers, 65536-row head), 24-token prompt, 128 greedy tokens
  C4  the C3 model, 512-token batched prefill, then 64 greedy tokens
  C5  Qwen2 7B-shape .qwb (28 layers, 152064-row head), context 4096, 32-token prompt, 256 greedy tokens
Seeds of the synthetic models and prompts are fixed below."""
import ctypes as C
import os

import numpy as np
import pytest

from helpers import GOLDEN, REF_DIR, oracle, pkg, ptr, synth

pytestmark = pytest.mark.gpu


def ref_lib(name):
    path = os.path.join(REF_DIR, f"libref_{name}.so")
    if not os.path.exists(path):
        pytest.skip(f"{path} not built (needs the reference sources at build time)")
    L = C.CDLL(path)
    vp, i32 = C.c_void_p, C.c_int
    if name == "qwen":
        L.refq_open.restype = vp
        L.refq_open.argtypes = [C.c_char_p, i32]
        L.refq_forward.restype = C.POINTER(C.c_float)
        L.refq_forward.argtypes = [vp, i32, i32]
        L.refq_head_k.argtypes = [vp]
        L.refq_head_ids.restype = C.POINTER(C.c_int32)
        L.refq_head_ids.argtypes = [vp]
        L.refq_kv.restype = C.POINTER(C.c_float)
        L.refq_kv.argtypes = [vp, i32]
        L.refq_argmax.argtypes = [vp, i32]
    else:
        L.refr_open.restype = vp
        L.refr_open.argtypes = [C.c_char_p]
        L.refr_forward.restype = C.POINTER(C.c_float)
        L.refr_forward.argtypes = [vp, i32, i32]
        L.refr_vocab.argtypes = [vp]
        L.refr_seq_len.argtypes = [vp]
        L.refr_kv.restype = C.POINTER(C.c_float)
        L.refr_kv.argtypes = [vp, i32]
        L.refr_argmax.argtypes = [vp, i32]
    return L


class RefQwen:
    """qwen.c's build_transformer / forward / generate (qwen.c:320-330, 490-573, 669-712) at -t 0"""

    def __init__(self, path, ctx):
        self.L = ref_lib("qwen")
        self.h = self.L.refq_open(os.fsencode(path), ctx)
        self.n = self.L.refq_head_k(self.h)
        self.head_ids = np.ctypeslib.as_array(self.L.refq_head_ids(self.h), shape=(self.n,)).copy()
        self.ctx = ctx

    def forward(self, token, pos):
        return np.ctypeslib.as_array(self.L.refq_forward(self.h, int(token), int(pos)), shape=(self.n,)).copy()

    def generate(self, prompt, steps):
        """(generated ids, logits of every position run) with qwen.c's prompt forcing and stop rules"""
        ids, logits, token = [], [], prompt[0]
        for pos in range(self.ctx):
            lg = self.forward(token, pos)
            logits.append(lg)
            if pos < len(prompt) - 1:
                token = prompt[pos + 1]
                continue
            nxt = int(self.head_ids[int(np.argmax(lg))])  # first maximum, as sample_argmax
            if nxt in (151645, 151643):
                break
            ids.append(nxt)
            if len(ids) >= steps:
                break
            token = nxt
        return ids, np.array(logits)

    def kv(self, which, layer, kv_dim, rows):
        base = np.ctypeslib.as_array(self.L.refq_kv(self.h, which), shape=((layer + 1) * self.ctx * kv_dim,))
        return base[layer * self.ctx * kv_dim:][:rows * kv_dim].copy()


class RefRunq:
    """runq.c's build_transformer / forward (runq.c:359-367, 477-615), generate at -t 0 (runq.c:982-1036)"""

    def __init__(self, path):
        self.L = ref_lib("runq")
        self.h = self.L.refr_open(os.fsencode(path))
        self.n = self.L.refr_vocab(self.h)
        self.seq_len = self.L.refr_seq_len(self.h)

    def generate(self, prompt, steps):
        ids, logits, token, pos = [], [], prompt[0], 0
        while pos < steps:
            lg = np.ctypeslib.as_array(self.L.refr_forward(self.h, int(token), pos), shape=(self.n,)).copy()
            logits.append(lg)
            nxt = prompt[pos + 1] if pos < len(prompt) - 1 else int(np.argmax(lg))
            pos += 1
            if nxt == 1:
                break
            if pos >= len(prompt):
                ids.append(nxt)
            token = nxt
        return ids, np.array(logits)

    def kv(self, which, layer, kv_dim, rows):
        base = np.ctypeslib.as_array(self.L.refr_kv(self.h, which), shape=((layer + 1) * self.seq_len * kv_dim,))
        return base[layer * self.seq_len * kv_dim:][:rows * kv_dim].copy()


def first_difference(got, ref):
    for pos, (g, r) in enumerate(zip(got, ref)):
        if not np.array_equal(g, r):
            k = int(np.argmax(g != r))
            return f"position {pos}: first differing logit {k}: {g[k]!r} vs {r[k]!r}"
    return None


def check_bitwise(model, ref, ids_g, lg_g, ids_r, lg_r, rows):
    """logits of every position, ids, and every layer's K and V rows 0 .. rows-1, bit for bit"""
    assert len(lg_g) == len(lg_r), (len(lg_g), len(lg_r))
    assert first_difference(lg_g, lg_r) is None, first_difference(lg_g, lg_r)
    assert list(ids_g) == list(ids_r)
    I = model.info
    kv_dim = I.dim // I.n_heads * I.n_kv_heads
    for layer in range(I.n_layers):
        for which in (1, 2):
            got = model.read_state(which, layer, rows * kv_dim)
            assert np.array_equal(got, ref.kv(which - 1, layer, kv_dim, rows)), (which, layer)


def test_ref_expf_on_the_device_matches_the_c_library():
    """the strict mode's expf on the device: bit for bit the C library's, over a strided sample of all 2^32
    patterns and every float of [-24, 0] with the last 4 mantissa bits fixed"""
    L = oracle()
    u = np.arange(0, 1 << 32, 257, dtype=np.uint64).astype(np.uint32)
    lo, hi = np.float32(-24.0).view(np.uint32), np.float32(-0.0).view(np.uint32)
    u = np.concatenate([u, np.arange(hi, lo + 1, 16, dtype=np.uint64).astype(np.uint32)])
    for chunk in np.array_split(u, 4):
        x = chunk.view(np.float32)
        want = np.empty_like(x)
        L.or_expf(ptr(x), x.size, ptr(want))
        got = pkg().ref_expf(x)
        same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
        assert same.all(), x[~same][:8]


@pytest.mark.parametrize("name,ctx", [("qwb", 64), ("bin", 0)])
def test_strict_tiny_models_equal_the_reference_binaries_bitwise(name, ctx):
    """the reference binaries' own --logits dumps and ids (tests/golden/tiny_*), bit for bit, through the
    captured step graph and through eager forward() calls"""
    import json
    meta = json.load(open(os.path.join(GOLDEN, "tiny_ref.json")))[name]
    m = pkg().Model(os.path.join(GOLDEN, f"tiny.{name}"), ctx or 1024)
    m.set_strict(True)
    assert m.strict
    max_new = meta["n"] if name == "qwb" else meta["steps"] - len(meta["prompt"]) + 1
    r = m.generate(meta["prompt"], max_new, logits=True)
    ref = np.fromfile(os.path.join(GOLDEN, f"tiny_{name}_ref.logits"), "<f4").reshape(-1, m.info.n_logits)
    n = min(len(ref), len(r["logits"]))
    assert list(r["ids"]) == meta["ids"]
    assert first_difference(r["logits"][:n], ref[:n]) is None
    seq = list(meta["prompt"]) + list(r["ids"])
    eager = np.array([m.forward(seq[p], p) for p in range(n)])
    m.close()
    assert np.array_equal(eager, ref[:n])


def test_strict_mode_switches_both_ways():
    """fast -> strict -> fast on one model: each mode's results are those of a model opened in that mode
    (the step graphs are re-captured)"""
    import json
    meta = json.load(open(os.path.join(GOLDEN, "tiny_ref.json")))["qwb"]
    path = os.path.join(GOLDEN, "tiny.qwb")
    m = pkg().Model(path, 64)
    fast0 = m.generate(meta["prompt"], meta["n"], logits=True)["logits"]
    m.set_strict(True)
    strict = m.generate(meta["prompt"], meta["n"], logits=True)["logits"]
    m.set_strict(False)
    fast1 = m.generate(meta["prompt"], meta["n"], logits=True)["logits"]
    m.close()
    ref = np.fromfile(os.path.join(GOLDEN, "tiny_qwb_ref.logits"), "<f4").reshape(-1, 256)
    assert np.array_equal(fast0, fast1)
    assert np.array_equal(strict, ref[:len(strict)])


@pytest.fixture(scope="module")
def c3_model(tmp_path_factory):
    return synth("qwb", str(tmp_path_factory.mktemp("c3") / "c3.qwb"), "c3", 31)


def c3_prompt(head_ids, n, seed):
    return [int(v) for v in np.random.default_rng(seed).choice(head_ids, n, replace=False)]


def test_strict_c3_full_depth_128_tokens(c3_model):
    ctx = 24 + 128
    ref = RefQwen(c3_model, ctx)
    prompt = c3_prompt(ref.head_ids, 24, 32)
    ids_r, lg_r = ref.generate(prompt, 128)
    assert len(ids_r) == 128 and len(lg_r) == 24 + 127  # the head leaves out the stop ids
    m = pkg().Model(c3_model, ctx)
    m.set_strict(True)
    r = m.generate(prompt, 128, logits=True)
    check_bitwise(m, ref, r["ids"], r["logits"], ids_r, lg_r, len(lg_r))
    m.close()


def test_strict_c4_prefill_512_then_64_tokens(c3_model):
    """a 512-token prompt through the batched prefill (int8 MFMA GEMMs, strict attention), then 64 greedy
    decode steps: the prefill's last-position logits, every later position's logits (eager forward() over the
    prefilled cache), the ids of llm_generate's prefill path, and all K/V rows, bit for bit"""
    ctx = 512 + 64
    ref = RefQwen(c3_model, ctx)
    prompt = c3_prompt(ref.head_ids, 512, 33)
    ids_r, lg_r = ref.generate(prompt, 64)
    assert len(ids_r) == 64 and len(lg_r) == 512 + 63
    m = pkg().Model(c3_model, ctx)
    m.set_strict(True)
    lg = m.prefill(prompt)
    assert np.array_equal(lg, lg_r[511]), first_difference([lg], [lg_r[511]])
    seq = prompt + ids_r
    later = [m.forward(seq[p], p) for p in range(512, len(lg_r))]
    assert first_difference(later, lg_r[512:]) is None, first_difference(later, lg_r[512:])
    r = m.generate(prompt, 64)
    assert list(r["ids"]) == ids_r
    # the cache after generate(): the prefill's rows 0..511, then the decode steps' rows
    I = m.info
    kv_dim = I.dim // I.n_heads * I.n_kv_heads
    for layer in range(I.n_layers):
        for which in (1, 2):
            got = m.read_state(which, layer, (len(lg_r)) * kv_dim)
            assert np.array_equal(got, ref.kv(which - 1, layer, kv_dim, len(lg_r))), (which, layer)
    m.close()


def test_strict_c5_full_workload_256_tokens_context_4096(tmp_path):
    """the whole C5 workload: a 32-token prompt and 256 greedy tokens with a 4096-position cache (positions up
    to 287), every logit, id and K/V row bit for bit"""
    import time
    p = synth("qwb", str(tmp_path / "c5.qwb"), "c5", 35)
    ctx = 4096
    ref = RefQwen(p, ctx)
    prompt = c3_prompt(ref.head_ids, 32, 36)
    t = time.time()
    ids_r, lg_r = ref.generate(prompt, 256)
    print(f"C5 reference: {len(ids_r)} ids over {len(lg_r)} positions in {time.time() - t:.1f} s", flush=True)
    assert len(lg_r) >= 32 + 64  # a stop id (in the untrimmed head) may end the stream early, at both sides
    m = pkg().Model(p, ctx)
    m.set_strict(True)
    r = m.generate(prompt, 256, logits=True)
    check_bitwise(m, ref, r["ids"], r["logits"], ids_r, lg_r, len(lg_r))
    m.close()


@pytest.mark.parametrize("preset,seed", [("c1", 37), ("c2", 38)])
def test_strict_runq_full_context(tmp_path, preset, seed):
    """llama2.c shapes run to seq_len positions (256 for 288/6L, 1024 for 768/12L: the KV cache fills)"""
    p = synth("bin", str(tmp_path / f"{preset}.bin"), preset, seed)
    ref = RefRunq(p)
    prompt = [1] + [int(v) for v in np.random.default_rng(seed).integers(3, ref.n, 7)]
    steps = ref.seq_len
    ids_r, lg_r = ref.generate(prompt, steps)
    print(f"{preset} reference: {len(ids_r)} ids over {len(lg_r)} positions")
    assert len(lg_r) >= steps // 2  # BOS may end the stream early, at both sides
    m = pkg().Model(p, 0)
    m.set_strict(True)
    r = m.generate(prompt, steps - len(prompt) + 1, logits=True)
    check_bitwise(m, ref, r["ids"], r["logits"], ids_r, lg_r, len(lg_r))
    m.close()
