"""Batched prefill (int8 MFMA GEMM, per-token steps, causal attention) on the MI355X.

The prefill GEMM adds the group terms ((float)ival * ws) * xs of every (row, token) in group order, which is
the reference's matmul (qwen.c:436-456, runq.c:429-458) exactly: the bar for it is bitwise equality with the
oracle's sequential matvec, token by token.  The whole prefill is held to the model bars of
test_gpu_model.py: logits within 1e-3 of the reference on the tiny models, the same greedy ids when the
generation continues from it, and the per-position decode path's KV cache within fp32 reordering."""
import json
import os

import numpy as np
import pytest

from helpers import GOLDEN, OracleModel, f16_scales, oracle, pkg, ptr, rel_err, synth

pytestmark = pytest.mark.gpu
TOL = 1e-3
META = json.load(open(os.path.join(GOLDEN, "tiny_ref.json")))


def golden(name, n):
    return np.fromfile(os.path.join(GOLDEN, f"tiny_{name}_ref.logits"), dtype="<f4").reshape(-1, n)


# 0: the library's choice; 10 TA + TB: one wave per 16 TA rows x 16 TB tokens
SHAPES = [0, 11, 12, 14, 21, 22, 24, 41, 42]


def check_qwen_gemm(w, s, xq, xs, M, n, d, bits, rb, shape):
    y = pkg().prefill_gemm(w, s, xq, xs, M, n, d, bits, 32, rb, shape)
    for m in range(M):
        o = np.empty(d, np.float32)
        oracle().or_matvec4(ptr(o), ptr(w), ptr(s), ptr(xq[m]), ptr(xs[m]), n, d, bits)
        assert np.array_equal(y[m].view(np.uint32), o.view(np.uint32)), m


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("M,n,d,bits,rb", [(1, 96, 36, 4, 16), (7, 96, 36, 8, 16), (33, 896, 128, 4, 16),
                                           (64, 896, 64, 8, 16), (40, 4864, 32, 4, 8), (5, 256, 20, 4, 16),
                                           (70, 128, 100, 4, 8), (96, 64, 12288, 4, 16), (64, 896, 16384, 4, 16),
                                           (64, 160, 16384, 8, 16)])
def test_prefill_gemm_bit_exact_qwen(M, n, d, bits, rb, shape):
    """group counts below, at and above the 4 waves the K groups are dealt over; grids of 1024 tiles and more;
    rows and tokens that fill no tile, one tile, or end inside one"""
    rng = np.random.default_rng(100 + M + n + d + bits)
    w = rng.integers(0, 256, size=d * n * bits // 8, dtype=np.uint8)
    s = f16_scales(rng, d * n // 32)
    xq = rng.integers(-128, 128, size=(M, n), dtype=np.int8)
    xs = rng.uniform(1e-3, 1e-1, size=(M, n // 32)).astype(np.float32)
    check_qwen_gemm(w, s, xq, xs, M, n, d, bits, rb, shape)


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("bits", [4, 8])
def test_prefill_gemm_bit_exact_special_scales(bits, shape):
    """fp16 scales of every exponent field (zero, subnormals, up to 65504) and both signs, row by row; the
    extreme int8 activations and weights (every group sum at its largest magnitude in some rows): the
    one-instruction product with the biased MFMA start must round like ((float)ival) * ws for all of them"""
    M, n, d = 40, 256, 64
    rng = np.random.default_rng(7 + bits)
    w = rng.integers(0, 256, size=d * n * bits // 8, dtype=np.uint8)
    if bits == 4:
        w.reshape(d, n // 2)[:8] = 0x88        # int4 -8 everywhere
    else:
        w.reshape(d, n)[:8] = 0x80             # int8 -128 everywhere
    s = f16_scales(rng, d * n // 32, special_rows=1, ng=n // 32)
    xq = rng.integers(-128, 128, size=(M, n), dtype=np.int8)
    xq[:4] = -128
    xq[4:8] = 127
    xs = rng.uniform(1e-3, 1e-1, size=(M, n // 32)).astype(np.float32)
    check_qwen_gemm(w, s, xq, xs, M, n, d, bits, 16, shape)


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("M,n,d,gs,rb", [(9, 288, 32, 32, 64), (33, 768, 96, 64, 64), (17, 768, 64, 32, 16),
                                         (64, 288, 16384, 32, 64), (64, 192, 16384, 64, 64)])
def test_prefill_gemm_bit_exact_runq(M, n, d, gs, rb, shape):
    rng = np.random.default_rng(200 + M + n + d + gs)
    wq = rng.integers(-128, 128, size=d * n, dtype=np.int8)
    ws = rng.uniform(1e-4, 2e-2, size=d * n // gs).astype(np.float32)
    xq = rng.integers(-128, 128, size=(M, n), dtype=np.int8)
    xs = rng.uniform(1e-3, 1e-1, size=(M, n // gs)).astype(np.float32)
    y = pkg().prefill_gemm(wq, ws, xq, xs, M, n, d, 0, gs, rb, shape)
    for m in range(M):
        o = np.empty(d, np.float32)
        oracle().or_matvec_runq(ptr(o), ptr(wq), ptr(ws), ptr(xq[m]), ptr(xs[m]), n, d, gs)
        assert np.array_equal(y[m].view(np.uint32), o.view(np.uint32)), m


@pytest.mark.parametrize("name,ctx", [("qwb", 64), ("bin", 0)])
def test_prefill_logits_against_reference(name, ctx):
    """the prompt as one batch: the last position's logits against the reference binary's"""
    m = pkg().Model(os.path.join(GOLDEN, f"tiny.{name}"), ctx or 1024)
    ref = golden(name, m.info.n_logits)
    prompt = META[name]["prompt"]
    lg = m.prefill(prompt)
    m.close()
    assert rel_err(lg, ref[len(prompt) - 1]) < TOL


@pytest.mark.parametrize("name,ctx", [("qwb", 64), ("bin", 0)])
def test_generate_through_prefill_matches_reference_ids(name, ctx):
    m = pkg().Model(os.path.join(GOLDEN, f"tiny.{name}"), ctx or 1024)
    meta = META[name]
    max_new = meta["n"] if name == "qwb" else meta["steps"] - len(meta["prompt"]) + 1
    r = m.generate(meta["prompt"], max_new)
    m.close()
    assert list(r["ids"]) == meta["ids"]


def kv_rows(m, n_pos):
    kv = m.info.dim // m.info.n_heads * m.info.n_kv_heads
    return [(m.read_state(1, l)[:n_pos * kv], m.read_state(2, l)[:n_pos * kv]) for l in range(m.info.n_layers)]


def test_prefill_equals_the_per_position_path_across_chunks(tmp_path):
    """a 600-token prompt (two prefill chunks: 512 + 88) against 600 decode steps: logits of the last position,
    and every layer's K/V rows position by position.  Layer 0's rows agree to fp32 rounding; later layers may
    differ at the few positions where an activation re-quantized between the two paths' different fp32 sum
    orders crossed an int8 boundary (the flip-limited bar of test_gpu_model.py)"""
    p = synth("qwb", str(tmp_path / "long.qwb"), "tiny", 31, "max_seq=700")
    a, b = pkg().Model(p, 700), pkg().Model(p, 700)
    hid = a.head_ids
    ids = [int(hid[v]) for v in np.random.default_rng(8).integers(0, len(hid), 600)]
    lg_pf = a.prefill(ids)
    for pos, t in enumerate(ids):
        lg_fw = b.forward(t, pos)
    assert rel_err(lg_pf, lg_fw) < TOL
    kv = a.info.dim // a.info.n_heads * a.info.n_kv_heads
    for layer, ((ka, va), (kb, vb)) in enumerate(zip(kv_rows(a, 600), kv_rows(b, 600))):
        for x, y in ((ka, kb), (va, vb)):
            x, y = x.reshape(600, kv), y.reshape(600, kv)
            e = np.abs(x - y).max(1) / np.abs(y).max(1)
            if layer == 0:
                assert e.max() < 1e-5, e.max()
            assert e.max() < 2e-2 and (e > 1e-4).sum() <= 6, (layer, e.max(), (e > 1e-4).sum())
    a.close()
    b.close()


@pytest.mark.parametrize("n,strict", [(512, False), (40, False), (512, True)])
def test_prefill_swiglu_epilogue_equals_the_separate_kernel(monkeypatch, tmp_path, n, strict):
    """the gate/up GEMM's SwiGLU + int8 quantization epilogue against the separate SwiGLU kernel
    (LLM_PF_SWIGLU=0): the same float operations in the same order, so the prefill logits and every layer's K/V
    rows are bitwise equal (512 tokens: 32 x 32 tiles, two waves per quantization group; 40 tokens: 16 x 16
    tiles, four waves, a partial token tile; and the strict mode, whose SiLU takes the reference's expf)"""
    p = synth("qwb", str(tmp_path / "sw.qwb"), "c3", 41, "layers=2", "vocab=4096", "head_k=4096")
    ids = [int(v) for v in np.random.default_rng(12).integers(0, 4096, n)]
    runs = []
    for setting in ("0", "1"):
        monkeypatch.setenv("LLM_PF_SWIGLU", setting)
        m = pkg().Model(p, 600)
        if strict:
            m.set_strict(True)
        lg = m.prefill(ids)
        runs.append((lg, kv_rows(m, n)))
        m.close()
    assert np.array_equal(runs[0][0], runs[1][0])
    for (ka, va), (kb, vb) in zip(runs[0][1], runs[1][1]):
        assert np.array_equal(ka, kb) and np.array_equal(va, vb)


@pytest.mark.parametrize("fmt,n,strict", [("qwb", 512, False), ("qwb", 600, False), ("qwb", 40, True),
                                          ("bin", 300, False), ("bin", 150, True)])
def test_prefill_qkv_epilogue_equals_the_separate_kernel(monkeypatch, tmp_path, fmt, n, strict):
    """bias, RoPE and the q / K / V writes in the QKV GEMM's epilogue against the separate kernel
    (LLM_PF_QKV=0): the same float operations, so the prefill logits and every layer's K/V rows are bitwise
    equal.  NeoX pairs (.qwb: a row's partner 8 rows away, in the lane across the halves of the MFMA tile)
    and interleaved pairs (.bin: the adjacent row, in the same lane), one prefill chunk and two (600 tokens:
    the second chunk's RoPE positions start at 512), and the strict mode"""
    if fmt == "qwb":
        p = synth("qwb", str(tmp_path / "q.qwb"), "c3", 51, "layers=2", "vocab=4096", "head_k=4096")
    else:
        p = synth("bin", str(tmp_path / "q.bin"), "tiny", 52, "dim=256", "heads=4", "kv_heads=2", "gs=64",
                  "hidden=256", "layers=2", "vocab=512", "max_seq=700")
    ids = [int(v) for v in np.random.default_rng(13).integers(0, 512 if fmt == "bin" else 4096, n)]
    runs = []
    for setting in ("0", "1"):
        monkeypatch.setenv("LLM_PF_QKV", setting)
        m = pkg().Model(p, 700)
        if strict:
            m.set_strict(True)
        lg = m.prefill(ids)
        runs.append((lg, kv_rows(m, n)))
        m.close()
    assert np.array_equal(runs[0][0], runs[1][0])
    for (ka, va), (kb, vb) in zip(runs[0][1], runs[1][1]):
        assert np.array_equal(ka, kb) and np.array_equal(va, vb)


def test_prefill_c3_shapes_two_layers(tmp_path):
    """Qwen2-0.5B layer shapes, two layers: prefill logits of a 40-token prompt against the oracle's forced
    prompt (flip-limited bar: see test_gpu_model.py)"""
    p = synth("qwb", str(tmp_path / "c3l2.qwb"), "c3", 21, "layers=2")
    om = OracleModel(p, 64)
    ids = [int(om.head_ids[v]) for v in np.random.default_rng(9).integers(0, om.n, 40)]
    for pos, t in enumerate(ids):
        ref = om.forward(t, pos)
    om.close()
    m = pkg().Model(p, 64)
    lg = m.prefill(ids)
    m.close()
    assert rel_err(lg, ref) < 2e-2


@pytest.mark.parametrize("fmt,shape,n", [("qwb", ("dim=896", "heads=14", "kv_heads=2"), 150),
                                         ("qwb", ("dim=512", "heads=4", "kv_heads=2"), 140),
                                         ("qwb", ("dim=384", "heads=8", "kv_heads=8"), 70),
                                         ("qwb", ("dim=256", "heads=8", "kv_heads=2"), 90),
                                         ("bin", ("dim=256", "heads=4", "kv_heads=4", "gs=64"), 150)])
def test_prefill_attention_head_shapes(tmp_path, fmt, shape, n):
    """head sizes 64 (7 query heads per kv head), 128, 48 (no grouping) and 32, and a runq model with
    quantization groups of 64 (one group per head), one layer, prompts that span two or three attention
    slices of 64 positions: prefill logits against as many decode steps.  The attention kernels write the o
    projection's int8 input themselves (groups inside a head) or through the slice merge.  The trimmed head
    (256 rows) is smaller than the layer matrices, which the loader's staging area must still hold."""
    extra = ["hidden=256", "layers=1", "vocab=512", "max_seq=200"] + (["head_k=256"] if fmt == "qwb" else [])
    p = synth(fmt, str(tmp_path / f"h.{fmt}"), "tiny", 5, *shape, *extra)
    a, b = pkg().Model(p, 200), pkg().Model(p, 200)
    hid = a.head_ids if fmt == "qwb" else np.arange(512)
    ids = [int(hid[v]) for v in np.random.default_rng(8).integers(0, len(hid), n)]
    lg_pf = a.prefill(ids)
    for pos, t in enumerate(ids):
        lg_fw = b.forward(t, pos)
    a.close()
    b.close()
    assert rel_err(lg_pf, lg_fw) < TOL


@pytest.mark.parametrize("shape", [("dim=256", "heads=8", "kv_heads=2"), ("dim=512", "heads=8", "kv_heads=2"),
                                   ("dim=512", "heads=4", "kv_heads=2")])
def test_prefill_split_bf16_attention_against_the_fp32_products(monkeypatch, tmp_path, shape):
    """head sizes 32, 64 and 128: the slice kernel's products on bf16 MFMA over three-piece splits of the fp32
    operands (the default) and on fp32 MFMA (LLM_PF_FLASH_BF=0), two layers, a 200-token prompt (four slices of
    64 positions), each against as many decode steps.  Layer 0's K/V rows come before any attention and are
    bitwise equal in both modes.  After that the paths differ from the decode path where an activation
    re-quantized after different fp32 sum orders crossed an int8 boundary: the logits and layer 1's rows are
    held to the flip-limited bar of test_gpu_model.py in both modes, and the split products may not move more
    of layer 1's positions than the fp32 products do (twice as many, plus a few: the counts are small).  The
    one-layer logits bar (1e-3) for the split products is test_prefill_attention_head_shapes."""
    extra = ["hidden=256", "layers=2", "vocab=512", "max_seq=256", "head_k=256"]
    p = synth("qwb", str(tmp_path / "bf.qwb"), "tiny", 17, *shape, *extra)
    b = pkg().Model(p, 256)
    hid = b.head_ids
    ids = [int(hid[v]) for v in np.random.default_rng(21).integers(0, len(hid), 200)]
    for pos, t in enumerate(ids):
        lg_fw = b.forward(t, pos)
    rows_fw = kv_rows(b, 200)
    b.close()
    lg, rows, flips = {}, {}, {}
    for bf in ("0", "1"):
        monkeypatch.setenv("LLM_PF_FLASH_BF", bf)
        m = pkg().Model(p, 256)
        lg[bf] = m.prefill(ids)
        rows[bf] = kv_rows(m, 200)
        m.close()
        assert rel_err(lg[bf], lg_fw) < 2e-2, bf
        kv = len(rows[bf][0][0]) // 200
        (ka, va), (kb, vb) = rows[bf][1], rows_fw[1]
        e = np.maximum(np.abs(ka - kb).reshape(200, kv).max(1) / np.abs(kb).reshape(200, kv).max(1),
                       np.abs(va - vb).reshape(200, kv).max(1) / np.abs(vb).reshape(200, kv).max(1))
        assert e.max() < 2e-2, (bf, e.max())
        flips[bf] = int((e > 1e-4).sum())
    print("layer-1 positions moved past 1e-4 (fp32, split):", flips["0"], flips["1"])
    for x, y in zip(rows["0"][0], rows["1"][0]):
        assert np.array_equal(x, y)
    assert flips["1"] <= 2 * flips["0"] + 6, flips
