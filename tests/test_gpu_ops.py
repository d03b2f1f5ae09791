"""Device stages against the oracle on the same seeded inputs (MI355X).

Bars: int8 quantization and int32 group sums bit-exact; fpga_matvec (runq flavour) bit-exact, the reference
testbench's bar (hls/matvec_tb.cpp:82-83); fpga_matvec4 (qwen flavour) within |out - exact| <= 1e-5 *
sum_g |term_g|, the reference testbench's bar (hls4/matvec4_tb.cpp:19, 67-79)."""
import ctypes as C
import os

import numpy as np
import pytest

from helpers import GOLDEN, exact_terms, f16_scales, oracle, pkg, ptr, synth, unpack_q4

pytestmark = pytest.mark.gpu
OPS = np.load(os.path.join(GOLDEN, "ops.npz"))


def oracle_quantize(x, flavor, gs):
    q, s = np.empty(x.size, np.int8), np.empty(x.size // gs, np.float32)
    if flavor == 0:
        oracle().or_quantize_qwen(ptr(q), ptr(s), ptr(x), x.size)
    else:
        oracle().or_quantize_runq(ptr(q), ptr(s), ptr(x), x.size, gs)
    return q, s


def test_quantize_golden_bit_exact():
    P = pkg()
    x = OPS["q_x"]
    q, s = P.quantize(x, 0, 32)
    assert np.array_equal(q, OPS["qwen_q"]) and np.array_equal(s.view(np.uint32), OPS["qwen_s"].view(np.uint32))
    for gs in (32, 64):
        q, s = P.quantize(x, 1, gs)
        assert np.array_equal(q, OPS[f"runq{gs}_q"])
        assert np.array_equal(s.view(np.uint32), OPS[f"runq{gs}_s"].view(np.uint32))


@pytest.mark.parametrize("seed", range(4))
def test_quantize_random_bit_exact(seed):
    P = pkg()
    rng = np.random.default_rng(100 + seed)
    n = 4864
    x = (rng.standard_normal(n) * np.exp(rng.uniform(-20, 20, size=n))).astype(np.float32)
    x[rng.integers(0, n, 50)] = 0.0
    for flavor, gs in ((0, 32), (1, 32), (1, 64)):
        q, s = P.quantize(x, flavor, gs)
        oq, os_ = oracle_quantize(x, flavor, gs)
        assert np.array_equal(q, oq), (flavor, gs)
        assert np.array_equal(s.view(np.uint32), os_.view(np.uint32)), (flavor, gs)


@pytest.mark.parametrize("n,d,bits,gs", [(96, 5, 4, 32), (96, 5, 8, 32), (896, 128, 4, 32), (896, 64, 8, 32),
                                         (4864, 32, 4, 32), (8192, 4, 4, 32), (18944, 8, 4, 32),
                                         (768, 24, 0, 64), (288, 7, 0, 32)])
def test_group_dots_bit_exact(n, d, bits, gs):
    rng = np.random.default_rng(n * 7 + d)
    wb = 8 if bits == 0 else bits
    w = rng.integers(0, 256, size=d * n * wb // 8, dtype=np.uint8)
    xq = rng.integers(-128, 128, size=n, dtype=np.int8)
    got = pkg().group_dots(w, xq, n, d, bits, gs)
    wv = unpack_q4(w, d, n) if bits == 4 else w.view(np.int8).reshape(d, n).astype(np.int16)
    want = (wv.reshape(d, n // gs, gs).astype(np.int64) * xq.reshape(1, n // gs, gs)).sum(2)
    assert np.array_equal(got, want)


@pytest.fixture(scope="module")
def drv():
    d = pkg().DropIn()
    yield d
    d.close()


def run_matvec4(drv, w, s, xq, xs, n, d, bits):
    _, pw = drv.put(w)
    _, ps = drv.put(s)
    _, px = drv.put(xq)
    _, pxs = drv.put(xs)
    out, po = drv.alloc(d * 4)
    assert drv.matvec4(pw, ps, px, pxs, po, n, d, bits) == 0
    return out.view(np.float32)[:d].copy()


QUICK = [(96, 5, 4), (96, 5, 8), (896, 128, 4), (896, 64, 8), (4864, 32, 4), (8192, 4, 4)]
ALL = [(896, 896, 4), (896, 128, 4), (896, 4864, 4), (4864, 896, 4), (896, 49152, 8), (18944, 512, 4),
       (3584, 1024, 8), (32768, 24, 4), (32768, 24, 8)]


@pytest.mark.parametrize("n,d,bits", QUICK + ALL)
def test_matvec4_testbench_bar(drv, n, d, bits):
    rng = np.random.default_rng(1234 + n + d + bits)
    w = rng.integers(0, 256, size=d * n * bits // 8, dtype=np.uint8)
    s = f16_scales(rng, d * n // 32)
    xq = rng.integers(-128, 128, size=n, dtype=np.int8)
    xs = rng.uniform(1e-3, 1e-1, size=n // 32).astype(np.float32)
    out = run_matvec4(drv, w, s, xq, xs, n, d, bits)
    wv = unpack_q4(w, d, n) if bits == 4 else w.view(np.int8).reshape(d, n)
    ref, mag, _ = exact_terms(wv, s.view(np.float16).astype(np.float32), xq, xs)
    err = np.abs(out.astype(np.float64) - ref)
    assert (err <= 1e-5 * mag).all(), float((err / np.maximum(mag, 1e-30)).max())
    # and against the oracle's sequential sum (same bar)
    o = np.empty(d, np.float32)
    oracle().or_matvec4(ptr(o), ptr(w), ptr(s), ptr(xq), ptr(xs), n, d, bits)
    assert (np.abs(out.astype(np.float64) - o) <= 2e-5 * mag).all()


@pytest.mark.parametrize("bits", [4, 8])
def test_matvec4_special_fp16_scales(drv, bits):
    """row i's scales have exponent field i % 31: zero, subnormals, up to 65504 (hls4/matvec4_tb.cpp:88-97, 143-144)"""
    rng = np.random.default_rng(77 + bits)
    n, d = 64, 31
    w = rng.integers(0, 256, size=d * n * bits // 8, dtype=np.uint8)
    s = f16_scales(rng, d * n // 32, special_rows=1, ng=n // 32)
    xq = rng.integers(-128, 128, size=n, dtype=np.int8)
    xs = rng.uniform(1e-3, 1e-1, size=n // 32).astype(np.float32)
    out = run_matvec4(drv, w, s, xq, xs, n, d, bits)
    wv = unpack_q4(w, d, n) if bits == 4 else w.view(np.int8).reshape(d, n)
    ref, mag, _ = exact_terms(wv, s.view(np.float16).astype(np.float32), xq, xs)
    assert (np.abs(out - ref) <= 1e-5 * mag).all()


def qwb_matrix(path, kind, layer):
    """matrix `kind` (0..6: wq, wk, wv, wo, w1 gate, w2 down, w3 up) of `layer`, or the head (kind 7), read from
    a .qwb the way the reference testbench walks it (hls4/matvec4_tb.cpp:102-126): every array padded to 64
    bytes; the per-layer vectors (two norms, the q/k/v biases), the output norm and the head ids, then the
    matrices as weight plane + fp16 scale plane.  Returns (weights, scales, n, d, bits)."""
    with open(path, "rb") as f:
        f.seek(8)
        dim, hid, L, nh, nkv, vocab, head_k, ctx, gs, emb_bits = np.frombuffer(f.read(40), "<i4")
        kv = dim // nh * nkv
        off = 256

        def take(nbytes):
            nonlocal off
            at = off
            off += nbytes + (-(off + nbytes) & 63)
            return at
        for n in (dim, dim, dim, kv, kv):
            for _ in range(L):
                take(4 * n)
        take(4 * dim)
        take(4 * head_k)
        shapes = [(dim, dim), (kv, dim), (kv, dim), (dim, dim), (hid, dim), (dim, hid), (hid, dim)]
        for i in range(7 * L + 1):
            rows, n = shapes[i // L] if i < 7 * L else (head_k, dim)
            bits = 4 if i < 7 * L else int(emb_bits)
            wo, so = take(rows * n * bits // 8), take(rows * n // 32 * 2)
            if i == kind * L + layer:
                f.seek(wo)
                w = np.frombuffer(f.read(rows * n * bits // 8), np.uint8)
                f.seek(so)
                s = np.frombuffer(f.read(rows * n // 32 * 2), np.uint16)
                return w, s, int(n), int(rows), bits
    raise ValueError("no such matrix")


@pytest.fixture(scope="module")
def c3_qwb(tmp_path_factory):
    # the reference testbench's real-matrix file is the 24-layer Qwen2.5-0.5B .qwb with a 49152-row head; the
    # same shapes and layout, seeded synthetic Q4_0 / Q8_0 data (no model files here)
    p = str(tmp_path_factory.mktemp("realmat") / "c3h49k.qwb")
    return synth("qwb", p, "c3", 17, "vocab=65536", "head_k=49152")


@pytest.mark.parametrize("name,kind,layer", [("blk.0 attn_q", 0, 0), ("blk.0 attn_k", 1, 0),
                                             ("blk.23 ffn_gate", 4, 23), ("blk.0 ffn_down", 5, 0),
                                             ("blk.12 ffn_up", 6, 12), ("output head", 7, 0)])
def test_matvec4_testbench_real_matrices(drv, c3_qwb, name, kind, layer):
    """the testbench's real-matrix mode (hls4/matvec4_tb.cpp:150-164): the matrices it names, read from the
    file, through the drop-in with its activation distributions (xq uniform in [-128, 127], xs in [1e-3, 1e-1])
    and its bar, |out - ref| <= 1e-5 * sum_g |term_g| per row, and against the oracle's sequential sum"""
    w, s, n, d, bits = qwb_matrix(c3_qwb, kind, layer)
    rng = np.random.default_rng(4321 + kind * 100 + layer)
    xq = rng.integers(-128, 128, size=n, dtype=np.int8)
    xs = rng.uniform(1e-3, 1e-1, size=n // 32).astype(np.float32)
    out = run_matvec4(drv, w, s, xq, xs, n, d, bits)
    wv = unpack_q4(w, d, n) if bits == 4 else w.view(np.int8).reshape(d, n)
    ref, mag, _ = exact_terms(wv, s.view(np.float16).astype(np.float32), xq, xs)
    err = np.abs(out.astype(np.float64) - ref)
    assert (err <= 1e-5 * mag).all(), (name, float((err / np.maximum(mag, 1e-30)).max()))
    o = np.empty(d, np.float32)
    oracle().or_matvec4(ptr(o), ptr(w), ptr(s), ptr(xq), ptr(xs), n, d, bits)
    assert (np.abs(out.astype(np.float64) - o) <= 2e-5 * mag).all(), name


@pytest.mark.parametrize("k", range(5))
def test_matvec4_golden(drv, k):
    n, d, bits = (int(v) for v in OPS[f"m{k}_shape"])
    out = run_matvec4(drv, OPS[f"m{k}_w"], OPS[f"m{k}_s"], OPS[f"m{k}_xq"], OPS[f"m{k}_xs"], n, d, bits)
    ref = OPS[f"m{k}_out"]
    wv = unpack_q4(OPS[f"m{k}_w"], d, n) if bits == 4 else OPS[f"m{k}_w"].view(np.int8).reshape(d, n)
    _, mag, _ = exact_terms(wv, OPS[f"m{k}_s"].view(np.float16).astype(np.float32), OPS[f"m{k}_xq"], OPS[f"m{k}_xs"])
    assert (np.abs(out.astype(np.float64) - ref) <= 2e-5 * mag).all()


MATVEC_TB = [(288, 288, 32), (288, 768, 32), (768, 288, 32), (768, 768, 64), (768, 2048, 64), (2048, 768, 64),
             (768, 32000, 64), (96, 7, 32), (768, 32000, 32),
             # the largest n (MATVEC_HIP_MAX_N): activations take more than one prologue pass per thread
             (32768, 40, 64), (32768, 9, 32)]


@pytest.mark.parametrize("n,d,gs", MATVEC_TB)
def test_matvec_runq_bit_exact(drv, n, d, gs):
    """hls/matvec_tb.cpp:56-66 distributions, out == runq.c matmul() exactly"""
    rng = np.random.default_rng(1234 + n * 3 + d + gs)
    wq = rng.integers(-128, 128, size=d * n, dtype=np.int8)
    xq = rng.integers(-128, 128, size=n, dtype=np.int8)
    ws = rng.uniform(1e-4, 2e-2, size=d * n // gs).astype(np.float32)
    xs = rng.uniform(1e-3, 1e-1, size=n // gs).astype(np.float32)
    _, pw = drv.put(wq)
    _, ps = drv.put(ws)
    _, px = drv.put(xq)
    _, pxs = drv.put(xs)
    out, po = drv.alloc(d * 4)
    assert drv.matvec(pw, ps, px, pxs, po, n, d, gs) == 0
    got = out.view(np.float32)[:d]
    ref = np.empty(d, np.float32)
    oracle().or_matvec_runq(ptr(ref), ptr(wq), ptr(ws), ptr(xq), ptr(xs), n, d, gs)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("offset", [4, 8, 12])
def test_matvec_runq_unaligned_activations(drv, offset):
    """xq at a device address that is only 4-byte aligned (the reference checks no alignment, matvec_fpga.cpp:178-182)"""
    n, d, gs = 768, 96, 32
    rng = np.random.default_rng(99 + offset)
    wq = rng.integers(-128, 128, size=d * n, dtype=np.int8)
    xq = rng.integers(-128, 128, size=n, dtype=np.int8)
    ws = rng.uniform(1e-4, 2e-2, size=d * n // gs).astype(np.float32)
    xs = rng.uniform(1e-3, 1e-1, size=n // gs).astype(np.float32)
    _, pw = drv.put(wq)
    _, ps = drv.put(ws)
    xbuf, px = drv.alloc(n + 64)
    xbuf[offset:offset + n] = xq.view(np.uint8)
    _, pxs = drv.put(xs)
    out, po = drv.alloc(d * 4)
    assert drv.matvec(pw, ps, px + offset, pxs, po, n, d, gs) == 0
    ref = np.empty(d, np.float32)
    oracle().or_matvec_runq(ptr(ref), ptr(wq), ptr(ws), ptr(xq), ptr(xs), n, d, gs)
    assert np.array_equal(out.view(np.float32)[:d].view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("k", range(3))
def test_matvec_runq_golden(drv, k):
    n, d, gs = (int(v) for v in OPS[f"r{k}_shape"])
    _, pw = drv.put(OPS[f"r{k}_wq"])
    _, ps = drv.put(OPS[f"r{k}_ws"])
    _, px = drv.put(OPS[f"r{k}_xq"])
    _, pxs = drv.put(OPS[f"r{k}_xs"])
    out, po = drv.alloc(d * 4)
    assert drv.matvec(pw, ps, px, pxs, po, n, d, gs) == 0
    assert np.array_equal(out.view(np.float32)[:d].view(np.uint32), OPS[f"r{k}_out"].view(np.uint32))


def test_weights_stay_resident_activations_do_not(drv):
    """second call with new activations in the same buffers: weights are not re-read from the host,
    activations are"""
    rng = np.random.default_rng(9)
    n, d = 896, 64
    w = rng.integers(0, 256, size=d * n // 2, dtype=np.uint8)
    s = f16_scales(rng, d * n // 32)
    vw, pw = drv.put(w)
    _, ps = drv.put(s)
    vx, px = drv.put(rng.integers(-128, 128, size=n, dtype=np.int8))
    vxs, pxs = drv.put(rng.uniform(1e-3, 1e-1, size=n // 32).astype(np.float32))
    out, po = drv.alloc(d * 4)
    assert drv.matvec4(pw, ps, px, pxs, po, n, d, 4) == 0
    xq2 = rng.integers(-128, 128, size=n, dtype=np.int8)
    vx[:n] = xq2.view(np.uint8)
    assert drv.matvec4(pw, ps, px, pxs, po, n, d, 4) == 0
    got = out.view(np.float32)[:d].copy()
    xs = vxs.view(np.float32)[:n // 32].copy()
    ref, mag, _ = exact_terms(unpack_q4(w, d, n), s.view(np.float16).astype(np.float32), xq2, xs)
    assert (np.abs(got - ref) <= 1e-5 * mag).all()


def test_argument_errors(drv, capfd):
    _, p = drv.alloc(1 << 16)
    assert drv.matvec4(p + 8, p, p, p, p, 32, 1, 4) == -1      # not 64-byte aligned
    assert drv.matvec4(p, p, p, p, p, 48, 1, 4) == -1          # n % 32
    assert drv.matvec4(p, p, p, p, p, 32, 1, 5) == -1          # wbits
    assert drv.matvec4(p, p, p, p, p, 32, 0, 4) == -1          # d
    assert drv.matvec4(p, p, p, p, p, 65536, 1, 4) == -1       # n above the library maximum
    assert drv.matvec(p, p, p, p, p, 96, 1, 48) == -1          # gs
    assert drv.matvec4(1 << 40, p, p, p, p, 32, 1, 4) == -1    # address outside every buffer
    err = capfd.readouterr().err
    assert "unsupported" in err and "not inside a buffer" in err


def test_forced_timeout_reports_minus_one(capfd):
    """FPGA_TIMEOUT_MS=0: the completion wait gives up at once and the call fails like the reference's 5 s
    ap_done time-out (matvec_fpga.cpp:156-170, 226-230); the kernel itself runs normally"""
    P = pkg()
    L = P.lib()
    L.fpga_close()
    os.environ["FPGA_TIMEOUT_MS"] = "0"
    try:
        d = P.DropIn()
        rng = np.random.default_rng(3)
        n, rows = 4096, 4096
        _, pw = d.put(rng.integers(0, 256, size=rows * n // 2, dtype=np.uint8))
        _, ps = d.put(f16_scales(rng, rows * n // 32))
        _, px = d.put(rng.integers(-128, 128, size=n, dtype=np.int8))
        _, pxs = d.put(rng.uniform(1e-3, 1e-1, size=n // 32).astype(np.float32))
        _, po = d.alloc(rows * 4)
        r = d.matvec4(pw, ps, px, pxs, po, n, rows, 4)
        d.close()
    finally:
        del os.environ["FPGA_TIMEOUT_MS"]
    assert r == -1 and "did not finish" in capfd.readouterr().err
