"""CPU checks of the product library and tools: it loads, exports every declared entry point, rejects bad
calls before touching a device, and the model writer is deterministic and writes the reference layout."""
import os
import re
import struct

import numpy as np
import pytest

from helpers import GOLDEN, REPO, SYNTH, pkg, synth


def declared_functions():
    names = []
    for h in ("matvec_fpga.h", "llm_hip.h"):
        text = open(os.path.join(REPO, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^[a-z][\w\s\*]*?\b(\w+)\s*\([^;{]*\)\s*;", text, flags=re.M):
            names.append(m.group(1))
    return names


def test_library_exports_every_declared_function():
    L = pkg().lib()
    names = declared_functions()
    assert {"fpga_open", "fpga_alloc", "fpga_alloc_try", "fpga_matvec", "fpga_matvec4", "fpga_close",
            "llm_open", "llm_generate"} <= set(names)
    for n in names:
        assert hasattr(L, n), n


def test_calls_before_open_fail_like_the_reference(capfd):
    L = pkg().lib()
    assert L.fpga_matvec4(0, 0, 0, 0, 0, 32, 1, 4) == -1
    assert L.fpga_matvec(0, 0, 0, 0, 0, 32, 1, 32) == -1
    import ctypes as C
    phys = C.c_uint64(0)
    assert not L.fpga_alloc_try(64, C.byref(phys))
    assert not L.fpga_alloc(64, C.byref(phys))
    err = capfd.readouterr().err
    assert "fpga_open() not called" in err
    L.fpga_close()  # safe without open, and twice
    L.fpga_close()


def gemv_shape(rows, n, gs, wbits, sf32, rb, role, ordered, cus=256):
    import ctypes as C
    out = (C.c_int * 4)()
    rc = pkg().lib().mvh_gemv_shape(rows, n, gs, wbits, sf32, rb, role, ordered, cus, out)
    return rc, tuple(out)


@pytest.mark.parametrize("name,dims,gs,wbits,sf32,rb,role,ordered", [
    ("runq 4096 gate/up", (2 * 11008, 4096), 64, 8, 1, 8, 2, 1),
    ("runq 4096 down", (4096, 11008), 64, 8, 1, 8, 3, 1),
    ("runq 8192 qkv", (8192 + 2 * 1024, 8192), 64, 8, 1, 8, 0, 1),
    ("qwen 896 strict gate/up", (2 * 4864, 896), 32, 4, 0, 16, 2, 3),
    ("qwen 3584 strict down", (3584, 18944), 32, 4, 0, 8, 3, 3),
    ("qwen 3584 strict head", (65536, 3584), 32, 8, 0, 16, 4, 3),
    ("qwen 8192 strict qkv", (8192 + 2 * 1024, 8192), 32, 4, 0, 16, 0, 3),
])
def test_ordered_gemv_shapes_keep_their_products_in_lds(name, dims, gs, wbits, sf32, rb, role, ordered):
    """every ordered shape the library picks adds each row's group products in group order from LDS: one
    iteration's products (nb row-blocks x rb rows x ng + 1 padded groups of fp32) within 64 KiB"""
    rows, n = dims
    rc, (kw, nb, grid, ordq) = gemv_shape(rows, n, gs, wbits, sf32, rb, role, ordered)
    assert rc == 0 and grid >= 1 and ordq == 1, (name, kw, nb, grid, ordq)
    assert nb * rb * (n // gs + 1) * 4 <= 65536, name


def test_ordered_gemv_without_an_ordered_shape_is_refused():
    """a gate/up whose SwiGLU epilogue fixes the row-blocks per iteration (gs / (rb / 2)) with too many groups
    for LDS has no ordered shape: llama2.c .bin at dim 8192 (8-row blocks, groups of 64) and a .qwb at dim
    8192 in the strict mode (16-row blocks, groups of 32) are refused (grid 0), not summed out of order; the
    same .qwb matrix in the fast mode and a drop-in GEMV (64-row blocks, one row per lane) keep a shape"""
    assert gemv_shape(2 * 28672, 8192, 64, 8, 1, 8, 2, 1)[0] == 1
    assert gemv_shape(2 * 29568, 8192, 32, 4, 0, 16, 2, 3)[0] == 1
    assert gemv_shape(2 * 29568, 8192, 32, 4, 0, 16, 2, 0)[0] == 0
    rc, (kw, nb, grid, ordq) = gemv_shape(4096, 65536, 32, 4, 0, 64, 5, 1)
    assert rc == 0 and kw == 1 and ordq == 0 and grid >= 1
    assert gemv_shape(4096, 4096, 48, 4, 0, 64, 5, 1)[0] == -1


def test_synth_is_deterministic(tmp_path):
    for fmt, name in (("qwb", "tiny.qwb"), ("bin", "tiny.bin")):
        p = synth(fmt, str(tmp_path / name), "tiny", 1)
        assert open(p, "rb").read() == open(os.path.join(GOLDEN, name), "rb").read()


def walk_qwb(path):
    """the file walk of qwen.c:237-262 (and tools/qwb_check.py): every array on 64 bytes, size must match"""
    b = open(path, "rb").read()
    assert b[:4] == b"QWB1" and struct.unpack_from("<I", b, 4)[0] == 1
    dim, hid, L, nh, nkv, vocab, head_k, ctx, gs, eb = struct.unpack_from("<10i", b, 8)
    theta, eps = struct.unpack_from("<2f", b, 48)
    kv = dim // nh * nkv
    off = 256
    pad = lambda n: (n + 63) & ~63
    for n in [dim] * (2 * L) + [dim] * L + [kv] * (2 * L) + [dim]:
        off += pad(4 * n)
    head_ids = np.frombuffer(b, np.int32, head_k, off)
    off += pad(4 * head_k)
    for d, n in [(dim, dim)] * L + [(kv, dim)] * (2 * L) + [(dim, dim)] * L + [(hid, dim)] * L + [(dim, hid)] * L + \
            [(hid, dim)] * L:
        off += pad(d * n // 2) + pad(d * n // 16)
    for rows in (head_k, vocab):
        off += pad(rows * dim) + pad(rows * dim // 16)
    return dict(size=len(b), walked=off, head_ids=head_ids, cfg=(dim, hid, L, nh, nkv, vocab, head_k, ctx, gs, eb),
                theta=theta, eps=eps)


def test_qwb_layout_and_head_ids(tmp_path):
    w = walk_qwb(os.path.join(GOLDEN, "tiny.qwb"))
    assert w["walked"] == w["size"]
    ids = w["head_ids"]
    assert (np.diff(ids) > 0).all() and 151643 not in ids and 151645 not in ids
    p = synth("qwb", str(tmp_path / "c3small.qwb"), "c3", 3, "layers=1", "vocab=151936", "head_k=4096")
    w = walk_qwb(p)
    assert w["walked"] == w["size"] and w["cfg"][:7] == (896, 4864, 1, 14, 2, 151936, 4096)
    assert abs(w["theta"] - 1e6) < 1 and abs(w["eps"] - 1e-6) < 1e-12
    assert 151643 not in w["head_ids"] and 151645 not in w["head_ids"] and (np.diff(w["head_ids"]) > 0).all()


def test_q4_generator_follows_q4_0(tmp_path):
    """nibbles are q + 8 of llama.cpp's Q4_0 (d = max/-8): the extreme element of each block quantizes to -8"""
    p = synth("qwb", str(tmp_path / "t.qwb"), "tiny", 9)
    b = open(p, "rb").read()
    dim = 128
    L = 2
    kv = 64
    off = 256
    pad = lambda n: (n + 63) & ~63
    off += pad(4 * dim) * 2 * L + pad(4 * dim) * L + pad(4 * kv) * 2 * L + pad(4 * dim) + pad(4 * 256)
    w = np.frombuffer(b, np.uint8, dim * dim // 2, off)
    s = np.frombuffer(b, np.float16, dim * dim // 32, off + pad(dim * dim // 2))
    v = np.empty(dim * dim, np.int8)
    v[0::2], v[1::2] = w & 15, w >> 4
    v = np.where(v >= 8, v - 16, v).reshape(-1, 32)
    assert ((v == -8).any(1)).all()          # the block's largest-magnitude value maps to -8
    assert (np.abs(s.astype(np.float32)) > 0).all()


def test_bin_layout(tmp_path):
    b = open(os.path.join(GOLDEN, "tiny.bin"), "rb").read()
    magic, ver, dim, hid, L, nh, nkv, vocab, seq, shared, gs = struct.unpack_from("<Ii7iBi", b, 0)
    assert magic == 0x616B3432 and ver == 2 and shared == 1 and gs == 32
    kv = dim * nkv // nh
    size = 256 + 4 * (2 * L * dim + dim)
    for nel in [vocab * dim] + [dim * dim] * L + [dim * kv] * (2 * L) + [dim * dim] * L + [dim * hid] * (3 * L):
        size += nel + nel // gs * 4
    assert size == len(b)
