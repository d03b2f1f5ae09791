"""Shared test helpers: the package bindings, the oracle (oracle/liboracle.so, the CPU checker) and the
reference's own functions (oracle/_ref/, present where the reference sources were available to build them)."""
import ctypes as C
import importlib.util
import os
import subprocess

import numpy as np

TESTS = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(TESTS)
GOLDEN = os.path.join(TESTS, "golden")
PKG_DIR = os.path.join(REPO, "local-llama-pynq-z2_amd")
REF_DIR = os.path.join(REPO, "oracle", "_ref")
SYNTH = os.path.join(PKG_DIR, "host", "synth")

_pkg = None
_oracle = None


def pkg():
    global _pkg
    if _pkg is None:
        spec = importlib.util.spec_from_file_location("llm_hip", os.path.join(PKG_DIR, "__init__.py"))
        _pkg = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(_pkg)
    return _pkg


def ptr(a):
    return a.ctypes.data_as(C.c_void_p)


def oracle():
    global _oracle
    if _oracle is None:
        path = os.path.join(REPO, "oracle", "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} missing: run make -C oracle")
        L = C.CDLL(path)
        vp, i32 = C.c_void_p, C.c_int
        L.or_f16.restype = C.c_float
        L.or_f16.argtypes = [C.c_uint16]
        L.or_f32_to_f16.restype = C.c_uint16
        L.or_f32_to_f16.argtypes = [C.c_float]
        L.or_quantize_qwen.argtypes = [vp, vp, vp, i32]
        L.or_quantize_runq.argtypes = [vp, vp, vp, i32, i32]
        L.or_matvec4.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32]
        L.or_matvec4_groups.argtypes = [vp, vp, vp, i32, i32, i32]
        L.or_matvec_runq.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32]
        L.or_matvec_runq_groups.argtypes = [vp, vp, vp, i32, i32, i32]
        L.or_rmsnorm.argtypes = [vp, vp, vp, i32, C.c_float]
        L.or_softmax.argtypes = [vp, i32]
        L.or_expf.argtypes = [vp, i32, vp]
        L.or_rope_angles.argtypes = [vp, vp, i32, i32, C.c_float]
        L.or_rope_neox.argtypes = [vp, i32, i32, vp, vp]
        L.or_rope_runq.argtypes = [vp, vp, i32, i32, i32, i32]
        L.or_argmax.argtypes = [vp, i32]
        L.or_random_u32.restype = C.c_uint
        L.or_random_u32.argtypes = [C.POINTER(C.c_ulonglong)]
        L.or_random_f32.restype = C.c_float
        L.or_random_f32.argtypes = [C.POINTER(C.c_ulonglong)]
        L.or_sample.argtypes = [vp, i32, C.c_float, C.c_float, C.POINTER(C.c_ulonglong)]
        L.or_open.restype = vp
        L.or_open.argtypes = [C.c_char_p, i32]
        L.or_forward.restype = C.POINTER(C.c_float)
        L.or_forward.argtypes = [vp, i32, i32]
        L.or_n_logits.argtypes = [vp]
        L.or_head_ids.restype = C.POINTER(C.c_int32)
        L.or_head_ids.argtypes = [vp]
        L.or_ctx.argtypes = [vp]
        L.or_kind.argtypes = [vp]
        L.or_generate_greedy.argtypes = [vp, vp, i32, i32, vp, i32]
        L.or_close.argtypes = [vp]
        _oracle = L
    return _oracle


class OracleModel:
    def __init__(self, path, ctx=1024):
        self.L = oracle()
        self.h = self.L.or_open(os.fsencode(path), ctx)
        assert self.h, f"oracle cannot open {path}"
        self.n = self.L.or_n_logits(self.h)
        hid = self.L.or_head_ids(self.h)
        self.head_ids = np.ctypeslib.as_array(hid, shape=(self.n,)).copy() if hid else np.arange(self.n)

    def forward(self, token, pos):
        return np.ctypeslib.as_array(self.L.or_forward(self.h, int(token), int(pos)), shape=(self.n,)).copy()

    def generate(self, prompt, steps):
        p = np.asarray(prompt, np.int32)
        out = np.zeros(4096, np.int32)
        k = self.L.or_generate_greedy(self.h, ptr(p), len(p), steps, ptr(out), out.size)
        return out[:k].copy()

    def close(self):
        if self.h:
            self.L.or_close(self.h)
            self.h = None


def ref_lib(name):
    """oracle/_ref/libref_<name>.so (the reference's own functions), or None when not built"""
    path = os.path.join(REF_DIR, f"libref_{name}.so")
    if not os.path.exists(path):
        return None
    return C.CDLL(path)


def synth(fmt, path, preset, seed=1, *overrides):
    subprocess.run([SYNTH, fmt, path, preset, str(seed), *overrides], check=True, capture_output=True)
    return path


def rel_err(a, b):
    """max |a - b| relative to the largest |b| (the logits-vector scale)"""
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def q4_weights(rng, d, n):
    return rng.integers(0, 256, size=d * n // 2, dtype=np.uint8)


def f16_scales(rng, count, special_rows=0, ng=1):
    """random sign, exponent 5..10, random mantissa (hls4/matvec4_tb.cpp:88-97); with special_rows,
    row i's scales get exponent field i % 31: zero, subnormals, up to 65504"""
    if special_rows:
        e = (np.arange(count) // ng) % 31
    else:
        e = rng.integers(5, 11, size=count)
    return ((rng.integers(0, 2, size=count) << 15) | (e << 10) | rng.integers(0, 1024, size=count)).astype(np.uint16)


def unpack_q4(w, d, n):
    """signed int4 values of a .qwb plane (element 2i in the low nibble of byte i)"""
    b = np.asarray(w, np.uint8).reshape(d, n // 2)
    lo, hi = (b & 15).astype(np.int16), (b >> 4).astype(np.int16)
    v = np.empty((d, n), np.int16)
    v[:, 0::2], v[:, 1::2] = lo, hi
    return np.where(v >= 8, v - 16, v)


def exact_terms(wvals, ws_f32, xq, xs, gs=32):
    """per-row exact reference in float64 and the sum of |term| (hls4/matvec4_tb.cpp:67-77)"""
    d, n = wvals.shape
    ng = n // gs
    isum = (wvals.reshape(d, ng, gs).astype(np.int64) * xq.reshape(1, ng, gs).astype(np.int64)).sum(2)
    t = isum * ws_f32.reshape(d, ng).astype(np.float64) * xs.reshape(1, ng).astype(np.float64)
    return t.sum(1), np.abs(t).sum(1), isum
