"""ctypes bindings of libmatvec_hip.so, the MI355X replacement for the reference's FPGA backend.

The library is C (include/matvec_fpga.h: the reference's six-function driver API; include/llm_hip.h: the
device-resident token loop).  These bindings are what the Python tests and bench.py call; the C hosts in
host/ and the reference's own hosts link the library directly.  Nothing here computes: every call goes
through the C ABI, and loading fails loudly when the built library is missing.

The directory name is not a Python identifier, so callers load this file by path, e.g.
    spec = importlib.util.spec_from_file_location("llm_hip", ".../local-llama-pynq-z2_amd/__init__.py")
"""
import ctypes as C
import os

import numpy as np

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
LIB_PATH = os.path.join(PKG_DIR, "libmatvec_hip.so")
HOST_DIR = os.path.join(PKG_DIR, "host")
MAX_N = 32768

_lib = None


class LlmInfo(C.Structure):
    _fields_ = [("kind", C.c_int), ("dim", C.c_int), ("hidden_dim", C.c_int), ("n_layers", C.c_int),
                ("n_heads", C.c_int), ("n_kv_heads", C.c_int), ("vocab_size", C.c_int), ("n_logits", C.c_int),
                ("ctx", C.c_int), ("group_size", C.c_int), ("rope_theta", C.c_float), ("rms_eps", C.c_float),
                ("gemv_bytes_per_token", C.c_double), ("weight_bytes", C.c_double)]


class LlmTiming(C.Structure):
    _fields_ = [("n_prompt", C.c_int), ("n_generated", C.c_int), ("n_forward", C.c_int),
                ("prompt_ms", C.c_double), ("decode_ms", C.c_double)]


class LlmKernelStat(C.Structure):
    _fields_ = [("name", C.c_char * 40), ("launches", C.c_int), ("total_ms", C.c_double),
                ("bytes_per_launch", C.c_double)]


def build_hint():
    return "build it first: python -c 'import __graft_entry__ as g; g.build()' (or make -C local-llama-pynq-z2_amd)"


def lib():
    """The loaded libmatvec_hip.so, with argument types set.  Raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing; {build_hint()}")
    L = C.CDLL(LIB_PATH)
    u64, i32, vp, sz = C.c_uint64, C.c_int, C.c_void_p, C.c_size_t
    L.fpga_open.restype = i32
    L.fpga_alloc.restype = vp
    L.fpga_alloc.argtypes = [sz, C.POINTER(u64)]
    L.fpga_alloc_try.restype = vp
    L.fpga_alloc_try.argtypes = [sz, C.POINTER(u64)]
    L.fpga_matvec.argtypes = [u64, u64, u64, u64, u64, i32, i32, i32]
    L.fpga_matvec.restype = i32
    L.fpga_matvec4.argtypes = [u64, u64, u64, u64, u64, i32, i32, i32]
    L.fpga_matvec4.restype = i32
    L.fpga_close.restype = None
    L.llm_open.restype = vp
    L.llm_open.argtypes = [C.c_char_p, i32]
    L.llm_get_info.argtypes = [vp, C.POINTER(LlmInfo)]
    L.llm_head_ids.restype = C.POINTER(C.c_int32)
    L.llm_head_ids.argtypes = [vp]
    L.llm_forward.argtypes = [vp, i32, i32, vp]
    L.llm_generate.argtypes = [vp, vp, i32, i32, vp, vp, C.POINTER(LlmTiming)]
    L.llm_continue.argtypes = [vp, i32, vp, i32, i32, i32, vp, C.POINTER(LlmTiming)]
    L.llm_decode_replay.argtypes = [vp, i32, C.POINTER(C.c_double)]
    L.llm_profile.argtypes = [vp, i32, C.POINTER(LlmKernelStat), i32]
    L.llm_profile_graph.argtypes = [vp, i32, i32, C.POINTER(LlmKernelStat), i32, C.POINTER(C.c_double)]
    L.llm_prefill.argtypes = [vp, vp, i32, vp]
    L.llm_close.argtypes = [vp]
    L.llm_close.restype = None
    L.llm_read_state.argtypes = [vp, i32, i32, vp, sz]
    L.mvh_quantize.argtypes = [vp, i32, i32, i32, vp, vp]
    L.mvh_group_dots.argtypes = [vp, vp, i32, i32, i32, i32, vp]
    L.mvh_prefill_gemm.argtypes = [vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, vp]
    L.llm_set_prefill.argtypes = [vp, i32]
    L.llm_set_sampler.argtypes = [vp, C.c_float, C.c_float, C.c_ulonglong]
    L.llm_sampler_state.argtypes = [vp, C.POINTER(C.c_ulonglong)]
    L.mvh_sample.argtypes = [vp, i32, i32, C.c_float, C.c_float, C.POINTER(C.c_ulonglong), vp]
    L.mvh_sample_noalloc.argtypes = [vp, i32, i32, C.c_float, C.c_float, C.POINTER(C.c_ulonglong), vp]
    L.mvh_sample_strict.argtypes = [vp, i32, i32, C.c_float, C.c_float, C.POINTER(C.c_ulonglong), vp]
    L.mvh_sample_strict_skew.argtypes = [vp, i32, i32, C.c_float, C.c_float, C.POINTER(C.c_ulonglong), vp, i32]
    L.mvh_ref_expf.argtypes = [vp, i32, vp]
    L.mvh_read_floor.argtypes = [C.c_size_t, i32, i32, i32, i32, C.POINTER(C.c_float)]
    L.mvh_ref_expf_host.argtypes = [vp, i32, vp]
    L.mvh_seq_sum.argtypes = [vp, i32, i32, i32, vp]
    L.llm_set_strict.argtypes = [vp, i32]
    L.llm_get_strict.argtypes = [vp]
    _lib = L
    return L


def _ptr(a):
    return a.ctypes.data_as(C.c_void_p)


# ---- test hooks -----------------------------------------------------------------------------------------

def quantize(x, flavor, gs=32):
    """Device activation quantization: flavor 0 = qwen.c:354-364, 1 = runq.c:244-270."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    q = np.empty(x.size, np.int8)
    s = np.empty(x.size // gs, np.float32)
    if lib().mvh_quantize(_ptr(x), x.size, flavor, gs, _ptr(q), _ptr(s)) != 0:
        raise RuntimeError("mvh_quantize failed")
    return q, s


def group_dots(w, xq, n, d, bits, gs=32):
    """Exact int32 group sums through the GEMV's dot-product code: [d, n/gs]."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    xq = np.ascontiguousarray(xq, dtype=np.int8)
    out = np.empty((d, n // gs), np.int32)
    if lib().mvh_group_dots(_ptr(w), _ptr(xq), n, d, bits, gs, _ptr(out)) != 0:
        raise RuntimeError("mvh_group_dots failed")
    return out


def prefill_gemm(w, ws, xq, xs, M, n, d, bits, gs=32, rb=16, shape=0):
    """The prefill GEMM (int8 MFMA) on caller data: [M, d] float32.  bits 4/8: qwen planes with fp16 scales;
    bits 0: runq int8 with fp32 scales, group gs.  shape: 0 the library's choice, 10 TA + TB one wave per
    16 TA rows x 16 TB tokens (TA 1, 2; TB 1, 2, 4)."""
    w = np.ascontiguousarray(w).view(np.uint8)
    ws = np.ascontiguousarray(ws)
    xq = np.ascontiguousarray(xq, dtype=np.int8)
    xs = np.ascontiguousarray(xs, dtype=np.float32)
    y = np.empty((M, d), np.float32)
    if lib().mvh_prefill_gemm(_ptr(w), _ptr(ws), _ptr(xq), _ptr(xs), M, n, d, bits, gs, rb, shape, _ptr(y)) != 0:
        raise RuntimeError("mvh_prefill_gemm failed")
    return y


def sample(logits, temperature, topp, seed, noalloc=False, strict=False, skew=None):
    """The on-device sampler on caller logits [count, n] (or [n]), drawn in order with one RNG state seeded by
    `seed`: (rows, the advanced RNG state).  noalloc: the entry point that allocates no device memory; strict:
    the strict mode's draw (the reference's sample() operation for operation); skew: the strict draw with its
    segment predictions moved by that many ulps (its term-by-term path)."""
    lg = np.ascontiguousarray(np.atleast_2d(logits), dtype=np.float32)
    rows = np.empty(lg.shape[0], np.int32)
    st = C.c_ulonglong(seed)
    args = [_ptr(lg), lg.shape[1], lg.shape[0], temperature, topp, C.byref(st), _ptr(rows)]
    if skew is not None:
        name, args = "mvh_sample_strict_skew", args + [skew]
    else:
        name = "mvh_sample_strict" if strict else "mvh_sample_noalloc" if noalloc else "mvh_sample"
    if getattr(lib(), name)(*args) != 0:
        raise RuntimeError(name + " failed")
    return rows, st.value


def read_floor(nbytes, copies, blocks, nt=True, reps=20):
    """µs per launch of a plain streaming read of nbytes (one launch per distinct buffer, in a graph)"""
    us = C.c_float(0)
    if lib().mvh_read_floor(nbytes, copies, blocks, int(nt), reps, C.byref(us)) != 0:
        raise RuntimeError("mvh_read_floor failed")
    return us.value


def seq_sum(x, which="block", threads=512):
    """the strict mode's sequential fp32 sum ((0 + x[0]) + x[1]) + ... on the device: which "block" (the block's
    speculative segments, `threads` threads), "wave" (one wave's chain) or "thread" (one thread's chain)"""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(1, np.float32)
    w = {"block": 0, "wave": 1, "thread": 2}[which]
    if lib().mvh_seq_sum(_ptr(x), x.size, w, threads, _ptr(out)) != 0:
        raise RuntimeError("mvh_seq_sum failed")
    return out[0]


def ref_expf(x, host=False):
    """expf as the reference's C library evaluates it (the strict mode's softmax and SiLU): on the device, or
    the same restatement compiled for the host CPU with host=True"""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    fn = lib().mvh_ref_expf_host if host else lib().mvh_ref_expf
    if fn(_ptr(x), x.size, _ptr(y)) != 0:
        raise RuntimeError("mvh_ref_expf failed")
    return y


# ---- drop-in driver API -----------------------------------------------------------------------------------

class DropIn:
    """The reference's driver API (fpga_open / fpga_alloc / fpga_matvec[4] / fpga_close) through ctypes."""

    def __init__(self):
        self.L = lib()
        if self.L.fpga_open() != 0:
            raise RuntimeError("fpga_open failed")
        self.bufs = []

    def alloc(self, nbytes):
        """(numpy uint8 view of the host buffer, device address)"""
        phys = C.c_uint64(0)
        p = self.L.fpga_alloc(nbytes, C.byref(phys))
        if not p:
            raise MemoryError("fpga_alloc failed")
        view = np.ctypeslib.as_array((C.c_uint8 * nbytes).from_address(p))
        self.bufs.append(view)
        return view, phys.value

    def put(self, arr, align=64):
        """copy an array into a new buffer; returns (view, device address)"""
        b = np.ascontiguousarray(arr).view(np.uint8).reshape(-1)
        view, phys = self.alloc(max(b.size, 1))
        view[:b.size] = b
        return view, phys

    def matvec4(self, w, ws, xq, xs, out, n, d, wbits):
        return self.L.fpga_matvec4(w, ws, xq, xs, out, n, d, wbits)

    def matvec(self, wq, ws, xq, xs, out, n, d, gs):
        return self.L.fpga_matvec(wq, ws, xq, xs, out, n, d, gs)

    def close(self):
        self.bufs = []
        self.L.fpga_close()


# ---- device-resident model -----------------------------------------------------------------------------------

class Model:
    """A .qwb or llama2.c .bin model resident in HBM (llm_open)."""

    def __init__(self, path, ctx=1024):
        self.L = lib()
        self.h = self.L.llm_open(os.fsencode(path), ctx)
        if not self.h:
            raise RuntimeError(f"llm_open({path}) failed")
        self.info = LlmInfo()
        self.L.llm_get_info(self.h, C.byref(self.info))
        hid = self.L.llm_head_ids(self.h)
        n = self.info.n_logits
        self.head_ids = np.ctypeslib.as_array(hid, shape=(n,)).copy() if hid else np.arange(n, dtype=np.int32)

    def forward(self, token, pos):
        lg = np.empty(self.info.n_logits, np.float32)
        if self.L.llm_forward(self.h, int(token), int(pos), _ptr(lg)) != 0:
            raise RuntimeError("llm_forward failed")
        return lg

    def generate(self, prompt, max_new, logits=False):
        """greedy ids (and the logits of every position run, when asked)"""
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.empty(max_new, np.int32)
        lg = np.empty((len(p) + max_new) * self.info.n_logits, np.float32) if logits else None
        t = LlmTiming()
        n = self.L.llm_generate(self.h, _ptr(p), len(p), max_new, _ptr(out), _ptr(lg) if logits else None,
                                C.byref(t))
        if n < 0:
            raise RuntimeError("llm_generate failed")
        res = {"ids": out[:n].copy(), "timing": t}
        if logits:
            res["logits"] = lg[:t.n_forward * self.info.n_logits].reshape(t.n_forward, self.info.n_logits)
        return res

    def continue_at(self, pos0, tokens, max_new, stop_id=-1):
        """the tokens forced from position pos0 over the cache earlier calls left, then up to max_new generated
        ids until stop_id (-1: the format's stop ids)"""
        p = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.empty(max_new, np.int32)
        t = LlmTiming()
        n = self.L.llm_continue(self.h, pos0, _ptr(p), len(p), max_new, stop_id, _ptr(out), C.byref(t))
        if n < 0:
            raise RuntimeError("llm_continue failed")
        return {"ids": out[:n].copy(), "timing": t}

    def decode_replay(self, steps):
        ms = C.c_double(0)
        if self.L.llm_decode_replay(self.h, steps, C.byref(ms)) != 0:
            raise RuntimeError("llm_decode_replay failed")
        return ms.value

    def profile(self, steps):
        st = (LlmKernelStat * 16)()
        n = self.L.llm_profile(self.h, steps, st, 16)
        if n < 0:
            raise RuntimeError("llm_profile failed")
        return [{"name": st[i].name.decode(), "launches": st[i].launches, "total_ms": st[i].total_ms,
                 "bytes_per_launch": st[i].bytes_per_launch} for i in range(n)]

    def profile_graph(self, steps, rounds=3):
        """per-kernel-kind device time inside the replayed step graph (see llm_profile_graph); returns
        (records, median step ms)"""
        st = (LlmKernelStat * 16)()
        step = C.c_double(0.0)
        n = self.L.llm_profile_graph(self.h, steps, rounds, st, 16, C.byref(step))
        if n < 0:
            raise RuntimeError("llm_profile_graph failed")
        return [{"name": st[i].name.decode(), "launches": st[i].launches, "total_ms": st[i].total_ms,
                 "bytes_per_launch": st[i].bytes_per_launch} for i in range(n)], step.value

    def read_state(self, which, layer=0, count=None):
        n = self.info.dim if which == 0 else self.info.ctx * (self.info.dim // self.info.n_heads * self.info.n_kv_heads)
        if count is not None:
            n = min(n, count)
        out = np.empty(n, np.float32)
        if self.L.llm_read_state(self.h, which, layer, _ptr(out), n) != 0:
            raise RuntimeError("llm_read_state failed")
        return out

    def set_sampler(self, temperature, topp=0.9, seed=1):
        """temperature > 0: generate() draws tokens on the device (temperature, top-p, xorshift coin from
        seed); 0: greedy"""
        if self.L.llm_set_sampler(self.h, temperature, topp, seed) != 0:
            raise RuntimeError("llm_set_sampler failed")

    def sampler_state(self):
        st = C.c_ulonglong(0)
        if self.L.llm_sampler_state(self.h, C.byref(st)) != 0:
            raise RuntimeError("llm_sampler_state failed")
        return st.value

    def set_strict(self, on):
        """reference-order mode: logits bitwise those of the reference's strict-IEEE build (llm_set_strict)"""
        if self.L.llm_set_strict(self.h, 1 if on else 0) != 0:
            raise RuntimeError("llm_set_strict failed")

    @property
    def strict(self):
        return self.L.llm_get_strict(self.h) == 1

    def set_prefill(self, on):
        """whether generate() runs the prompt as one batched prefill (default) or one step per position"""
        self.L.llm_set_prefill(self.h, 1 if on else 0)

    def prefill(self, ids):
        """batched prefill of positions 0..len(ids)-1; the logits of the last position"""
        p = np.ascontiguousarray(ids, dtype=np.int32)
        lg = np.empty(self.info.n_logits, np.float32)
        if self.L.llm_prefill(self.h, _ptr(p), len(p), _ptr(lg)) != 0:
            raise RuntimeError("llm_prefill failed")
        return lg

    def close(self):
        if self.h:
            self.L.llm_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
