"""Writes the committed golden fixtures of tests/golden/ from the reference's own compiled C.

Run from the repository root after `make -C oracle all ref` and `make -C local-llama-pynq-z2_amd host/synth`
(it needs oracle/_ref/, which is built from the reference sources):
    python tests/golden/make_golden.py
The reference's tests hold no golden vectors (its checks compare the FPGA kernel with the CPU function on
the fly), so every expected output here comes from running the reference code itself:
  - tiny.qwb / tiny.bin: seeded synthetic models (host/synth), small enough to commit,
  - *_ref.logits / *_ref.json: the reference binaries' --logits dump, greedy ids and sampled ids (temperature,
    top-p or the plain cdf walk, seeded xorshift coin) on those models,
  - ops.npz: the reference's quantize() and matmul() (qwen.c and runq.c, through oracle/_ref/libref_*.so)
    on seeded inputs, crafted edge groups and the reference testbench's special fp16 scales.
"""
import ctypes as C
import json
import os
import subprocess
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
REF = os.path.join(REPO, "oracle", "_ref")
SYNTH = os.path.join(REPO, "local-llama-pynq-z2_amd", "host", "synth")

QWEN_PROMPT = [5, 77, 300, 12]
BIN_PROMPT = [1, 50, 60, 70]


def run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True, check=True)
    return r.stdout.strip(), r.stderr


def ptr(a):
    return a.ctypes.data_as(C.c_void_p)


def quantize_inputs(rng):
    """seeded groups plus crafted edge groups (n multiple of 64)"""
    xs = [rng.standard_normal(64 * 8).astype(np.float32) * 3]
    g = np.zeros(64, np.float32)
    xs.append(g)                                                   # all zero: scale 0, q 0
    t = np.linspace(-1, 1, 64).astype(np.float32)
    t[0] = 127.0
    t[1:] = np.arange(63, dtype=np.float32) - 31.5                 # halves: roundf away from zero
    xs.append(t)
    xs.append(np.full(64, 1e-39, np.float32))                      # subnormal inputs
    xs.append(np.array([(-1) ** i * 1e-40 * (i + 1) for i in range(64)], np.float32))
    xs.append((rng.standard_normal(64) * 1e30).astype(np.float32))  # huge values
    xs.append(np.where(np.arange(64) % 2 == 0, 1.0, -1.0).astype(np.float32) * 0.5)
    return np.concatenate(xs)


def main():
    out = {}
    os.chdir(REPO)
    tq, tb = os.path.join(HERE, "tiny.qwb"), os.path.join(HERE, "tiny.bin")
    run([SYNTH, "qwb", tq, "tiny", "1"])
    run([SYNTH, "bin", tb, "tiny", "1"])
    ids, err = run([os.path.join(REF, "qwen"), tq, "--ids", ",".join(map(str, QWEN_PROMPT)), "-t", "0", "-n", "20",
                    "-c", "64", "--logits", os.path.join(HERE, "tiny_qwb_ref.logits")])
    out["qwb"] = {"prompt": QWEN_PROMPT, "ids": [int(v) for v in ids.split(",")], "n": 20, "ctx": 64}
    ids, err = run([os.path.join(REF, "qwen"), tq, "--ids", ",".join(map(str, QWEN_PROMPT)), "-t", "0.9", "-p",
                    "0.9", "-s", "42", "-n", "20", "-c", "64"])
    out["qwb_sampled"] = {"prompt": QWEN_PROMPT, "ids": [int(v) for v in ids.split(",")], "n": 20, "ctx": 64,
                          "t": 0.9, "p": 0.9, "seed": 42}
    ids, err = run([os.path.join(REF, "qwen"), tq, "--ids", ",".join(map(str, QWEN_PROMPT)), "-t", "1.0", "-p",
                    "1.0", "-s", "7", "-n", "20", "-c", "64"])
    out["qwb_sampled_mult"] = {"prompt": QWEN_PROMPT, "ids": [int(v) for v in ids.split(",")], "n": 20, "ctx": 64,
                               "t": 1.0, "p": 1.0, "seed": 7}
    ids, err = run([os.path.join(REF, "runq_ids"), tb, "--ids", ",".join(map(str, BIN_PROMPT)), "-n", "32",
                    "--logits", os.path.join(HERE, "tiny_bin_ref.logits")])
    out["bin"] = {"prompt": BIN_PROMPT, "ids": [int(v) for v in ids.split(",")], "steps": 32}
    ids, err = run([os.path.join(REF, "runq_ids"), tb, "--ids", ",".join(map(str, BIN_PROMPT)), "-n", "32",
                    "-t", "0.8", "-p", "0.9", "-s", "5"])
    out["bin_sampled"] = {"prompt": BIN_PROMPT, "ids": [int(v) for v in ids.split(",")], "steps": 32,
                          "t": 0.8, "p": 0.9, "seed": 5}
    with open(os.path.join(HERE, "tiny_ref.json"), "w") as f:
        json.dump(out, f, indent=1)

    # per-function vectors from the reference functions
    Q = C.CDLL(os.path.join(REF, "libref_qwen.so"))
    R = C.CDLL(os.path.join(REF, "libref_runq.so"))
    Q.refq_f16.restype = C.c_float
    Q.refq_f16.argtypes = [C.c_uint16]
    rng = np.random.default_rng(20261201)
    x = quantize_inputs(rng)
    qq, qs = np.empty(x.size, np.int8), np.empty(x.size // 32, np.float32)
    Q.refq_quantize(ptr(qq), ptr(qs), ptr(x), C.c_int(x.size))
    rq32, rs32 = np.empty(x.size, np.int8), np.empty(x.size // 32, np.float32)
    R.refr_quantize(ptr(rq32), ptr(rs32), ptr(x), C.c_int(x.size), C.c_int(32))
    rq64, rs64 = np.empty(x.size, np.int8), np.empty(x.size // 64, np.float32)
    R.refr_quantize(ptr(rq64), ptr(rs64), ptr(x), C.c_int(x.size), C.c_int(64))
    f16 = np.array([Q.refq_f16(h) for h in range(0, 65536, 7) if ((h >> 10) & 31) != 31], np.float32)
    # matmul cases: (n, d, bits) for qwen, (n, d, gs) for runq; special scales give row i exponent i % 31
    arrays = dict(q_x=x, qwen_q=qq, qwen_s=qs, runq32_q=rq32, runq32_s=rs32, runq64_q=rq64, runq64_s=rs64,
                  f16_bits=np.array([h for h in range(0, 65536, 7) if ((h >> 10) & 31) != 31], np.uint16),
                  f16_vals=f16)
    for k, (n, d, bits, special) in enumerate([(96, 5, 4, 0), (96, 5, 8, 0), (896, 16, 4, 0), (64, 31, 4, 1),
                                               (64, 31, 8, 1)]):
        w = rng.integers(0, 256, size=d * n * bits // 8, dtype=np.uint8)
        ng = n // 32
        e = (np.arange(d * ng) // ng % 31) if special else rng.integers(5, 11, size=d * ng)
        s = ((rng.integers(0, 2, size=d * ng) << 15) | (e << 10) | rng.integers(0, 1024, size=d * ng)).astype(np.uint16)
        xq = rng.integers(-128, 128, size=n, dtype=np.int8)
        xs = rng.uniform(1e-3, 1e-1, size=ng).astype(np.float32)
        o = np.empty(d, np.float32)
        Q.refq_matmul(ptr(o), ptr(w), ptr(s), C.c_int(n), C.c_int(d), C.c_int(bits), ptr(xq), ptr(xs))
        arrays.update({f"m{k}_w": w, f"m{k}_s": s, f"m{k}_xq": xq, f"m{k}_xs": xs, f"m{k}_out": o,
                       f"m{k}_shape": np.array([n, d, bits], np.int32)})
    for k, (n, d, gs) in enumerate([(96, 7, 32), (288, 64, 32), (768, 32, 64)]):
        wq = rng.integers(-128, 128, size=d * n, dtype=np.int8)
        ws = rng.uniform(1e-4, 2e-2, size=d * n // gs).astype(np.float32)
        xq = rng.integers(-128, 128, size=n, dtype=np.int8)
        xs = rng.uniform(1e-3, 1e-1, size=n // gs).astype(np.float32)
        o = np.empty(d, np.float32)
        R.refr_matmul(ptr(o), ptr(xq), ptr(xs), ptr(wq), ptr(ws), C.c_int(n), C.c_int(d), C.c_int(gs))
        arrays.update({f"r{k}_wq": wq, f"r{k}_ws": ws, f"r{k}_xq": xq, f"r{k}_xs": xs, f"r{k}_out": o,
                       f"r{k}_shape": np.array([n, d, gs], np.int32)})
    np.savez_compressed(os.path.join(HERE, "ops.npz"), **arrays)
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    sys.exit(main())
