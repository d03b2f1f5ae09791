"""The strict mode's draw on the MI355X: the reference's sample() operation for operation.

Bar: bitwise.  Every draw's row and the RNG state after it equal those of the reference's own sample()
(qwen.c:647-654 compiled from the reference's source into oracle/_ref/libref_qwen.so, refq_sample) and of the
oracle's restatement (or_sample), over flat, moderate, peaked, tie-heavy and masked logits, from a few hundred
rows to the Qwen2 vocabulary (152,064), for the plain walk and for top-p.  The draw's sequential sums run
through speculative segments whose misses fall back to term-by-term adds (both paths are exact); the
flat logits of a large vocabulary exercise long sums, the tie-heavy ones long runs of equal keys in the
sort.  Then a whole sampled generation in the strict mode against the reference program's stream
(qwen -t 0.7 -p 0.8 -s 42 on a Qwen2-0.5B-shape model)."""
import ctypes as C
import os
import subprocess

import numpy as np
import pytest

from helpers import REF_DIR, oracle, pkg, ptr, ref_lib, synth
from test_gpu_sample import logit_sets

pytestmark = pytest.mark.gpu


def reference_rows(fn, logits, temperature, topp, seed):
    st = C.c_ulonglong(seed)
    rows = []
    for lg in logits:
        x = np.array(lg, np.float32)
        rows.append(fn(ptr(x), x.size, C.c_float(temperature), C.c_float(topp), C.byref(st)))
    return np.array(rows), st.value


@pytest.mark.parametrize("n", [256, 4097, 65536, 152064])
@pytest.mark.parametrize("topp", [0.0, 0.5, 0.8, 0.95, 1.0])
def test_strict_draw_is_the_reference_sample(n, topp):
    ref = ref_lib("qwen")
    fns = [("oracle", oracle().or_sample)] + ([("reference", ref.refq_sample)] if ref else [])
    rng = np.random.default_rng(n + int(topp * 1000))
    count = 4 if n > 60000 else 8
    print(f"n={n} topp={topp}", flush=True)
    for kind, lg in logit_sets(n, count, rng).items():
        for temp, seed in ((0.7, 42), (1.0, 2**63 + 5), (1.6, 9)):
            got, st_g = pkg().sample(lg, temp, topp, seed, strict=True)
            for name, fn in fns:
                want, st_w = reference_rows(fn, lg, temp, topp, seed)
                assert st_g == st_w, (name, kind, temp)
                assert list(got) == list(want), (name, kind, temp, list(got), list(want))


@pytest.mark.parametrize("skew", [12, 40, -300])
@pytest.mark.parametrize("n", [4097, 152064])
def test_strict_draw_term_by_term_path(n, skew):
    """predicted segment starts moved by `skew` ulps: some starts (12) or none (40, -300) among the candidates,
    so the walks take the term-by-term path for those segments; the draws stay the reference's"""
    rng = np.random.default_rng(n + 31 * abs(skew))
    lg = logit_sets(n, 3, rng)
    for kind in ("flat", "moderate", "ties"):
        for topp in (0.0, 0.8):
            got, st_g = pkg().sample(lg[kind], 0.9, topp, 7, skew=skew)
            want, st_w = reference_rows(oracle().or_sample, lg[kind], 0.9, topp, 7)
            assert st_g == st_w and list(got) == list(want), (kind, topp)


def test_the_fast_draw_differs_where_the_strict_one_does_not():
    """the fast mode's exact fixed-point sums misplace some draws of a large flat vocabulary that the
    reference's fp32 sums place elsewhere; the strict draw follows the reference in all of them"""
    rng = np.random.default_rng(5)
    lg = rng.standard_normal((24, 152064)).astype(np.float32) * 0.05
    want, _ = reference_rows(oracle().or_sample, lg, 1.0, 0.0, 3)
    fast, _ = pkg().sample(lg, 1.0, 0.0, 3)
    strict, _ = pkg().sample(lg, 1.0, 0.0, 3, strict=True)
    print("fast draws off the reference's:", int(np.sum(fast != want)), "of", len(want))
    assert list(strict) == list(want)
    assert np.any(fast != want)


def test_strict_draw_all_equal_logits():
    """n equal probabilities: every row a candidate, the sort keeps row order, and the reference's drifting
    fp32 running sum of 0.001 decides the row"""
    lg = np.zeros((16, 1000), np.float32)
    for topp in (0.5, 0.0):
        got, st_g = pkg().sample(lg, 1.0, topp, 99, strict=True)
        want, st_w = reference_rows(oracle().or_sample, lg, 1.0, topp, 99)
        assert st_g == st_w and list(got) == list(want)


def test_strict_sampled_generation_matches_reference_stream(tmp_path):
    """the Qwen2-0.5B-shape model (24 layers, 65536-row head) sampled in the strict mode (temperature 0.7,
    top-p 0.8, seed 42) through the step graph: the reference's qwen.c (strict IEEE build) prints the same ids"""
    exe = os.path.join(REF_DIR, "qwen")
    if not os.path.exists(exe):
        pytest.skip(f"{exe} not built")
    from test_lib import walk_qwb
    p = synth("qwb", str(tmp_path / "c3.qwb"), "c3", 41)
    hid = walk_qwb(p)["head_ids"]
    prompt = [int(v) for v in np.random.default_rng(42).choice(hid, 24, replace=False)]
    r = subprocess.run([exe, p, "--ids", ",".join(map(str, prompt)), "-t", "0.7", "-p", "0.8", "-s", "42", "-n", "32",
                        "-c", "128"], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    want = [int(v) for v in r.stdout.strip().split(",") if v]
    m = pkg().Model(p, 128)
    m.set_strict(True)
    m.set_sampler(0.7, 0.8, 42)
    got = list(m.generate(prompt, 32)["ids"])
    m.close()
    print("reference", want, "\ndevice   ", got)
    assert got == want
