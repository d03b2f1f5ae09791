"""The on-device sampler (temperature, softmax, top-p or the plain cdf walk, xorshift64* coin) on the MI355X.

Oracle: or_sample, the CPU restatement of qwen.c:591-654 / runq.c:843-967, pinned to the reference's own
sample() and to the reference binaries' sampled ids (test_oracle.py).

Bar.  The RNG stream is bit-exact (same coins, same final state) and the selection logic is the reference's.
The sampled row is the oracle's except where the reference's own fp32 arithmetic decides: it walks one
sequential fp32 cumulative sum (after a sequential softmax sum), whose rounding error grows like sqrt(n)
ulps over random terms and linearly over repeated equal terms (a tie-heavy vocabulary), while the device
takes segment prefixes plus in-segment walks of at most ceil(n / 1024) terms.  Over a large vocabulary that
error reaches a visible fraction of one row's probability, so a coin close to a cdf boundary can land on a
neighbouring row on one side and not the other.  A differing draw is accepted only if the device's row is
the correct choice in float64 arithmetic (softmax, candidate order, cutoff and cumulative sums of the
reference's algorithm recomputed in float64, within eps = 8e-6, or a row whose probability equals the
correct row's to 1e-5); the reference's sequential softmax sum alone is off by up to ~2e-4 of the total over
such a vocabulary, which rescales every probability it divides;
draws over n = 256 must all be identical, and at least 75% of the draws over n = 4097 except the tie-heavy
ones.  Over 65536 and more rows the reference's own softmax sum and cdf are off by several rows' probability
(it misplaces about a third of its draws there against float64), so only the float64 check applies."""
import ctypes as C
import json
import os

import numpy as np
import pytest

from helpers import GOLDEN, oracle, pkg, ptr

pytestmark = pytest.mark.gpu
META = json.load(open(os.path.join(GOLDEN, "tiny_ref.json")))


def oracle_rows(logits, temperature, topp, seed):
    """the oracle's rows, its final RNG state, and per draw (probabilities, coin)"""
    st = C.c_ulonglong(seed)
    rows, draws = [], []
    for lg in logits:
        x = np.array(lg, np.float32)
        before = C.c_ulonglong(st.value)
        coin = oracle().or_random_f32(C.byref(before))
        rows.append(oracle().or_sample(ptr(x), x.size, C.c_float(temperature), C.c_float(topp), C.byref(st)))
        draws.append((exact_probs(lg, temperature), coin))
    return np.array(rows), st.value, draws


def exact_probs(logits, temperature):
    """the reference's softmax of logits / temperature (the division in fp32, as qwen.c:648) in float64"""
    x = (np.asarray(logits, np.float32) / np.float32(temperature)).astype(np.float64)
    e = np.exp(x - x.max())
    return e / e.sum()


def exact_choice(p, coin, topp, row):
    """whether `row` is the draw of the reference's algorithm evaluated in float64 (p = exact_probs; within eps
    of every cdf decision), see the module docstring"""
    eps = 8e-6
    n = p.size
    if topp <= 0 or topp >= 1:
        cdf = np.cumsum(p)
        lo = cdf[row - 1] if row > 0 else 0.0
        return lo - eps <= coin <= cdf[row] + eps or (row == n - 1 and coin >= cdf[-1] - eps)
    p32 = p.astype(np.float32)
    cand = np.nonzero(p32 >= np.float32((1 - np.float32(topp)) / np.float32(n - 1)))[0]
    order = cand[np.lexsort((cand, -p32[cand]))]
    cdf = np.cumsum(p[order])
    last = min(int(np.searchsorted(cdf, topp, side="right")), cdf.size - 1)
    where = np.nonzero(order == row)[0]
    if where.size == 0:
        return False
    k = int(where[0])
    cuts = [last]  # the cut itself may sit on a boundary: one more or one fewer candidate
    if cdf[last] - topp <= eps and last + 1 < cdf.size:
        cuts.append(last + 1)
    if last > 0 and topp - cdf[last - 1] <= eps:
        cuts.append(last - 1)
    for l in cuts:
        r = coin * cdf[l]
        lo = cdf[k - 1] if k > 0 else 0.0
        if k <= l and lo - eps <= r <= cdf[k] + eps:
            return True
        # an equal-probability neighbour in the order (a swap within rounding)
        j = int(np.searchsorted(cdf, r, side="right"))
        if j < cdf.size and abs(p[order[j]] - p[row]) <= 1e-5 * p[row]:
            return True
    return False


def logit_sets(n, count, rng):
    """flat (near-uniform), moderate, peaked, with exact ties, and with a -inf tail"""
    out = {
        "flat": rng.standard_normal((count, n)).astype(np.float32) * 0.05,
        "moderate": rng.standard_normal((count, n)).astype(np.float32) * 2.0,
        "peaked": rng.standard_normal((count, n)).astype(np.float32) * 12.0,
    }
    t = np.round(rng.standard_normal((count, n)) * 2).astype(np.float32)  # few distinct values: many ties
    out["ties"] = t
    m = rng.standard_normal((count, n)).astype(np.float32) * 3.0
    m[:, n // 2:] = -np.inf
    out["masked"] = m
    return out


# 256 and 4097 rows: one workgroup; 8192 and more: the many-workgroup draw (9999: a last chunk of 15 rows,
# a last vector of 3)
@pytest.mark.parametrize("n", [256, 4097, 8192, 9999, 65536, 152064])
@pytest.mark.parametrize("topp", [0.0, 0.5, 0.9, 0.99, 1.0])
def test_device_sampler_matches_oracle(n, topp):
    rng = np.random.default_rng(n * 7 + int(topp * 100))
    count = 8 if n > 60000 else 12
    for kind, lg in logit_sets(n, count, rng).items():
        same = total = 0
        for temp, seed in ((0.3, 11), (0.9, 12345), (1.7, 2**63 + 5)):
            got, st_g = pkg().sample(lg, temp, topp, seed)
            want, st_o, draws = oracle_rows(lg, temp, topp, seed)
            assert st_g == st_o, (kind, temp)
            for k, (d, o) in enumerate(zip(got, want)):
                if d == o:
                    continue
                p, coin = draws[k]
                print(f"n={n} topp={topp} {kind} T={temp} draw {k}: device {d} oracle {o} (p {p[d]:.3e} / {p[o]:.3e})")
                assert n > 256 and exact_choice(p, coin, topp, int(d)), (kind, temp, k, d, o)
            same += int(np.sum(got == want))
            total += got.size
        if n <= 4097 and kind != "ties":
            assert same >= 0.75 * total, (kind, same, total)


def test_all_equal_logits_take_ties_in_index_order():
    """top-p over n equal probabilities: every row is a candidate and equal probabilities keep row order (as
    the reference's qsort over its row-ordered candidates does for equal keys), so the draw is the row
    floor(coin * cumulative / p) of the prefix.  The reference's fp32 running sum of 0.001 drifts by a
    fraction of a row over 500 terms, so its row can be one off; the device's is the exact one."""
    lg = np.zeros((32, 1000), np.float32)
    got, st_g = pkg().sample(lg, 1.0, 0.5, 99)
    want, st_o, draws = oracle_rows(lg, 1.0, 0.5, 99)
    assert st_g == st_o
    assert np.abs(got - want).max() <= 1
    for row, (p, coin) in zip(got, draws):
        assert exact_choice(p, coin, 0.5, int(row))
    assert got.max() <= 501  # the prefix passes topp = 0.5 after ~500 equal candidates


def test_sampled_generation_over_a_large_vocabulary_matches_the_draws_of_the_same_logits(tmp_path):
    """vocabularies of 8192 rows and more take the many-workgroup draw; inside the step graph it must draw
    what sample() draws from the same logits and seed (sample() itself is held to the oracle above): the
    generated ids are those rows mapped through head_ids.  Top-p, then the plain walk on the same model, then
    top-p again (the sampled step graphs hold one path's launches and are captured again on a switch)"""
    from helpers import synth
    p = synth("qwb", str(tmp_path / "v.qwb"), "c3", 61, "layers=2", "vocab=16384", "head_k=16384")
    m = pkg().Model(p, 128)
    m.set_prefill(False)
    prompt = [int(v) for v in np.random.default_rng(3).integers(0, 16384, 8)]
    hid = np.asarray(m.head_ids)
    for temp, topp, seed in ((0.8, 0.9, 77), (1.1, 1.0, 78), (0.6, 0.5, 79)):
        m.set_sampler(temp, topp, seed)
        r = m.generate(prompt, 12, logits=True)
        ids = list(r["ids"])
        lg = np.asarray(r["logits"])[len(prompt) - 1:len(prompt) - 1 + len(ids)]
        rows, _ = pkg().sample(lg, temp, topp, seed)
        assert [int(hid[k]) for k in rows] == ids, (temp, topp)
    m.close()


@pytest.mark.parametrize("name,prefill", [("qwb_sampled", True), ("qwb_sampled", False), ("qwb_sampled_mult", True),
                                          ("bin_sampled", True)])
def test_sampled_generation_matches_reference_ids(name, prefill):
    """llm_generate with the device sampler in the step graph against the reference binaries' sampled ids;
    the RNG state afterwards is the seed advanced once per generated token"""
    meta = META[name]
    runq = name.startswith("bin")
    m = pkg().Model(os.path.join(GOLDEN, "tiny.bin" if runq else "tiny.qwb"), 1024 if runq else meta["ctx"])
    m.set_prefill(prefill)
    m.set_sampler(meta["t"], meta["p"], meta["seed"])
    max_new = meta["steps"] - len(meta["prompt"]) + 1 if runq else meta["n"]
    r = m.generate(meta["prompt"], max_new)
    state = m.sampler_state()
    m.set_sampler(0.0)
    greedy = m.generate(meta["prompt"], 4)
    m.close()
    assert list(r["ids"]) == meta["ids"]
    st = C.c_ulonglong(meta["seed"])
    for _ in range(len(meta["ids"])):
        oracle().or_random_u32(C.byref(st))
    assert state == st.value
    base = META["bin" if runq else "qwb"]
    assert list(greedy["ids"]) == base["ids"][:4]  # temperature 0: back to the argmax
