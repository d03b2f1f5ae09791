"""The strict mode's sequential fp32 sums on the MI355X, each device form on its own (mvh_seq_sum).

The reference adds a sum's terms one after another in fp32: rmsnorm's sum of squares (qwen.c:339), the softmax
denominator (qwen.c:349), a row's group products (qwen.c:441-452).  The device computes the first two by
speculative segments (the block's waves each start 64 candidate chains around a predicted start, one wave
walks them) or by one wave's chain, the third by one thread's chain.  Bar: bitwise, for every length and
every block size, against the definition s_k = fl(s_{k-1} + a_k) (numpy's float32 accumulate, checked
against a plain Python loop of float32 adds first).  The cases push each path: lengths at and around the
segment and batch edges, ties and exact halves, subnormals, inf, NaN and overflow, mixed signs with
cancellation, and sums whose drift from the exact value leaves every candidate (the term-by-term path)."""
import numpy as np
import pytest

from helpers import pkg

pytestmark = pytest.mark.gpu


def seq_ref(a):
    a = np.asarray(a, np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        return np.cumsum(a, dtype=np.float32)[-1] if a.size else np.float32(0)


def same(x, y):
    x, y = np.float32(x), np.float32(y)
    return (np.isnan(x) and np.isnan(y)) or x.view(np.uint32) == y.view(np.uint32)


def cases():
    rng = np.random.default_rng(20)
    out = []
    lengths = [1, 2, 3, 15, 16, 17, 28, 31, 32, 33, 47, 48, 49, 63, 64, 65, 112, 127, 152, 255, 256, 257, 288, 511,
               513, 592, 767, 768, 769, 896, 1000, 2047, 3584, 4096, 4864, 8192]
    for n in lengths:
        x = rng.standard_normal(n).astype(np.float32)
        out.append((f"squares n={n}", x * x))
        out.append((f"small squares n={n}", (x * 0.02) ** 2))
        out.append((f"exps n={n}", np.exp(x * 6).astype(np.float32)))
        out.append((f"signed n={n}", x))
    out.append(("all 0.75", np.full(1000, 0.75, np.float32)))
    out.append(("eighths", (rng.integers(0, 8, 3000) * 0.125).astype(np.float32)))
    out.append(("powers of two", (2.0 ** rng.integers(-1, 19, 2000)).astype(np.float32)))
    out.append(("subnormals", np.ldexp(rng.integers(1, 4, 777), -140).astype(np.float32)))
    out.append(("zeros then squares", np.concatenate([np.zeros(300, np.float32), rng.random(600, np.float32)])))
    out.append(("inf", np.array([1, np.inf, 2], np.float32)))
    out.append(("nan", np.array([1, 2, np.nan, 3], np.float32)))
    out.append(("overflow", np.array([3.4e38, 3.4e38, 1], np.float32)))
    out.append(("nan deep", np.where(np.arange(3000) == 1500, np.nan, 1).astype(np.float32)))
    out.append(("inf deep", np.where(np.arange(3000) == 700, np.inf, 0.5).astype(np.float32)))
    # one large term, then terms just under / over half an ulp of it: the running sum stays put (or creeps)
    # while the exact sum grows, far past every candidate window
    for f in (0.49, 0.51, 0.75):
        a = np.full(4864, np.ldexp(f, -24), np.float32)
        a[0] = 1
        out.append((f"drift {f}", a))
    out.append(("alternating", np.where(np.arange(2000) % 2, -1, 1 + 1e-7 * np.arange(2000)).astype(np.float32)))
    a = np.full(896, 1e-3, np.float32)
    a[::7] = 1e6
    out.append(("spikes", a))
    return out


def test_reference_definition_is_a_loop_of_float32_adds():
    rng = np.random.default_rng(3)
    for n in (1, 5, 300):
        a = rng.standard_normal(n).astype(np.float32)
        s = np.float32(0)
        for v in a:
            s = np.float32(s + v)
        assert same(s, seq_ref(a))


@pytest.mark.parametrize("threads", [64, 128, 256, 448, 512, 1024])
def test_block_sum_is_the_sequential_sum(threads):
    for name, a in cases():
        got = pkg().seq_sum(a, "block", threads)
        assert same(got, seq_ref(a)), (name, threads, float(got), float(seq_ref(a)))


@pytest.mark.parametrize("which", ["wave", "thread"])
def test_chain_sums_are_the_sequential_sum(which):
    for name, a in cases():
        got = pkg().seq_sum(a, which)
        assert same(got, seq_ref(a)), (name, which, float(got), float(seq_ref(a)))


def test_bad_arguments_are_refused():
    with pytest.raises(RuntimeError):
        pkg().seq_sum(np.ones(10, np.float32), "block", 100)
    with pytest.raises(RuntimeError):
        pkg().seq_sum(np.ones(8193, np.float32), "wave")
