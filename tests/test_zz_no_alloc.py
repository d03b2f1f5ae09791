"""mvh_sample_noalloc (the sampler entry point that allocates no device memory) against mvh_sample, the
entry point it varies: the same rows and the same advanced RNG state, bit for bit, on two calls in a row,
the second with a smaller input (so what the first call left in the shared scratch array must not leak into
the second); and sizes beyond the scratch array rejected with an error before any device work."""
import numpy as np
import pytest

from helpers import pkg

pytestmark = pytest.mark.gpu


def test_noalloc_sampler_equals_the_allocating_sampler():
    P = pkg()
    rng = np.random.default_rng(11)
    for count, n, temperature, topp, seed in ((6, 152064, 0.8, 0.9, 42), (3, 4097, 1.0, 1.0, 7)):
        lg = (rng.standard_normal((count, n)) * 2).astype(np.float32)
        rows_a, st_a = P.sample(lg, temperature, topp, seed)
        rows_b, st_b = P.sample(lg, temperature, topp, seed, noalloc=True)
        assert list(rows_a) == list(rows_b), (count, n)
        assert st_a == st_b


def test_noalloc_sampler_rejects_sizes_beyond_its_scratch():
    P = pkg()
    with pytest.raises(RuntimeError):
        P.sample(np.zeros((1, 262145), np.float32), 1.0, 0.9, 1, noalloc=True)  # a row over 262144 logits
    with pytest.raises(RuntimeError):
        P.sample(np.zeros((14, 152064), np.float32), 1.0, 0.9, 1, noalloc=True)  # over 2^21 staged logits
