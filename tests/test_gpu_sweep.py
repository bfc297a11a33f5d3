"""Seeded random sweep of the HIP path against the fp64 oracle: 150 shapes
(dense and varlen, d 64 and 128, every rank tier from 8 to 64, GQA groups of
1 to 3 with any number of graph heads, causal or not), lengths drawn with the
32 / 64 / 128 / 256 / 512-token tile edges and their neighbours
over-represented.  Each shape is checked to the same bounds as the other
parity tests (FNA2/validate_fna2.py:115-122 tolerances)."""
import numpy as np
import pytest

from tests import test_gpu_parity as T

pytestmark = pytest.mark.gpu

EDGES = [1, 31, 32, 33, 63, 64, 65, 127, 128, 129, 255, 256, 257, 511, 512, 513]


def _case(gpu, seed):
    rng = np.random.default_rng(seed)
    D = int(rng.choice([64, 128]))
    H_KV = int(rng.integers(1, 3))
    Hq = H_KV * int(rng.integers(1, 4))
    H_G = int(rng.integers(0, Hq + 1))
    R = 8 * int(rng.integers(1, 9)) if H_G else 0
    causal = bool(rng.integers(0, 2))
    if rng.random() < 0.3:
        B = int(rng.integers(1, 3))
        S = int(rng.choice(EDGES)) if rng.random() < 0.5 else int(rng.integers(1, 700))
        T._dense_case(gpu, B, Hq, S, D, H_KV, H_G, R, causal, seed=seed)
    else:
        n = int(rng.integers(1, 8))
        lengths = [int(rng.choice(EDGES)) if rng.random() < 0.5 else int(rng.integers(0, 900))
                   for _ in range(n)]
        if sum(lengths) == 0:
            lengths[0] = 17
        T._varlen_case(gpu, lengths, Hq, D, H_KV, H_G, R, causal, seed=seed)


@pytest.mark.parametrize("first", range(5000, 5150, 10))
def test_random_shapes(gpu, first):
    for seed in range(first, first + 10):
        print(f"sweep seed {seed}", flush=True)
        _case(gpu, seed)
