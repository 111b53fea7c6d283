"""The CPU orders the reference's act_order depends on, checked against torch itself:
act_square's column sum (gptq_plus_utils.py:856) and argsort's tie order (:1046).  The HIP
kernels implement these models; the GPU tests then compare the kernels with torch directly."""
import numpy as np
import pytest
import torch

from tests._cpu_order import (adversarial_keys, column_sum_model, heap_sort_runs, model_covers,
                              std_sort)


@pytest.mark.parametrize("n,C", [(32768, 256), (2048, 96), (1000, 64), (37, 64), (12305, 32),
                                 (5000, 13), (4097, 77), (300, 3), (40000, 250), (600000, 40),
                                 (17, 2), (70001, 130)])
def test_column_sum_model_matches_torch(n, C):
    rng = np.random.default_rng(n * 1000 + C)
    x = (rng.standard_normal((n, C), dtype=np.float32) * 3).astype(np.float16).astype(np.float32)
    x[rng.integers(0, n, 3), rng.integers(0, C, 3)] *= 50
    assert model_covers(C)
    e = column_sum_model(x * x)
    for th in (1, 4, 8):
        prev = torch.get_num_threads()
        torch.set_num_threads(th)
        try:
            t = (torch.from_numpy(x) ** 2).sum(0).numpy()
        finally:
            torch.set_num_threads(prev)
        assert np.array_equal(t, e), (n, C, th, int((t != e).sum()))


def test_column_sum_model_is_not_a_plain_loop():
    """The cascade differs from a left-to-right sum (so the check above has teeth)."""
    rng = np.random.default_rng(1)
    x = rng.standard_normal((32768, 64), dtype=np.float32)
    sq = x * x
    plain = np.zeros(64, np.float32)
    for r in range(sq.shape[0]):
        plain = (plain + sq[r]).astype(np.float32)
    assert not np.array_equal(plain, column_sum_model(sq))


@pytest.mark.parametrize("seed", range(12))
def test_std_sort_model_matches_torch_argsort(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(2, 3000))
    nv = int(rng.integers(1, max(2, n)))
    keys = (rng.integers(0, nv, n) * 0.5).astype(np.float32)
    if seed % 3 == 0:
        keys[rng.integers(0, n, 3)] = np.nan
    t = torch.argsort(torch.from_numpy(keys), descending=True).numpy()
    assert np.array_equal(std_sort(keys), t)


@pytest.mark.parametrize("n", [64, 700, 2000])
def test_std_sort_model_heap_branch(n):
    keys = adversarial_keys(n)
    assert heap_sort_runs(keys) >= 1
    t = torch.argsort(torch.from_numpy(keys), descending=True).numpy()
    assert np.array_equal(std_sort(keys), t)


def test_torch_argsort_is_not_stable_on_ties():
    keys = np.repeat(np.arange(200, dtype=np.float32), 5)
    t = torch.argsort(torch.from_numpy(keys), descending=True).numpy()
    assert not np.array_equal(t, np.argsort(-keys, kind="stable"))
    assert np.array_equal(t, std_sort(keys))
