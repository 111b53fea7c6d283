"""The oracle's record_ratio report and tests/_util.flip_report, on the CPU.

record_ratio returns w / scale, the value torch.round rounds for each code
(quant_utils.py:477, gptq_plus_utils.py:1306-1310): it must change no result, and rounding it
half to even and clamping must give the codes back, in the fast per-channel path, with static
groups (act_order) and in the atomic block.  flip_report is checked on hand-made codes whose
ratios sit at known distances from the rounding midpoint."""
import copy

import numpy as np
import pytest
import torch

from oracle.gptqplus_cpu import GPTQPlusOracle, make_quantizer
from tests._util import flip_report


def _oracle(seed, R=32, C=96, G=2, sym=False):
    r = np.random.Generator(np.random.PCG64(seed))
    X = torch.from_numpy(r.standard_normal((4, 64, C)).astype(np.float32))
    W = torch.from_numpy(r.standard_normal((R, C)).astype(np.float32) * 0.05)
    s = torch.from_numpy(r.lognormal(size=(4, 64, G)).astype(np.float32))
    o = GPTQPlusOracle(W, s, torch.zeros(R, C), G, 0.0, 0.0)
    o.quantizer = make_quantizer(4, sym)
    o.add_batch(X)
    o.finalize_hessian()
    return o


@pytest.mark.parametrize("kw", [
    dict(groupsize=-1, actorder=True, static_groups=True),
    dict(groupsize=32, actorder=True, static_groups=True),
    dict(groupsize=32, actorder=False, static_groups=False, blocksize=32, block_atomic_quant=True),
    dict(groupsize=-1, actorder=False, blocksize=32, block_atomic_quant=True),
])
def test_record_ratio_rounds_to_the_codes(kw):
    o = _oracle(5)
    kw = dict(dict(blocksize=32, percdamp=0.01), **kw)
    a = copy.deepcopy(o).fasterquant(**kw)
    b = copy.deepcopy(o).fasterquant(record_ratio=True, **kw)
    assert torch.equal(a.W_int, b.W_int) and torch.equal(a.Q, b.Q) and a.ratio is None
    maxq = int(o.quantizer.maxq)
    assert torch.equal(torch.clamp(torch.round(b.ratio), -(maxq + 1), maxq), b.W_int)


def test_flip_report_classifies_distances():
    ref = torch.zeros(3, 6)
    gpu = ref.clone()
    ratio = torch.full((3, 6), 0.25)
    # row 0: an exact tie (2.5 rounds to 2 half to even; the other side gave 3)
    ratio[0, 1], ref[0, 1], gpu[0, 1] = 2.5, 2.0, 3.0
    # row 1: 3 ulps above the midpoint 1.5, then a later flip in the same row
    r1 = np.float32(1.5)
    for _ in range(3):
        r1 = np.nextafter(r1, np.float32(2.0))
    ratio[1, 2], ref[1, 2], gpu[1, 2] = float(r1), 2.0, 1.0
    ratio[1, 4], ref[1, 4], gpu[1, 4] = 0.2, 0.0, 1.0
    rep = flip_report(gpu, ref, ratio)
    assert rep["flips"] == 3 and rep["primary"] == 2 and rep["exact_ties"] == 1
    assert rep["primary_exact_ties"] == 1 and rep["primary_ulps_le_1"] == 1 and rep["primary_ulps_le_16"] == 2
    assert rep["primary_ulps_max"] == pytest.approx(3.0)
    assert rep["all_dist_max"] == pytest.approx(0.3, abs=1e-6)
    # the act_order column order decides which flip of a row is the first
    perm = torch.tensor([5, 4, 3, 2, 1, 0])
    rep_p = flip_report(gpu, ref, ratio, perm)
    assert rep_p["primary"] == 2 and rep_p["primary_dist_max"] == pytest.approx(0.3, abs=1e-6)
    assert flip_report(ref, ref, ratio) == {"flips": 0, "exact_ties": 0, "primary": 0}
