"""Pin the classic-GPTQ oracle (oracle/gptq_cpu.py) to golden vectors written by the reference's
own GPTQ class (gptq_utils/gptq_utils.py:23-180), bit for bit."""
import numpy as np
import pytest
import torch

from oracle.gptq_cpu import GPTQOracle
from oracle.gptqplus_cpu import make_quantizer
from tests.golden.fixtures import GoldenSet

CASES = GoldenSet.load().gptq_cases


def run_gptq_oracle(case, H=None):
    """The oracle on a golden case; H (finalized, [C, C]) replaces the accumulated Hessian."""
    m = case.meta
    g = GPTQOracle(case.t("W"))
    g.quantizer = make_quantizer(m["bits"], m["sym"], m.get("mse", False))
    X = case.t("X")
    for j in range(X.shape[0]):
        g.add_batch(X[j].unsqueeze(0))
    if H is not None:
        g.H = H.clone()
    H = g.H.clone()
    res = g.fasterquant(blocksize=m["B"], percdamp=0.01, groupsize=m["gs"], actorder=m["act"],
                        static_groups=m.get("static", m["act"]))
    return g, H, res


@pytest.mark.parametrize("case", CASES, ids=[c.name for c in CASES])
def test_gptq_bitexact(case):
    g, H, res = run_gptq_oracle(case)
    assert torch.equal(H, case.H()[0])
    assert torch.equal(res.Q, case.t("Q"))
    assert torch.equal(res.W_int.to(torch.int8), case.t("W_int"))
    assert torch.equal(res.Scale, case.t("Scale"))
    assert torch.equal(g.quantizer.scale, case.t("qscale"))
    assert torch.equal(g.quantizer.zero, case.t("qzero"))


def test_gptq_golden_cover_the_branches():
    metas = [c.meta for c in CASES]
    assert any(m["gs"] != -1 and not m.get("static", m["act"]) and m["gs"] < m["B"] for m in metas)
    assert any(m["gs"] != -1 and not m.get("static", m["act"]) and m["gs"] > m["B"] for m in metas)
    assert any(m["gs"] != -1 and m.get("static", m["act"]) for m in metas)
    assert any(m["N"] == 0 for m in metas)                       # RTN fallback (H == 0)
    assert any(m.get("dead") for m in metas) and any(m.get("mse") for m in metas)
    assert any(m["C"] % m["B"] for m in metas)


def test_gptq_running_mean_is_the_scaled_gram_matrix():
    """The per-sample running mean equals 2/N * sum x x^T (the product runs in fp32, as in the
    reference, so the bar is fp32 rounding)."""
    r = np.random.default_rng(5)
    X = torch.from_numpy(r.standard_normal((6, 8, 12)))
    g = GPTQOracle(torch.zeros(3, 12))
    for j in range(6):
        g.add_batch(X[j].unsqueeze(0).float())
    Xf = X.reshape(-1, 12)
    torch.testing.assert_close(g.H.double(), 2.0 / 6 * Xf.T @ Xf, rtol=1e-5, atol=1e-5)
