"""Pin the CPU oracle to golden vectors produced by the reference implementation itself.

The oracle runs the reference's torch op sequence on CPU, so on the same inputs it must
reproduce every recorded tensor bit for bit (H, act_square, quantizer params, per-subgroup
Hinv_init / Hinv / beta / Z / GHinv / perm, and the final Q / codes / scale).
"""
import numpy as np
import pytest
import torch

from oracle.gptqplus_cpu import GPTQPlusOracle, make_quantizer, safe_beta_from_reference_loss
from tests.golden.fixtures import GoldenSet, quadratic_refresh

CASES = GoldenSet.load().cases


def _run(case, inject_H=False):
    m = case.meta
    W = case.t("W")
    g = GPTQPlusOracle(W, case.t("s"), case.t("grad"), m["G"], m["alpha"], m["ref_loss"])
    g.quantizer = make_quantizer(m["bits"], m["sym"], m.get("mse", False))
    X = case.t("X")
    for j in range(0, X.shape[0], 4):
        g.add_batch(X[j:j + 4])
    g.finalize_hessian()
    if inject_H:
        g.H = case.H().clone()
        g.act_square = case.t("act_square").clone()
    extra = dict(m.get("fq", {}))
    if m.get("mode") in ("block_gd", "block_backward"):
        extra["gradient_refresh_fn"] = quadratic_refresh(case.t("X"), W, case.t("grad"))
    res = g.fasterquant(blocksize=m["B"], percdamp=0.01, groupsize=m["gs"], actorder=m["act"],
                        static_groups=m["act"], block_atomic_quant=m["atomic"],
                        g_update_mode=m.get("mode", "frozen"), **extra)
    return g, res


@pytest.mark.parametrize("case", CASES, ids=[c.name for c in CASES])
def test_hessian_bitexact(case):
    g, _ = _run(case)
    assert torch.equal(g.H, case.H())
    assert torch.equal(g.act_square, case.t("act_square"))


@pytest.mark.parametrize("case", CASES, ids=[c.name for c in CASES])
def test_fasterquant_bitexact(case):
    g, res = _run(case, inject_H=True)
    m = case.meta
    assert torch.equal(g.quantizer.scale, case.t("qscale"))
    assert torch.equal(g.quantizer.zero, case.t("qzero"))
    for s, rec in enumerate(res.subgroups):
        assert torch.equal(rec.Hinv_init, case.sub(s, "Hinv_init")), f"Hinv_init sub{s}"
        assert torch.equal(rec.Hinv, case.sub(s, "Hinv_upper_cholesky")), f"Hinv sub{s}"
        assert torch.equal(rec.beta, case.sub(s, "beta")), f"beta sub{s}"
        assert torch.equal(rec.Z, case.sub(s, "Z_initial")), f"Z sub{s}"
        assert torch.equal(rec.GHinv, case.sub(s, "GHinv_initial")), f"GHinv sub{s}"
        if m["act"]:
            assert torch.equal(rec.perm, case.sub(s, "perm")), f"perm sub{s}"
        fb = case.arrays.get(f"sub{s}_identity_fallback")
        assert rec.identity_fallback == bool(fb)
    assert torch.equal(res.Q, case.t("Q"))
    assert torch.equal(res.W_int.to(torch.int8), case.t("W_int"))
    assert torch.equal(res.W_int, case.t("W_int").float())
    assert torch.equal(res.Scale, case.t("Scale"))


def test_golden_cover_the_branches():
    """The fixture set exercises the branches only an import of the reference pins."""
    names = {c.name for c in CASES}
    metas = [c.meta for c in CASES]
    assert any(m["atomic"] and m["gs"] != -1 and not m["act"] for m in metas)      # atomic+dynamic
    assert any(m["atomic"] and m["gs"] != -1 and m["act"] for m in metas)          # atomic+static
    assert any(m["alpha"] > 0 for m in metas)                                       # beta != 0
    assert any(not m["sym"] for m in metas)                                         # asym quirk
    assert any(m["C"] % m["B"] for m in metas)                                      # ragged last block
    assert sum(bool(m.get("mse")) for m in metas) >= 3                              # clip search
    assert {m.get("mode") for m in metas} >= {"surrogate_block", "surrogate_online", "block_gd",
                                              "block_backward"}
    fq = [m.get("fq", {}) for m in metas]
    assert {f.get("grad_optimizer") for f in fq} >= {"sgd", "adam", "h_adam"}
    assert {f.get("grad_reg_strategy") for f in fq} >= {"none", "l2", "hessian", "quant_error_gate",
                                                        "quant_error_gate_optimized"}
    assert "g1_sym4_indefinite_identity" in names
    ident = GoldenSet.load().by_name("g1_sym4_indefinite_identity")
    assert bool(ident.arrays["sub0_identity_fallback"])
    gp = GoldenSet.load().by_name("g4_asym4_perchan_act_gplus")
    b = np.concatenate([gp.arrays[f"sub{s}_beta"] for s in range(4)])
    assert b.min() > 0 and b.max() < 0.1                   # small, non-zero first-order term
    big = GoldenSet.load().by_name("g2_sym4_atomic_static_gplus")
    b = np.concatenate([big.arrays[f"sub{s}_beta"] for s in range(2)])
    assert b.max() > 0.9                                   # the ratio clamp near beta = 1


def test_safe_beta_vectors(golden):
    for k in range(4):
        G = torch.from_numpy(golden.beta[f"beta{k}_G"])
        Hi = torch.from_numpy(golden.beta[f"beta{k}_Hinv_init"])
        ref_loss, alpha = golden.beta[f"beta{k}_params"].tolist()
        beta, gh = safe_beta_from_reference_loss(G, Hi, ref_loss, alpha)
        assert torch.equal(beta, torch.from_numpy(golden.beta[f"beta{k}_beta"]))
        assert torch.equal(gh, torch.from_numpy(golden.beta[f"beta{k}_ghinv_init"]))
