"""Pin the CPU oracle by mathematics that is independent of its own formulas.

Each check is chosen so that a plausible slip (a dropped saliency factor, a transposed
operand, non-cumulative damping, a wrong rounding mode, a sign error in the GPTQ+ term)
fails at least one of them.
"""
import numpy as np
import pytest
import scipy.linalg
import torch

from oracle.gptqplus_cpu import (GPTQPlusOracle, WeightQuantizerOracle, hessian_inverse_with_fallback,
                                 make_quantizer)


def _rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


# ----------------------------------------------------------------------------- Hessian
def test_hessian_matches_fp64_outer_product_sum():
    rng = _rng(1)
    N, T, C, G = 6, 10, 12, 3
    X = rng.standard_normal((N, T, C)).astype(np.float32)
    s = rng.lognormal(size=(N, T, G)).astype(np.float32)
    W = rng.standard_normal((G * 2, C)).astype(np.float32)
    g = GPTQPlusOracle(torch.from_numpy(W), torch.from_numpy(s), torch.zeros(G * 2, C), G, 0.0, 0.0)
    g.add_batch(torch.from_numpy(X[:4]))
    g.add_batch(torch.from_numpy(X[4:]))
    g.finalize_hessian()
    # brute force: H_g = sum_t s_tg x_t x_t^T / (N*T), act = sum_t x_t^2 / T
    Xd = X.reshape(-1, C).astype(np.float64)
    sd = s.reshape(-1, G).astype(np.float64)
    for gi in range(G):
        ref = np.zeros((C, C))
        for t in range(Xd.shape[0]):
            ref += sd[t, gi] * np.outer(Xd[t], Xd[t])
        ref /= N * T
        np.testing.assert_allclose(g.H[gi].numpy(), ref, rtol=2e-6, atol=1e-6)
        assert torch.equal(g.H[gi], g.H[gi].T)
    np.testing.assert_allclose(g.act_square.numpy(), (Xd ** 2).sum(0) / T, rtol=1e-6)


def test_hessian_saliency_scale_and_sink_drop():
    rng = _rng(2)
    X = rng.standard_normal((2, 8, 5)).astype(np.float32)
    s = np.ones((2, 6, 1), np.float32)          # saliency shorter than T: the 2 sink tokens drop
    g = GPTQPlusOracle(torch.zeros(1, 5), torch.from_numpy(s), torch.zeros(1, 5), 1, 0.0, 0.0,
                       hessian_saliency_scale=4.0)
    g.add_batch(torch.from_numpy(X))
    g.finalize_hessian()
    Xk = X[:, 2:, :].reshape(-1, 5).astype(np.float64)
    np.testing.assert_allclose(g.H[0].numpy(), Xk.T @ Xk / 12 / 4.0, rtol=2e-6)
    np.testing.assert_allclose(g.act_square.numpy(), (Xk ** 2).sum(0) / 6, rtol=2e-6)


def test_finalize_errors():
    g = GPTQPlusOracle(torch.zeros(2, 3), torch.ones(1, 4, 1), torch.zeros(2, 3), 1, 0.0, 0.0)
    with pytest.raises(RuntimeError):
        g.finalize_hessian()
    g.add_batch(torch.ones(1, 4, 3))
    g.finalize_hessian()
    with pytest.raises(RuntimeError):
        g.add_batch(torch.ones(1, 4, 3))


# ----------------------------------------------------------------------------- quantizer
@pytest.mark.parametrize("row,bits,sym,scale,zero", [
    ([-1.0, 0.5, 2.0], 4, True, 2.0 / 7, 0.0),
    ([-3.0, 0.5, 2.0], 3, True, 3.0 / 3, 0.0),
    ([0.0, 0.0, 0.0], 4, False, 2.0 / 15, 7.0),        # (-1, +1) branch; 1/fl32(2/15) = 7.4999996 -> 7
    ([1.0, 2.0, 3.0], 4, False, 3.0 / 15, 0.0),        # xmin clipped at 0
    ([-2.0, -1.0, -0.5], 4, False, 2.0 / 15, 15.0),    # xmax clipped at 0
    ([1e-9, -1e-9, 0.0], 4, True, 1e-5 / 7, 0.0),      # clamp(min=1e-5)
])
def test_find_params_known_answers(row, bits, sym, scale, zero):
    q = make_quantizer(bits, sym)
    q.find_params(torch.tensor([row], dtype=torch.float32))
    assert q.scale.shape == (1, 1)
    assert abs(q.scale.item() - scale) <= 1e-7 * max(scale, 1e-6)
    assert q.zero.item() == zero


@pytest.mark.parametrize("sym,scale,zero", [(True, 3.0 / 7, 0.0), (False, 4.0 / 15, 4.0)])
def test_find_params_per_tensor_known_answer(sym, scale, zero):
    """perchannel=False: one range over the whole tensor (min -1.0 in row 1, max 3.0 in row 0),
    repeated for every row -- rows with their own ranges would give other values."""
    q = make_quantizer(4, sym, perchannel=False)
    q.find_params(torch.tensor([[0.5, 3.0], [-1.0, 0.25], [0.1, 0.2]], dtype=torch.float32))
    assert q.scale.shape == (3, 1) and q.zero.shape == (3, 1)
    assert torch.allclose(q.scale.flatten(), torch.full((3,), scale), rtol=1e-7, atol=0)
    assert torch.equal(q.zero.flatten(), torch.full((3,), zero))


@pytest.mark.parametrize("sym,row,scale,zero", [
    # asym: each run's own range, not widened to 0 (that would give 2/15, 0 and 5/15, 0)
    (False, [1.0, 2.0, 3.0, 5.0], [1 / 15, 1 / 15, 2 / 15, 2 / 15], [-15.0, -15.0, -22.0, -22.0]),
    # sym: max(|min|, max) of the run, also for an all-negative run
    (True, [-1.0, -4.0, 0.5, 0.25], [4 / 7, 4 / 7, 0.5 / 7, 0.5 / 7], [0.0] * 4),
])
def test_find_params_weight_groupwise_known_answers(sym, row, scale, zero):
    q = make_quantizer(4, sym, weight_groupsize=2)
    q.find_params(torch.tensor([row, row], dtype=torch.float32))
    assert q.scale.shape == (2, 4) and q.zero.shape == (2, 4)
    assert torch.allclose(q.scale, torch.tensor([scale, scale]), rtol=1e-6, atol=0)
    assert torch.equal(q.zero, torch.tensor([zero, zero]))


@pytest.mark.parametrize("sym", [True, False])
def test_find_params_weight_groupwise_mse_reduces_to_per_row(sym):
    """Runs that hold both signs have the same range with or without the widening to 0, so the
    groupwise clip search of a run equals the per-channel search (golden-pinned) on the run
    taken as a row of its own."""
    r = _rng(11)
    x = torch.from_numpy(r.standard_normal((6, 32)).astype(np.float32))
    x[:, 0::8] = -x[:, 0::8].abs() - 0.1
    x[:, 1::8] = x[:, 1::8].abs() + 0.1
    qg = make_quantizer(4, sym, mse=True, weight_groupsize=8)
    qg.find_params(x)
    qr = make_quantizer(4, sym, mse=True)
    qr.find_params(x.reshape(-1, 8))
    assert torch.equal(qg.scale.reshape(-1, 8), qr.scale.reshape(-1, 1).expand(-1, 8))
    assert torch.equal(qg.zero.reshape(-1, 8), qr.zero.reshape(-1, 1).expand(-1, 8))


@pytest.mark.parametrize("bits,sym", [(4, True), (4, False), (3, True), (2, False)])
def test_fake_quantize_is_nearest_grid_point(bits, sym):
    """Brute force over every code: fake_quantize picks the nearest point of
    scale * [-(maxq+1), maxq] (ties to the even code), whatever ``sym`` says."""
    rng = _rng(3 + bits)
    x = torch.from_numpy((rng.standard_normal((64, 40)) * 0.05).astype(np.float32))
    q = make_quantizer(bits, sym)
    q.find_params(x)
    deq, codes, scale = q.fake_quantize(x)
    maxq = int(q.maxq)
    grid = torch.arange(-(maxq + 1), maxq + 1, dtype=torch.float64)
    ratio = (x.double() / scale.double())
    dist = (ratio.unsqueeze(-1) - grid).abs()
    best = dist.min(-1).values
    cand = dist <= best.unsqueeze(-1) + 1e-9
    # among equally near codes prefer the even one (round half to even)
    even = cand & (grid.remainder(2) == 0)
    pick = torch.where(even.any(-1, keepdim=True), even, cand).double().argmax(-1)
    expect = grid[pick]
    mism = (codes.double() != expect)
    # only fp32-vs-fp64 ratio rounding at exact .5 boundaries may differ
    assert mism.sum().item() == 0
    assert torch.equal(deq, (scale * codes))
    assert codes.min() >= -(maxq + 1) and codes.max() <= maxq


def test_fake_quantize_grid_roundtrip():
    q = make_quantizer(4, True)
    q.scale = torch.full((3, 1), 0.125)
    q.maxq = torch.tensor(7)
    k = torch.arange(-8, 8, dtype=torch.float32)
    x = (0.125 * k).expand(3, -1).clone()
    deq, codes, _ = q.fake_quantize(x)
    assert torch.equal(codes[0], k) and torch.equal(deq, x)


# ----------------------------------------------------------------------------- Cholesky chain
def test_hessian_inverse_against_scipy_fp64():
    rng = _rng(5)
    C = 48
    A = rng.standard_normal((200, C)).astype(np.float32)
    A[:, 3] *= 20
    H = torch.from_numpy((A.T @ A / 200).astype(np.float32))
    Hinv_init, Hinv, p, fb, attempts = hessian_inverse_with_fallback(H, 0.01)
    assert (p, fb, attempts) == (0.01, False, 1)
    Hd = H.double().numpy()
    Hd = Hd + 0.01 * np.mean(np.diag(H.numpy())).astype(np.float64) * np.eye(C)
    inv = np.linalg.inv(Hd)
    U = scipy.linalg.cholesky(inv, lower=False)
    np.testing.assert_allclose(Hinv_init.double().numpy(), inv, rtol=0, atol=2e-5 * np.abs(inv).max())
    np.testing.assert_allclose(Hinv.double().numpy(), U, rtol=0, atol=2e-5 * np.abs(U).max())
    assert torch.equal(Hinv, torch.triu(Hinv)) and (torch.diag(Hinv) > 0).all()


def _expected_attempts(diag, p0=0.01, inc=0.0015):
    """Retry schedule for a diagonal H with one negative pivot, in float64:
    the damping is re-added to the SAME working matrix each attempt (cumulative)."""
    d = np.array(diag, dtype=np.float64)
    p, n = p0, 0
    while 1 > p > 0:
        n += 1
        d = d + p * d.mean()
        if (d > 0).all():
            return n, p, False
        p += inc
    return n, p, True


@pytest.mark.parametrize("neg", [0.05, 0.3, 5.0])
def test_damping_retry_is_cumulative(neg):
    diag = [-neg, 1.0, 1.0, 1.0, 2.0]
    H = torch.diag(torch.tensor(diag, dtype=torch.float64))
    n, p, fb = _expected_attempts(diag)
    Hinv_init, Hinv, p_got, fb_got, attempts = hessian_inverse_with_fallback(H, 0.01)
    assert attempts == n and fb_got == fb and abs(p_got - p) < 1e-12
    if fb:
        assert torch.equal(Hinv, torch.eye(5, dtype=torch.float64))


def test_damping_must_be_positive():
    with pytest.raises(ValueError):
        hessian_inverse_with_fallback(torch.eye(3), 0.0)


# ----------------------------------------------------------------------------- fasterquant
def _oracle_from_H(W, H, act, G=1, alpha=0.0, ref_loss=0.0, grad=None, bits=4, sym=True, dtype=torch.float64):
    R, C = W.shape
    g = GPTQPlusOracle(W, torch.ones(1, 1, G), torch.zeros(R, C) if grad is None else grad, G,
                       alpha, ref_loss, dtype=dtype)
    g.H = (H if H.dim() == 3 else H[None]).to(dtype).clone()
    g.act_square = act.to(dtype).clone()
    g._finalized = True
    g.quantizer = make_quantizer(bits, sym)
    return g


def _obs_textbook(W, H, percdamp, maxq, scale):
    """Sequential Optimal Brain Surgeon quantization (GPTQ paper, Frantar et al. 2022, eq. 2-3)
    with an explicitly maintained inverse of the remaining-columns Hessian, in float64."""
    W = W.copy()
    C = W.shape[1]
    Hd = H + percdamp * np.mean(np.diag(H)) * np.eye(C)
    Hi = np.linalg.inv(Hd)
    codes = np.zeros_like(W)
    for q in range(C):
        c = np.clip(np.round(W[:, q] / scale[:, 0]), -(maxq + 1), maxq)
        codes[:, q] = c
        e = (W[:, q] - c * scale[:, 0]) / Hi[q, q]
        W[:, q + 1:] -= np.outer(e, Hi[q, q + 1:])
        Hi = Hi - np.outer(Hi[:, q], Hi[q, :]) / Hi[q, q]
        Hi[q, :] = 0
        Hi[:, q] = 0
    return codes


def test_fasterquant_equals_textbook_obs_fp64():
    rng = _rng(7)
    R, C = 24, 20
    A = rng.standard_normal((300, C))
    H = A.T @ A / 300
    W = rng.standard_normal((R, C)) * 0.02
    g = _oracle_from_H(torch.from_numpy(W), torch.from_numpy(H), torch.ones(C))
    res = g.fasterquant(blocksize=8, percdamp=0.01, actorder=False)
    scale = g.quantizer.scale.numpy()
    codes = _obs_textbook(W, H, 0.01, 7, scale)
    assert np.array_equal(res.W_int.numpy(), codes)


def test_identity_hessian_reduces_to_rtn():
    rng = _rng(8)
    W = torch.from_numpy((rng.standard_normal((16, 40)) * 0.02).astype(np.float32))
    g = _oracle_from_H(W, torch.eye(40), torch.ones(40), dtype=torch.float32)
    res = g.fasterquant(blocksize=16, actorder=False)
    q = make_quantizer(4, True)
    q.find_params(W)
    deq, codes, _ = q.fake_quantize(W)
    assert torch.equal(res.W_int, codes) and torch.equal(res.Q_fp32, deq)


def _gplus_problem(seed=9, R=12, C=24, G=2):
    rng = _rng(seed)
    A = rng.standard_normal((200, C))
    H = np.stack([A.T @ (A * rng.lognormal(size=(200, 1))) / 200 for _ in range(G)])
    W = torch.from_numpy(rng.standard_normal((R, C)) * 0.02)
    grad = torch.from_numpy(rng.standard_normal((R, C)))
    act = torch.from_numpy(rng.permutation(C).astype(np.float64) + 1.0)
    return torch.from_numpy(H), W, grad, act


def test_gptqplus_frozen_is_blocksize_invariant_fp64():
    """In exact arithmetic count*GHinv_rest - (Z1*D)Hinv equals the per-column GHinv1
    subtractions, so the frozen GPTQ+ column-loop result does not depend on the block size."""
    H, W, grad, act = _gplus_problem()
    outs = []
    for B in (1, 8, W.shape[1]):
        g = _oracle_from_H(W, H, act, G=2, alpha=0.05, ref_loss=3e5, grad=grad)
        res = g.fasterquant(blocksize=B, actorder=True)
        assert torch.cat([r.beta for r in res.subgroups]).min() > 0.01   # first-order term is on
        outs.append(res)
    for r in outs[1:]:
        assert torch.equal(r.W_int, outs[0].W_int)
        torch.testing.assert_close(r.Q_fp32, outs[0].Q_fp32, rtol=0, atol=1e-12)


def test_atomic_blocksize_one_equals_column_loop_fp64():
    """With one column per block the atomic triangular solve is the column loop's error
    recursion, so atomic B=1 reproduces the (block-size invariant) column-loop result."""
    H, W, grad, act = _gplus_problem(seed=12)
    ref = _oracle_from_H(W, H, act, G=2, alpha=0.05, ref_loss=3e5, grad=grad).fasterquant(
        blocksize=8, actorder=True)
    at = _oracle_from_H(W, H, act, G=2, alpha=0.05, ref_loss=3e5, grad=grad).fasterquant(
        blocksize=1, actorder=True, block_atomic_quant=True)
    assert torch.equal(at.W_int, ref.W_int)
    torch.testing.assert_close(at.Q_fp32, ref.Q_fp32, rtol=0, atol=1e-12)


def test_gptqplus_term_changes_result_and_sign():
    """beta > 0 must move the result, and in the direction of -G Hinv (a sign slip flips it)."""
    rng = _rng(10)
    R, C = 8, 16
    A = rng.standard_normal((100, C))
    H = torch.from_numpy(A.T @ A / 100)[None]
    W = torch.from_numpy(rng.standard_normal((R, C)) * 0.02)
    grad = torch.from_numpy(rng.standard_normal((R, C)))
    act = torch.ones(C, dtype=torch.float64)
    base = _oracle_from_H(W, H, act).fasterquant(blocksize=4)
    g = _oracle_from_H(W, H, act, alpha=0.05, ref_loss=3e5, grad=grad)
    res = g.fasterquant(blocksize=4)
    assert not torch.equal(res.W_int, base.W_int)
    # first-order objective: <G, Q - W> decreases when the gradient term is on
    assert (grad * (res.Q_fp32 - W)).sum() < (grad * (base.Q_fp32 - W)).sum()


def test_atomic_err_solves_triangular_system():
    rng = _rng(11)
    Hinv1 = np.triu(rng.standard_normal((6, 6))) + 4 * np.eye(6)
    res = rng.standard_normal((5, 6))
    err = torch.linalg.solve_triangular(torch.from_numpy(Hinv1).T, torch.from_numpy(res).T, upper=False).T
    np.testing.assert_allclose(err.numpy() @ Hinv1, res, atol=1e-12)


def test_dynamic_groups_require_groupsize_equal_blocksize():
    g = _oracle_from_H(torch.zeros(2, 8, dtype=torch.float64), torch.eye(8)[None], torch.ones(8))
    with pytest.raises(ValueError):
        g.fasterquant(blocksize=4, groupsize=2, actorder=False, static_groups=False)
