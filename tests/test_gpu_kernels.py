"""GPU parity of each HIP entry point against the CPU oracle on identical seeded inputs.

Tolerances: integer / index outputs (codes, perm, find_params) are bit-exact; Hessian
rel-Frobenius <= 1e-5 (fp32 MFMA vs MKL fp32 summation order); H^-1 and its upper factor
rel-Frobenius <= 1e-4 vs the oracle's fp32 LAPACK chain (the kernel factorises in fp64, so it
is also checked <= 1e-5 against a float64 reference).
"""
import numpy as np
import pytest
import scipy.linalg
import torch

from gptq_plus_mp_quant_amd import _native as nat
from gptq_plus_mp_quant_amd import kernels as K
from oracle.gptqplus_cpu import (GPTQPlusOracle, gradient_terms, hessian_inverse_with_fallback,
                                 make_quantizer)
from tests._util import rel_fro, rng, synth

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _oracle_hessian(X, s, G, chunks):
    o = GPTQPlusOracle(torch.zeros(G, X.shape[-1]), s, torch.zeros(G, X.shape[-1]), G, 0.0, 0.0)
    for c in chunks:
        o.add_batch(X[c])
    o.finalize_hessian()
    return o.H, o.act_square


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("C,G", [(256, 1), (200, 3), (136, 4)])
def test_hessian_accum_and_finalize(dtype, C, G):
    X, _, s, _ = synth(11 + C + G, 8, C, G, 6, 96, x_dtype=dtype)
    chunks = [slice(0, 4), slice(4, 6)]
    H = torch.zeros(G, C, C, device=DEV)
    act = torch.zeros(C, device=DEV)
    for c in chunks:
        x = X[c].reshape(-1, C).to(DEV)
        sal = s[c].reshape(-1, G).to(DEV).contiguous()
        K.hessian_accum(x, sal, H, act)
    ntok = 6 * 96
    K.hessian_finalize(H, act, float(6) * (ntok / 6), 1.0, ntok / 6)
    torch.cuda.synchronize()
    Ho, acto = _oracle_hessian(X.float(), s, G, chunks)
    assert rel_fro(H, Ho) <= 1e-5
    assert rel_fro(act, acto) <= 1e-5
    assert torch.equal(H, H.transpose(1, 2))
    # float64 brute force
    Xd = X.double().reshape(-1, C)
    sd = s.double().reshape(-1, G)
    for g in range(G):
        ref = (Xd * sd[:, g:g + 1]).T @ Xd / ntok
        assert rel_fro(H[g], ref) <= 1e-5


def test_hessian_is_deterministic_and_scaled():
    X, _, s, _ = synth(5, 8, 384, 2, 4, 128)
    outs = []
    for _ in range(2):
        H = torch.zeros(2, 384, 384, device=DEV)
        act = torch.zeros(384, device=DEV)
        K.hessian_accum(X.reshape(-1, 384).to(DEV), s.reshape(-1, 2).to(DEV).contiguous(), H, act)
        K.hessian_finalize(H, act, 512.0, 4.0, 128.0)
        outs.append((H.clone(), act.clone()))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    o = GPTQPlusOracle(torch.zeros(2, 384), s, torch.zeros(2, 384), 2, 0.0, 0.0, hessian_saliency_scale=4.0)
    o.add_batch(X)
    o.finalize_hessian()
    assert rel_fro(outs[0][0], o.H) <= 1e-5


@pytest.mark.parametrize("C,G", [(1000, 3), (384, 2)])   # larger first: the second reuses its workspace
def test_hessian_tail_slices_match_whole_items(C, G):
    """fp32-MFMA kernel: the split of a partly filled last round into token slices (workspace
    given) changes only the summation order: same result as whole items to fp32 rounding, and
    bitwise reproducible from call to call.  (The split-operand kernel's slices are covered in
    test_gpu_hessian_split.py.)"""
    r = rng(40 + C)
    n = 4096
    x = torch.from_numpy(r.standard_normal((n, C), dtype=np.float32)).half().to(DEV)
    sal = torch.from_numpy(r.lognormal(size=(n, G)).astype(np.float32)).to(DEV)
    ws, nbytes = K.hessian_workspace(x, G)
    assert nbytes > 0                                  # this shape has a partial last round
    outs = []
    for use_ws in (False, True, True):
        H = torch.zeros(G, C, C, device=DEV)
        act = torch.zeros(C, device=DEV)
        with K.hessian_math("fp32"):
            nat.call("rq_hessian_accum", nat.ptr(x), nat.RQ_F16, n, C, C, nat.ptr(sal), G, G, nat.ptr(H),
                     nat.ptr(act), nat.ptr(ws) if use_ws else None, nbytes if use_ws else 0,
                     nat.stream_of(x.device))
        outs.append((H, act))
    torch.cuda.synchronize()
    assert torch.equal(outs[1][0], outs[2][0]) and torch.equal(outs[1][1], outs[2][1])
    iu = torch.triu_indices(C, C)
    for g in range(G):
        a, b = outs[0][0][g][iu[0], iu[1]], outs[1][0][g][iu[0], iu[1]]
        assert rel_fro(b, a) <= 1e-5      # the Hessian bar: fp32 sums of 4096 terms, other order
    assert rel_fro(outs[1][1], outs[0][1]) <= 1e-5
    # (the second split call reuses the workspace: equal results show the per-item counters
    # were left zero by the first)


@pytest.mark.parametrize("C,G", [(300, 2), (64, 1), (129, 3)])
def test_finalize_exact_on_symmetric_input(C, G):
    """On a symmetric H the reference's 0.5 * (H + H^T) is the identity, so finalize must equal
    (H / h_div) / hessian_saliency_scale evaluated on the CPU bit for bit (ragged 64-tiles)."""
    r = rng(C + G)
    A = torch.from_numpy(r.standard_normal((G, C, C)).astype(np.float32))
    Hs = A + A.transpose(1, 2)
    H = Hs.to(DEV).contiguous()
    act = torch.ones(C, device=DEV)
    K.hessian_finalize(H, act, 3.0, 7.0, 2.0)
    torch.cuda.synchronize()
    assert torch.equal(H.cpu(), (Hs / 3.0) / 7.0)


def test_finalize_sanitises_nonfinite():
    H = torch.eye(70, device=DEV).repeat(2, 1, 1)
    H[1, 3, 40] = float("nan")
    H[0, 5, 5] = float("inf")
    act = torch.ones(70, device=DEV)
    bad = torch.zeros(1, dtype=torch.int32, device=DEV)
    K.hessian_finalize(H, act, 2.0, 1.0, 2.0, bad)
    torch.cuda.synchronize()
    assert int(bad.item()) == 3
    assert torch.isfinite(H).all()
    assert H[1, 3, 40] == 0 and H[1, 40, 3] == 0 and H[0, 5, 5] == 0 and H[0, 6, 6] == 0.5


def test_finalize_keeps_nonfinite_unsanitised():
    """sanitize=False (classic GPTQ): the same count, the entries (and their mirrors) kept."""
    H = torch.eye(70, device=DEV).repeat(2, 1, 1)
    H[1, 3, 40] = float("nan")
    H[0, 5, 5] = float("inf")
    bad = torch.zeros(1, dtype=torch.int32, device=DEV)
    K.hessian_finalize(H, None, 2.0, 1.0, 1.0, bad, sanitize=False)
    torch.cuda.synchronize()
    assert int(bad.item()) == 3
    assert bool(H[1, 3, 40].isnan()) and bool(H[1, 40, 3].isnan()) and H[0, 5, 5] == float("inf")
    assert int((~torch.isfinite(H)).sum()) == 3 and H[0, 6, 6] == 0.5


@pytest.mark.parametrize("sym", [True, False])
@pytest.mark.parametrize("mse", [False, True])
def test_find_params_weight_groupwise_matches_oracle(sym, mse):
    """weight_groupsize > 0 on an fp32 weight: the per-run fit expanded per element equals the
    oracle's find_params_weight_groupwise bit for bit (one-sign, all-zero and NaN runs
    included); 16-bit tensors and ragged run lengths raise."""
    from gptq_plus_mp_quant_amd import WeightQuantizer
    r = rng(21 + sym + 2 * mse)
    W = torch.from_numpy(r.standard_normal((40, 96)).astype(np.float32) * 0.03)
    W[2, :16] = W[2, :16].abs() + 0.01
    W[3, 16:32] = -W[3, 16:32].abs() - 0.01
    W[5, 32:48] = 0
    W[7, 50] = float("nan")
    q = WeightQuantizer()
    q.configure(4, perchannel=True, sym=sym, mse=mse, weight_groupsize=16)
    q.find_params(W.to(DEV))
    o = make_quantizer(4, sym, mse, weight_groupsize=16)
    o.find_params(W.clone())
    assert q.scale.shape == W.shape and q.zero.shape == W.shape
    torch.testing.assert_close(q.scale.cpu(), o.scale, rtol=0, atol=0, equal_nan=True)
    torch.testing.assert_close(q.zero.cpu(), o.zero, rtol=0, atol=0, equal_nan=True)
    with pytest.raises(NotImplementedError):
        q.find_params(W.to(DEV).half())
    q2 = WeightQuantizer()
    q2.configure(4, perchannel=True, sym=sym, weight_groupsize=7)
    with pytest.raises(RuntimeError):
        q2.find_params(W.to(DEV))


@pytest.mark.parametrize("bits,sym", [(4, True), (4, False), (3, True), (2, False), (8, True), (8, False)])
@pytest.mark.parametrize("gs", [-1, 32])
def test_find_params_bitexact(bits, sym, gs):
    r = rng(bits * 10 + sym)
    W = torch.from_numpy(r.standard_normal((77, 160)).astype(np.float32) * 0.03).to(torch.float16)
    W[3] = 0                       # all-zero row
    W[5] = W[5].abs()              # non-negative row: xmin clipped at 0
    W[9, 7] = float("nan")         # NaN propagates like torch.min / max
    q = make_quantizer(bits, sym)
    scale, zero = K.find_params(W.to(DEV), int(q.maxq), sym, gs)
    groups = range(0, 160, gs) if gs > 0 else [0]
    for k, c0 in enumerate(groups):
        qo = make_quantizer(bits, sym)
        qo.find_params(W.float()[:, c0:c0 + gs] if gs > 0 else W.float())
        assert torch.equal(scale[k].cpu(), qo.scale.flatten()) or torch.allclose(
            scale[k].cpu(), qo.scale.flatten(), rtol=0, atol=0, equal_nan=True)
        assert torch.allclose(zero[k].cpu(), qo.zero.flatten(), rtol=0, atol=0, equal_nan=True)


@pytest.mark.parametrize("bits,sym", [(4, True), (4, False), (3, True), (3, False)])
@pytest.mark.parametrize("gs", [-1, 64])
def test_find_params_mse_matches_oracle(bits, sym, gs):
    """The --w_clip grid search: the chosen (scale, zero) must equal the oracle's, except
    where two candidates' error sums tie to within summation-order rounding (reported)."""
    r = rng(100 + bits * 10 + sym)
    W = torch.from_numpy(r.standard_normal((96, 256)).astype(np.float32) * 0.03).to(torch.float16)
    W[3] = 0
    q = make_quantizer(bits, sym, mse=True)
    scale, zero = K.find_params_mse(W.to(DEV), int(q.maxq), sym, group_size=gs)
    groups = range(0, 256, gs) if gs > 0 else [0]
    maxq = float(q.maxq)

    def clip_err(x, s_, z_):
        # the search's objective (quant_utils.py:431-444) in fp64
        x, s_, z_ = x.double(), float(s_), float(z_)
        if sym:
            qv = s_ * torch.clamp(torch.round(x / s_), -(maxq + 1), maxq)
        else:
            qv = s_ * (torch.clamp(torch.round(x / s_) + z_, 0, maxq) - z_)
        return float(((qv - x).abs() ** 2.4).sum())

    mism = 0
    for k, c0 in enumerate(groups):
        Wg = W.float()[:, c0:c0 + gs] if gs > 0 else W.float()
        qo = make_quantizer(bits, sym, mse=True)
        qo.find_params(Wg)
        diff = (scale[k].cpu() != qo.scale.flatten()) | (zero[k].cpu() != qo.zero.flatten())
        mism += int(diff.sum())
        for r_ in torch.nonzero(diff).flatten().tolist():
            # a different choice is allowed only between candidates of equal error
            e_gpu = clip_err(Wg[r_], scale[k, r_].cpu(), zero[k, r_].cpu())
            e_ora = clip_err(Wg[r_], qo.scale.flatten()[r_], qo.zero.flatten()[r_])
            assert abs(e_gpu - e_ora) <= 1e-5 * e_ora, (r_, e_gpu, e_ora)
    n = 96 * len(groups)
    print(f"mse search: {mism}/{n} (row, group) choices differ from the oracle")
    assert mism <= max(1, n // 100)


def test_act_order_perm_matches_cpu_argsort():
    """perm is torch's CPU argsort(descending=True), ties in its (unstable) order, NaN first."""
    r = rng(3)
    a = torch.from_numpy(r.integers(0, 40, size=3000).astype(np.float32))
    a[17] = float("nan")
    a[2999] = float("nan")
    a[100] = -0.0
    perm, invperm = K.act_order_perm(a.to(DEV))
    ref = torch.argsort(a, descending=True)
    assert not torch.equal(ref, torch.argsort(a, descending=True, stable=True))
    assert torch.equal(perm.cpu(), ref)
    assert torch.equal(invperm.cpu(), torch.argsort(ref))
    b = torch.from_numpy(r.standard_normal(4096).astype(np.float32))
    assert torch.equal(K.act_order_perm(b.to(DEV))[0].cpu(), torch.argsort(b, descending=True))
    # the 70B down_proj width plus one (global-memory variant), heavy ties
    c = torch.from_numpy(r.integers(0, 300, size=28673).astype(np.float32))
    c[r.choice(28673, 5, replace=False)] = float("nan")
    perm, invperm = K.act_order_perm(c.to(DEV))
    ref = torch.argsort(c, descending=True)
    assert torch.equal(perm.cpu(), ref) and torch.equal(invperm.cpu(), torch.argsort(ref))


def _spd(seed, C, outlier=20.0):
    r = rng(seed)
    A = r.standard_normal((4 * C, C)).astype(np.float32)
    A[:, r.choice(C, 3, replace=False)] *= outlier
    return torch.from_numpy((A.T @ (A * r.lognormal(size=(4 * C, 1)).astype(np.float32)) / (4 * C)).astype(np.float32))


@pytest.mark.parametrize("C", [64, 200, 300, 520, 777, 1000, 1536])
def test_cholesky_chain(C):
    H = _spd(C, C)
    Hinv_init_o, Hinv_o, p, fb, att = hessian_inverse_with_fallback(H, 0.01)
    Hw = H.to(DEV).clone()
    ws = K.chol_workspace(C, DEV)
    Hinv = torch.empty(C, C, device=DEV)
    Hinit = torch.empty(C, C, device=DEV)
    hdiag = torch.empty(C, device=DEV)
    info = K.chol_hinv_attempt(Hw, 0.01, ws, Hinv, Hinit, Hinv_diag=hdiag)
    torch.cuda.synchronize()
    assert int(info.item()) == 0
    assert rel_fro(Hinv, Hinv_o) <= 1e-4
    assert rel_fro(Hinit, Hinv_init_o) <= 1e-4
    # the diagonal output (column norms of L^-1) against the formed H^-1: fp64 sums in two
    # orders, rounded to fp32 -- equal up to one fp32 rounding step
    assert float(((hdiag - torch.diagonal(Hinit)).abs() / torch.diagonal(Hinit)).max()) <= 2 ** -23
    assert torch.equal(Hinv, torch.triu(Hinv)) and (torch.diag(Hinv) > 0).all()
    assert torch.equal(Hinit, Hinit.T)
    # float64 truth on the same damped matrix
    Hd = Hw.double().cpu().numpy()
    inv = np.linalg.inv(Hd)
    U = scipy.linalg.cholesky(inv, lower=False)
    assert rel_fro(Hinit, torch.from_numpy(inv)) <= 1e-5
    assert rel_fro(Hinv, torch.from_numpy(U)) <= 1e-5
    d_true = torch.from_numpy(np.diag(inv).copy())
    assert float(((hdiag.double().cpu() - d_true).abs() / d_true).max()) <= 1e-5
    # damping applied in place exactly like the reference's first attempt
    Hd_ref = H.clone()
    idx = torch.arange(C)
    Hd_ref[idx, idx] += 0.01 * torch.mean(torch.diag(H))
    assert rel_fro(Hw, Hd_ref) <= 1e-7


@pytest.mark.parametrize("C", [8200, 8520])
def test_cholesky_chain_wide_panels(C):
    """C >= 8192 runs 512-wide panels (K = 512 panel updates, 4-row tile bands), each factored
    as two 256-wide halves joined by a rank-256 update, with a ragged last panel (C = 8200: 8
    columns, one pass; C = 8520: 328 columns, halves of 256 and 72); checked against the float64
    upper Cholesky factor of H_work^-1 (numpy / scipy on the host)."""
    g = torch.Generator(device=DEV)
    g.manual_seed(C)
    A = torch.randn(2 * C, C, device=DEV, generator=g)
    A[:, :3] *= 20.0
    H = (A.T @ (A * torch.rand(2 * C, 1, device=DEV, generator=g))) / (2 * C)
    del A
    Hw = H.clone()
    ws = K.chol_workspace(C, DEV)
    Hinv = torch.empty(C, C, device=DEV)
    hdiag = torch.empty(C, device=DEV)
    info = K.chol_hinv_attempt(Hw, 0.01, ws, Hinv, None, Hinv_diag=hdiag)
    torch.cuda.synchronize()
    assert int(info.item()) == 0
    assert torch.equal(Hinv, torch.triu(Hinv)) and bool((torch.diag(Hinv) > 0).all())
    Hd = Hw.double().cpu().numpy()
    inv = np.linalg.inv(Hd)
    U_true = torch.from_numpy(scipy.linalg.cholesky(inv, lower=False))
    err = rel_fro(Hinv, U_true)
    d_true = torch.from_numpy(np.diag(inv).copy())
    derr = float(((hdiag.double().cpu() - d_true).abs() / d_true).max())
    print(f"C={C}: rel-Frobenius vs float64 truth {err:.2e}, diag(H^-1) max rel {derr:.2e}")
    assert err <= 1e-5 and derr <= 1e-5


def test_cholesky_lookahead_repeatable():
    """The chain overlaps each panel's far trailing update (second stream) with the next panel's
    factorisation; the results must not depend on how the two interleave.  C = 14336 (28
    panels of 512, the down_proj width): six attempts on the same matrices give the same bits.
    Regression check for a staging-ring race (a stage refilled by one wave's direct-to-LDS
    load before another wave's read of it had completed) that concurrent kernels exposed."""
    C, nb = 14336, 4
    g = torch.Generator(device=DEV)
    g.manual_seed(5)
    A = torch.randn(2 * C, C, device=DEV, generator=g)
    H = (A.T @ A) / (2 * C)
    del A
    Hs = H.unsqueeze(0).repeat(nb, 1, 1).contiguous()
    del H
    ws = K.chol_workspace(C, DEV, nb)
    Hinv = torch.empty(nb, C, C, device=DEV)
    hd = torch.empty(nb, C, device=DEV)
    ref = None
    for rep in range(6):
        Hw = Hs.clone()
        info = K.chol_hinv_attempt(Hw, [0.01] * nb, ws, Hinv, None, Hinv_diag=hd)
        torch.cuda.synchronize()
        assert info.tolist() == [0] * nb
        if ref is None:
            ref = (Hinv.clone(), hd.clone())
        else:
            assert torch.equal(Hinv, ref[0]) and torch.equal(hd, ref[1]), f"attempt {rep} differs"
        del Hw


@pytest.mark.parametrize("C", [200, 600])
def test_cholesky_batch_independent_entries(C):
    """Batched attempt: each matrix gets its own damping, skipped entries stay untouched, and a
    non-positive-definite entry fails alone (C = 600 runs the rank-256 panel updates)."""
    Hs = [_spd(7, C), _spd(8, C), -torch.eye(C), _spd(9, C)]
    damps = [0.01, 0.02, 0.01, 0.0]          # last entry skipped
    Hw = torch.stack(Hs).to(DEV).contiguous()
    before = Hw.clone()
    ws = K.chol_workspace(C, DEV, 4)
    Hinv = torch.zeros(4, C, C, device=DEV)
    Hinit = torch.zeros(4, C, C, device=DEV)
    hdiag = torch.zeros(4, C, device=DEV)
    info = K.chol_hinv_attempt(Hw, damps, ws, Hinv, Hinit, Hinv_diag=hdiag)
    torch.cuda.synchronize()
    codes = info.tolist()
    assert codes[0] == 0 and codes[1] == 0 and codes[2] > 0 and codes[3] == -1
    assert torch.equal(Hw[3], before[3]) and not Hinv[3].any() and not hdiag[3].any()
    for b in (0, 1):
        Hi_o, Hv_o, *_ = hessian_inverse_with_fallback(Hs[b], damps[b])
        assert rel_fro(Hinv[b], Hv_o) <= 1e-4 and rel_fro(Hinit[b], Hi_o) <= 1e-4
        assert rel_fro(hdiag[b], torch.diagonal(Hi_o)) <= 1e-5


@pytest.mark.parametrize("neg", [0.05, 0.3, 5.0])
def test_cholesky_retry_schedule(neg):
    """Indefinite diagonal H: the damping retries (cumulative on the same working copy)
    must stop at the same attempt as the reference's loop, or fall back to identity."""
    from gptq_plus_mp_quant_amd.gptq_plus import hessian_inverse_chain
    d = torch.tensor([-neg, 1.0, 1.0, 1.0, 2.0] * 16)
    H = torch.diag(d)
    _, _, p_o, fb_o, att_o = hessian_inverse_with_fallback(H, 0.01)
    Hw = H.to(DEV).clone()
    Hinv = torch.empty(80, 80, device=DEV)
    (p, fb, att), = hessian_inverse_chain(DEV, Hw, Hinv, None, K.chol_workspace(80, DEV), 0.01)
    assert (att, fb) == (att_o, fb_o) and abs(p - p_o) < 1e-12
    if fb:
        assert torch.equal(Hinv.cpu(), torch.eye(80))


def test_cholesky_near_singular_dense():
    """A dense H whose damped working copy is positive definite by a margin of ~1e-8 of its
    norm: the reference's fp32 chain (potrf, cholesky_inverse, potrf) breaks down at
    damp_percent 0.01 and succeeds on the retry at 0.0115; the fp64 factorisation succeeds at
    0.01 (the documented difference in the number of retries).  Pinned: the oracle's attempt
    count, this build's, the factor at 0.01 against fp64 truth on the same damped matrix, and
    the factor at the oracle's damping against the oracle's."""
    from gptq_plus_mp_quant_amd.gptq_plus import hessian_inverse_chain
    C = 64
    r = rng(0)
    Q, _ = np.linalg.qr(r.standard_normal((C, C)))
    lam = np.linspace(1.0, 2.0, C)
    delta = 1e-6
    lam[0] = -0.01 * (1 - delta) * lam[1:].sum() / (C + 0.01 * (1 - delta))   # lam_min = -(1 - delta) damp
    H = torch.from_numpy((Q * lam) @ Q.T).float()
    _, Hv_o, p_o, fb_o, att_o = hessian_inverse_with_fallback(H, 0.01)
    # 2 attempts on the x86 hosts measured (MKL); the breakdown depends on the LAPACK build
    print(f"near-singular C={C}: fp32 reference chain attempts {att_o} (damp {p_o:.4f})", flush=True)
    assert not fb_o

    ws = K.chol_workspace(C, DEV)
    Hw = H.to(DEV).clone()
    Hinv = torch.empty(C, C, device=DEV)
    (p, fb, att), = hessian_inverse_chain(DEV, Hw, Hinv, None, ws, 0.01)
    assert (att, fb) == (1, False) and abs(p - 0.01) < 1e-12 and att_o >= att
    Hd = Hw.double().cpu()                            # the damped working copy the chain factored
    assert float(torch.linalg.eigvalsh(Hd)[0]) > 0.0
    U = torch.linalg.cholesky(torch.cholesky_inverse(torch.linalg.cholesky(Hd)), upper=True)
    assert rel_fro(Hinv, U.float()) <= 1e-5

    if att_o > 1:                                     # at the reference's final damping both agree
        Hw2 = H.to(DEV).clone()
        Hinv2 = torch.empty(C, C, device=DEV)
        (p2, fb2, att2), = hessian_inverse_chain(DEV, Hw2, Hinv2, None, ws, p_o)
        assert (att2, fb2) == (1, False)
        assert rel_fro(Hinv2, Hv_o) <= 1e-4


def _check_terms(G, Hinv, beta, Z, GH, beta_o):
    """beta against the oracle's to an absolute 2^-21: the reference's 1 - sqrt(1 - ratio) in
    fp32 cancels (beta ~ 1e-4 keeps ~10 of its 24 bits), so a last-bit difference of ratio --
    from c summed in another order -- moves beta by up to an ulp of 1.  Z and GHinv follow beta
    linearly, so they are checked against the oracle's products formed with the kernel's beta
    (fp32 on the CPU: 1e-5)."""
    beta_c = beta.cpu()
    assert float((beta_c - beta_o).abs().max()) <= 2.0 ** -21
    Z_o = G.matmul(Hinv.T) * beta_c.unsqueeze(1)
    assert rel_fro(Z, Z_o) <= 1e-5
    assert rel_fro(GH, Z.cpu().matmul(Hinv)) <= 1e-5


@pytest.mark.parametrize("alpha,ref_loss", [(0.0, 0.0), (0.05, 3e5), (0.05, 0.0)])
@pytest.mark.parametrize("nt", [False, True], ids=["tile64", "nt128"])
def test_gptqplus_terms(alpha, ref_loss, nt):
    """One subgroup against the oracle; nt: with the Hinv^T workspace the beta_mode 1 products
    run on the batched 128-tile NT kernel (C = 192 is a multiple of 16), else on 64-tiles."""
    C, R_s = 192, 48
    H = _spd(99, C)
    Hinit_o, Hinv_o, *_ = hessian_inverse_with_fallback(H, 0.01)
    Gs = torch.from_numpy(rng(4).standard_normal((R_s, C)).astype(np.float32))
    a_eff = alpha / (R_s * 2 * C) if alpha > 0 else 0.0
    beta_o, Z_o, GH_o, _ = gradient_terms(Gs, Hinit_o, Hinv_o, alpha, ref_loss, R_s * 2, C)
    mode = 1 if alpha > 0 else 0
    beta = torch.empty(R_s if mode else 1, device=DEV)
    Z = torch.empty(R_s, C, device=DEV)
    GH = torch.empty(R_s, C, device=DEV)
    GH0 = torch.empty(R_s, C, device=DEV) if mode else None
    HinvT = torch.empty(C, C, device=DEV) if (mode and nt) else None
    nz = torch.zeros(1, dtype=torch.int32, device=DEV)
    # beta_mode 1 takes diag(H^-1) and forms G Hinv_init as (G Hinv^T) Hinv (Hinv^T Hinv = Hinv_init
    # up to the oracle's fp32 factorisation, so the bars below also bound that rewrite)
    hdiag = torch.diagonal(Hinit_o).contiguous().to(DEV) if mode else None
    K.gptqplus_terms(Gs.to(DEV), hdiag, Hinv_o.to(DEV), a_eff, ref_loss, mode, beta, Z, GH, GH0, nz, HinvT)
    torch.cuda.synchronize()
    if alpha > 0 and ref_loss > 0:
        assert beta_o.min() > 0.0 and int(nz.item()) == 1
        _check_terms(Gs, Hinv_o, beta, Z, GH, beta_o)
    else:
        assert float(beta[0]) == 0.0 and int(nz.item()) == 0
        assert not Z.any() and not GH.any()


def test_gptqplus_terms_batched_nt():
    """Three subgroups in one call (ragged R_s = 200 against the 128-row tiles, C = 400 with a
    ragged last column tile): each against the oracle's terms of its own (H^-1, G rows), and
    the NT-kernel results against the 64-tile path on the same inputs."""
    C, R_s, nsub = 400, 200, 3
    Gs = torch.from_numpy(rng(6).standard_normal((nsub * R_s, C)).astype(np.float32))
    ref, hinvs, diags = [], [], []
    for b in range(nsub):
        Hinit_o, Hinv_o, *_ = hessian_inverse_with_fallback(_spd(120 + b, C), 0.01)
        ref.append(gradient_terms(Gs[b * R_s:(b + 1) * R_s], Hinit_o, Hinv_o, 0.05, 3e5, nsub * R_s, C))
        hinvs.append(Hinv_o)
        diags.append(torch.diagonal(Hinit_o))
    Hinv = torch.stack(hinvs).to(DEV).contiguous()
    hdiag = torch.stack(diags).to(DEV).contiguous()
    a_eff = 0.05 / (nsub * R_s * C)
    outs, errs = [], []
    for HinvT in (torch.empty(nsub, C, C, device=DEV), None):
        beta = torch.empty(nsub * R_s, device=DEV)
        Z = torch.empty(nsub * R_s, C, device=DEV)
        GH = torch.empty(nsub * R_s, C, device=DEV)
        GH0 = torch.empty(nsub * R_s, C, device=DEV)
        nz = torch.full((nsub,), 7, dtype=torch.int32, device=DEV)
        K.gptqplus_terms(Gs.to(DEV), hdiag, Hinv, a_eff, 3e5, 1, beta, Z, GH, GH0, nz, HinvT)
        torch.cuda.synchronize()
        assert nz.tolist() == [1] * nsub
        if HinvT is not None:
            assert torch.equal(HinvT.cpu(), Hinv.cpu().transpose(1, 2))
        for b in range(nsub):
            rows = slice(b * R_s, (b + 1) * R_s)
            beta_o, Z_o, GH_o, GH0_o = ref[b]
            errs.append(dict(nt=HinvT is not None, sub=b, gh0=rel_fro(GH0[rows], GH0_o),
                             beta_abs=float((beta[rows].cpu() - beta_o).abs().max()), beta_max=float(beta_o.max())))
            _check_terms(Gs[rows], hinvs[b], beta[rows], Z[rows], GH[rows], beta_o)
        outs.append((beta, Z, GH, GH0))
    for e in errs:
        print(e)
        assert e["gh0"] <= 1e-5, e
    # the two kernel paths: GH0 (before the cancellation) to 1e-5, beta to the same 2^-21
    assert rel_fro(outs[0][3], outs[1][3]) <= 1e-5
    assert float((outs[0][0] - outs[1][0]).abs().max()) <= 2.0 ** -21


def test_gptqplus_terms_zero_beta_nonfinite():
    """beta = 0 (alpha = 0): Z = (G Hinv^T) * 0 is zero except where a product or partial sum
    is not finite, where the reference yields NaN: rows with inf / NaN in G, and a row whose
    (same-sign) products overflow fp32.  The kernel skips the product only when it can show Z
    is zero.  Rows with finite G stay exactly zero; each bad row holds NaN in Z (the product
    skips the structurally zero part of Hinv, so the NaN positions inside a bad row may be
    fewer than the reference's) and is all NaN in GHinv = Z Hinv, as in the oracle."""
    C, R_s = 192, 48
    H = _spd(98, C)
    Hinit_o, Hinv_o, *_ = hessian_inverse_with_fallback(H, 0.01)
    Gs = torch.from_numpy(rng(5).standard_normal((R_s, C)).astype(np.float32))
    Gs[3, 17] = float("inf")
    Gs[10, 0] = float("nan")
    h0 = Hinv_o[0].double()
    Gs[20] = (torch.sign(h0) * min(3.0e38, 5.0e38 / float(h0.abs().sum()))).float()
    bad = [3, 10, 20]
    good = [r for r in range(R_s) if r not in bad]
    beta_o, Z_o, GH_o, _ = gradient_terms(Gs, Hinit_o, Hinv_o, 0.0, 0.0, R_s * 2, C)
    assert bool(Z_o[20, 0].isnan())                # the overflow row does overflow
    beta = torch.empty(1, device=DEV)
    Z = torch.empty(R_s, C, device=DEV)
    GH = torch.empty(R_s, C, device=DEV)
    nz = torch.zeros(1, dtype=torch.int32, device=DEV)
    K.gptqplus_terms(Gs.to(DEV), None, Hinv_o.to(DEV), 0.0, 0.0, 0, beta, Z, GH, None, nz)
    torch.cuda.synchronize()
    Zc, GHc = Z.cpu(), GH.cpu()
    assert float(beta[0]) == 0.0 and int(nz.item()) == 1
    for z, gh in ((Zc, GHc), (Z_o, GH_o)):
        assert not z[good].any() and not gh[good].any()
        for r in bad:
            assert z[r].isnan().any() and gh[r].isnan().all()
    assert bool(Zc[20, 0].isnan())


@pytest.mark.parametrize("G,R_s,C,i1,cnt,gmode,sos", [
    (2, 96, 300, 64, 64, 0, 1.0),        # frozen, ragged row and column tiles
    (4, 256, 1024, 128, 128, 0, 1.0),    # frozen, interior tiles
    (2, 96, 640, 128, 128, 1, 1.0),      # surrogate_block: gh_eff = GH + beta (W - W_anchor)
    (1, 200, 516, 0, 128, 3, 0.7),       # block_gd: the W update scaled by second_order_scale
    (2, 64, 300, 100, 60, 0, 1.0),       # count % 8 != 0: the general kernel runs instead
])
def test_trailing_update_with_z(G, R_s, C, i1, cnt, gmode, sos):
    """The outer update with the GPTQ+ terms (gptq_plus_utils.py:1500-1570) against the
    reference's expressions evaluated by torch on the CPU:
      G_Update = count * gh_eff - einsum("ij,j,jk->ik", Z1, D, Hinv[i1:i2, i2:])
      W[:, i2:] -= Err1 @ Hinv[i1:i2, i2:] + G_Update       (x second_order_scale in block_gd)
      GH[:, i2:] -= Z[:, i1:i2] @ Hinv[i1:i2, i2:]
    bit for bit where the k-ordered kernel runs (count % 8 == 0), within 1e-6 otherwise.  (The
    bit-exact cases keep C - i2 a multiple of 16 or, for the shapes measured, 12: MKL on the
    AMD host sums some narrower column remainders with separate multiplies and adds, where it
    otherwise forms the fused chain, so the CPU reference itself changes with the host there.)"""
    r = rng(8 + cnt + gmode)
    Hinv = torch.from_numpy(np.triu(r.standard_normal((G, C, C))).astype(np.float32) * 0.1)
    W = torch.from_numpy(r.standard_normal((G * R_s, C)).astype(np.float32))
    GH = torch.from_numpy(r.standard_normal((G * R_s, C)).astype(np.float32) * 1e-3)
    Z = torch.from_numpy(r.standard_normal((G * R_s, C)).astype(np.float32) * 1e-3)
    err = torch.from_numpy(r.standard_normal((G * R_s, cnt)).astype(np.float32))
    anchor = W + torch.from_numpy(r.standard_normal((G * R_s, C)).astype(np.float32) * 1e-2)
    beta = torch.from_numpy(r.uniform(0, 0.5, G * R_s).astype(np.float32))
    Wd, GHd = W.to(DEV), GH.to(DEV)
    nz = torch.ones(1, dtype=torch.int32, device=DEV)
    surr = gmode in (1, 2)
    K.trailing_update(Wd, GHd, Z.to(DEV), Hinv.to(DEV), R_s, i1, cnt, err.to(DEV), nz, gmode,
                      anchor=anchor.to(DEV) if surr else None, beta=beta.to(DEV) if surr else None,
                      second_order_scale=sos)
    torch.cuda.synchronize()
    i2 = i1 + cnt
    D = torch.arange(cnt - 1, -1, -1, dtype=torch.float32)                    # :1175
    for s in range(G):
        rows = slice(s * R_s, (s + 1) * R_s)
        Hb = Hinv[s, i1:i2, i2:]
        Z1 = Z[rows, i1:i2]
        ghr = GH[rows, i2:]
        if surr:                                                              # :580-584
            ghr = ghr + beta[rows].unsqueeze(1) * (W[rows, i2:] - anchor[rows, i2:])
        gup = cnt * ghr - torch.einsum("ij,j,jk->ik", Z1, D, Hb)
        tot = err[rows].matmul(Hb) + gup
        W_ref = W[rows, i2:] - (sos * tot if gmode == 3 else tot)
        GH_ref = GH[rows, i2:] - Z1.matmul(Hb)
        if cnt % 8 == 0:
            assert torch.equal(Wd[rows, i2:].cpu(), W_ref)
            assert torch.equal(GHd[rows, i2:].cpu(), GH_ref)
        else:
            assert rel_fro(Wd[rows, i2:], W_ref) <= 1e-6
            assert rel_fro(GHd[rows, i2:], GH_ref) <= 1e-6
        assert torch.equal(Wd[rows, :i2].cpu(), W[rows, :i2])
        assert torch.equal(GHd[rows, :i2].cpu(), GH[rows, :i2])


@pytest.mark.parametrize("G,R_s,C,B,qmode,atomic", [
    (2, 96, 328, 128, "channel", False),     # last block 72 wide
    (1, 200, 280, 128, "static", False),     # last block 24 wide (the narrow column loop)
    (3, 48, 384, 128, "dynamic", False),
    (2, 64, 264, 64, "channel", True),       # atomic blocks, 64 wide
    (4, 40, 256, 32, "static", True),
])
def test_quant_block_lookahead_equals_two_calls(G, R_s, C, B, qmode, atomic):
    """rq_quant_block_lookahead (block k's W-only trailing update and block k+1's column loop in
    one launch) against rq_trailing_update + rq_quant_block over a whole column loop: codes,
    every block's err and the working weight equal bit for bit."""
    r = rng(70 + C + B)
    R = G * R_s
    Hs = torch.stack([_spd(80 + g, C) for g in range(G)]).to(DEV).contiguous()
    ws = K.chol_workspace(C, DEV, G)
    Hinv = torch.empty(G, C, C, device=DEV)
    info = K.chol_hinv_attempt(Hs.clone(), [0.01] * G, ws, Hinv)
    assert info.tolist() == [0] * G
    W0 = torch.from_numpy(r.standard_normal((R, C)).astype(np.float32)).to(DEV)
    maxq, sym = 7, 0
    nblocks = (C + B - 1) // B
    scale = col_group = dyn = None
    qm = {"channel": nat.RQ_QMODE_CHANNEL, "static": nat.RQ_QMODE_STATIC, "dynamic": nat.RQ_QMODE_DYNAMIC}[qmode]
    if qmode == "channel":
        scale = (W0.abs().amax(1) / maxq).contiguous()
    elif qmode == "static":
        ng = (C + 63) // 64
        scale = torch.from_numpy(r.uniform(0.2, 0.6, (ng, R)).astype(np.float32)).to(DEV).reshape(-1)
        col_group = (torch.arange(C, device=DEV) // 64).to(torch.int32)
    zero = torch.zeros_like(W0)
    nz0 = torch.zeros(1, dtype=torch.int32, device=DEV)
    out = {}
    for mode in ("two_calls", "lookahead"):
        Wp = W0.clone()
        codes = torch.zeros((R, C), dtype=torch.int16, device=DEV)
        errs = [torch.empty((R, B), device=DEV) for _ in range(2)]
        dyn = torch.zeros((nblocks, R), device=DEV) if qmode == "dynamic" else None
        seen = []
        for b, i1 in enumerate(range(0, C, B)):
            i2 = min(i1 + B, C)
            at = atomic and i2 < C
            ds = dyn[b] if dyn is not None else None
            e = errs[b % 2]
            if mode == "two_calls" or b == 0:
                K.quant_block(Wp, Hinv, zero, zero, R_s, i1, i2 - i1, qm, scale, col_group, ds, maxq, sym, at,
                              nz0, codes, e)
            if i2 < C:
                if mode == "two_calls":
                    K.trailing_update(Wp, zero, zero, Hinv, R_s, i1, i2 - i1, e, nz0, z_zero=True)
                else:
                    n2 = min(i2 + B, C)
                    K.quant_block_lookahead(Wp, Hinv, R_s, i1, i2 - i1, e, n2 - i2, qm, scale, col_group,
                                            dyn[b + 1] if dyn is not None else None, maxq, sym,
                                            atomic and n2 < C, codes, errs[(b + 1) % 2])
            if mode == "two_calls" or b == 0:
                seen.append(e.reshape(-1)[:R * (i2 - i1)].clone())
            if mode == "lookahead" and i2 < C:
                n2 = min(i2 + B, C)
                seen.append(errs[(b + 1) % 2].reshape(-1)[:R * (n2 - i2)].clone())
        torch.cuda.synchronize()
        out[mode] = (Wp, codes, seen, dyn)
    a, b = out["two_calls"], out["lookahead"]
    assert torch.equal(a[1], b[1]), "codes"
    assert len(a[2]) == len(b[2]) == nblocks
    for k, (x, y) in enumerate(zip(a[2], b[2])):
        assert torch.equal(x, y), f"err of block {k}"
    assert torch.equal(a[0], b[0]), "working weight"
    if qmode == "dynamic":
        assert torch.equal(a[3], b[3])
    assert not zero.any()


@pytest.mark.parametrize("G,R_s,C,i1,cnt,gmode,sos", [
    (2, 96, 300, 64, 64, 0, 1.0),        # ragged row and column tiles
    (4, 256, 1024, 128, 128, 0, 1.0),    # interior 128x128 tiles only
    (1, 200, 516, 0, 128, 3, 0.7),       # block_gd: the update scaled by second_order_scale
    (3, 130, 392, 256, 8, 0, 1.0),       # a single 8-deep K step
    (2, 64, 300, 100, 60, 0, 1.0),       # count % 8 != 0: the general kernel runs instead
])
def test_trailing_update_w_only(G, R_s, C, i1, cnt, gmode, sos):
    """Z identically zero (z_zero=True): W[:, i2:] -= f err Hinv[i1:i2, i2:].  Where the W-only
    kernel runs (count % 8 == 0) it forms the product as a k-ordered fused multiply-add chain,
    like torch's CPU matmul, so W equals the reference expression evaluated on the CPU bit for
    bit; the general kernel (and count % 8 != 0) is checked against float64 and that result."""
    r = rng(10 + cnt)
    Hinv = torch.from_numpy(np.triu(r.standard_normal((G, C, C))).astype(np.float32) * 0.1)
    W = torch.from_numpy(r.standard_normal((G * R_s, C)).astype(np.float32))
    err = torch.from_numpy(r.standard_normal((G * R_s, cnt)).astype(np.float32))
    zero = torch.zeros_like(W).to(DEV)
    nz0 = torch.zeros(1, dtype=torch.int32, device=DEV)
    Hd, ed = Hinv.to(DEV), err.to(DEV)
    Wf, Wg = W.to(DEV), W.to(DEV)
    K.trailing_update(Wf, zero, zero, Hd, R_s, i1, cnt, ed, nz0, gmode, second_order_scale=sos, z_zero=True)
    K.trailing_update(Wg, zero, zero, Hd, R_s, i1, cnt, ed, nz0, gmode, second_order_scale=sos)
    torch.cuda.synchronize()
    i2 = i1 + cnt
    f = sos if gmode == 3 else 1.0
    for s in range(G):
        rows = slice(s * R_s, (s + 1) * R_s)
        ref = W[rows, i2:].double() - f * (err[rows].double() @ Hinv[s, i1:i2, i2:].double())
        assert rel_fro(Wf[rows, i2:], ref) <= 1e-6
        assert rel_fro(Wf[rows, i2:], Wg[rows, i2:]) <= 1e-6
        assert torch.equal(Wf[rows, :i2].cpu(), W[rows, :i2])
        if cnt % 8 == 0:
            second = err[rows].matmul(Hinv[s, i1:i2, i2:])                    # :1512-1519
            exact = W[rows, i2:] - (f * second if gmode == 3 else second)
            assert torch.equal(Wf[rows, i2:].cpu(), exact)
    assert not zero.any()


@pytest.mark.parametrize("R_s,C,wdt,ldpad,perm_on", [
    (40, 136, torch.float16, 0, True),      # 16-byte rows, 256 threads
    (33, 130, torch.bfloat16, 3, True),     # row length / stride not whole 16 bytes: element loads
    (9, 20000, torch.float16, 0, True),     # fp16 rows above 32 KB (1024 threads), fp32 G rows above 64 KB
    (6, 45000, torch.float32, 0, False),    # fp32 rows above 160 KB: the column kernels
    (5, 1, torch.float32, 0, True),         # C = 1: no index scratch in H_sub
])
def test_prepare_subgroup_gathers_exact(R_s, C, wdt, ldpad, perm_on):
    """rq_prepare_subgroup against torch indexing, bit for bit: W_sub = W[:, perm] with dead
    columns (H_g[p, p] == 0) zeroed, G_sub = G[:, perm], H_sub = H_g[perm][:, perm] with a dead
    diagonal set to 1; then rq_writeback's un-permute of int16 codes against torch."""
    r = rng(R_s + C)
    ld = C + ldpad
    Wfull = torch.from_numpy(r.standard_normal((R_s, ld)).astype(np.float32)).to(wdt)
    W = Wfull.to(DEV)[:, :C] if ldpad else Wfull.to(DEV)
    G = torch.from_numpy(r.standard_normal((R_s, C)).astype(np.float32)).to(DEV)
    d = torch.from_numpy(r.standard_normal(C).astype(np.float32) ** 2 + 0.5)
    dead = torch.from_numpy(r.random(C) < 0.1)
    d[dead] = 0.0
    if C <= 2048:
        A = torch.from_numpy(r.standard_normal((C, C)).astype(np.float32)) * 0.01
        Hg = (A + A.T)
        Hg[torch.arange(C), torch.arange(C)] = d
        Hg[dead, :] = 0.0
        Hg[:, dead] = 0.0
    else:
        Hg = None
    perm = torch.from_numpy(r.permutation(C)).to(torch.int64) if perm_on else torch.arange(C)
    W_sub = torch.full((R_s, C), 7.0, device=DEV)
    G_sub = torch.full((R_s, C), 7.0, device=DEV)
    if Hg is not None:
        Hg_d = Hg.to(DEV).contiguous()
        H_sub = torch.empty(C, C, device=DEV)
    else:                                             # diagonal H: the W / G gathers are the point
        Hg_d = torch.zeros(C, C, device=DEV)
        Hg_d[torch.arange(C), torch.arange(C)] = d.to(DEV)
        H_sub = torch.empty(C, C, device=DEV)
    K.prepare_subgroup(W, G, Hg_d, perm.to(DEV) if perm_on else None, W_sub, G_sub, H_sub)
    torch.cuda.synchronize()
    Wc = W.float().cpu()
    pd = perm
    exp_W = Wc[:, pd].clone()
    exp_W[:, dead[pd]] = 0.0
    assert torch.equal(W_sub.cpu(), exp_W)
    assert torch.equal(G_sub.cpu(), G.cpu()[:, pd])
    if C <= 20000:                                    # H_sub checked where the host copies stay small
        pg = pd.to(DEV)
        exp_H = Hg_d[pg][:, pg]
        dd = dead[pd].nonzero().flatten().to(DEV)
        exp_H[dd, dd] = 1.0
        assert torch.equal(H_sub, exp_H)
    del Hg_d, H_sub

    # write-back: codes in the permuted order -> q[:, c] = fp16(scale[r] * codes[r, invperm[c]])
    codes = torch.from_numpy(r.integers(-8, 8, size=(R_s, C)).astype(np.int16)).to(DEV)
    codes[0, 0] = -32768                              # a NaN weight
    scale = torch.from_numpy(r.random(R_s).astype(np.float32) * 0.1 + 0.01).to(DEV)
    invperm = torch.argsort(perm).to(DEV)
    q = torch.empty(R_s, C, dtype=torch.float16, device=DEV)
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    K.writeback(codes, invperm, nat.RQ_QMODE_CHANNEL, scale, None, None, 128, q, nan_flag=flag)
    torch.cuda.synchronize()
    cf = codes.cpu().float()
    cf[codes.cpu() == -32768] = float("nan")
    exp_q = (scale.cpu().unsqueeze(1) * cf[:, invperm.cpu()]).to(torch.float16)
    torch.testing.assert_close(q.cpu(), exp_q, rtol=0, atol=0, equal_nan=True)
    assert int(flag.item()) == 1
