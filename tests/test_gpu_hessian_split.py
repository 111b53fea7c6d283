"""The split-operand Hessian kernels (the default for fp16 and bf16 X; for fp32 X the opt-in
"split16" mode's kernel, the default there being the fp32-MFMA kernel) against exact
arithmetic and the fp32-MFMA kernel.

The reference forms H = X^T (s * X) in fp32 (gptq_plus_utils.py:842-847): each product is
x * fl32(x * s).  The exact value of that sum is computed here in float64 (each product of an
fp16 / bf16 x and an fp32 w is exact in float64, and float64 sums of a few thousand terms are
accurate to ~1e-13 relative), and both kernels are held to it.  Bars: rel-Frobenius <= 1e-6
(fp32 accumulation over n tokens), per-entry error <= 1e-5 of sqrt(|H_ii H_jj|) on inputs with
column magnitudes over twelve decades, and the split kernel with exact products (bf16, or
fp16 with "split16x3", the default) no less accurate than the fp32 kernel (within 1.5x); the
opt-in fp16 two-piece products ("split16", each within 2^-23 relative) within 2x of it.  Results are bitwise reproducible, and non-finite inputs give
non-finite entries in the same places as the fp32 kernel."""
import numpy as np
import pytest
import torch

from gptq_plus_mp_quant_amd import kernels as K
from tests._util import rel_fro, rng

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _run(x, sal, mode):
    n, C = x.shape
    G = sal.shape[1]
    H = torch.zeros(G, C, C, device=DEV)
    a = torch.zeros(C, device=DEV)
    with K.hessian_math(mode):
        K.hessian_accum(x.to(DEV), sal.to(DEV).contiguous(), H, a)
    torch.cuda.synchronize()
    iu = torch.triu_indices(C, C)
    return H.cpu(), a.cpu(), iu


def _exact(x, sal):
    """sum_t x_ti * fl32(x_tj * s_t) in float64 (upper triangle is what the kernels form)."""
    xf = x.float()
    out = []
    for g in range(sal.shape[1]):
        w = (xf * sal[:, g:g + 1]).double()               # fl32(x * s), exactly representable
        out.append(xf.double().T @ w)
    return torch.stack(out), (xf.double() ** 2).sum(0)


def _upper(H, iu):
    return H[:, iu[0], iu[1]]


@pytest.mark.parametrize("mode", ["split16", "split16x3"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("n,C,G", [(4096, 512, 2), (2048, 1000, 3), (33, 385, 1), (5, 130, 2), (300, 17, 1)])
def test_split_matches_exact_sum(mode, dtype, n, C, G):
    r = rng(1000 + n + C + G)
    X = r.standard_normal((n, C), dtype=np.float32)
    X[:, r.choice(C, min(8, C), replace=False)] *= 20.0
    x = torch.from_numpy(X).to(dtype)
    sal = torch.from_numpy(np.minimum(r.lognormal(size=(n, G)), 10.0).astype(np.float32))
    ref, act_ref = _exact(x, sal)
    Hs, acts, iu = _run(x, sal, mode)
    Hf, actf, _ = _run(x, sal, "fp32")
    es = rel_fro(_upper(Hs, iu), _upper(ref, iu))
    ef = rel_fro(_upper(Hf, iu), _upper(ref, iu))
    print(f"{mode} {dtype} n={n} C={C} G={G}: rel err split {es:.3e}  fp32 {ef:.3e}")
    assert es <= 1e-6 and ef <= 1e-6
    two_piece = mode == "split16" and dtype == torch.float16
    assert es <= (2.0 if two_piece else 1.5) * ef + 1e-8
    assert rel_fro(acts, act_ref) <= 1e-6


@pytest.mark.parametrize("mode", ["split16", "split16x3"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_split_wide_dynamic_range(mode, dtype):
    """Columns from 1e-5 to 1e4 in magnitude (fp16: up to near its 65504 limit) and saliencies
    from 1e-3 to 1e3: x * s overflows fp16, and small columns fall far below the scaled range of
    the large ones.  The per-column exponent keeps every entry at fp32 accuracy."""
    r = rng(77)
    n, C, G = 2048, 384, 2
    mags = np.logspace(-5, 4, C).astype(np.float32)
    r.shuffle(mags)
    X = r.standard_normal((n, C)).astype(np.float32) * mags
    if dtype == torch.float16:
        X = np.clip(X, -60000, 60000)
    x = torch.from_numpy(X).to(dtype)
    sal = torch.from_numpy(np.exp(r.uniform(np.log(1e-3), np.log(1e3), size=(n, G))).astype(np.float32))
    ref, _ = _exact(x, sal)
    Hs, _, iu = _run(x, sal, mode)
    Hf, _, _ = _run(x, sal, "fp32")
    d = torch.sqrt(torch.diagonal(ref, dim1=1, dim2=2).abs())
    norm = d[:, :, None] * d[:, None, :]
    es = float(((Hs.double() - ref).abs() / norm)[:, iu[0], iu[1]].max())
    ef = float(((Hf.double() - ref).abs() / norm)[:, iu[0], iu[1]].max())
    print(f"{mode} {dtype}: max normalised entry error split {es:.3e}  fp32 {ef:.3e}")
    assert es <= 1e-5 and ef <= 1e-5


@pytest.mark.parametrize("mode", ["split16", "split16x3"])
def test_split_is_deterministic_and_tail_sliced(mode):
    """C = 1000, G = 3 has fewer items than one round, so every item runs as token slices."""
    r = rng(9)
    n, C, G = 4096, 1000, 3
    x = torch.from_numpy(r.standard_normal((n, C), dtype=np.float32)).half()
    sal = torch.from_numpy(r.lognormal(size=(n, G)).astype(np.float32))
    a = _run(x, sal, mode)
    b = _run(x, sal, mode)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    ref, _ = _exact(x, sal)
    assert rel_fro(_upper(a[0], a[2]), _upper(ref, a[2])) <= 1e-6


@pytest.mark.parametrize("mode", ["split16", "split16x3"])
def test_split_nonfinite_like_fp32(mode):
    r = rng(13)
    n, C = 256, 300
    X = r.standard_normal((n, C), dtype=np.float32)
    X[17, 5] = np.inf
    X[200, 250] = -np.inf
    x = torch.from_numpy(X).half()
    sal = torch.from_numpy(r.lognormal(size=(n, 1)).astype(np.float32))
    Hs, _, iu = _run(x, sal, mode)
    Hf, _, _ = _run(x, sal, "fp32")
    bs = ~torch.isfinite(_upper(Hs, iu))
    bf = ~torch.isfinite(_upper(Hf, iu))
    assert bf.any() and torch.equal(bs, bf)
    ok = ~bf
    assert rel_fro(_upper(Hs, iu)[ok], _upper(Hf, iu)[ok]) <= 1e-6


@pytest.mark.parametrize("n,C,G", [(256, 4096, 4), (512, 6000, 2)])
def test_split_multi_round_matches_exact_sum(n, C, G):
    """Calls whose whole items span several rounds of the GPU's workgroup slots, which the split
    kernel issues as one dispatch per round with the tail's token slices in the last: at C = 4096,
    G = 4, 544 items (two rounds and 32 items in 4 slices each); at C = 6000 (a ragged last tile),
    G = 2, 600 items (two rounds and 88 items in 2 slices each).  Every tile must be formed once:
    a missing or repeated tile would move H by far more than the fp32 bar."""
    r = rng(2000 + n + C + G)
    X = r.standard_normal((n, C), dtype=np.float32)
    X[:, r.choice(C, 8, replace=False)] *= 20.0
    x = torch.from_numpy(X).half()
    sal = torch.from_numpy(np.minimum(r.lognormal(size=(n, G)), 10.0).astype(np.float32))
    H, a, iu = _run(x, sal, "split16x3")
    xd = x.to(DEV).double()
    for g in range(G):
        w = (x.to(DEV).float() * sal[:, g:g + 1].to(DEV)).double()     # fl32(x * s), exact in fp64
        ref = (xd.T @ w).cpu()
        err = rel_fro(H[g][iu[0], iu[1]], ref[iu[0], iu[1]])
        print(f"multi-round n={n} C={C} G={G} group {g}: rel-Frobenius {err:.2e}", flush=True)
        assert err <= 1e-6, (g, err)
    assert torch.equal(a, (x.float() ** 2).sum(0)) or rel_fro(a, (x.double() ** 2).sum(0)) <= 1e-6


def test_multi_target_split_equals_separate():
    r = rng(21)
    n, C = 1024, 640
    x = torch.from_numpy(r.standard_normal((n, C), dtype=np.float32)).half().to(DEV)
    sals = [torch.from_numpy(r.lognormal(size=(n, 2)).astype(np.float32)).to(DEV) for _ in range(3)]
    Hm = [torch.zeros(2, C, C, device=DEV) for _ in range(3)]
    am = [torch.zeros(C, device=DEV) for _ in range(3)]
    K.hessian_accum_multi(x, sals, Hm, am)
    for t in range(3):
        H = torch.zeros(2, C, C, device=DEV)
        a = torch.zeros(C, device=DEV)
        K.hessian_accum(x, sals[t], H, a)
        torch.cuda.synchronize()
        iu = torch.triu_indices(C, C)
        assert rel_fro(_upper(Hm[t], iu), _upper(H, iu)) <= 1e-6
        assert torch.equal(am[t], a)


@pytest.mark.parametrize("n,C,G", [(4096, 512, 2), (2048, 1000, 3), (33, 385, 1), (5, 130, 2), (300, 17, 1)])
def test_split_fp32_x_matches_exact_sum(n, C, G):
    """fp32 X on the split path: x as two fp16 pieces (22 of its 24 bits) against the in-kernel
    two-piece w, three MFMAs per product (each product within ~2^-20.5 relative of the
    reference's).  The exact sums are still exact in float64 (24 x 24-bit products).  Bars:
    rel-Frobenius <= 1e-6 like the other split modes, and act_square equal to the fp32 kernel's
    bit for bit (both reproduce the reference's CPU summation order)."""
    r = rng(3000 + n + C + G)
    X = r.standard_normal((n, C), dtype=np.float32)
    X[:, r.choice(C, min(8, C), replace=False)] *= 20.0
    x = torch.from_numpy(X)
    sal = torch.from_numpy(np.minimum(r.lognormal(size=(n, G)), 10.0).astype(np.float32))
    ref, act_ref = _exact(x, sal)
    Hs, acts, iu = _run(x, sal, "split16")
    Hf, actf, _ = _run(x, sal, "fp32")
    Hd, actd, _ = _run(x, sal, "split16x3")
    es = rel_fro(_upper(Hs, iu), _upper(ref, iu))
    ef = rel_fro(_upper(Hf, iu), _upper(ref, iu))
    print(f"fp32 X n={n} C={C} G={G}: rel err split {es:.3e}  fp32 {ef:.3e}")
    assert es <= 1e-6 and ef <= 1e-6
    assert torch.equal(acts, actf) and rel_fro(acts, act_ref) <= 1e-6
    # the default mode runs fp32 X on the fp32 MFMA kernel: the same bits
    assert torch.equal(_upper(Hd, iu), _upper(Hf, iu)) and torch.equal(actd, actf)


def test_split_fp32_x_wide_dynamic_range():
    """fp32 columns from 1e-15 to 1e15 and saliencies from 1e-3 to 1e3: the per-column
    exponents of the row pieces and of w keep every entry at fp32 accuracy (normalised by
    sqrt(|H_ii H_jj|), as for the 16-bit inputs)."""
    r = rng(78)
    n, C, G = 2048, 384, 2
    mags = np.logspace(-15, 15, C).astype(np.float32)
    r.shuffle(mags)
    x = torch.from_numpy(r.standard_normal((n, C)).astype(np.float32) * mags)
    sal = torch.from_numpy(np.exp(r.uniform(np.log(1e-3), np.log(1e3), size=(n, G))).astype(np.float32))
    ref, _ = _exact(x, sal)
    Hs, _, iu = _run(x, sal, "split16")
    Hf, _, _ = _run(x, sal, "fp32")
    d = torch.sqrt(torch.diagonal(ref, dim1=1, dim2=2).abs())
    norm = d[:, :, None] * d[:, None, :]
    es = float(((Hs.double() - ref).abs() / norm)[:, iu[0], iu[1]].max())
    ef = float(((Hf.double() - ref).abs() / norm)[:, iu[0], iu[1]].max())
    print(f"fp32 X wide range: max normalised entry error split {es:.3e}  fp32 {ef:.3e}")
    assert es <= 1e-5 and ef <= 1e-5


def test_split_fp32_x_deterministic_nonfinite_and_multi_target():
    """Bitwise reproducible (C = 1000, G = 3 runs as token slices); an inf input gives
    non-finite entries in the same places as the fp32 kernel; the multi-target launch agrees
    with separate calls."""
    r = rng(91)
    n, C, G = 4096, 1000, 3
    x = torch.from_numpy(r.standard_normal((n, C), dtype=np.float32))
    sal = torch.from_numpy(r.lognormal(size=(n, G)).astype(np.float32))
    a = _run(x, sal, "split16")
    b = _run(x, sal, "split16")
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    X = r.standard_normal((256, 300), dtype=np.float32)
    X[17, 5] = np.inf
    X[200, 250] = -np.inf
    xi = torch.from_numpy(X)
    si = torch.from_numpy(r.lognormal(size=(256, 1)).astype(np.float32))
    Hs, _, iu = _run(xi, si, "split16")
    Hf, _, _ = _run(xi, si, "fp32")
    bs, bf = ~torch.isfinite(_upper(Hs, iu)), ~torch.isfinite(_upper(Hf, iu))
    assert bf.any() and torch.equal(bs, bf)
    assert rel_fro(_upper(Hs, iu)[~bf], _upper(Hf, iu)[~bf]) <= 1e-6
    xd = x[:1024, :640].contiguous().to(DEV)
    sals = [torch.from_numpy(r.lognormal(size=(1024, 2)).astype(np.float32)).to(DEV) for _ in range(3)]
    Hm = [torch.zeros(2, 640, 640, device=DEV) for _ in range(3)]
    am = [torch.zeros(640, device=DEV) for _ in range(3)]
    K.hessian_accum_multi(xd, sals, Hm, am)
    for t in range(3):
        H = torch.zeros(2, 640, 640, device=DEV)
        ac = torch.zeros(640, device=DEV)
        K.hessian_accum(xd, sals[t], H, ac)
        torch.cuda.synchronize()
        iu2 = torch.triu_indices(640, 640)
        # (another target count splits the tail into other token slices: fp32 sums in another order)
        assert rel_fro(_upper(Hm[t], iu2), _upper(H, iu2)) <= 1e-6 and torch.equal(am[t], ac)
