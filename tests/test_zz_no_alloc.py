"""rq_hessian_accum_noalloc, the variant of rq_hessian_accum that allocates nothing (its
workspace is the library's per-GPU scratch array), through the C ABI against rq_hessian_accum:

- given a workspace of the scratch's size, rq_hessian_accum makes the same kernel choices, so
  H and act_square must be equal bit for bit;
- against rq_hessian_accum with its full workspace (which may also split the last round of
  tiles along the tokens, or pick another kernel) H's upper triangle must agree to rel.
  Frobenius 1e-5 (the suite's bar for H) and act_square exactly;
- two calls in a row on different shapes (the second smaller), each accumulated over two
  chunks, and fp16 / bf16 / fp32 inputs, in the default and the opt-in split16 Hessian mode;
- a chunk needing more than RQ_NOALLOC_SCRATCH_BYTES is refused with RQ_EINVAL before any
  launch.
"""
import ctypes

import pytest
import torch

from gptq_plus_mp_quant_amd import _native as nat
from gptq_plus_mp_quant_amd import kernels as K

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _inputs(ntok, C, G, dtype, seed):
    gen = torch.Generator(device=DEV)
    gen.manual_seed(seed)
    x = (torch.randn((2, ntok, C), generator=gen, device=DEV) * 2).to(dtype)
    s = torch.exp(torch.randn((2, ntok, G), generator=gen, device=DEV))
    return x, s


def _run(x, s, mode, ws_bytes=None):
    _, ntok, C = x.shape
    G = s.shape[2]
    H = torch.zeros((G, C, C), device=DEV)
    act = torch.zeros(C, device=DEV)
    lib = nat.load()
    for k in range(2):
        xk, sk = x[k], s[k].contiguous()
        args = (nat.ptr(xk), nat.dtype_code(xk.dtype), ntok, C, C, nat.ptr(sk), G, G, nat.ptr(H), nat.ptr(act))
        if mode == "noalloc":
            rc = lib.rq_hessian_accum_noalloc(*args, nat.stream_of(DEV))
        else:
            need = int(lib.rq_hessian_workspace_bytes(ntok, C, G, nat.dtype_code(xk.dtype))) if ws_bytes is None \
                else ws_bytes
            ws = torch.zeros(need, dtype=torch.uint8, device=DEV)
            rc = lib.rq_hessian_accum(*args, nat.ptr(ws), need, nat.stream_of(DEV))
        assert rc == nat.RQ_OK, (mode, rc)
    torch.cuda.synchronize()
    return H, act


@pytest.mark.parametrize("dtype,math", [(torch.float16, "split16x3"), (torch.bfloat16, "split16x3"),
                                        (torch.float32, "split16x3"), (torch.float16, "split16"),
                                        (torch.float32, "split16")])
def test_noalloc_matches_workspace_entry(dtype, math):
    for ntok, C, G, seed in ((9000, 1536, 4, 1), (700, 200, 3, 2)):
        print(f"noalloc: ntok={ntok} C={C} G={G} {dtype} {math}", flush=True)
        x, s = _inputs(ntok, C, G, dtype, seed)
        with K.hessian_math(math):
            H_n, a_n = _run(x, s, "noalloc")
            H_w, a_w = _run(x, s, "workspace", ws_bytes=nat.RQ_NOALLOC_SCRATCH_BYTES)
            H_f, a_f = _run(x, s, "workspace")
        assert torch.equal(H_n, H_w) and torch.equal(a_n, a_w)
        assert torch.equal(a_n, a_f)
        # the upper triangle (what rq_hessian_accum defines; finalize mirrors it): the two
        # workspaces may choose different kernels (fp32 X in the split16 mode: its split kernel
        # needs more than the scratch at the first shape), whose lower triangles hold different
        # partial values
        iu = torch.triu_indices(C, C, device=DEV)
        Hn_u, Hf_u = H_n[:, iu[0], iu[1]].double(), H_f[:, iu[0], iu[1]].double()
        err = float((Hn_u - Hf_u).norm() / Hf_u.norm())
        assert err <= 1e-5, err


def test_noalloc_rejects_oversize():
    """Buffers sized for the shape the call states (x [ntok, C] of ones, s [ntok, 1], H [1, C, C]),
    so that a guard that let the call through would compute a non-zero H within bounds and fail
    the assertions, rather than touch memory past the tensors."""
    C = 1024
    ntok = (nat.RQ_NOALLOC_SCRATCH_BYTES // (2 * C)) + 4096          # the chunk copy alone is larger
    x = torch.ones((ntok, C), dtype=torch.float16, device=DEV)
    s = torch.ones((ntok, 1), device=DEV)
    H = torch.zeros((1, C, C), device=DEV)
    lib = nat.load()
    rc = lib.rq_hessian_accum_noalloc(nat.ptr(x), nat.RQ_F16, ntok, C, C, nat.ptr(s), 1, 1, nat.ptr(H), None,
                                      nat.stream_of(DEV))
    assert rc == nat.RQ_EINVAL
    torch.cuda.synchronize()
    assert float(H.abs().sum()) == 0.0                                # nothing ran
