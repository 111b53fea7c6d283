"""act_order inputs bit for bit (gptq_plus_utils.py:856, 1046, 1050).

* act_square: the HIP reduction equals torch's CPU `(x.float() ** 2).sum(0)` added per
  add_batch call, exactly (both Hessian kernels, fp16 / bf16 / fp32 inputs, partial blocks, the
  level-5 cascade of > 2^19 tokens, ragged widths, and the no-workspace path through the C ABI).
* perm: equals torch's CPU `argsort(key, descending=True)` exactly -- ties in the order its
  introsort leaves them, NaN first, the heap-sort branch on adversarial keys -- on the LDS
  (C <= 16384) and global-memory variants; invperm = argsort(perm).
"""
import ctypes

import numpy as np
import pytest
import torch

from gptq_plus_mp_quant_amd import _native as nat
from gptq_plus_mp_quant_amd import kernels as K
from tests._cpu_order import adversarial_keys, model_covers

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _cpu_act(chunks):
    act = torch.zeros(chunks[0].shape[1], dtype=torch.float32)
    for x in chunks:
        act.add_((x.float() ** 2).sum(0))
    return act


def _gpu_act(chunks, math="split16"):
    C = chunks[0].shape[1]
    H = torch.zeros((1, C, C), device=DEV)
    act = torch.zeros(C, device=DEV)
    with K.hessian_math(math):
        for x in chunks:
            xd = x.to(DEV)
            s = torch.ones((x.shape[0], 1), device=DEV)
            K.hessian_accum(xd, s, H, act)
    torch.cuda.synchronize()
    return act.cpu()


@pytest.mark.parametrize("ntok,C,dtype,math", [
    (32768, 256, torch.float16, "split16"),
    (32768 + 100, 4096, torch.float16, "split16"),
    (5000, 96, torch.float16, "split16"),
    (300, 64, torch.bfloat16, "split16"),
    (4097, 77, torch.float16, "split16"),
    (1000, 35, torch.float16, "fp32"),
    (12305, 160, torch.float32, "split16"),
    (4096, 200, torch.float16, "fp32"),
    (600000, 64, torch.float16, "split16"),
    (17, 32, torch.float16, "split16"),
])
def test_act_square_matches_cpu_sum(ntok, C, dtype, math):
    assert model_covers(C)
    gen = torch.Generator().manual_seed(ntok + C)
    chunks = []
    for k in range(2):
        x = torch.randn((ntok, C), generator=gen) * 3
        x[:, :4] *= 20                       # outlier channels
        chunks.append(x.to(dtype))
    print(f"act_square ntok={ntok} C={C} {dtype} {math}", flush=True)
    ref = _cpu_act(chunks)
    got = _gpu_act(chunks, math)
    bad = int((got != ref).sum())
    assert bad == 0, f"{bad}/{C} act_square entries differ from the CPU sum"


def test_act_square_no_workspace_path():
    """Without a workspace the one-pass kernel runs (fp32 Hessian kernel); same bits."""
    gen = torch.Generator().manual_seed(3)
    x = (torch.randn((7001, 104), generator=gen) * 2).half()
    assert model_covers(x.shape[1])
    ref = _cpu_act([x])
    xd = x.to(DEV)
    C = x.shape[1]
    H = torch.zeros((1, C, C), device=DEV)
    act = torch.zeros(C, device=DEV)
    s = torch.ones((x.shape[0], 1), device=DEV)
    nat.call("rq_hessian_accum", nat.ptr(xd), nat.RQ_F16, x.shape[0], C, C, nat.ptr(s), 1, 1, nat.ptr(H),
             nat.ptr(act), None, 0, nat.stream_of(DEV))
    torch.cuda.synchronize()
    assert torch.equal(act.cpu(), ref)


def _check_perm(keys):
    perm, invperm = K.act_order_perm(keys.to(DEV))
    torch.cuda.synchronize()
    ref = torch.argsort(keys, descending=True)
    p = perm.cpu()
    bad = int((p != ref).sum())
    assert bad == 0, f"{bad}/{keys.numel()} perm positions differ from torch's CPU argsort"
    assert torch.equal(invperm.cpu(), torch.argsort(ref))


@pytest.mark.parametrize("C", [1, 2, 3, 16, 17, 100, 511, 513, 1025, 4096, 8193, 14336, 16384, 16385, 28672])
def test_perm_ties_and_nan(C):
    gen = torch.Generator().manual_seed(C)
    keys = torch.randint(0, max(2, C // 7), (C,), generator=gen).float() * 0.25
    if C > 8:
        keys[torch.randint(0, C, (3,), generator=gen)] = float("nan")
        keys[torch.randint(0, C, (2,), generator=gen)] = -0.0
    print(f"perm C={C}", flush=True)
    _check_perm(keys)


@pytest.mark.parametrize("C", [4096, 14336, 28672])
def test_perm_act_square_like(C):
    """chi^2-like sums on a fine grid: a few dozen exact ties among many near ties."""
    gen = torch.Generator().manual_seed(C + 1)
    v = 262144 + torch.randn(C, generator=gen, dtype=torch.float64) * 724
    v[torch.randint(0, C, (8,), generator=gen)] *= 400
    keys = (v.float() / 2048).float()
    _check_perm(keys)


@pytest.mark.parametrize("C", [64, 700, 3000, 17000])
def test_perm_heap_branch(C):
    keys = torch.from_numpy(adversarial_keys(C))
    _check_perm(keys)
    # ties on top of the adversarial shape
    _check_perm(torch.floor(keys / 3))


def test_perm_bad_args():
    lib = nat.load()
    assert lib.rq_act_order_perm(None, 4, None, None, None) == nat.RQ_EINVAL
    k = torch.zeros(70000, device=DEV)
    p = torch.empty(70000, dtype=torch.int64, device=DEV)
    assert lib.rq_act_order_perm(ctypes.c_void_p(k.data_ptr()), 70000, ctypes.c_void_p(p.data_ptr()),
                                 ctypes.c_void_p(p.data_ptr()), None) == nat.RQ_EINVAL
