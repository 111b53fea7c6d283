"""Drop-in ``GPTQ`` (reference: gptq_utils/gptq_utils.py:23-180, the classic GPTQ class the
reference drives from ``gptq_fwrd`` :183-293) on the same gfx950 kernels as ``GPTQPlus``.

Same constructor, ``add_batch(inp, out)`` / ``fasterquant(blocksize, percdamp, groupsize,
actorder, static_groups, export_to_et)`` / ``free()``, fields (``layer``, ``rows``,
``columns``, ``nsamples``, ``H``, ``quantizer``) and side effects:

* ``add_batch`` accumulates the Gram matrix of the inputs with one MFMA launch per call
  (``rq_hessian_accum`` with unit weights).  The reference keeps a running mean
  (``H *= n/(n+b)``, ``x <- sqrt(2/n) x``, :39-43), which equals ``2/n * sum x x^T``; here ``H``
  holds the plain sum (upper 128-tiles) until ``fasterquant`` scales and mirrors it once.
* ``fasterquant`` follows :45-171: RTN for an all-zero H, dead columns, static groups cut
  from the dead-fixed unpermuted weight, act_order by ``diag(H)``, the damped Cholesky chain
  with +0.0015 retries (``ValueError`` at 1, no identity fallback), the column loop with
  ``err = (w - q) / d`` (the GPTQ+ kernels with the first-order term off), dynamic groups
  re-fitted on the working weight at every group start, the trailing update, and the
  write-back.  As in the reference, ``export_to_et``'s ``int_weight`` / ``scale`` keep the
  act_order column order (only Q is un-permuted), and the quantizer left on the object is
  the last one used (the last dynamic fit, or the last static group).
"""
from __future__ import annotations

import logging

import torch

from . import _native as nat
from . import kernels as K
from .gptq_plus import GPTQPlus, hessian_inverse_chain


class GPTQ:
    # gptq_utils.py:23-31
    def __init__(self, layer):
        self.layer = layer
        self.dev = layer.weight.device
        nat.require_gpu(layer.weight, "layer.weight")
        nat.load()
        W = layer.weight.data
        self.rows, self.columns = W.shape[0], W.shape[1]
        self.H = torch.zeros((self.columns, self.columns), device=self.dev)
        self.nsamples = 0
        self.quantizer = None
        self._act = torch.zeros((self.columns,), device=self.dev)   # unused by GPTQ; kernel output
        self._ones = None
        self.perm = self.invperm = None
        self._codes_perm = None

    # gptq_utils.py:33-43
    @torch.no_grad()
    def add_batch(self, inp, out=None):
        if inp.dim() == 2:
            inp = inp.unsqueeze(0)
        nat.require_gpu(inp, "add_batch input")
        tmp = inp.shape[0]
        x = inp.reshape(-1, inp.shape[-1])
        if x.stride(1) != 1 or x.stride(0) < x.shape[1]:
            x = x.contiguous()
        if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            x = x.float()
        n = x.shape[0]
        if self._ones is None or self._ones.shape[0] < n:
            self._ones = torch.ones((n, 1), device=self.dev)
        K.hessian_accum(x, self._ones[:n], self.H.view(1, self.columns, self.columns), self._act)
        self.nsamples += tmp

    # gptq_utils.py:45-171
    @torch.no_grad()
    def fasterquant(self, blocksize=128, percdamp=0.01, groupsize=-1, actorder=False,
                    static_groups=False, export_to_et=False):
        q = self.quantizer
        if q is None or q.bits >= 16:
            raise ValueError("fasterquant needs a configured WeightQuantizer with bits < 16")
        if getattr(q, "weight_groupsize", -1) > 0:
            # one scale per weight element: the reference's column loop broadcasts it against a
            # column (gptq_utils.py:135-136) and fails
            raise ValueError("fasterquant: a quantizer with weight_groupsize > 0 has no per-row scale")
        if blocksize > 128 or blocksize <= 0:
            raise NotImplementedError("blocksize must be in [1, 128] on the HIP path")
        if actorder:
            K.check_act_order_width(self.columns)
        dev, R, C = self.dev, self.rows, self.columns
        f32 = dict(device=dev, dtype=torch.float32)
        W = self.layer.weight.data
        if W.stride(1) != 1:
            W = W.contiguous()
        if not q.ready():
            q.find_params(W)
        maxq, sym = int(q.maxq), int(bool(q.sym))

        # H = 2/n * sum x x^T, mirrored and left unsanitised (a non-finite H fails every
        # Cholesky retry and raises, :87-104); an all-zero H (no data) becomes the identity (RTN)
        H = self.H.view(1, C, C)
        self.H = None
        if self.nsamples > 0:
            K.hessian_finalize(H, None, self.nsamples / 2.0, 1.0, 1.0, sanitize=False)
        if self.nsamples == 0 or not bool(torch.any(H[0])):
            H[0].copy_(torch.eye(C, device=dev))
        # dead columns (:64-66), then act_order by the dead-fixed diag(H) (:75-80)
        Wp = torch.empty((R, C), **f32)
        H_work = torch.empty((1, C, C), **f32)
        K.prepare_subgroup(W, None, H[0], None, Wp, None, H_work[0])
        Wd = Wp                                                    # dead-fixed, unpermuted
        perm = invperm = None
        if actorder:
            perm, invperm = K.act_order_perm(torch.diagonal(H_work[0]).contiguous())
            Wp = torch.empty((R, C), **f32)
            K.prepare_subgroup(W, None, H[0], perm, Wp, None, H_work[0])

        qmode, scale_tab, zero_tab, col_group, dyn_fit = nat.RQ_QMODE_CHANNEL, None, None, None, False
        if groupsize == -1:
            scale_tab = q.scale.reshape(-1).to(**f32).contiguous()
        else:
            qmode = nat.RQ_QMODE_STATIC
            cols = perm if perm is not None else torch.arange(C, device=dev)
            if static_groups:
                # groups of the dead-fixed, unpermuted weight (:67-73)
                scale_tab, zero_tab = q.params_grouped(Wd, groupsize)
                col_group = (cols // groupsize).to(torch.int32).contiguous()
            else:
                # re-fitted on the working weight at each group start (:121-125), in the
                # (possibly permuted) column order
                ng = (C + groupsize - 1) // groupsize
                scale_tab = torch.empty((ng, R), **f32)
                zero_tab = torch.empty((ng, R), **f32)
                col_group = (torch.arange(C, device=dev) // groupsize).to(torch.int32).contiguous()
                dyn_fit = True

        del Wd
        Hinv_all = torch.empty((1, C, C), **f32)
        workspace = K.chol_workspace(C, dev, 1)
        hessian_inverse_chain(dev, H_work, Hinv_all, None, workspace, percdamp, identity_fallback=False)
        del workspace, H_work

        codes = torch.empty((R, C), dtype=torch.int16, device=dev)
        err = torch.empty((R, min(blocksize, C)), **f32)
        z_off = torch.zeros(1, dtype=torch.int32, device=dev)      # no first-order term
        for i1 in range(0, C, blocksize):
            i2 = min(i1 + blocksize, C)
            if dyn_fit:
                for g in range((i1 + groupsize - 1) // groupsize, (i2 + groupsize - 1) // groupsize):
                    s0 = g * groupsize
                    sc, zc = q.row_params(Wp[:, s0:min(s0 + groupsize, C)], R)
                    scale_tab[g].copy_(sc)
                    zero_tab[g].copy_(zc)
            # GH / Z are never read when the first-order flag is 0; Wp stands in for them
            K.quant_block(Wp, Hinv_all, Wp, Wp, R, i1, i2 - i1, qmode, scale_tab, col_group, None, maxq,
                          sym, False, z_off, codes, err)
            if i2 < C:
                K.trailing_update(Wp, Wp, Wp, Hinv_all, R, i1, i2 - i1, err, z_off, z_zero=True)

        Q = torch.empty((R, C), dtype=W.dtype, device=dev)
        nan_flag = torch.zeros(1, dtype=torch.int32, device=dev)
        K.writeback(codes, invperm, qmode, scale_tab, col_group, None, blocksize, Q, None, None, nan_flag)
        if export_to_et:
            # the reference un-permutes Q only (:157-163)
            w_int = torch.empty((R, C), **f32)
            scale_full = torch.empty((R, C), **f32)
            K.writeback(codes, None, qmode, scale_tab, col_group, None, blocksize,
                        torch.empty((R, C), dtype=W.dtype, device=dev), w_int, scale_full)
            self.layer.register_buffer("int_weight", w_int.reshape(self.layer.weight.shape))
            self.layer.register_buffer("scale", scale_full)
        self.layer.weight.data = Q.reshape(self.layer.weight.shape)
        # the quantizer the reference leaves on the object: the last group used
        if groupsize != -1:
            last = (int(perm[C - 1]) if (perm is not None and static_groups) else C - 1) // groupsize
            q.scale = scale_tab[last].reshape(-1, 1).clone()
            q.zero = zero_tab[last].reshape(-1, 1).clone()
        self.perm, self.invperm, self._codes_perm = perm, invperm, codes
        self.qmode, self.scale_table, self.col_group = qmode, scale_tab, col_group
        self.blocksize_used, self.groupsize_used = blocksize, groupsize
        self.dyn_scale = None
        if int(nan_flag.item()):
            logging.warning("NaN in weights")
            raise ValueError("NaN in weights")

    codes = GPTQPlus.codes
    export_packed = GPTQPlus.export_packed

    def free(self):
        self.H = None
        self.Losses = None
        self._codes_perm = None
        K.release_hessian_workspace(self.dev)
        torch.cuda.empty_cache()
