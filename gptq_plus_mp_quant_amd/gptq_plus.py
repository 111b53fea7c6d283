"""Drop-in ``GPTQPlus`` (reference: gptq_utils/gptq_plus_utils.py:430-1896) whose
arithmetic runs in the gfx950 HIP kernels of ``libgptqplus_hip.so``.

The constructor, ``add_batch`` / ``finalize_hessian`` / ``fasterquant`` / ``free`` signatures,
the public fields the layer-wise driver reads (``H``, ``act_square``, ``gradients``,
``saliencies``, ``reference_loss``, ``token_count``, ``index``, ``quantizer``), the error
behaviour and the side effects (``layer.weight.data`` replaced by the dequantized weight in
the layer dtype, ``int_weight`` / ``scale`` buffers with ``export_to_et``) follow the
reference.  Additionally exposed for inspection: ``perm``, ``invperm``, ``codes`` (natural
column order), ``subgroup_info`` (damping, retries, identity fallback, beta).

Every ``g_update_mode`` of the reference runs on the HIP path: ``"frozen"`` (default),
``"surrogate_block"``, ``"surrogate_online"``, and the refresh modes ``"block_gd"`` /
``"block_backward"``, whose layer backward is the caller's ``gradient_refresh_fn`` (called
with the current weight, on the GPU, like the reference does); the optimizer step,
regularizers and GPTQ+ term refresh around it are kernels; ``refresh_full_metrics`` fills the
``block_observer`` statistics (means, row norms, max and 0.99 quantile of the refreshed
gradient and of the update terms) with torch reductions on the GPU.  ``diagnostic_recorder``
dumps raise ``NotImplementedError`` rather than silently differing.
"""
from __future__ import annotations

import contextlib
import inspect
import logging
from typing import Optional

import torch

from . import _native as nat
from . import kernels as K
from .quant_utils import WeightQuantizer

_NULL = contextlib.nullcontext()
MAX_BLOCKSIZE = 128


def _section(rec, name):
    return rec.section(name) if rec is not None else _NULL


def hessian_inverse_chain(dev, H_work, Hinv_out, Hinv_init_out, workspace, percdamp,
                          damp_auto_increment=0.0015, log_context="", identity_fallback=True,
                          Hinv_diag_out=None):
    """The damped Cholesky chain with retries (gptq_plus_utils.py:494-561; classic GPTQ
    gptq_utils.py:87-106 has the same schedule but raises instead of the identity fallback).
    H_work [nb, C, C] (or [C, C]) is damped in place; Hinv_init_out (H^-1) and Hinv_diag_out
    (its diagonal, [nb, C]) are optional.  Returns [(damp, fallback, attempts)]."""
    damp0 = float(percdamp)
    if damp0 <= 0:
        raise ValueError(f"Quantization{log_context}: `damp_percent` must be positive. current is {damp0}")
    if H_work.dim() == 2:
        H_work, Hinv_out = H_work[None], Hinv_out[None]
        Hinv_init_out = None if Hinv_init_out is None else Hinv_init_out[None]
        Hinv_diag_out = None if Hinv_diag_out is None else Hinv_diag_out.reshape(1, -1)
    nb, C = H_work.shape[0], H_work.shape[-1]
    damp = [damp0] * nb
    attempts = [0] * nb
    status = ["run" if 1 > damp0 > 0 else "range"] * nb
    info = torch.zeros(nb, dtype=torch.int32, device=dev)
    while any(st == "run" for st in status):
        todo = [damp[b] if status[b] == "run" else 0.0 for b in range(nb)]
        for b in range(nb):
            attempts[b] += status[b] == "run"
        K.chol_hinv_attempt(H_work, todo, workspace, Hinv_out, Hinv_init_out, info, Hinv_diag_out)
        codes = info.tolist()
        for b in range(nb):
            if status[b] != "run":
                continue
            if codes[b] == 0:
                status[b] = "ok"
                continue
            logging.warning("Quantization%s subgroup=%d: Current `damp_percent = %.5f` is too low, "
                            "auto-incrementing by `%.5f`", log_context, b, damp[b], damp_auto_increment)
            damp[b] += damp_auto_increment
            if not (1 > damp[b] > 0):
                status[b] = "range"
    out = []
    for b in range(nb):
        if status[b] == "ok":
            out.append((damp[b], False, attempts[b]))
        elif damp[b] >= 1 and identity_fallback:
            logging.warning("Quantization%s subgroup=%d: `damp_percent` reached %.5f; falling back to "
                            "identity Hessian inverse for this subgroup.", log_context, b, damp[b])
            eye = torch.eye(C, device=dev)
            Hinv_out[b].copy_(eye)
            if Hinv_init_out is not None:
                Hinv_init_out[b].copy_(eye)
            if Hinv_diag_out is not None:
                Hinv_diag_out[b].fill_(1.0)
            out.append((damp[b], True, attempts[b]))
        else:
            raise ValueError(f"Quantization{log_context}: `damp_percent` must between 0 and 1. "
                             f"current is {damp[b]}")
    return out



def _quantile_large(t, q):
    """gptq_plus_utils.py:46-60: torch.quantile, or the k-th value where quantile refuses the size."""
    flat = t.reshape(-1)
    n = flat.numel()
    if n == 0:
        return None
    k = max(1, min(n, int(n * q + 0.5)))
    try:
        return torch.quantile(flat, q).item()
    except RuntimeError:
        return flat.kthvalue(k).values.item()


def _update_stats(t, name, outliers=False):
    """abs mean and mean row L2 norm of an update term (:1657-1668, :1759-1783); with outliers also
    its abs max and 0.99 quantile.  Keys as in the observer record (``<name>_abs_mean`` ...)."""
    t = t.float()
    a = t.abs()
    out = {f"{name}_abs_mean": a.mean().item(), f"{name}_mean_row_l2": torch.linalg.norm(t, dim=1).mean().item()}
    if outliers:
        out[f"{name}_abs_max"] = a.max().item()
        out[f"{name}_abs_q99"] = _quantile_large(a, 0.99)
    return out


def _grad_stats(g, grad_clip):
    """The refreshed gradient's trailing columns (:1448-1462, :1669-1681): abs mean, mean row L2
    norm, and abs mean after clamping to +-grad_clip (the abs mean when there is no clip)."""
    g = g.float()
    a = g.abs().mean().item()
    clipped = g.clamp(min=-grad_clip, max=grad_clip).abs().mean().item() \
        if grad_clip is not None and grad_clip > 0 else a
    return {"remaining_grad_abs_mean": a, "remaining_grad_mean_row_l2": torch.linalg.norm(g, dim=1).mean().item(),
            "remaining_grad_clipped_abs_mean": clipped}


class GPTQPlus:
    # gptq_plus_utils.py:431-487
    def __init__(self, layer, saliency: torch.Tensor, gradient: torch.Tensor, num_groups: int,
                 alpha: float, reference_loss: float, hessian_saliency_scale: float = 1.0):
        self.layer = layer
        self.dev = layer.weight.device
        nat.require_gpu(layer.weight, "layer.weight")
        nat.load()
        W = layer.weight.data
        self.rows, self.columns = W.shape[0], W.shape[1]
        self.num_groups = num_groups
        assert self.num_groups == saliency.shape[2], "Number of groups for GuidedQuant must match saliency shape!"
        self.alpha = alpha
        self.reference_loss = max(reference_loss, 0)
        self.hessian_saliency_scale = float(hessian_saliency_scale)
        self.saliencies = saliency.float()
        self.gradients = gradient.float()
        self.H = torch.zeros((self.num_groups, self.columns, self.columns), device=self.dev)
        self.act_square = torch.zeros((self.columns,), device=self.dev)
        self.nsamples = saliency.shape[0]
        self.index = 0
        self.token_count = 0
        self._finalized = False
        self.profile_recorder = None
        self.quantizer: Optional[WeightQuantizer] = None
        self.perm = None
        self.invperm = None
        self.subgroup_info = []
        self._codes_perm = None
        assert self.rows % self.num_groups == 0, (
            f"Number of rows ({self.rows}) must be divisible by num_groups ({self.num_groups})")

    # gptq_plus_utils.py:798-857
    @torch.no_grad()
    def add_batch(self, inp: torch.Tensor, out=None):
        if self._finalized:
            raise RuntimeError("add_batch called after finalize_hessian. Re-init GPTQPlus to reuse.")
        rec = self.profile_recorder
        with _section(rec, "add_batch.total"):
            if inp.dim() == 2:
                inp = inp.unsqueeze(0)
            else:
                assert inp.dim() == 3, "Input must be 2D or 3D. Got %dD." % inp.dim()
            x, s = self._take_saliency(inp)
            K.hessian_accum(x, s, self.H, self.act_square)
            self.token_count += x.shape[0]

    def _take_saliency(self, inp):
        """Advance the sample cursor like add_batch and return (x [n, C], sal [n, G])."""
        if self._finalized:
            raise RuntimeError("add_batch called after finalize_hessian. Re-init GPTQPlus to reuse.")
        if inp.dim() == 2:
            inp = inp.unsqueeze(0)
        nat.require_gpu(inp, "add_batch input")
        bsz = inp.shape[0]
        sal = self.saliencies[self.index:self.index + bsz]
        self.index += bsz
        if sal.dim() == 3 and inp.shape[1] > sal.shape[1]:
            inp = inp[:, inp.shape[1] - sal.shape[1]:]
        x = inp.reshape(-1, inp.shape[-1])
        if x.stride(1) != 1 or x.stride(0) < x.shape[1]:
            x = x.contiguous()
        if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            x = x.float()
        s = sal.reshape(-1, sal.shape[-1]).to(self.dev, torch.float32).contiguous()
        if s.shape[0] != x.shape[0]:
            raise ValueError(f"saliency rows ({s.shape[0]}) do not match tokens ({x.shape[0]})")
        return x, s

    # gptq_plus_utils.py:859-908 (single GPU: the all-reduces are identities)
    @torch.no_grad()
    def finalize_hessian(self):
        if self._finalized:
            return
        total_samples = float(self.index)
        total_tokens = float(self.token_count)
        if total_samples <= 0 or total_tokens <= 0:
            raise RuntimeError("finalize_hessian called before any add_batch ran.")
        seq_len = total_tokens / total_samples
        nonfinite = torch.zeros(1, dtype=torch.int32, device=self.dev)
        K.hessian_finalize(self.H, self.act_square, total_samples * seq_len, self.hessian_saliency_scale,
                           seq_len, nonfinite)
        n_bad = int(nonfinite.item())
        if n_bad:
            logging.warning("finalize_hessian: %d non-finite entries in H sanitised to 0 (module=%s)",
                            n_bad, self.layer.__class__.__name__)
        self._finalized = True

    # gptq_plus_utils.py:910-1896 (frozen mode)
    @torch.no_grad()
    def fasterquant(self, blocksize=128, percdamp=0.01, groupsize=-1, actorder=False,
                    static_groups=False, enable_gradient_update=True, g_update_mode="frozen",
                    export_to_et=False, profile_recorder=None, gradient_refresh_fn=None,
                    grad_lr=1e-3, grad_optimizer="sgd", curvature_damping=0.1,
                    grad_reg_strategy="none", grad_reg_lambda=0.0, grad_gate_floor=0.1,
                    grad_gate_sharpness=1.0, grad_gate_sine_amp=0.0, second_order_scale=1.0,
                    block_atomic_quant=False, block_observer=None, grad_clip=1.0,
                    diagnostic_recorder=None, slide_refresh_start=0, slide_refresh_block_total=None,
                    refresh_full_metrics=False, keep_hinv=False, inject=None):
        """Quantize ``layer.weight`` in place (gptq_plus_utils.py:910-1896).

        Extra keyword arguments (not in the reference):
          keep_hinv -- keep ``Hinv_all``, ``Hinv_init_all``, ``Z`` and ``GHinv`` on the object.
          inject    -- parity-test hook: ``{"perm": LongTensor[C], "hinv": [(Hinv_init, Hinv), ...],
                       "terms": [(beta, Z, GHinv), ...]}`` replaces the act_order permutation,
                       each subgroup's inverse factors and/or its GPTQ+ terms (as the reference's
                       _compute_gradient_terms returns them), so the block loop can be compared
                       against another implementation on identical inputs.
        """
        kw = {k: v for k, v in locals().items() if k != "self"}
        steps = self._fasterquant_steps(**kw)
        req = next(steps)
        if req is not None:
            req.run([req])
        for _ in steps:
            pass

    def _fasterquant_steps(self, blocksize, percdamp, groupsize, actorder, static_groups,
                           enable_gradient_update, g_update_mode, export_to_et, profile_recorder,
                           gradient_refresh_fn, grad_lr, grad_optimizer, curvature_damping,
                           grad_reg_strategy, grad_reg_lambda, grad_gate_floor, grad_gate_sharpness,
                           grad_gate_sine_amp, second_order_scale, block_atomic_quant, block_observer,
                           grad_clip, diagnostic_recorder, slide_refresh_start, slide_refresh_block_total,
                           refresh_full_metrics, keep_hinv, inject, alloc=None):
        """fasterquant as a generator that pauses once, at the damped Cholesky chain: it yields a
        ChainRequest (or None when inject supplies H^-1), whose chain the caller runs -- alone
        (fasterquant) or batched with other linears' (fasterquant_shared) -- and is then driven to
        the end.  ``alloc`` supplies this linear's H_work / Hinv_all / Hinv_init_all / diag(H^-1)
        as views into the caller's batched buffers."""
        rec = profile_recorder or self.profile_recorder
        inject = inject or {}
        inject_hinv = inject.get("hinv")
        self._validate(grad_reg_strategy, grad_reg_lambda, grad_gate_floor, grad_gate_sharpness,
                       grad_gate_sine_amp)
        if g_update_mode not in nat.GMODES:
            raise NotImplementedError(f"g_update_mode={g_update_mode!r} is not one of {sorted(nat.GMODES)}")
        gm_in, gm_out = nat.GMODES[g_update_mode]
        block_gd = g_update_mode == "block_gd"
        block_bw = g_update_mode == "block_backward"
        if block_gd and grad_optimizer not in K.OPTIMIZERS:
            raise ValueError(f"Unsupported `grad_optimizer={grad_optimizer}`. Expected one of: sgd, adam, h_adam.")
        if diagnostic_recorder is not None:
            raise NotImplementedError("diagnostic_recorder dumps are not produced by the HIP path")
        if not self._finalized:
            raise RuntimeError("fasterquant called before finalize_hessian")
        q = self.quantizer
        if q is None or q.bits >= 16:
            raise ValueError("fasterquant needs a configured WeightQuantizer with bits < 16")
        if getattr(q, "weight_groupsize", -1) > 0:
            # one scale per weight element: the reference's column loop fails on it
            # (gptq_plus_utils.py:1301-1315 broadcasts it against a column)
            raise ValueError("fasterquant: a quantizer with weight_groupsize > 0 has no per-row scale")
        if blocksize > MAX_BLOCKSIZE or blocksize <= 0:
            raise NotImplementedError(f"blocksize must be in [1, {MAX_BLOCKSIZE}] on the HIP path")
        if actorder:
            K.check_act_order_width(self.columns)

        dev, R, C, G = self.dev, self.rows, self.columns, self.num_groups
        R_s = R // G
        W = self.layer.weight.data
        if W.stride(1) != 1:
            W = W.contiguous()
        maxq = int(q.maxq)
        sym = int(bool(q.sym))
        f32 = dict(device=dev, dtype=torch.float32)

        with _section(rec, "fasterquant.total"):
            if not q.ready():
                with _section(rec, "fasterquant.quantizer_find_params_initial"):
                    q.find_params(W)
            dynamic_groups = groupsize != -1 and not static_groups
            if dynamic_groups and groupsize != blocksize:
                raise ValueError("`groupsize` must equal `blocksize` when using dynamic groups in GPTQ+. "
                                 f"Got groupsize={groupsize}, blocksize={blocksize}.")
            if dynamic_groups and grad_reg_strategy in {"quant_error_gate", "quant_error_gate_optimized"}:
                raise ValueError("Dynamic weight groups are not supported with quant_error_gate regularization yet.")

            if groupsize == -1:
                qmode = nat.RQ_QMODE_CHANNEL
                scale_tab = q.scale.reshape(-1).to(**f32).contiguous()
                if scale_tab.numel() != R:
                    raise ValueError("quantizer scale must hold one value per output row")
            elif static_groups:
                qmode = nat.RQ_QMODE_STATIC
                with _section(rec, "fasterquant.quantizer_build_groups"):
                    scale_tab, zero_tab = q.params_grouped(W, groupsize)
            else:
                qmode = nat.RQ_QMODE_DYNAMIC
                scale_tab = None

            # act_order: one permutation, argsort(act_square, descending), for every subgroup
            perm = invperm = None
            if actorder:
                if inject.get("perm") is not None:
                    perm = inject["perm"].to(dev, torch.int64).contiguous()
                    invperm = torch.argsort(perm)
                else:
                    perm, invperm = K.act_order_perm(self.act_square)
            col_group = None
            if qmode == nat.RQ_QMODE_STATIC:
                cols = perm if perm is not None else torch.arange(C, device=dev)
                col_group = (cols // groupsize).to(torch.int32).contiguous()

            Wp = torch.empty((R, C), **f32)
            Z = torch.empty((R, C), **f32)
            GH = torch.empty((R, C), **f32)
            Gs = torch.empty((R, C), **f32)
            beta_mode = 1 if (enable_gradient_update and self.alpha > 0) else 0
            alloc = alloc or {}
            Hinv_all = alloc["Hinv_all"] if "Hinv_all" in alloc else torch.empty((G, C, C), **f32)
            # H^-1 itself only for keep_hinv; the GPTQ+ step size needs just its diagonal
            Hinit_all = (alloc["Hinv_init_all"] if "Hinv_init_all" in alloc else torch.empty((G, C, C), **f32)) \
                if keep_hinv else None
            hdiag_all = (alloc["Hinv_diag"] if "Hinv_diag" in alloc else torch.empty((G, C), **f32)) \
                if beta_mode == 1 else None
            grads = self.gradients.to(**f32)
            if grads.stride(1) != 1:
                grads = grads.contiguous()
            # slice, dead-column fix and act_order gathers of every subgroup
            H_work = alloc["H_work"] if "H_work" in alloc else torch.empty((G, C, C), **f32)
            with _section(rec, "fasterquant.subgroup.slice_inputs"):
                for sub in range(G):
                    r0 = sub * R_s
                    K.prepare_subgroup(W[r0:], grads[r0:], self.H[sub], perm, Wp[r0:r0 + R_s],
                                       Gs[r0:r0 + R_s], H_work[sub])
            # surrogate inner loops refresh GHinv against the weight before the first block
            surrogate = gm_in in (nat.RQ_GMODE_SURROGATE_BLOCK, nat.RQ_GMODE_SURROGATE_ONLINE) or \
                gm_out in (nat.RQ_GMODE_SURROGATE_BLOCK, nat.RQ_GMODE_SURROGATE_ONLINE)
            anchor = Wp.clone() if surrogate else None
            # block_gd state (gptq_plus_utils.py:1024-1151): W_fp for l2 / hessian, the undamped
            # H_sub for hessian, H-Adam's curvature, the optimizer moments, the gate maps
            reg = grad_reg_strategy if block_gd else "none"
            W_fp = Wp.clone() if reg in ("l2", "hessian") else None
            H_reg = H_work.clone() if reg == "hessian" else None
            curvature = (K.kfac_curvature(H_work, curvature_damping)
                         if block_gd and grad_optimizer == "h_adam" else None)
            exp_avg = torch.zeros((R, C), **f32) if block_gd and grad_optimizer in ("adam", "h_adam") else None
            exp_avg_sq = torch.zeros((R, C), **f32) if block_gd and grad_optimizer == "adam" else None
            opt_step = 0
            gate_q = gate_s = gate_z = None
            if reg in ("quant_error_gate", "quant_error_gate_optimized"):
                if qmode == nat.RQ_QMODE_STATIC:
                    gate_q, gate_s, gate_z = nat.RQ_QMODE_STATIC, scale_tab, zero_tab
                else:
                    gate_q = nat.RQ_QMODE_CHANNEL
                    gate_s = q.scale.reshape(-1).to(**f32).contiguous()
                    gate_z = q.zero.reshape(-1).to(**f32).contiguous()
            # damped Cholesky chain, subgroups batched through every launch (the caller runs it:
            # this linear's alone, or batched with other linears')
            with _section(rec, "fasterquant.subgroup.compute_hinv"):
                if inject_hinv is None:
                    req = ChainRequest(dev, H_work, Hinv_all, Hinit_all, hdiag_all, percdamp)
                    yield req
                    chain = req.chain
                else:   # test hook: use given (Hinv_init, Hinv) pairs
                    yield None
                    chain = []
                    for sub in range(G):
                        Hinv_all[sub].copy_(inject_hinv[sub][1])
                        if Hinit_all is not None:
                            Hinit_all[sub].copy_(inject_hinv[sub][0])
                        if hdiag_all is not None:
                            hdiag_all[sub].copy_(torch.diagonal(inject_hinv[sub][0]))
                        chain.append((float(percdamp), False, 0))
            del H_work
            # GPTQ+ terms of every subgroup in one call (GH0 and Hinv^T: its workspaces)
            GH0 = torch.empty((R, C), **f32) if beta_mode == 1 else None
            HinvT = torch.empty((G, C, C), **f32) if beta_mode == 1 else None
            z_flags = torch.zeros(G, dtype=torch.int32, device=dev)
            alpha_eff = self.alpha / (R * C) if beta_mode == 1 else 0.0
            beta_all = torch.empty(R if beta_mode == 1 else 1, **f32)
            with _section(rec, "fasterquant.subgroup.init_ghinv"):
                K.gptqplus_terms(Gs, hdiag_all, Hinv_all, alpha_eff, float(self.reference_loss), beta_mode,
                                 beta_all, Z, GH, GH0, z_flags, HinvT)
            if beta_mode == 1 and self.reference_loss <= 0:
                beta_all = torch.zeros(R, **f32)
            self.subgroup_info = []
            for sub in range(G):
                r0 = sub * R_s
                beta = beta_all[r0:r0 + R_s] if beta_mode == 1 else beta_all
                if inject.get("terms") is not None:   # test hook: given (beta, Z, GHinv)
                    b_in, z_in, gh_in = inject["terms"][sub]
                    beta = b_in.to(**f32).reshape(-1).clone()
                    Z[r0:r0 + R_s].copy_(z_in)
                    GH[r0:r0 + R_s].copy_(gh_in)
                    zs = Z[r0:r0 + R_s]
                    z_flags[sub] = ((zs != 0) | torch.isnan(zs)).any().to(torch.int32)
                damp, fallback, attempts = chain[sub]
                self.subgroup_info.append(dict(damp_percent=damp, identity_fallback=fallback,
                                               attempts=attempts, beta=beta))
            if not block_bw:
                del Gs, GH0, HinvT
            beta_rows = None
            if surrogate:
                beta_rows = torch.zeros(R, **f32)
                if beta_mode == 1:
                    for sub, info in enumerate(self.subgroup_info):
                        beta_rows[sub * R_s:(sub + 1) * R_s].copy_(info["beta"])
            self.GHinv_initial = GH.clone() if keep_hinv else None
            z_any = torch.amax(z_flags).reshape(1).contiguous()
            z_zero = not bool(z_any.item())      # one read-back: Z identically zero

            codes = torch.empty((R, C), dtype=torch.int16, device=dev)
            err = torch.empty((R, min(blocksize, C)), **f32)
            nblocks = (C + blocksize - 1) // blocksize
            dyn_scale = torch.empty((nblocks, R), **f32) if qmode == nat.RQ_QMODE_DYNAMIC else None
            n_refresh_total = max(nblocks - 1, 0)
            sos = float(second_order_scale) if block_gd else 1.0

            def snapshot(i_q):
                # the caller's layer sees each subgroup's current weight, quantized columns
                # replaced by Q, in the layer's own column order (:1412-1420, :1578-1588)
                return K.current_weight(Wp, codes, i_q, qmode, scale_tab, col_group, dyn_scale,
                                        blocksize, invperm=invperm).reshape(self.layer.weight.shape)

            def refreshed(grad):
                grad = grad.to(dev).float().reshape(R, C)
                return grad if grad.is_contiguous() else grad.contiguous()

            # Frozen mode with the GPTQ+ terms identically zero and no refresh between blocks: one
            # launch per block quantises block k+1 while block k's wide update runs
            # (rq_quant_block_lookahead; equal bit for bit to the two calls per block below)
            lookahead = (gm_in == nat.RQ_GMODE_FROZEN and gm_out == nat.RQ_GMODE_FROZEN and z_zero
                         and not (block_bw or block_gd) and nblocks > 1 and blocksize % 8 == 0
                         and C % 4 == 0
                         and not (qmode == nat.RQ_QMODE_DYNAMIC and (q.mse or not q.perchannel)))
            if lookahead:
                with _section(rec, "fasterquant.block_loop"):
                    errs = (err, torch.empty_like(err))
                    for bidx, i1 in enumerate(range(0, C, blocksize)):
                        i2 = min(i1 + blocksize, C)
                        atomic = bool(block_atomic_quant) and i2 < C
                        ds = dyn_scale[bidx] if dyn_scale is not None else None
                        if bidx == 0:
                            K.quant_block(Wp, Hinv_all, GH, Z, R_s, i1, i2 - i1, qmode, scale_tab, col_group,
                                          ds, maxq, sym, atomic, z_any, codes, errs[0], gm_in, anchor,
                                          beta_rows, sos)
                        if i2 < C:
                            n2 = min(i2 + blocksize, C)
                            K.quant_block_lookahead(Wp, Hinv_all, R_s, i1, i2 - i1, errs[bidx % 2], n2 - i2,
                                                    qmode, scale_tab, col_group,
                                                    dyn_scale[bidx + 1] if dyn_scale is not None else None,
                                                    maxq, sym, bool(block_atomic_quant) and n2 < C, codes,
                                                    errs[(bidx + 1) % 2])
            with _section(rec, "fasterquant.block_loop"):
                for bidx, i1 in enumerate(range(0, C, blocksize) if not lookahead else ()):
                    i2 = min(i1 + blocksize, C)
                    count = i2 - i1
                    atomic = bool(block_atomic_quant) and i2 < C
                    if qmode == nat.RQ_QMODE_DYNAMIC and (q.mse or not q.perchannel):
                        # dynamic groups with the clip search, or one scale per subgroup block
                        # (perchannel=False): find_params on the block start
                        # (gptq_plus_utils.py:1208-1209), then quantize with those row scales
                        bscale, _ = q.row_params(Wp[:, i1:i2], R_s)
                        dyn_scale[bidx].copy_(bscale)
                        K.quant_block(Wp, Hinv_all, GH, Z, R_s, i1, count, nat.RQ_QMODE_CHANNEL,
                                      dyn_scale[bidx], None, None, maxq, sym, atomic, z_any, codes, err,
                                      gm_in, anchor, beta_rows, sos)
                    else:
                        K.quant_block(Wp, Hinv_all, GH, Z, R_s, i1, count, qmode, scale_tab, col_group,
                                      dyn_scale[bidx] if dyn_scale is not None else None, maxq, sym,
                                      atomic, z_any, codes, err, gm_in, anchor, beta_rows, sos)
                    if block_bw and enable_gradient_update:
                        # block_backward (:1408-1448): gradient at the current weight, then
                        # beta / Z / GHinv recomputed and the anchor moved to the current weight
                        if gradient_refresh_fn is None:
                            raise ValueError("`gradient_refresh_fn` must be provided for g_update_mode='block_backward'.")
                        with _section(rec, "fasterquant.block.true_gradient_refresh"):
                            grad, meta = gradient_refresh_fn(snapshot(i2))
                            K.gather_cols(refreshed(grad), perm, out=Gs)
                            beta_all = torch.empty(R if beta_mode == 1 else 1, **f32)
                            K.gptqplus_terms(Gs, hdiag_all, Hinv_all, alpha_eff, float(self.reference_loss),
                                             beta_mode, beta_all, Z, GH, GH0, z_flags, HinvT)
                            if beta_mode == 1 and self.reference_loss > 0:
                                beta_rows.copy_(beta_all)
                            z_any = torch.amax(z_flags).reshape(1).contiguous()
                            z_zero = not bool(z_any.item())
                            K.current_weight(Wp, codes, i2, qmode, scale_tab, col_group, dyn_scale,
                                             blocksize, out=anchor)
                        stats = {}
                        if refresh_full_metrics and i2 < C:
                            stats = _grad_stats(Gs[:, i2:], grad_clip)
                        if block_observer is not None:
                            block_observer(self._observer_record(i1, i2, blocksize, meta, block_gd=False,
                                                                 stats=stats))
                    if i2 < C:
                        K.trailing_update(Wp, GH, Z, Hinv_all, R_s, i1, count, err, z_any, gm_out,
                                          anchor, beta_rows, sos, z_zero=z_zero)
                    if block_gd and enable_gradient_update and i2 < C:
                        # block_gd (:1572-1834): one optimizer step on the trailing columns
                        if gradient_refresh_fn is None:
                            raise ValueError("`gradient_refresh_fn` must be provided for g_update_mode='block_gd'.")
                        with _section(rec, "fasterquant.block.true_gradient_refresh"):
                            total = (slide_refresh_block_total if slide_refresh_block_total is not None
                                     else n_refresh_total)
                            idx = slide_refresh_start + i1 // blocksize
                            slide_alpha = 1.0 - idx / max(total - 1, 1) if total > 1 else 1.0
                            grad, meta = gradient_refresh_fn(snapshot(i2), slide_alpha=slide_alpha)
                            grad = refreshed(grad)
                        with _section(rec, "fasterquant.block.outer_update_grad_descent"):
                            hreg = None
                            if reg == "hessian":
                                diff = K.current_weight(Wp, codes, i2, qmode, scale_tab, col_group,
                                                        dyn_scale, blocksize, sub_ref=W_fp)
                                hreg = K.hessian_reg_gemm(diff, H_reg, R_s, i2)
                                del diff
                            if grad_optimizer != "sgd":
                                opt_step += 1
                            stats, parts = {}, None
                            if refresh_full_metrics:
                                # the applied second-order step (:1546-1553) and the refreshed
                                # gradient's trailing columns, permuted (:1626-1681)
                                second = torch.cat([sos * err[r0:r0 + R_s, :count].matmul(
                                    Hinv_all[s_][i1:i2, i2:]) for s_, r0 in enumerate(range(0, R, R_s))])
                                stats.update(_update_stats(second, "second_order_update", outliers=True))
                                gperm = grad if perm is None else grad.index_select(1, perm)
                                stats.update(_grad_stats(gperm[:, i2:], grad_clip))
                                del second, gperm
                                parts = torch.empty((4, R, C - i2), **f32)
                            K.block_gd_step(Wp, R_s, i2, grad, perm, grad_optimizer, opt_step, grad_lr,
                                            grad_clip, exp_avg, exp_avg_sq, curvature, reg,
                                            grad_reg_lambda, W_fp, hreg, gate_q or 0, gate_s, gate_z,
                                            col_group, maxq, sym, grad_gate_floor, grad_gate_sharpness,
                                            grad_gate_sine_amp, stats_parts=parts)
                            if parts is not None:
                                # :1759-1783: the optimizer step, the applied update, the
                                # regularizer and sine parts
                                stats.update(_update_stats(parts[0], "first_order_raw"))
                                stats.update(_update_stats(parts[1], "first_order_update", outliers=True))
                                stats.update(_update_stats(parts[2], "regularizer_update"))
                                stats.update(_update_stats(parts[3], "sine_regularizer_update"))
                                del parts
                        if block_observer is not None:
                            block_observer(self._observer_record(i1, i2, blocksize, meta, block_gd=True,
                                                                 stats=stats))

            with _section(rec, "fasterquant.write_layer_weight"):
                Q = torch.empty((R, C), dtype=W.dtype, device=dev)
                w_int = torch.empty((R, C), **f32) if export_to_et else None
                scale_full = torch.empty((R, C), **f32) if export_to_et else None
                nan_flag = torch.zeros(1, dtype=torch.int32, device=dev)
                K.writeback(codes, invperm, qmode, scale_tab, col_group, dyn_scale, blocksize, Q,
                            w_int, scale_full, nan_flag)
                if export_to_et:
                    self.layer.register_buffer("int_weight", w_int.reshape(self.layer.weight.shape))
                    self.layer.register_buffer("scale", scale_full)
                self.layer.weight.data = Q.reshape(self.layer.weight.shape)

        self.perm, self.invperm = perm, invperm
        self._codes_perm = codes
        self.qmode, self.scale_table, self.col_group, self.dyn_scale = qmode, scale_tab, col_group, dyn_scale
        self.blocksize_used, self.groupsize_used = blocksize, groupsize
        self.Hinv_all = Hinv_all if keep_hinv else None
        self.Hinv_init_all = Hinit_all if keep_hinv else None
        self.Z = Z if keep_hinv else None
        if int(nan_flag.item()):
            logging.warning("NaN in weights")
            raise ValueError("NaN in weights")

    @staticmethod
    def _chol_batch(C, G, dev):
        return _chol_batch(C, G, dev)

    @property
    def codes(self):
        """Integer codes (int16) in natural column order, shape (R, C)."""
        if self._codes_perm is None:
            return None
        return self._codes_perm if self.invperm is None else self._codes_perm[:, self.invperm]

    def _observer_record(self, i1, i2, blocksize, meta, block_gd, stats=None):
        """The per-block dict the reference hands to ``block_observer`` (:1462-1496,
        :1784-1817); the refresh_full_metrics statistics come from ``stats`` (None when absent,
        as in the reference with the flag off)."""
        rec = {"block_idx": i1 // blocksize, "col_start": i1, "col_end": i2,
               "remaining_columns": self.columns - i2}
        for k in ("remaining_grad_abs_mean", "remaining_grad_clipped_abs_mean", "remaining_grad_mean_row_l2",
                  "second_order_update_abs_mean", "second_order_update_mean_row_l2",
                  "second_order_update_abs_max", "second_order_update_abs_q99", "first_order_raw_abs_mean",
                  "first_order_raw_mean_row_l2", "first_order_update_abs_mean",
                  "first_order_update_mean_row_l2", "first_order_update_abs_max",
                  "first_order_update_abs_q99", "regularizer_update_abs_mean",
                  "regularizer_update_mean_row_l2", "sine_regularizer_update_abs_mean",
                  "sine_regularizer_update_mean_row_l2"):
            rec[k] = (stats or {}).get(k)
        keys = ["mean_refresh_loss", "train_mean_refresh_loss", "val_mean_refresh_loss",
                "refresh_subset_mean_refresh_loss"]
        if block_gd:
            keys += ["slide_alpha", "mean_refresh_loss_current", "mean_refresh_loss_next"]
        for k in keys:
            rec[k] = None if meta is None else meta.get(k)
        return rec

    @staticmethod
    def _validate(grad_reg_strategy, grad_reg_lambda=0.0, grad_gate_floor=0.1, grad_gate_sharpness=1.0,
                  grad_gate_sine_amp=0.0):
        # gptq_plus_utils.py:658-677
        valid = {"none", "l2", "hessian", "quant_error_gate", "quant_error_gate_optimized"}
        if grad_reg_strategy not in valid:
            raise ValueError(f"Unsupported `grad_reg_strategy={grad_reg_strategy}`.")
        if grad_reg_lambda < 0:
            raise ValueError(f"`grad_reg_lambda` must be non-negative. Got {grad_reg_lambda}.")
        if not (0.0 <= grad_gate_floor <= 1.0):
            raise ValueError(f"`grad_gate_floor` must be in [0, 1]. Got {grad_gate_floor}.")
        if grad_gate_sharpness < 0:
            raise ValueError(f"`grad_gate_sharpness` must be non-negative. Got {grad_gate_sharpness}.")
        if grad_gate_sine_amp < 0:
            raise ValueError(f"`grad_gate_sine_amp` must be non-negative. Got {grad_gate_sine_amp}.")

    # gptq_plus_utils.py:2357-2361
    def export_packed(self):
        """Packed form of the quantized weight (call after ``fasterquant``, before ``free``):
        see ``gptq_plus_mp_quant_amd.export.export_packed``."""
        from .export import export_packed
        return export_packed(self)

    def free(self):
        # gptq_plus_utils.py:2357-2361: drop the Hessians and return cached device memory
        # (the library's cached Hessian workspace included) to the device
        self.H = None
        self.Losses = None
        self._codes_perm = None
        self.Hinv_all = None
        K.release_hessian_workspace(self.dev)
        torch.cuda.empty_cache()


def _chol_batch(C, G, dev):
    """How many subgroup matrices to factorise per launch sequence: all of them (at most
    RQ_CHOL_MAXBATCH, the library's limit) when their fp64 workspaces fit in 40 % of the device
    memory not yet held by PyTorch's caching allocator, fewer otherwise.  Memory the allocator
    caches but does not use counts as free (mem_get_info alone would count it as used)."""
    per = int(nat.load().rq_chol_workspace_bytes(C))
    free, _ = torch.cuda.mem_get_info(dev)
    free += torch.cuda.memory_reserved(dev) - torch.cuda.memory_allocated(dev)
    return max(1, min(G, nat.RQ_CHOL_MAXBATCH, int(0.4 * free) // per))


class ChainRequest:
    """One linear's damped Cholesky chain, as fasterquant pauses for it: H_work [G, C, C] (damped
    in place), Hinv_all [G, C, C] (the upper factors), optional Hinv_init_all and diag(H^-1)
    outputs.  ``run`` factorises a list of requests with the same C as one batch of launch
    sequences (gptq_plus_utils.py:494-561 per subgroup: each keeps its own damping schedule) and
    leaves each request's [(damp, identity_fallback, attempts)] in ``chain``."""

    def __init__(self, dev, H_work, Hinv_all, Hinv_init_all, Hinv_diag, percdamp):
        self.dev, self.H_work, self.Hinv_all = dev, H_work, Hinv_all
        self.Hinv_init_all, self.Hinv_diag, self.percdamp = Hinv_init_all, Hinv_diag, percdamp
        self.chain = None

    @staticmethod
    def run(reqs):
        reqs = [r for r in reqs if r is not None]
        if not reqs:
            return
        dev, C = reqs[0].dev, reqs[0].H_work.shape[-1]
        # one batch when the requests' buffers are consecutive views of one allocation
        # (fasterquant_shared), else one batch per request
        groups, cur = [], [reqs[0]]
        for r in reqs[1:]:
            prev = cur[-1]
            same = all((getattr(r, a) is None) == (getattr(prev, a) is None)
                       for a in ("Hinv_init_all", "Hinv_diag")) and r.percdamp == prev.percdamp
            contiguous = same and all(
                getattr(r, a) is None or
                getattr(r, a).data_ptr() == getattr(prev, a).data_ptr() +
                getattr(prev, a).numel() * getattr(prev, a).element_size()
                for a in ("H_work", "Hinv_all", "Hinv_init_all", "Hinv_diag"))
            if contiguous:
                cur.append(r)
            else:
                groups.append(cur)
                cur = [r]
        groups.append(cur)
        for grp in groups:
            G = sum(r.H_work.shape[0] for r in grp)
            view = lambda a: None if getattr(grp[0], a) is None else \
                getattr(grp[0], a).as_strided((G,) + tuple(getattr(grp[0], a).shape[1:]),
                                              getattr(grp[0], a).stride())
            H_work, Hinv_all, Hinit, hdiag = (view(a) for a in ("H_work", "Hinv_all", "Hinv_init_all",
                                                                 "Hinv_diag"))
            nb = _chol_batch(C, G, dev)
            workspace = K.chol_workspace(C, dev, nb)
            chain = []
            for b0 in range(0, G, nb):
                b1 = min(G, b0 + nb)
                chain += hessian_inverse_chain(dev, H_work[b0:b1], Hinv_all[b0:b1],
                                               None if Hinit is None else Hinit[b0:b1], workspace,
                                               grp[0].percdamp,
                                               Hinv_diag_out=None if hdiag is None else hdiag[b0:b1])
            del workspace
            o = 0
            for r in grp:
                g = r.H_work.shape[0]
                r.chain = chain[o:o + g]
                o += g


@torch.no_grad()
def fasterquant_shared(gptqs, **kwargs):
    """``fasterquant(**kwargs)`` for several GPTQPlus objects of the same in_features (q/k/v, or
    gate/up), their damped Cholesky chains run as one batch: each linear's work up to the chain
    (find_params, act_order, the subgroup gathers) runs first, then the chains of all their
    subgroups go through the same launch sequences (each subgroup keeps its own damping schedule,
    gptq_plus_utils.py:494-561), then each linear's block loop and write-back.  The results are
    those of calling fasterquant on each object in turn, bit for bit."""
    gptqs = list(gptqs)
    if not gptqs:
        return
    C, dev = gptqs[0].columns, gptqs[0].dev
    if any(g.columns != C or g.dev != dev for g in gptqs):
        raise ValueError("fasterquant_shared: all modules must share in_features and device")
    inject = kwargs.get("inject") or {}
    if inject.get("hinv") is not None:
        for g in gptqs:
            g.fasterquant(**kwargs)
        return
    keep = bool(kwargs.get("keep_hinv", False))
    Gt = sum(g.num_groups for g in gptqs)
    f32 = dict(device=dev, dtype=torch.float32)
    H_work = torch.empty((Gt, C, C), **f32)
    Hinv_all = torch.empty((Gt, C, C), **f32)
    Hinit = torch.empty((Gt, C, C), **f32) if keep else None
    hdiag = torch.empty((Gt, C), **f32)
    sig = inspect.signature(GPTQPlus.fasterquant)
    sig.bind(None, **kwargs)                     # unknown arguments fail here, as in fasterquant
    full = {k: p.default for k, p in sig.parameters.items() if k != "self"}
    full.update(kwargs)
    steps, reqs, o = [], [], 0
    for g in gptqs:
        G = g.num_groups
        alloc = dict(H_work=H_work[o:o + G], Hinv_all=Hinv_all[o:o + G], Hinv_diag=hdiag[o:o + G])
        if Hinit is not None:
            alloc["Hinv_init_all"] = Hinit[o:o + G]
        o += G
        st = g._fasterquant_steps(alloc=alloc, **full)
        steps.append(st)
        reqs.append(next(st))
    ChainRequest.run(reqs)
    del H_work
    for st in steps:
        for _ in st:
            pass


@torch.no_grad()
def add_batch_shared(gptqs, inp, out=None):
    """``add_batch(inp, out)`` for several GPTQPlus objects whose modules receive the same input
    (q/k/v, or gate/up: their forward hooks in gptq_plus_utils.py:6991-7003 see one tensor).

    Each object advances its own saliency cursor and accumulates its own H / act_square exactly
    as its own add_batch would (same kernel, same tile order, so the result is bitwise the
    same), but X is streamed once for all of them: one launch for up to 32 (module, group)
    Hessians.
    """
    gptqs = list(gptqs)
    if not gptqs:
        return
    C = gptqs[0].columns
    if any(g.columns != C or g.dev != gptqs[0].dev for g in gptqs):
        raise ValueError("add_batch_shared: all modules must share in_features and device")
    parts = [g._take_saliency(inp) for g in gptqs]
    x0 = parts[0][0]
    batch, used = [], 0
    for g, (x, s) in zip(gptqs, parts):
        if x.shape != x0.shape:
            raise ValueError("add_batch_shared: the modules' saliencies keep different token counts")
        if g.num_groups > 32:                  # its own launch(es)
            K.hessian_accum(x0, s, g.H, g.act_square)
            continue
        if batch and used + g.num_groups > 32:
            K.hessian_accum_multi(x0, [b[1] for b in batch], [b[0].H for b in batch],
                                  [b[0].act_square for b in batch])
            batch, used = [], 0
        batch.append((g, s))
        used += g.num_groups
    if batch:
        K.hessian_accum_multi(x0, [b[1] for b in batch], [b[0].H for b in batch],
                              [b[0].act_square for b in batch])
    for g in gptqs:
        g.token_count += x0.shape[0]
