"""CPU restatement of the GPTQ+ per-linear quantization hot path (TEST INFRASTRUCTURE ONLY).

This module is the parity oracle.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker (or as the
timed CPU baseline) -- never as the thing that produces product results.  The product
path lives in ``gptq_plus_mp_quant_amd`` and runs hand-written gfx950 HIP kernels.

It restates, op for op and in the same torch call order on CPU tensors, the reference:

* ``WeightQuantizer.configure / find_params / fake_quantize / ready``
  -- ``utils/quant_utils.py:300-331, 390-457, 471-486``
* ``compute_safe_beta_from_reference_loss`` -- ``gptq_utils/gptq_plus_utils.py:174-194``
* ``GPTQPlus.__init__ / add_batch / finalize_hessian`` -- ``gptq_plus_utils.py:431-487, 798-908``
* ``GPTQPlus._compute_hessian_inverse_with_fallback`` -- ``gptq_plus_utils.py:494-561``
* ``GPTQPlus._compute_gradient_terms`` -- ``gptq_plus_utils.py:563-578``
* ``GPTQPlus.fasterquant`` for every ``g_update_mode``: frozen (default), surrogate_block,
  surrogate_online (``_current_ghinv`` :580-584), block_backward and block_gd (the optimizer
  step and regularizers :587-796, refresh :1408-1448, :1572-1848; the layer backward is the
  caller's ``gradient_refresh_fn``): find_params,
  static / dynamic groups, dead columns, act_order, per-subgroup state, the in-block
  column loop, the block-atomic variant, the trailing (outer) update, un-permute and
  write-back -- ``gptq_plus_utils.py:910-1396, 1500-1570, 1850-1896``.

One deviation, opt-in: ``dtype`` lets the same sequence run in float64 (used by the
closed-form pinning tests).  One report, opt-in: ``fasterquant(record_ratio=True)`` also
returns the value ``w / scale`` that each code rounds (the operand of ``torch.round`` at
quant_utils.py:477 / gptq_plus_utils.py:1306-1310), computed by the same division, so code
flips against another implementation can be classified as exact rounding ties or
near-boundary flips; it changes no computed value.

Parity pinning (see ``tests/test_oracle_*.py``): golden vectors written by importing the
reference (``tests/golden/make_golden.py``), fp64 brute-force Hessians, scipy fp64
Cholesky/inverse, textbook sequential OBS on tiny inputs, RTN reduction at H = I,
blocksize invariance of the frozen GPTQ+ update, and the atomic triangular-solve identity.
"""
from __future__ import annotations

import copy
import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional

import torch


# ---------------------------------------------------------------------------------------
# WeightQuantizer  (utils/quant_utils.py:300-486)
# ---------------------------------------------------------------------------------------
class WeightQuantizerOracle:
    """Per-channel min/max weight quantizer, restating ``WeightQuantizer``.

    ``configure`` -> quant_utils.py:309-331; ``find_params`` -> :390-457 (the ``mse`` grid
    search :422-448 included); ``fake_quantize`` -> :471-480 (note: it ignores ``zero`` and
    clamps to ``[-(maxq+1), maxq]`` even for ``sym=False``); ``ready`` -> :485-486.
    """

    def __init__(self, shape: int = 1):
        self.maxq = torch.tensor(0)
        self.scale = torch.zeros(shape)
        self.zero = torch.zeros(shape)
        self.bits = 16

    def configure(self, bits, perchannel=False, sym=True, mse=False, norm=2.4, grid=50,
                  maxshrink=0.5, weight_groupsize=-1):
        self.bits = bits
        self.perchannel = perchannel
        self.sym = sym
        self.mse = mse
        self.norm = norm
        self.grid = grid
        self.maxshrink = maxshrink
        self.weight_groupsize = weight_groupsize
        # quant_utils.py:327-331
        self.maxq = torch.tensor(2 ** (bits - 1) - 1) if sym else torch.tensor(2 ** bits - 1)

    def find_params(self, x: torch.Tensor) -> None:
        # quant_utils.py:390-457 (per-channel / per-tensor branch)
        if self.bits == 16:
            return
        if self.weight_groupsize > 0:
            self.find_params_weight_groupwise(x)
            return
        self.maxq = self.maxq.to(x.device)
        shape = x.shape
        x = x.flatten(1) if self.perchannel else x.flatten().unsqueeze(0)
        zeros = torch.zeros(x.shape[0], device=x.device, dtype=x.dtype)
        xmin = torch.minimum(x.min(1)[0], zeros)
        xmax = torch.maximum(x.max(1)[0], zeros)
        if self.sym:
            self.scale = torch.maximum(torch.abs(xmin), xmax).clamp(min=1e-5) / self.maxq
            self.zero = torch.zeros_like(self.scale)
        else:
            both_zero = (xmin == 0) & (xmax == 0)
            xmin[both_zero] = -1
            xmax[both_zero] = +1
            self.scale = (xmax - xmin).clamp(min=1e-5) / self.maxq
            self.zero = torch.round(-xmin / self.scale)
        if self.mse:
            self._mse_search(x, xmin, xmax)
        if not self.perchannel:
            self.scale = self.scale.repeat(shape[0])
            self.zero = self.zero.repeat(shape[0])
        out_shape = [-1] + [1] * (len(shape) - 1)
        self.scale = self.scale.reshape(out_shape)
        self.zero = self.zero.reshape(out_shape)

    def _mse_search(self, x, xmin, xmax):
        # quant_utils.py:422-448: shrink grid over (xmin, xmax), |q - x|^norm row error.
        best = torch.full([x.shape[0]], float("inf"), device=x.device, dtype=x.dtype)
        steps = int(self.maxshrink * self.grid)
        for i in range(steps):
            for j in range(steps):
                xmin1 = (1 - i / self.grid) * xmin
                xmax1 = (1 - j / self.grid) * xmax
                if self.sym:
                    scale1 = torch.maximum(torch.abs(xmin1), xmax1).clamp(min=1e-5) / self.maxq
                    zero1 = torch.zeros_like(scale1)
                    s = scale1.unsqueeze(1)
                    q = s * torch.clamp(torch.round(x / s), -(self.maxq + 1), self.maxq)
                else:
                    scale1 = (xmax1 - xmin1) / self.maxq
                    zero1 = torch.round(-xmin1 / scale1)
                    s, z = scale1.unsqueeze(1), zero1.unsqueeze(1)
                    q = s * (torch.clamp(torch.round(x / s) + z, 0, self.maxq) - z)
                q -= x
                q.abs_()
                q.pow_(self.norm)
                err = torch.sum(q, 1)
                better = err < best
                if torch.any(better):
                    best[better] = err[better]
                    self.scale[better] = scale1[better]
                    self.zero[better] = zero1[better]

    def find_params_weight_groupwise(self, x: torch.Tensor) -> None:
        # quant_utils.py:333-388: per (row, run of weight_groupsize columns) min / max taken as
        # they are (no widening to 0), in x's own dtype, optional shrink-grid search per run;
        # scale / zero repeated over each run, in x's shape
        wg = self.weight_groupsize
        init_shape = x.shape
        x = x.reshape(x.shape[-2], x.shape[-1] // wg, wg)
        xmax = torch.amax(x, dim=-1, keepdim=True)
        xmin = torch.amin(x, dim=-1, keepdim=True)
        if self.sym:
            self.scale = torch.maximum(torch.abs(xmin), xmax).clamp(min=1e-5) / self.maxq
            self.zero = torch.zeros_like(self.scale)
        else:
            both_zero = (xmin == 0) & (xmax == 0)
            xmin[both_zero] = -1
            xmax[both_zero] = +1
            self.scale = (xmax - xmin).clamp(min=1e-5) / self.maxq
            self.zero = torch.round(-xmin / self.scale)
        self.scale = self.scale.repeat(1, 1, wg)
        self.zero = self.zero.repeat(1, 1, wg)
        if self.mse:
            best = torch.full([x.shape[0], x.shape[1]], float("inf"), device=x.device).type_as(x)
            steps = int(self.maxshrink * self.grid)
            for i in range(steps):
                for j in range(steps):
                    xmin1 = (1 - i / self.grid) * xmin
                    xmax1 = (1 - j / self.grid) * xmax
                    if self.sym:
                        scale1 = torch.maximum(torch.abs(xmin1), xmax1).clamp(min=1e-5) / self.maxq
                        zero1 = torch.zeros_like(scale1)
                        scale1 = scale1.repeat(1, 1, wg)
                        zero1 = zero1.repeat(1, 1, wg)
                        q = scale1 * torch.clamp(torch.round(x / scale1), -(self.maxq + 1), self.maxq)
                    else:
                        scale1 = (xmax1 - xmin1) / self.maxq
                        zero1 = torch.round(-xmin1 / scale1)
                        scale1 = scale1.repeat(1, 1, wg)
                        zero1 = zero1.repeat(1, 1, wg)
                        q = scale1 * (torch.clamp(torch.round(x / scale1) + zero1, 0, self.maxq) - zero1)
                    q -= x
                    q.abs_()
                    q.pow_(self.norm)
                    err = torch.sum(q, -1)
                    better = err < best
                    if torch.any(better):
                        best[better] = err[better]
                        self.scale[better] = scale1[better]
                        self.zero[better] = zero1[better]
        self.scale = self.scale.reshape(init_shape)
        self.zero = self.zero.reshape(init_shape)

    def fake_quantize(self, x, st_idx=None, end_idx=None):
        # quant_utils.py:471-480
        if self.ready() and self.bits < 16:
            scale = self.scale.to(x.device)
            if st_idx is not None and end_idx is not None:
                scale = scale[st_idx:end_idx]
            q = torch.clamp(torch.round(x / scale), -(self.maxq + 1), self.maxq)
            return (scale * q).to(x.dtype), q, scale
        return None, None, None

    def ready(self):
        return torch.all(self.scale != 0)


# ---------------------------------------------------------------------------------------
# GPTQ+ first-order term helpers
# ---------------------------------------------------------------------------------------
def safe_beta_from_reference_loss(gradients_sub, hinv_init, reference_loss, alpha):
    """gptq_plus_utils.py:174-194 (``compute_safe_beta_from_reference_loss``)."""
    ghinv_init = gradients_sub.matmul(hinv_init)
    if reference_loss <= 0:
        return torch.zeros(gradients_sub.shape[0], dtype=gradients_sub.dtype), ghinv_init
    c = (gradients_sub * ghinv_init).sum(dim=1) - (
        (ghinv_init ** 2) / torch.diagonal(hinv_init).unsqueeze(0)).mean(1)
    target = 2 * alpha * reference_loss
    c = torch.clamp(c, min=target)
    ratio = torch.where(c > 0, target / c, torch.zeros_like(c))
    ratio = torch.clamp(ratio, min=0.0, max=1.0)
    beta = 1 - torch.sqrt(torch.clamp(1 - ratio, min=0.0))
    beta = torch.nan_to_num(beta, nan=0.0, posinf=1.0, neginf=0.0)
    return beta, ghinv_init


def hessian_inverse_with_fallback(H_sub, percdamp=0.01, damp_auto_increment=0.0015):
    """gptq_plus_utils.py:494-561.  Returns (Hinv_init, Hinv_upper, damp_percent, identity_fallback, attempts).

    Damping is cumulative across retries on the same working copy; ``damp_percent >= 1``
    gives the identity fallback.
    """
    damp_percent = float(percdamp)
    if damp_percent <= 0:
        raise ValueError(f"`damp_percent` must be positive. current is {damp_percent}")
    H_work = H_sub.clone()
    idx = torch.arange(H_work.shape[0])
    attempts = 0
    while 1 > damp_percent > 0:
        attempts += 1
        try:
            damp = damp_percent * torch.mean(torch.diag(H_work))
            H_work[idx, idx] += damp
            chol = torch.linalg.cholesky(H_work)
            Hinv_init = torch.cholesky_inverse(chol)
            Hinv = torch.linalg.cholesky(Hinv_init, upper=True)
            if not torch.isfinite(Hinv_init).all() or not torch.isfinite(Hinv).all():
                raise torch._C._LinAlgError("non-finite Hinv")
            return Hinv_init, Hinv, damp_percent, False, attempts
        except torch._C._LinAlgError:
            damp_percent += damp_auto_increment
    if damp_percent >= 1:
        eye = torch.eye(H_sub.shape[0], dtype=H_sub.dtype)
        return eye, eye, damp_percent, True, attempts
    raise ValueError(f"`damp_percent` must between 0 and 1. current is {damp_percent}")


def gradient_terms(gradients_sub, Hinv_init, Hinv, alpha, reference_loss, rows, columns,
                   enable_gradient_update=True):
    """gptq_plus_utils.py:563-578.  Returns (beta, Z, GHinv, GHinv_init)."""
    if enable_gradient_update and alpha > 0:
        a = alpha / (rows * columns)
        beta, GHinv_init = safe_beta_from_reference_loss(gradients_sub, Hinv_init, reference_loss, a)
    else:
        beta = torch.zeros([1]).to(gradients_sub)
        GHinv_init = gradients_sub.matmul(Hinv_init)
    beta_view = beta.unsqueeze(1)
    Z = gradients_sub.matmul(Hinv.T) * beta_view
    GHinv = Z.matmul(Hinv)
    return beta, Z, GHinv, GHinv_init


def _current_ghinv(base, current_weight, ref_weight, beta_view, refresh_mode):
    """gptq_plus_utils.py:580-584."""
    if refresh_mode == "frozen":
        return base
    return base + beta_view * (current_weight - ref_weight)


# ---------------------------------------------------------------------------------------
# block_gd: optimizer step and first-order regularizers on the trailing columns
# ---------------------------------------------------------------------------------------
def kfac_curvature_diag(in_features, input_sq, damping=0.1):
    """gptq_utils/gptq_plus_utils.py:4601-4640 without an output factor (the call at :1148
    passes None): the mean-normalised input diagonal as a [1, C] row, plus ``damping``."""
    a = input_sq.to(dtype=torch.float32).clamp_min(0.0)
    a = a / a.mean().clamp_min(1e-12)
    curvature = a.view(1, in_features)
    if damping and damping > 0:
        curvature = curvature + float(damping)
    return curvature


def make_opt_state(weight_sub, grad_optimizer, curvature_full=None):
    """gptq_plus_utils.py:587-605."""
    if grad_optimizer not in {"sgd", "adam", "h_adam"}:
        raise ValueError(f"Unsupported `grad_optimizer={grad_optimizer}`.")
    st = {"type": grad_optimizer, "step": 0}
    if grad_optimizer in ("adam", "h_adam"):
        st["exp_avg"] = torch.zeros_like(weight_sub)
    if grad_optimizer == "adam":
        st["exp_avg_sq"] = torch.zeros_like(weight_sub)
    if grad_optimizer == "h_adam":
        if curvature_full is None:
            raise ValueError("h_adam requires `curvature_full` (KFAC curvature diagonal).")
        st["curvature"] = curvature_full
    return st


def clear_opt_state(opt, c0, c1):
    """gptq_plus_utils.py:607-614."""
    if opt is None or c1 <= c0:
        return
    if opt["type"] in ("adam", "h_adam"):
        opt["exp_avg"][:, c0:c1].zero_()
    if opt["type"] == "adam":
        opt["exp_avg_sq"][:, c0:c1].zero_()


def opt_update(opt, grad_sub, c0, lr, grad_clip=1.0, b1=0.9, b2=0.999, eps=1e-8):
    """gptq_plus_utils.py:616-655: the step for columns [c0, C)."""
    g = grad_sub[:, c0:]
    if g.numel() == 0:
        return g
    if grad_clip is not None and grad_clip > 0:
        g = g.clamp(min=-grad_clip, max=grad_clip)
    if opt["type"] == "sgd":
        return lr * g
    opt["step"] += 1
    m = opt["exp_avg"][:, c0:]
    m.mul_(b1).add_(g, alpha=1 - b1)
    bc1 = 1 - b1 ** opt["step"]
    if opt["type"] == "h_adam":
        denom = opt["curvature"][:, c0:].sqrt() + eps
        return (lr / bc1) * (m / denom)
    v = opt["exp_avg_sq"][:, c0:]
    v.mul_(b2).addcmul_(g, g, value=1 - b2)
    bc2 = 1 - b2 ** opt["step"]
    denom = v.sqrt() / math.sqrt(bc2)
    denom.add_(eps)
    return (lr / bc1) * (m / denom)


def validate_regularizer(strategy, lam=0.0, floor=0.1, sharp=1.0, sine_amp=0.0):
    """gptq_plus_utils.py:657-678."""
    valid = {"none", "l2", "hessian", "quant_error_gate", "quant_error_gate_optimized"}
    if strategy not in valid:
        raise ValueError(f"Unsupported `grad_reg_strategy={strategy}`.")
    if lam < 0:
        raise ValueError(f"`grad_reg_lambda` must be non-negative. Got {lam}.")
    if not (0.0 <= floor <= 1.0):
        raise ValueError(f"`grad_gate_floor` must be in [0, 1]. Got {floor}.")
    if sharp < 0:
        raise ValueError(f"`grad_gate_sharpness` must be non-negative. Got {sharp}.")
    if sine_amp < 0:
        raise ValueError(f"`grad_gate_sine_amp` must be non-negative. Got {sine_amp}.")


def gate_quant_maps(base_q, weight_sub, groupsize, r0, r1, groups=None, perm=None):
    """gptq_plus_utils.py:680-710: per-element (scale, zero) of the quantizer grid."""
    gs = torch.zeros_like(weight_sub)
    gz = torch.zeros_like(weight_sub)
    if groupsize == -1:
        gs.copy_(base_q.scale[r0:r1].expand_as(weight_sub))
        gz.copy_(base_q.zero[r0:r1].expand_as(weight_sub))
        return gs, gz
    if groups is None:
        raise ValueError("`groups` must be provided when groupsize != -1.")
    ids = (torch.arange(weight_sub.shape[1]) if perm is None else perm) // groupsize
    for gid, gq in enumerate(groups):
        mask = ids == gid
        n = int(mask.sum().item())
        if n == 0:
            continue
        gs[:, mask] = gq.scale[r0:r1].expand(-1, n)
        gz[:, mask] = gq.zero[r0:r1].expand(-1, n)
    return gs, gz


def nearest_quant_grid(w, scale, zero, maxq, sym):
    """gptq_plus_utils.py:712-719."""
    scale = scale.clamp(min=1e-8)
    if sym:
        return scale * torch.clamp(torch.round(w / scale), -(maxq + 1), maxq)
    q = torch.clamp(torch.round(w / scale) + zero, 0, maxq)
    return scale * (q - zero)


def sine_regularizer_update(w, scale, zero, sym, amp):
    """gptq_plus_utils.py:721-728."""
    scale = scale.clamp(min=1e-8)
    phase = 2 * math.pi * (w / scale) if sym else 2 * math.pi * ((w / scale) + zero)
    return amp * (2 * math.pi / scale) * torch.sin(phase)


def apply_regularizer(st, current, upd, c0, lr, strategy, lam, floor, sharp, sine_amp, maxq, sym):
    """gptq_plus_utils.py:730-796: returns (update, gate part, sine part)."""
    if upd.numel() == 0:
        return upd, upd, torch.zeros_like(upd)
    validate_regularizer(strategy, lam, floor, sharp, sine_amp)
    cur = current[:, c0:]
    if strategy == "none":
        z = torch.zeros_like(upd)
        return upd, z, z
    if strategy == "l2":
        reg = lr * lam * (cur - st["full_precision_weight"][:, c0:])
        return upd + reg, reg, torch.zeros_like(reg)
    if strategy == "hessian":
        diff = current - st["full_precision_weight"]
        reg = lr * lam * diff.matmul(st["hessian_reg"][:, c0:])
        return upd + reg, reg, torch.zeros_like(reg)
    sc = st["gate_scale"][:, c0:]
    zr = st["gate_zero"][:, c0:]
    qn = nearest_quant_grid(cur, sc, zr, maxq, sym)
    dist = (cur - qn).abs() / sc.clamp(min=1e-8)
    gate = floor + (1.0 - floor) * (1.0 - torch.exp(-sharp * dist))
    gated = upd * gate
    gate_part = gated - upd
    if strategy == "quant_error_gate":
        return gated, gate_part, torch.zeros_like(gate_part)
    sine = lr * sine_regularizer_update(cur, sc, zr, sym, sine_amp)
    return gated + sine, gate_part, sine


# ---------------------------------------------------------------------------------------
# refresh_full_metrics statistics and the block_observer record
# ---------------------------------------------------------------------------------------
def quantile_large(tensor, q):
    """gptq_plus_utils.py:46-60."""
    flat = tensor.reshape(-1)
    n = flat.numel()
    if n == 0:
        return None
    k = max(1, min(n, int(n * q + 0.5)))
    try:
        return torch.quantile(flat, q).item()
    except RuntimeError:
        return flat.kthvalue(k).values.item()


def _update_term_stats(chunks, name, outliers):
    """gptq_plus_utils.py:1657-1668, 1764-1798: abs mean and mean row L2 norm of the rows of all
    subgroups, with outliers also the abs max and the 0.99 quantile."""
    cat = torch.cat(chunks, dim=0).float()
    a = cat.abs()
    out = {f"{name}_abs_mean": a.mean().item(),
           f"{name}_mean_row_l2": torch.linalg.norm(cat, dim=1).mean().item()}
    if outliers:
        out[f"{name}_abs_max"] = a.max().item()
        out[f"{name}_abs_q99"] = quantile_large(a, 0.99)
    return out


def _trailing_grad_stats(chunks, grad_clip):
    """gptq_plus_utils.py:1451-1467, 1669-1687."""
    cat = torch.cat(chunks, dim=0).float()
    out = {"remaining_grad_abs_mean": cat.abs().mean().item(),
           "remaining_grad_mean_row_l2": torch.linalg.norm(cat, dim=1).mean().item()}
    if grad_clip is not None and grad_clip > 0:
        out["remaining_grad_clipped_abs_mean"] = cat.clamp(min=-grad_clip, max=grad_clip).abs().mean().item()
    else:
        out["remaining_grad_clipped_abs_mean"] = out["remaining_grad_abs_mean"]
    return out


_STAT_KEYS = ("remaining_grad_abs_mean", "remaining_grad_clipped_abs_mean", "remaining_grad_mean_row_l2",
              "second_order_update_abs_mean", "second_order_update_mean_row_l2",
              "second_order_update_abs_max", "second_order_update_abs_q99", "first_order_raw_abs_mean",
              "first_order_raw_mean_row_l2", "first_order_update_abs_mean", "first_order_update_mean_row_l2",
              "first_order_update_abs_max", "first_order_update_abs_q99", "regularizer_update_abs_mean",
              "regularizer_update_mean_row_l2", "sine_regularizer_update_abs_mean",
              "sine_regularizer_update_mean_row_l2")


def _observer_record(i1, i2, blocksize, columns, meta, stats, block_gd):
    """The dict handed to block_observer (gptq_plus_utils.py:1462-1496 block_backward,
    1784-1817 block_gd); statistics not computed are None."""
    rec = {"block_idx": i1 // blocksize, "col_start": i1, "col_end": i2, "remaining_columns": columns - i2}
    for k in _STAT_KEYS:
        rec[k] = stats.get(k)
    keys = ["mean_refresh_loss", "train_mean_refresh_loss", "val_mean_refresh_loss",
            "refresh_subset_mean_refresh_loss"]
    if block_gd:
        keys += ["slide_alpha", "mean_refresh_loss_current", "mean_refresh_loss_next"]
    for k in keys:
        rec[k] = None if meta is None else meta.get(k)
    return rec


# ---------------------------------------------------------------------------------------
# GPTQPlus (all g_update modes; the layer backward comes from the caller's refresh fn)
# ---------------------------------------------------------------------------------------
@dataclass
class SubgroupRecord:
    row_start: int
    row_end: int
    perm: Optional[torch.Tensor]
    invperm: Optional[torch.Tensor]
    Hinv_init: torch.Tensor
    Hinv: torch.Tensor
    damp_percent: float
    identity_fallback: bool
    attempts: int
    beta: torch.Tensor
    Z: torch.Tensor
    GHinv: torch.Tensor
    W_sub_initial: torch.Tensor


@dataclass
class FasterquantResult:
    Q: torch.Tensor            # (R, C) dequantized weight in the layer dtype (natural order)
    Q_fp32: torch.Tensor       # (R, C) same before the dtype cast
    W_int: torch.Tensor        # (R, C) integer-valued codes (compute dtype), natural order
    Scale: torch.Tensor        # (R, C) per-element scale, natural order
    subgroups: List[SubgroupRecord] = field(default_factory=list)
    ratio: Optional[torch.Tensor] = None   # (R, C) w / scale each code rounds (record_ratio)


class GPTQPlusOracle:
    """Restates ``GPTQPlus`` (gptq_plus_utils.py:430-1896) for the default frozen mode.

    ``weight`` is the layer weight (R, C) (any float dtype); ``saliency`` (N, T, G);
    ``gradient`` (R, C).  ``quantizer`` must be assigned and configured by the caller,
    exactly as ``build_gptq_for_subset`` does (gptq_plus_utils.py:6981-6987).
    """

    def __init__(self, weight, saliency, gradient, num_groups, alpha, reference_loss,
                 hessian_saliency_scale=1.0, dtype=torch.float32):
        self.weight = weight.clone()
        self.rows, self.columns = weight.shape
        self.dtype = dtype
        self.num_groups = num_groups
        assert self.num_groups == saliency.shape[2], "Number of groups must match saliency shape"
        self.alpha = alpha
        self.reference_loss = max(reference_loss, 0)
        self.hessian_saliency_scale = float(hessian_saliency_scale)
        self.saliencies = saliency.to(dtype)
        self.gradients = gradient.to(dtype)
        self.H = torch.zeros((num_groups, self.columns, self.columns), dtype=dtype)
        self.act_square = torch.zeros((self.columns,), dtype=dtype)
        self.nsamples = saliency.shape[0]
        self.index = 0
        self.token_count = 0
        self._finalized = False
        self.quantizer: Optional[WeightQuantizerOracle] = None
        assert self.rows % self.num_groups == 0, "rows must be divisible by num_groups"

    # gptq_plus_utils.py:798-857
    @torch.no_grad()
    def add_batch(self, inp, out=None, hessian=True):
        """``hessian=False`` (test option) skips the H product and keeps everything else, for
        full-size checks that take H from elsewhere."""
        if self._finalized:
            raise RuntimeError("add_batch called after finalize_hessian. Re-init GPTQPlus to reuse.")
        if inp.dim() == 2:
            inp = inp.unsqueeze(0)
        assert inp.dim() == 3
        bsz = inp.shape[0]
        sal = self.saliencies[self.index:self.index + bsz]
        self.index += bsz
        if sal.dim() == 3 and inp.shape[1] > sal.shape[1]:
            inp = inp[:, inp.shape[1] - sal.shape[1]:]
        inp = inp.reshape(-1, inp.shape[-1]).to(self.dtype)
        sal = sal.reshape(-1, sal.shape[-1]).to(self.dtype)
        n_tokens = inp.shape[0]
        if hessian:
            weighted = inp.unsqueeze(0).mul(sal.transpose(0, 1).unsqueeze(-1))
            block = torch.bmm(inp.transpose(0, 1).unsqueeze(0).expand(self.num_groups, -1, -1), weighted)
            self.H.add_(block)
        self.act_square.add_((inp ** 2).sum(0))
        self.token_count += n_tokens

    # gptq_plus_utils.py:859-908 (world size 1: the all-reduces are identities)
    @torch.no_grad()
    def finalize_hessian(self):
        if self._finalized:
            return
        total_samples = float(self.index)
        total_tokens = float(self.token_count)
        if total_samples <= 0 or total_tokens <= 0:
            raise RuntimeError("finalize_hessian called before any add_batch ran.")
        seq_len = total_tokens / total_samples
        self.H.div_(total_samples * seq_len)
        if self.hessian_saliency_scale != 1.0:
            self.H.div_(self.hessian_saliency_scale)
        self.act_square.div_(seq_len)
        self.H = 0.5 * (self.H + self.H.transpose(-1, -2))
        if not torch.isfinite(self.H).all():
            self.H = torch.nan_to_num(self.H, nan=0.0, posinf=0.0, neginf=0.0)
        self._finalized = True

    # gptq_plus_utils.py:910-1896, frozen mode only
    @torch.no_grad()
    def fasterquant(self, blocksize=128, percdamp=0.01, groupsize=-1, actorder=False,
                    static_groups=False, enable_gradient_update=True, g_update_mode="frozen",
                    block_atomic_quant=False, gradient_refresh_fn=None,
                    grad_lr=1e-3, grad_optimizer="sgd", curvature_damping=0.1,
                    grad_reg_strategy="none", grad_reg_lambda=0.0, grad_gate_floor=0.1,
                    grad_gate_sharpness=1.0, grad_gate_sine_amp=0.0, second_order_scale=1.0,
                    grad_clip=1.0, slide_refresh_start=0,
                    slide_refresh_block_total=None, block_observer=None,
                    refresh_full_metrics=False, record_ratio=False) -> FasterquantResult:
        # g_update modes: gptq_plus_utils.py:1190-1199, 1360-1367 (inner), 1408-1448
        # (block_backward refresh), 1500-1570 (outer), 1572-1848 (block_gd step)
        if g_update_mode not in ("frozen", "surrogate_block", "surrogate_online", "block_gd",
                                 "block_backward"):
            raise NotImplementedError(f"g_update_mode={g_update_mode!r}")
        validate_regularizer(grad_reg_strategy, grad_reg_lambda, grad_gate_floor,   # :942-948
                             grad_gate_sharpness, grad_gate_sine_amp)
        block_gd = g_update_mode == "block_gd"
        block_bw = g_update_mode == "block_backward"
        inner_mode = "surrogate_online" if block_bw else "frozen" if block_gd else g_update_mode
        online = inner_mode == "surrogate_online"
        outer_mode = ("frozen" if g_update_mode in ("frozen", "block_backward", "block_gd")
                      else "surrogate_block")                          # :1500
        sos = second_order_scale
        dt = self.dtype
        W = self.weight.clone().to(dt)
        quantizer = self.quantizer
        Q_final = torch.zeros_like(W)
        W_int_final = torch.zeros_like(W)
        Scale_final = torch.zeros_like(W)

        if not quantizer.ready():
            quantizer.find_params(W)                                   # :978-980

        dynamic_groups = groupsize != -1 and not static_groups         # :982-992
        if dynamic_groups and groupsize != blocksize:
            raise ValueError("`groupsize` must equal `blocksize` when using dynamic groups in GPTQ+.")
        if dynamic_groups and grad_reg_strategy in {"quant_error_gate", "quant_error_gate_optimized"}:
            raise ValueError("Dynamic weight groups are not supported with quant_error_gate regularization yet.")
        need_hreg = grad_reg_strategy == "hessian"                     # :1024-1026
        need_fp = grad_reg_strategy in {"l2", "hessian"}
        need_gate = grad_reg_strategy in {"quant_error_gate", "quant_error_gate_optimized"}

        shared_groups = None
        if groupsize != -1 and static_groups:                          # :994-1002
            shared_groups = []
            for col_start in range(0, self.columns, groupsize):
                col_end = min(col_start + groupsize, self.columns)
                qz = copy.deepcopy(quantizer)
                qz.find_params(W[:, col_start:col_end])
                shared_groups.append(qz)

        fast = groupsize == -1 and quantizer.bits < 16 and bool(quantizer.ready())   # :1008-1020
        if fast:
            fast_scale_full = quantizer.scale
            fast_maxq = int(quantizer.maxq.item())
            fast_lo = -(fast_maxq + 1)

        rows_per_sub = self.rows // self.num_groups
        states = []
        records: List[SubgroupRecord] = []
        for sub in range(self.num_groups):                             # :1027-1162
            r0, r1 = sub * rows_per_sub, (sub + 1) * rows_per_sub
            W_sub = W[r0:r1, :].clone()
            H_sub = self.H[sub].clone()
            G_sub = self.gradients[r0:r1, :].to(dt).clone()
            dead = torch.diag(H_sub) == 0
            H_sub[dead, dead] = 1
            W_sub[:, dead] = 0
            perm = invperm = None
            if actorder:
                perm = torch.argsort(self.act_square, descending=True)
                W_sub = W_sub[:, perm]
                H_sub = H_sub[perm][:, perm]
                G_sub = G_sub[:, perm]
                invperm = torch.argsort(perm)
            h_diag = torch.diagonal(H_sub).clone() if (block_gd and grad_optimizer == "h_adam") else None
            hessian_reg = H_sub.clone() if need_hreg else None         # :1061-1065
            gate_scale = gate_zero = None
            if need_gate:                                              # :1066-1078
                gate_scale, gate_zero = gate_quant_maps(quantizer, W_sub, groupsize, r0, r1,
                                                        shared_groups, perm)
            Hinv_init, Hinv, damp, fallback, attempts = hessian_inverse_with_fallback(H_sub, percdamp)
            beta, Z, GHinv, _ = gradient_terms(G_sub, Hinv_init, Hinv, self.alpha, self.reference_loss,
                                               self.rows, self.columns, enable_gradient_update)
            records.append(SubgroupRecord(r0, r1, perm, invperm, Hinv_init, Hinv, damp, fallback,
                                          attempts, beta, Z.clone(), GHinv.clone(), W_sub.clone()))
            states.append(dict(r0=r0, r1=r1, W_sub=W_sub, Hinv=Hinv, Z=Z, GHinv=GHinv, perm=perm,
                               anchor=W_sub.clone(), beta_view=beta.unsqueeze(1), Hinv_init=Hinv_init,
                               full_precision_weight=W_sub.clone() if need_fp else None,
                               hessian_reg=hessian_reg, gate_scale=gate_scale, gate_zero=gate_zero,
                               opt=make_opt_state(W_sub, grad_optimizer,
                                                  kfac_curvature_diag(self.columns, h_diag, curvature_damping)
                                                  if grad_optimizer == "h_adam" else None)
                               if block_gd else None,
                               invperm=invperm, Q=torch.zeros_like(W_sub),
                               W_int=torch.zeros_like(W_sub), Scale=torch.zeros_like(W_sub),
                               Ratio=torch.zeros_like(W_sub) if record_ratio else None,
                               fast_scale=fast_scale_full[r0:r1] if fast else None))

        n_blocks = (self.columns + blocksize - 1) // blocksize         # :1165-1167
        n_refresh_total = max(n_blocks - 1, 0)
        maxq_int = int(quantizer.maxq.item())

        def snapshot(cur_of):
            # weight_snapshot rows = each subgroup's current weight, un-permuted (:1412-1420)
            snap = self.weight.clone().to(dt)
            for st in states:
                cur = cur_of(st)
                snap[st["r0"]:st["r1"], :] = cur[:, st["invperm"]] if actorder else cur
            return snap

        for i1 in range(0, self.columns, blocksize):                   # :1169
            i2 = min(i1 + blocksize, self.columns)
            count = i2 - i1
            atomic = block_atomic_quant and i2 < self.columns          # :1174
            D = torch.arange(count - 1, -1, -1).to(W)
            block_states = []
            for st in states:
                W1 = st["W_sub"][:, i1:i2].clone()
                W_block_start = W1.clone()
                Q1 = torch.zeros_like(W1)
                W_int1 = torch.zeros_like(W1)
                Scale1 = torch.zeros_like(W1)
                Err1 = torch.zeros_like(W1)
                Hinv1 = st["Hinv"][i1:i2, i1:i2]
                GHinv1 = st["GHinv"][:, i1:i2].clone()
                Z1 = st["Z"][:, i1:i2]
                W_ref1 = st["anchor"][:, i1:i2]
                GHinv1_eff = _current_ghinv(GHinv1, W1 if online else W_block_start, W_ref1,
                                            st["beta_view"], inner_mode)
                dyn_q = None
                if dynamic_groups:                                     # :1202-1209
                    dyn_q = copy.deepcopy(quantizer)
                    dyn_q.find_params(W_block_start)
                if st["fast_scale"] is not None:
                    Scale1.copy_(st["fast_scale"].expand_as(Scale1))

                def column_quantizer(i):
                    if dyn_q is not None:
                        return dyn_q, None, None
                    if groupsize != -1:
                        idx = i1 + i
                        if actorder:
                            idx = st["perm"][idx]
                        return shared_groups[idx // groupsize], st["r0"], st["r1"]
                    return quantizer, st["r0"], st["r1"]

                if atomic:                                             # :1238-1288
                    if groupsize == -1:
                        q, iw, sc = quantizer.fake_quantize(W_block_start, st_idx=st["r0"], end_idx=st["r1"])
                        Q1.copy_(q)
                        W_int1.copy_(iw)
                        Scale1.copy_(sc.expand_as(W_block_start))
                        if record_ratio:
                            st["Ratio"][:, i1:i2] = W_block_start / sc
                    else:
                        for i in range(count):
                            qz, a, b = column_quantizer(i)
                            q, iw, sc = qz.fake_quantize(W_block_start[:, i].unsqueeze(1), st_idx=a, end_idx=b)
                            Q1[:, i] = q.flatten()
                            W_int1[:, i] = iw.flatten()
                            Scale1[:, i] = sc.flatten()
                            if record_ratio:
                                st["Ratio"][:, i1 + i] = (W_block_start[:, i].unsqueeze(1) / sc).flatten()
                    residual = W_block_start - Q1 - GHinv1_eff
                    Err1.copy_(torch.linalg.solve_triangular(Hinv1.T, residual.T, upper=False).T)
                else:                                                  # :1296-1367
                    for i in range(count):
                        w = W1[:, i]
                        d = Hinv1[i, i]
                        w_col = w.unsqueeze(1)
                        if st["fast_scale"] is not None:
                            fs = st["fast_scale"]
                            iw = torch.clamp(torch.round(w_col / fs), fast_lo, fast_maxq)
                            q_fake = (fs * iw).to(w_col.dtype)
                            sc = fs
                        else:
                            qz, a, b = column_quantizer(i)
                            q_fake, iw, sc = qz.fake_quantize(w_col, st_idx=a, end_idx=b)
                        if record_ratio:
                            st["Ratio"][:, i1 + i] = (w_col / sc).flatten()
                        q = q_fake.flatten()
                        Q1[:, i] = q
                        W_int1[:, i] = iw.flatten()
                        if st["fast_scale"] is None:
                            Scale1[:, i] = sc.flatten()
                        err1 = (w - q - GHinv1_eff[:, i]) / d
                        upd = err1.unsqueeze(1).matmul(Hinv1[i, i:].unsqueeze(0))
                        if block_gd:                                   # :1344-1349
                            W1[:, i:] -= sos * (upd + GHinv1_eff[:, i:])
                        else:
                            W1[:, i:] -= upd + GHinv1_eff[:, i:]
                        Err1[:, i] = err1
                        GHinv1[:, i:].sub_(Z1[:, i].unsqueeze(1).matmul(Hinv1[i, i:].unsqueeze(0)))
                        if inner_mode != "frozen":
                            GHinv1_eff = _current_ghinv(GHinv1, W1 if online else W_block_start, W_ref1,
                                                        st["beta_view"], inner_mode)
                st["Q"][:, i1:i2] = Q1
                st["W_int"][:, i1:i2] = W_int1
                st["Scale"][:, i1:i2] = Scale1
                if block_bw:                                           # :1389-1396
                    cur = st["W_sub"].clone()
                    if i1 > 0:
                        cur[:, :i1] = st["Q"][:, :i1]
                    cur[:, i1:i2] = Q1
                    st["current"] = cur
                block_states.append([st, Err1, Z1])

            if block_bw and enable_gradient_update:                     # :1408-1448
                if gradient_refresh_fn is None:
                    raise ValueError("`gradient_refresh_fn` must be provided for g_update_mode='block_backward'.")
                grad, meta = gradient_refresh_fn(snapshot(lambda st: st["current"]))
                grad = grad.to(dt)
                trailing = []
                for bs in block_states:
                    st = bs[0]
                    g_sub = grad[st["r0"]:st["r1"], :]
                    if actorder:
                        g_sub = g_sub[:, st["perm"]]
                    if refresh_full_metrics and g_sub[:, i2:].numel() > 0:
                        trailing.append(g_sub[:, i2:])
                    beta, Z, GHinv, _ = gradient_terms(g_sub, st["Hinv_init"], st["Hinv"], self.alpha,
                                                       self.reference_loss, self.rows, self.columns,
                                                       enable_gradient_update)
                    st["beta_view"] = beta.unsqueeze(1)
                    st["Z"], st["GHinv"] = Z, GHinv
                    st["anchor"] = st["current"].clone()
                    bs[2] = Z[:, i1:i2]
                if block_observer is not None:                         # :1448-1496
                    stats = _trailing_grad_stats(trailing, grad_clip) if trailing else {}
                    block_observer(_observer_record(i1, i2, blocksize, self.columns, meta, stats, False))

            second_chunks = []
            for st, Err1, Z1 in block_states:                          # :1500-1570
                GHinv_rest = _current_ghinv(st["GHinv"][:, i2:], st["W_sub"][:, i2:], st["anchor"][:, i2:],
                                            st["beta_view"], outer_mode)
                G_Update = count * GHinv_rest - torch.einsum("ij,j,jk->ik", Z1, D, st["Hinv"][i1:i2, i2:])
                second = Err1.matmul(st["Hinv"][i1:i2, i2:])
                if block_gd:
                    st["W_sub"][:, i2:] -= sos * (second + G_Update)
                    if refresh_full_metrics and second.numel() > 0:
                        second_chunks.append(sos * second)
                else:
                    st["W_sub"][:, i2:] -= second + G_Update
                st["GHinv"][:, i2:] -= st["Z"][:, i1:i2].matmul(st["Hinv"][i1:i2, i2:])
                if block_gd:
                    clear_opt_state(st["opt"], i1, i2)

            if block_gd and enable_gradient_update and i2 < self.columns:   # :1572-1848
                if gradient_refresh_fn is None:
                    raise ValueError("`gradient_refresh_fn` must be provided for g_update_mode='block_gd'.")

                def effective(st):
                    cur = st["W_sub"].clone()
                    cur[:, :i2] = st["Q"][:, :i2]
                    return cur
                refresh_idx = i1 // blocksize                          # :1600-1610
                total = slide_refresh_block_total if slide_refresh_block_total is not None else n_refresh_total
                idx = slide_refresh_start + refresh_idx
                slide_alpha = 1.0 - idx / max(total - 1, 1) if total > 1 else 1.0
                grad, meta = gradient_refresh_fn(snapshot(effective), slide_alpha=slide_alpha)
                grad = grad.to(dt)
                trailing, parts = [], ([], [], [], [])
                for st in states:                                      # :1688-1711
                    g_sub = grad[st["r0"]:st["r1"], :]
                    if actorder:
                        g_sub = g_sub[:, st["perm"]]
                    if refresh_full_metrics and g_sub[:, i2:].numel() > 0:
                        trailing.append(g_sub[:, i2:])
                    raw = opt_update(st["opt"], g_sub, i2, grad_lr, grad_clip=grad_clip)
                    upd, gate_part, sine_part = apply_regularizer(
                        st, effective(st), raw, i2, grad_lr, grad_reg_strategy, grad_reg_lambda,
                        grad_gate_floor, grad_gate_sharpness, grad_gate_sine_amp, maxq_int, quantizer.sym)
                    st["pending"] = upd
                    if refresh_full_metrics:                           # :1757-1763
                        if raw.numel() > 0:
                            parts[0].append(raw)
                        if upd.numel() > 0:
                            parts[1].append(upd)
                            parts[2].append(gate_part)
                            parts[3].append(sine_part)
                if block_observer is not None:                         # :1657-1817
                    stats = {}
                    if second_chunks:
                        stats.update(_update_term_stats(second_chunks, "second_order_update", True))
                    if trailing:
                        stats.update(_trailing_grad_stats(trailing, grad_clip))
                    for chunks, name, outl in zip(parts, ("first_order_raw", "first_order_update",
                                                          "regularizer_update", "sine_regularizer_update"),
                                                  (False, True, False, False)):
                        if chunks:
                            stats.update(_update_term_stats(chunks, name, outl))
                    block_observer(_observer_record(i1, i2, blocksize, self.columns, meta, stats, True))
                for st in states:                                      # :1828-1834
                    upd = st.pop("pending")
                    if upd.numel() > 0:
                        st["W_sub"][:, i2:] -= upd

        Ratio_final = torch.zeros_like(W) if record_ratio else None
        for st in states:                                              # :1850-1864
            Q, W_int_sub, Scale_sub = st["Q"], st["W_int"], st["Scale"]
            if actorder:
                Q = Q[:, st["invperm"]]
                W_int_sub = W_int_sub[:, st["invperm"]]
                Scale_sub = Scale_sub[:, st["invperm"]]
            Q_final[st["r0"]:st["r1"], :] = Q
            W_int_final[st["r0"]:st["r1"], :] = W_int_sub
            Scale_final[st["r0"]:st["r1"], :] = Scale_sub
            if record_ratio:
                Ratio_final[st["r0"]:st["r1"], :] = st["Ratio"][:, st["invperm"]] if actorder else st["Ratio"]

        Q_out = Q_final.reshape(self.weight.shape).to(self.weight.dtype)   # :1873-1875
        if torch.any(torch.isnan(Q_out)):
            raise ValueError("NaN in weights")
        return FasterquantResult(Q=Q_out, Q_fp32=Q_final, W_int=W_int_final, Scale=Scale_final,
                                 subgroups=records, ratio=Ratio_final)


# ---------------------------------------------------------------------------------------
# Convenience drivers used by tests and the CPU baseline
# ---------------------------------------------------------------------------------------
def make_quantizer(bits, sym=True, mse=False, perchannel=True, weight_groupsize=-1) -> WeightQuantizerOracle:
    q = WeightQuantizerOracle()
    q.configure(bits, perchannel=perchannel, sym=sym, mse=mse, weight_groupsize=weight_groupsize)
    return q


def run_linear(weight, X, saliency, gradient, num_groups, bits=4, sym=True, alpha=0.0,
               reference_loss=0.0, accum_bsz=16, blocksize=128, percdamp=0.01, groupsize=-1,
               actorder=True, static_groups=None, block_atomic_quant=False,
               g_update_mode="frozen", dtype=torch.float32):
    """Drive one linear like ``build_gptq_for_subset`` + ``accumulate_hessian_for_gptq`` +
    ``fasterquant`` (gptq_plus_utils.py:6954-7039, 7467-7502).  X is (N, T, C)."""
    if static_groups is None:
        static_groups = actorder
    g = GPTQPlusOracle(weight, saliency, gradient, num_groups, alpha, reference_loss, dtype=dtype)
    g.quantizer = make_quantizer(bits, sym)
    for j in range(0, X.shape[0], accum_bsz):
        g.add_batch(X[j:j + accum_bsz])
    g.finalize_hessian()
    res = g.fasterquant(blocksize=blocksize, percdamp=percdamp, groupsize=groupsize, actorder=actorder,
                        static_groups=static_groups, block_atomic_quant=block_atomic_quant,
                        g_update_mode=g_update_mode)
    return g, res


def reconstruction_error(W, Q, X):
    """Layer reconstruction error ||(W - Q) X^T||^2 / ||W X^T||^2 over tokens X (n, C), in float64."""
    W = W.double()
    Q = Q.double()
    X = X.reshape(-1, X.shape[-1]).double()
    num = ((W - Q) @ X.T).pow(2).sum()
    den = (W @ X.T).pow(2).sum()
    return float(num / den)


__all__ = [
    "WeightQuantizerOracle", "GPTQPlusOracle", "FasterquantResult", "SubgroupRecord",
    "safe_beta_from_reference_loss", "hessian_inverse_with_fallback", "gradient_terms",
    "make_quantizer", "run_linear", "reconstruction_error", "kfac_curvature_diag",
    "make_opt_state", "opt_update", "apply_regularizer", "gate_quant_maps", "nearest_quant_grid",
]
