"""Drop-in ``WeightQuantizer`` (reference: utils/quant_utils.py:300-486) whose ``find_params``
runs the gfx950 ``rq_find_params`` kernel.

Same constructor, ``configure`` arguments, attributes (``maxq``, ``scale``, ``zero``, ``bits``,
``perchannel``, ``sym``, ...) and method semantics as the reference.  ``find_params`` needs the
tensor on the GPU; ``mse=True`` runs the clip grid search kernel (``rq_find_params_mse``).
``weight_groupsize > 0`` (``find_params_weight_groupwise``: one scale per run of columns,
stored per element) runs the same kernels on the runs' own ranges, for fp32 tensors (the
reference fits 16-bit tensors in their own dtype; those raise ``NotImplementedError``).
"""
from __future__ import annotations

import torch

from . import _native as nat


def get_minq_maxq(bits, sym):
    """utils/quant_utils.py:21-29."""
    if sym:
        maxq = torch.tensor(2 ** (bits - 1) - 1)
        minq = -maxq - 1
    else:
        maxq = torch.tensor(2 ** bits - 1)
        minq = 0
    return minq, maxq


class WeightQuantizer(torch.nn.Module):
    def __init__(self, shape: int = 1) -> None:
        super().__init__()
        self.register_buffer("maxq", torch.tensor(0))
        self.register_buffer("scale", torch.zeros(shape))
        self.register_buffer("zero", torch.zeros(shape))
        self.bits = 16

    # utils/quant_utils.py:309-331
    def configure(self, bits, perchannel: bool = False, sym: bool = True, mse: bool = False,
                  norm: float = 2.4, grid: int = 50, maxshrink: float = 0.5,
                  weight_groupsize: int = -1) -> None:
        self.bits = bits
        self.perchannel = perchannel
        self.sym = sym
        self.mse = mse
        self.norm = norm
        self.grid = grid
        self.maxshrink = maxshrink
        self.weight_groupsize = weight_groupsize
        self.maxq = torch.tensor(2 ** (bits - 1) - 1) if sym else torch.tensor(2 ** bits - 1)

    def params_on(self, w: torch.Tensor, group_size: int = -1, clip_zero: bool = True):
        """Return (scale [ngroups, R], zero [ngroups, R]) for a 2-D weight without touching self
        (clip_zero: the range of each (row, group) includes 0, as in find_params; False: the
        group's own min / max, as in find_params_weight_groupwise)."""
        nat.require_gpu(w, "weight")
        if w.dim() != 2:
            raise ValueError("expected a 2-D weight")
        if w.stride(1) != 1:
            w = w.contiguous()
        R, C = w.shape
        gs = group_size if group_size > 0 else C
        ng = (C + gs - 1) // gs
        scale = torch.empty((ng, R), device=w.device, dtype=torch.float32)
        zero = torch.empty((ng, R), device=w.device, dtype=torch.float32)
        if self.mse:
            nat.call("rq_find_params_mse", nat.ptr(w), nat.dtype_code(w.dtype), R, C, w.stride(0), gs,
                     int(self.maxq), int(bool(self.sym)), int(bool(clip_zero)), float(self.norm), int(self.grid),
                     float(self.maxshrink), nat.ptr(scale), nat.ptr(zero), nat.stream_of(w.device))
        else:
            nat.call("rq_find_params", nat.ptr(w), nat.dtype_code(w.dtype), R, C, w.stride(0), gs,
                     int(self.maxq), int(bool(self.sym)), int(bool(clip_zero)), nat.ptr(scale), nat.ptr(zero),
                     nat.stream_of(w.device))
        return scale, zero

    def params_grouped(self, w: torch.Tensor, group_size: int):
        """(scale, zero) [ngroups, R] of the column groups of w, as ``find_params`` on each
        slice ``w[:, g0:g0 + group_size]`` (static groups, gptq_plus_utils.py:994-1002): per row,
        or with perchannel=False one value per group from the flattened slice, repeated over
        the rows."""
        if self.perchannel:
            return self.params_on(w, group_size)
        R, C = w.shape
        ng = (C + group_size - 1) // group_size
        scale = torch.empty((ng, R), device=w.device, dtype=torch.float32)
        zero = torch.empty((ng, R), device=w.device, dtype=torch.float32)
        for g in range(ng):
            sg, zg = self.params_on(w[:, g * group_size:(g + 1) * group_size].reshape(1, -1))
            scale[g].copy_(sg[0].expand(R))
            zero[g].copy_(zg[0].expand(R))
        return scale, zero

    def row_params(self, w: torch.Tensor, rows_per_fit: int):
        """(scale, zero) [R] for the block w [R, n] when ``find_params`` runs on each run of
        rows_per_fit rows (a GPTQ+ subgroup's block start, gptq_plus_utils.py:1202-1209): per row,
        or with perchannel=False one value per run of rows."""
        if self.perchannel:
            s, z = self.params_on(w)
            return s[0], z[0]
        R = w.shape[0]
        scale = torch.empty(R, device=w.device, dtype=torch.float32)
        zero = torch.empty(R, device=w.device, dtype=torch.float32)
        for r0 in range(0, R, rows_per_fit):
            r1 = min(R, r0 + rows_per_fit)
            sg, zg = self.params_on(w[r0:r1].reshape(1, -1))
            scale[r0:r1].copy_(sg[0].expand(r1 - r0))
            zero[r0:r1].copy_(zg[0].expand(r1 - r0))
        return scale, zero

    # utils/quant_utils.py:333-388
    def find_params_weight_groupwise(self, x) -> None:
        """One (scale, zero) per run of weight_groupsize columns of each row (x viewed as
        [x.shape[-2], -1, weight_groupsize]), from the run's own min / max (mse: the shrink-grid
        search per run), repeated over the run in x's shape."""
        nat.require_gpu(x, "x")
        wg = self.weight_groupsize
        rows, cols = x.shape[-2], x.shape[-1]
        if cols % wg or x.numel() != rows * cols:
            raise RuntimeError(f"shape '[{rows}, {cols // wg}, {wg}]' is invalid for input of size {x.numel()}")
        if x.dtype != torch.float32:
            raise NotImplementedError("weight_groupsize > 0 for a 16-bit tensor: the reference fits it in "
                                      "that dtype; pass a float32 tensor")
        w = x.reshape(rows, cols)
        if w.stride(1) != 1:
            w = w.contiguous()
        scale, zero = self.params_on(w, wg, clip_zero=False)          # [cols / wg, rows]
        self.scale = scale.t().repeat_interleave(wg, dim=1).reshape(x.shape)
        self.zero = zero.t().repeat_interleave(wg, dim=1).reshape(x.shape)

    # utils/quant_utils.py:390-457
    def find_params(self, x) -> None:
        if self.bits == 16:
            return
        nat.require_gpu(x, "x")
        self.maxq = self.maxq.to(x.device)
        if getattr(self, "weight_groupsize", -1) > 0:
            self.find_params_weight_groupwise(x)
            return
        shape = x.shape
        x2 = x.flatten(1) if self.perchannel else x.flatten().unsqueeze(0)
        scale, zero = self.params_on(x2)
        scale, zero = scale[0], zero[0]
        if not self.perchannel:
            scale = scale.repeat(shape[0])
            zero = zero.repeat(shape[0])
        out = [-1] + [1] * (len(shape) - 1)
        self.scale = scale.reshape(out)
        self.zero = zero.reshape(out)

    # utils/quant_utils.py:462-469
    def quantize(self, x):
        if self.ready() and self.bits < 16:
            scale = self.scale.to(x.device)
            if self.sym:
                return (scale * torch.clamp(torch.round(x / scale), -(self.maxq + 1), self.maxq)).to(x.dtype)
            zero = self.zero.to(x.device)
            q = torch.clamp(torch.round(x / scale) + zero, 0, self.maxq)
            return (scale * (q - zero)).to(x.dtype)
        return x

    # utils/quant_utils.py:471-480 (zero ignored, signed range even when sym=False)
    def fake_quantize(self, x, st_idx=None, end_idx=None):
        if self.ready() and self.bits < 16:
            scale = self.scale.to(x.device)
            if st_idx is not None and end_idx is not None:
                scale = scale[st_idx:end_idx]
            q = torch.clamp(torch.round(x / scale), -(self.maxq + 1), self.maxq)
            return (scale * q).to(x.dtype), q, scale
        return None, None, None

    def enabled(self):
        return self.maxq > 0

    def ready(self):
        return torch.all(self.scale != 0)
