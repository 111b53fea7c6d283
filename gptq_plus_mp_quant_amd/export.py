"""Packed export of GPTQ+ results and the ``quantizers`` dict.

The reference exports a quantized linear as two full fp32 [R, C] buffers, ``int_weight`` and
``scale`` (``export_to_et``, gptq_utils/gptq_plus_utils.py:1866-1871), and saves the
``quantizers`` dict (one ``WeightQuantizer`` per module) next to the fake-quantized
state_dict with ``torch.save`` (gptq_utils/main.py:68-71).  This module produces the compact
form of the same information, on the GPU:

* ``qweight`` -- int32 [R, ceil(C*nbits/32)]: every row an nbits-wide little-endian
  bitstream of the codes in natural column order, each stored as code + 2^(nbits-1)
  (``rq_pack_codes``).  nbits = bits for sym, bits + 1 for asym, because the asym
  fake_quantize clamps codes to the signed range [-(maxq+1), maxq] (quant_utils.py:477).
* ``scales`` -- float32 [ngroups, R]: one row per scale group (per-channel: 1 group;
  static groups: the C/groupsize column groups; dynamic groups: one per block).
* ``g_idx`` -- int32 [C]: the scale group of every natural column.

``dequantize_packed`` (``rq_unpack_dequant``) rebuilds the layer weight bit for bit.
``save_packed`` / ``load_packed`` store entries and quantizer states with safetensors, so
loading executes nothing from the file.
"""
from __future__ import annotations

import json
from typing import Dict, Optional, Tuple

import torch

from . import _native as nat
from . import kernels as K

FORMAT = "gptqplus-packed-v1"


def _nbits(bits: int, sym: bool) -> int:
    return int(bits) if sym else int(bits) + 1


def export_packed(gptq) -> Dict[str, object]:
    """Pack a ``GPTQPlus`` after ``fasterquant``.  Returns ``{"qweight", "scales", "g_idx",
    "nbits", "bits", "sym", "shape", "dtype"}``; raises if a code does not fit ``nbits``."""
    codes = getattr(gptq, "_codes_perm", None)
    if codes is None:
        raise RuntimeError("export_packed needs the codes of fasterquant (call it before free())")
    q = gptq.quantizer
    R, C = codes.shape
    dev = codes.device
    nbits = _nbits(q.bits, bool(q.sym))
    invperm = gptq.invperm
    if gptq.qmode == nat.RQ_QMODE_CHANNEL:
        scales = gptq.scale_table.reshape(1, R)
        g_idx = torch.zeros(C, dtype=torch.int32, device=dev)
    elif gptq.qmode == nat.RQ_QMODE_STATIC:
        # a scale table indexed by col_group[j] for the (permuted) column j: natural column c
        # reads col_group[invperm[c]] (GPTQ+ static groups give c // groupsize; classic GPTQ's
        # dynamic groups follow the permuted order)
        scales = gptq.scale_table
        g_idx = gptq.col_group[invperm] if invperm is not None else gptq.col_group
    else:
        # dynamic groups: one scale per block of the (permuted) column order
        scales = gptq.dyn_scale
        j = invperm if invperm is not None else torch.arange(C, device=dev)
        g_idx = (j // gptq.blocksize_used).to(torch.int32)
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    qweight = K.pack_codes(codes, nbits, invperm=invperm, range_flag=flag)
    if int(flag.item()):
        raise ValueError(f"a code does not fit {nbits} bits (NaN weight or inconsistent quantizer)")
    return dict(qweight=qweight, scales=scales.contiguous(), g_idx=g_idx.contiguous(), nbits=nbits,
                bits=int(q.bits), sym=bool(q.sym), shape=tuple(gptq.layer.weight.shape),
                dtype=str(gptq.layer.weight.dtype).replace("torch.", ""))


def dequantize_packed(entry: Dict[str, object], dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """Rebuild the dequantized weight (the ``layer.weight`` fasterquant wrote) from an entry."""
    dtype = dtype or getattr(torch, entry["dtype"])
    R = entry["qweight"].shape[0]
    C = entry["g_idx"].numel()
    q, _ = K.unpack_dequant(entry["qweight"], C, entry["nbits"], entry["scales"], entry["g_idx"], dtype)
    return q.reshape(entry["shape"]) if tuple(entry["shape"]) != (R, C) else q


def unpack_codes(entry: Dict[str, object]) -> torch.Tensor:
    """int16 codes [R, C] in natural column order."""
    C = entry["g_idx"].numel()
    _, codes = K.unpack_dequant(entry["qweight"], C, entry["nbits"], want_codes=True)
    return codes


def quantizer_state(quantizer) -> Dict[str, torch.Tensor]:
    """The tensors of one ``quantizers`` dict entry (``WeightQuantizer`` buffers)."""
    return {"scale": quantizer.scale.detach().float().contiguous(),
            "zero": quantizer.zero.detach().float().contiguous(),
            "maxq": torch.as_tensor(quantizer.maxq).detach().reshape(1).to(torch.int32)}


def save_packed(path: str, entries: Dict[str, Dict[str, object]],
                quantizers: Optional[Dict[str, object]] = None) -> None:
    """Write packed entries (and optionally the ``quantizers`` dict) to one safetensors file."""
    from safetensors.torch import save_file
    tensors, meta = {}, {"format": FORMAT}
    for name, e in entries.items():
        for key in ("qweight", "scales", "g_idx"):
            tensors[f"{name}.{key}"] = e[key].detach().contiguous().cpu()
        meta[name] = json.dumps({k: e[k] for k in ("nbits", "bits", "sym", "shape", "dtype")})
    for name, q in (quantizers or {}).items():
        for key, t in quantizer_state(q).items():
            tensors[f"w_quantizers.{name}.{key}"] = t.cpu()
    save_file(tensors, path, metadata=meta)


def load_packed(path: str, device="cuda") -> Tuple[Dict[str, Dict[str, object]], Dict[str, Dict[str, torch.Tensor]]]:
    """Read a file written by ``save_packed``: (entries, quantizer states)."""
    from safetensors import safe_open
    entries, quants = {}, {}
    with safe_open(path, framework="pt", device="cpu") as f:
        meta = f.metadata() or {}
        if meta.get("format") != FORMAT:
            raise ValueError(f"{path}: not a {FORMAT} file")
        for key in f.keys():
            t = f.get_tensor(key)
            if key.startswith("w_quantizers."):
                name, field = key[len("w_quantizers."):].rsplit(".", 1)
                quants.setdefault(name, {})[field] = t.to(device)
            else:
                name, field = key.rsplit(".", 1)
                entries.setdefault(name, {})[field] = t.to(device)
        for name, e in entries.items():
            info = json.loads(meta[name])
            info["shape"] = tuple(info["shape"])
            e.update(info)
    return entries, quants
