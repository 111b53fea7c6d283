"""ctypes binding of the C ABI in ``include/gptqplus_hip.h`` (library ``_lib/libgptqplus_hip.so``).

The library is the only compute path: if it is missing or cannot be loaded every call raises
``RuntimeError`` -- there is no silent fallback.  ``GPTQPLUS_HIP_LIB`` (environment) names
another build of the same library to load instead (e.g. a variant built for an A/B timing).
"""
from __future__ import annotations

import ctypes
import os
import re
from pathlib import Path

import torch

LIB_PATH = Path(os.environ.get("GPTQPLUS_HIP_LIB") or
                Path(__file__).resolve().parent / "_lib" / "libgptqplus_hip.so").resolve()
HEADER = Path(__file__).resolve().parent.parent / "include" / "gptqplus_hip.h"

RQ_OK, RQ_EINVAL, RQ_EHIP, RQ_ENOTSUP = 0, -1, -2, -3
RQ_F16, RQ_BF16, RQ_F32 = 0, 1, 2
RQ_QMODE_CHANNEL, RQ_QMODE_STATIC, RQ_QMODE_DYNAMIC = 0, 1, 2
RQ_GMODE_FROZEN, RQ_GMODE_SURROGATE_BLOCK, RQ_GMODE_SURROGATE_ONLINE, RQ_GMODE_BLOCK_GD = 0, 1, 2, 3
RQ_HMATH_SPLIT16, RQ_HMATH_FP32, RQ_HMATH_SPLIT16X3 = 0, 1, 2
RQ_NOALLOC_SCRATCH_BYTES = 128 << 20
RQ_CHOL_MAXBATCH = 64          # matrices per rq_chol_hinv_attempt call
RQ_ACT_ORDER_MAXC = 65536      # widest rq_act_order_perm
# g_update_mode -> (kernel mode of the in-block loop, kernel mode of the trailing update);
# gptq_plus_utils.py:1190 (inner) and :1500 (outer)
GMODES = {"frozen": (RQ_GMODE_FROZEN, RQ_GMODE_FROZEN),
          "surrogate_block": (RQ_GMODE_SURROGATE_BLOCK, RQ_GMODE_SURROGATE_BLOCK),
          "surrogate_online": (RQ_GMODE_SURROGATE_ONLINE, RQ_GMODE_SURROGATE_BLOCK),
          "block_gd": (RQ_GMODE_BLOCK_GD, RQ_GMODE_BLOCK_GD),
          "block_backward": (RQ_GMODE_SURROGATE_ONLINE, RQ_GMODE_FROZEN)}

_P, _I, _L, _D = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_double

# name -> (restype, argtypes); mirrors include/gptqplus_hip.h
SIGNATURES = {
    "rq_version": (_I, []),
    "rq_hessian_accum": (_I, [_P, _I, _L, _L, _I, _P, _L, _I, _P, _P, _P, _L, _P]),
    "rq_hessian_accum_noalloc": (_I, [_P, _I, _L, _L, _I, _P, _L, _I, _P, _P, _P]),
    "rq_hessian_workspace_bytes": (_L, [_L, _I, _I, _I]),
    "rq_hessian_math": (_I, [_I]),
    "rq_hessian_timing_events": (_I, [_P, _P]),
    "rq_hessian_accum_multi": (_I, [_P, _I, _L, _L, _I, _I, _P, _P, _P, _P, _P, _L, _P]),
    "rq_hessian_finalize": (_I, [_P, _P, _I, _I, _D, _D, _D, _I, _P, _P]),
    "rq_find_params": (_I, [_P, _I, _I, _I, _L, _I, _I, _I, _I, _P, _P, _P]),
    "rq_find_params_mse": (_I, [_P, _I, _I, _I, _L, _I, _I, _I, _I, _D, _I, _D, _P, _P, _P]),
    "rq_act_order_perm": (_I, [_P, _I, _P, _P, _P]),
    "rq_prepare_subgroup": (_I, [_P, _I, _L, _P, _L, _P, _I, _I, _P, _P, _L, _P, _L, _P, _P]),
    "rq_chol_workspace_bytes": (_L, [_I]),
    "rq_chol_hinv_attempt": (_I, [_P, _I, _I, _P, _P, _P, _P, _P, _P, _P]),
    "rq_gptqplus_terms": (_I, [_P, _L, _P, _P, _P, _I, _I, _I, _D, _D, _I, _P, _P, _P, _L, _P, _P, _P]),
    "rq_quant_block": (_I, [_P, _L, _P, _I, _P, _P, _L, _I, _I, _I, _I, _I, _P, _P, _P, _I, _I,
                            _I, _P, _P, _P, _I, _P, _L, _P, _D, _P]),
    "rq_quant_block_lookahead": (_I, [_P, _L, _P, _I, _I, _I, _I, _I, _P, _I, _I, _P, _P, _P, _I, _I, _I, _P,
                                      _P, _P]),
    "rq_trailing_update": (_I, [_P, _L, _P, _P, _L, _P, _I, _I, _I, _I, _I, _P, _P, _I, _I, _P, _L,
                                _P, _D, _P]),
    "rq_writeback": (_I, [_P, _I, _I, _P, _I, _P, _P, _P, _I, _P, _I, _L, _P, _P, _P, _P]),
    "rq_packed_words_per_row": (_L, [_I, _I]),
    "rq_pack_codes": (_I, [_P, _I, _I, _L, _P, _I, _P, _L, _P, _P]),
    "rq_unpack_dequant": (_I, [_P, _I, _I, _L, _I, _P, _L, _P, _P, _I, _L, _P, _P]),
    "rq_current_weight": (_I, [_P, _L, _P, _I, _I, _I, _I, _P, _P, _P, _I, _P, _P, _L, _P, _L, _P]),
    "rq_gather_cols": (_I, [_P, _L, _P, _I, _I, _P, _L, _P]),
    "rq_kfac_curvature": (_I, [_P, _I, _I, _D, _P, _P]),
    "rq_hessian_reg_gemm": (_I, [_P, _L, _P, _I, _I, _I, _I, _P, _L, _P]),
    "rq_block_gd_step": (_I, [_P, _L, _I, _I, _I, _I, _P, _L, _P, _I, _I, _D, _D, _P, _P, _P, _I, _D,
                              _P, _L, _P, _L, _I, _P, _P, _P, _I, _I, _D, _D, _D, _P, _P]),
}

_lib = None


def header_symbols():
    """Function names declared in include/gptqplus_hip.h."""
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t)\s+(rq_\w+)\s*\(", text, re.M)))


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"gptq_plus_mp_quant_amd: HIP library not built ({LIB_PATH}); run "
            "`python -m gptq_plus_mp_quant_amd.build` (hipcc, gfx950)")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def call(name, *args):
    rc = getattr(load(), name)(*args)
    if rc != RQ_OK:
        raise RuntimeError(f"{name} failed with status {rc}")
    return rc


def ptr(t):
    """Device pointer of a tensor (None -> NULL)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def dtype_code(dt):
    if dt == torch.float16:
        return RQ_F16
    if dt == torch.bfloat16:
        return RQ_BF16
    if dt == torch.float32:
        return RQ_F32
    raise TypeError(f"unsupported dtype {dt}; expected float16, bfloat16 or float32")


def require_gpu(t, what):
    if not (isinstance(t, torch.Tensor) and t.is_cuda):
        raise RuntimeError(f"{what} must be a tensor on a ROCm GPU (got "
                           f"{t.device if isinstance(t, torch.Tensor) else type(t)})")
