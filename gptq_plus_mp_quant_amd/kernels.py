"""Tensor-level wrappers of the C ABI (one function per entry point of include/gptqplus_hip.h).

Each wrapper validates shapes/dtypes on the host, passes raw device pointers and the current
HIP stream of the tensors' device, and raises ``RuntimeError`` on a non-zero status.
"""
from __future__ import annotations

import contextlib
import ctypes

import torch

from . import _native as nat

_f32 = torch.float32


def _stream(t):
    return nat.stream_of(t.device)


def _rowmajor(t, name):
    nat.require_gpu(t, name)
    if t.dim() != 2 or t.stride(1) != 1:
        raise ValueError(f"{name} must be a 2-D tensor with unit column stride")
    return t


def _cin(t, name, dtype=_f32):
    """Read-only operand: on the GPU, given dtype, dense row-major (copied if it is a view
    with other strides, e.g. the transposed result of torch.linalg.cholesky(upper=True))."""
    if t is None:
        return None
    nat.require_gpu(t, name)
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}")
    return t if t.is_contiguous() else t.contiguous()


def _cout(t, name, dtype=_f32):
    """Written operand: must already be dense row-major (the kernel writes through it)."""
    if t is None:
        return None
    nat.require_gpu(t, name)
    if t.dtype != dtype or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous {dtype} tensor")
    return t


_HWS = {}


def hessian_workspace(x, ntargets):
    """Grow-only workspace of the Hessian launches, one per (device, stream): the
    fragment-blocked copy of the chunk, the saliency copies, the pre-pass partials and the
    tail slices' partial tiles and counters (zero-filled on allocation; the kernels leave the
    counters zero).  Launches on one stream are ordered, so the calls on that stream share it;
    calls on another stream get their own."""
    need = int(nat.load().rq_hessian_workspace_bytes(x.shape[0], x.shape[1], int(ntargets),
                                                     nat.dtype_code(x.dtype)))
    if need <= 0:
        return None, 0
    dev = x.device.index if x.device.index is not None else torch.cuda.current_device()
    key = (dev, torch.cuda.current_stream(x.device).cuda_stream)
    ws = _HWS.get(key)
    if ws is None or ws.numel() < need:
        _HWS.pop(key, None)                       # the old one is released before the new one is made
        del ws
        ws = torch.zeros(need, dtype=torch.uint8, device=x.device)
        _HWS[key] = ws
    return ws, ws.numel()


def release_hessian_workspace(device=None):
    """Drop the cached Hessian workspaces (all devices, or one), e.g. when a linear is freed;
    the next launch allocates a new one of the size it needs.  Work already queued on a stream
    keeps its workspace alive through the caching allocator's stream semantics."""
    dev = None if device is None else (device.index if device.index is not None else torch.cuda.current_device())
    for key in [k for k in _HWS if dev is None or k[0] == dev]:
        del _HWS[key]


HESSIAN_MATH = {"split16": nat.RQ_HMATH_SPLIT16, "split16x3": nat.RQ_HMATH_SPLIT16X3, "fp32": nat.RQ_HMATH_FP32}


@contextlib.contextmanager
def hessian_math(mode):
    """Select the Hessian kernel inside the block: "split16x3" (default: each fp32 product
    exactly; fp16 / bf16 X from three 16-bit MFMA products, fp32 X on the fp32 MFMA kernel),
    "split16" (faster, narrower products: fp16 X from two 16-bit products, within 2^-23
    relative; bf16 X as the default; fp32 X on the fp32-X split kernel, three MFMAs per product,
    each within ~2^-20.5 relative) or "fp32" (fp32 MFMA for every input type).  The choice is
    process-wide."""
    lib = nat.load()
    prev = int(lib.rq_hessian_math(HESSIAN_MATH[mode]))
    if prev < 0:
        raise RuntimeError(f"rq_hessian_math failed with status {prev}")
    try:
        yield
    finally:
        lib.rq_hessian_math(prev)


def hessian_accum(x, sal, H, act_sq):
    """H[g] += X^T diag(sal[:, g]) X (upper tiles), act_sq += sum x^2.  x: [n, C], sal: [n, G]."""
    _rowmajor(x, "x")
    _rowmajor(sal, "sal")
    G, C, C2 = H.shape
    if C != C2 or x.shape[1] != C or sal.shape != (x.shape[0], G) or sal.dtype != _f32:
        raise ValueError("hessian_accum: shape mismatch")
    if not (H.is_contiguous() and H.dtype == _f32 and act_sq.is_contiguous() and act_sq.numel() == C):
        raise ValueError("hessian_accum: H / act_sq must be contiguous fp32")
    ws, nbytes = hessian_workspace(x, G)
    nat.call("rq_hessian_accum", nat.ptr(x), nat.dtype_code(x.dtype), x.shape[0], x.stride(0), C,
             nat.ptr(sal), sal.stride(0), G, nat.ptr(H), nat.ptr(act_sq), nat.ptr(ws), nbytes, _stream(x))


def hessian_accum_noalloc(x, sal, H, act_sq):
    """hessian_accum without a workspace: the library's per-GPU scratch array serves instead
    (rq_hessian_accum_noalloc; RuntimeError when the chunk needs more than
    RQ_NOALLOC_SCRATCH_BYTES of scratch).  Calls overlapping in time on one GPU race."""
    _rowmajor(x, "x")
    _rowmajor(sal, "sal")
    G, C, C2 = H.shape
    if C != C2 or x.shape[1] != C or sal.shape != (x.shape[0], G) or sal.dtype != _f32:
        raise ValueError("hessian_accum_noalloc: shape mismatch")
    if not (H.is_contiguous() and H.dtype == _f32 and (act_sq is None or
                                                       (act_sq.is_contiguous() and act_sq.numel() == C))):
        raise ValueError("hessian_accum_noalloc: H / act_sq must be contiguous fp32")
    nat.call("rq_hessian_accum_noalloc", nat.ptr(x), nat.dtype_code(x.dtype), x.shape[0], x.stride(0), C,
             nat.ptr(sal), sal.stride(0), G, nat.ptr(H), nat.ptr(act_sq), _stream(x))


def hessian_accum_multi(x, sals, Hs, acts):
    """One launch for several (module, group) targets sharing x [n, C]: for module m,
    Hs[m][g] += x^T diag(sals[m][:, g]) x and acts[m] += sum x^2 (acts[m] may be None)."""
    _rowmajor(x, "x")
    n, C = x.shape
    sal_p, ld, H_p, act_p = [], [], [], []
    for sal, H, act in zip(sals, Hs, acts):
        _rowmajor(sal, "sal")
        G = H.shape[0]
        if sal.shape != (n, G) or sal.dtype != _f32 or H.shape != (G, C, C) or not H.is_contiguous():
            raise ValueError("hessian_accum_multi: shape mismatch")
        for g in range(G):
            sal_p.append(sal.data_ptr() + 4 * g)
            ld.append(sal.stride(0))
            H_p.append(H[g].data_ptr())
            act_p.append(act.data_ptr() if (act is not None and g == 0) else 0)
    if len(H_p) > 32:
        raise ValueError("hessian_accum_multi: at most 32 (module, group) targets per launch")
    nt = len(H_p)
    P = ctypes.c_void_p
    ws, nbytes = hessian_workspace(x, nt)
    nat.call("rq_hessian_accum_multi", nat.ptr(x), nat.dtype_code(x.dtype), n, x.stride(0), C, nt,
             (P * nt)(*sal_p), (ctypes.c_int64 * nt)(*ld), (P * nt)(*H_p), (P * nt)(*act_p), nat.ptr(ws),
             nbytes, _stream(x))


def hessian_finalize(H, act_sq, h_div, sal_scale, seq_len, nonfinite=None, sanitize=True):
    """Mirror and scale H [G, C, C] in place; non-finite entries are counted into nonfinite
    and, with sanitize, zeroed."""
    G, C, _ = H.shape
    nat.call("rq_hessian_finalize", nat.ptr(H), nat.ptr(act_sq), G, C, float(h_div), float(sal_scale),
             float(seq_len), int(bool(sanitize)), nat.ptr(nonfinite), _stream(H))


def find_params(w, maxq, sym, group_size=-1, clip_zero=True):
    """Per-row (or per column group) min/max scale and zero: returns ([ng, R], [ng, R]).
    clip_zero: the range includes 0 (find_params); False: the groupwise fit."""
    _rowmajor(w, "w")
    R, C = w.shape
    gs = group_size if group_size > 0 else C
    ng = (C + gs - 1) // gs
    scale = torch.empty((ng, R), device=w.device, dtype=_f32)
    zero = torch.empty((ng, R), device=w.device, dtype=_f32)
    nat.call("rq_find_params", nat.ptr(w), nat.dtype_code(w.dtype), R, C, w.stride(0), gs, int(maxq),
             int(bool(sym)), int(bool(clip_zero)), nat.ptr(scale), nat.ptr(zero), _stream(w))
    return scale, zero


def find_params_mse(w, maxq, sym, norm=2.4, grid=50, maxshrink=0.5, group_size=-1, clip_zero=True):
    """find_params with the mse clip search: returns ([ng, R], [ng, R])."""
    _rowmajor(w, "w")
    R, C = w.shape
    gs = group_size if group_size > 0 else C
    ng = (C + gs - 1) // gs
    scale = torch.empty((ng, R), device=w.device, dtype=_f32)
    zero = torch.empty((ng, R), device=w.device, dtype=_f32)
    nat.call("rq_find_params_mse", nat.ptr(w), nat.dtype_code(w.dtype), R, C, w.stride(0), gs, int(maxq),
             int(bool(sym)), int(bool(clip_zero)), float(norm), int(grid), float(maxshrink), nat.ptr(scale),
             nat.ptr(zero), _stream(w))
    return scale, zero


def check_act_order_width(C):
    """act_order sorts at most RQ_ACT_ORDER_MAXC columns (rq_act_order_perm); the fasterquant
    entry points call this before any device work, so a wider linear is refused up front."""
    if C > nat.RQ_ACT_ORDER_MAXC:
        raise NotImplementedError(f"actorder=True supports at most {nat.RQ_ACT_ORDER_MAXC} input columns "
                                  f"on the HIP path (got {C})")


def act_order_perm(act_sq):
    C = act_sq.numel()
    check_act_order_width(C)
    perm = torch.empty(C, dtype=torch.int64, device=act_sq.device)
    invperm = torch.empty(C, dtype=torch.int64, device=act_sq.device)
    nat.call("rq_act_order_perm", nat.ptr(act_sq), C, nat.ptr(perm), nat.ptr(invperm), _stream(act_sq))
    return perm, invperm


def prepare_subgroup(w, grad, H_g, perm, W_sub, G_sub, H_sub):
    _rowmajor(w, "w")
    R_s, C = W_sub.shape
    nat.call("rq_prepare_subgroup", nat.ptr(w), nat.dtype_code(w.dtype), w.stride(0), nat.ptr(grad),
             grad.stride(0) if grad is not None else 0, nat.ptr(H_g), R_s, C, nat.ptr(perm),
             nat.ptr(W_sub), W_sub.stride(0), nat.ptr(G_sub), G_sub.stride(0) if G_sub is not None else 0,
             nat.ptr(H_sub), _stream(w))


def chol_workspace(C, device, nb=1):
    return torch.empty(nb * int(nat.load().rq_chol_workspace_bytes(C)), dtype=torch.uint8, device=device)


def chol_hinv_attempt(H_work, damp_percent, workspace, Hinv, Hinv_init=None, info=None, Hinv_diag=None):
    """One damping attempt for H_work [C, C] or a batch [nb, C, C]; damp_percent is a float or a
    list (entries <= 0 skip that matrix).  Optional outputs: Hinv_init (H^-1) and Hinv_diag
    (diag(H^-1), [C] or [nb, C]).  Returns the device info tensor [nb]."""
    batched = H_work.dim() == 3
    nb = H_work.shape[0] if batched else 1
    C = H_work.shape[-1]
    _cout(H_work, "H_work"), _cout(Hinv, "Hinv"), _cout(Hinv_init, "Hinv_init"), _cout(Hinv_diag, "Hinv_diag")
    if Hinv.numel() != nb * C * C or (Hinv_init is not None and Hinv_init.numel() != nb * C * C) or \
            (Hinv_diag is not None and Hinv_diag.numel() != nb * C):
        raise ValueError("chol_hinv_attempt: output shape mismatch")
    if workspace.numel() < nb * int(nat.load().rq_chol_workspace_bytes(C)):
        raise ValueError("chol_hinv_attempt: workspace too small")
    damps = list(damp_percent) if isinstance(damp_percent, (list, tuple)) else [float(damp_percent)] * nb
    if len(damps) != nb:
        raise ValueError("chol_hinv_attempt: one damp_percent per matrix")
    if info is None:
        info = torch.zeros(nb, dtype=torch.int32, device=H_work.device)
    arr = (ctypes.c_double * nb)(*[float(d) for d in damps])
    nat.call("rq_chol_hinv_attempt", nat.ptr(H_work), C, nb, arr, nat.ptr(workspace), nat.ptr(Hinv),
             nat.ptr(Hinv_init), nat.ptr(Hinv_diag), nat.ptr(info), _stream(H_work))
    return info


def gptqplus_terms(G, hinv_diag, Hinv, alpha_eff, reference_loss, beta_mode, beta, Z, GHinv,
                   GH0, z_nonzero, HinvT=None):
    """beta, Z = (G Hinv^T) beta and GHinv = Z Hinv for nsub = Hinv.shape[0] subgroups of
    R_s = G.shape[0] / nsub rows: Hinv [nsub, C, C], hinv_diag = diag(H^-1) [nsub, C]
    (beta_mode 1), GH0 [R, C] and HinvT [nsub, C, C] workspaces (beta_mode 1), z_nonzero [nsub]."""
    R, C = G.shape
    Hinv = Hinv.reshape(-1, C, C)
    nsub = Hinv.shape[0]
    if R % nsub:
        raise ValueError("gptqplus_terms: rows must split evenly over the subgroups")
    R_s = R // nsub
    G = _cin(G, "G")
    hinv_diag = _cin(hinv_diag, "hinv_diag")
    Hinv = _cin(Hinv, "Hinv")
    if hinv_diag is not None and hinv_diag.numel() != nsub * C:
        raise ValueError("gptqplus_terms: hinv_diag must hold C values per subgroup")
    if GH0 is not None and GH0.numel() != R * C:
        raise ValueError("gptqplus_terms: GH0 must be [R, C]")
    if HinvT is not None and HinvT.numel() != nsub * C * C:
        raise ValueError("gptqplus_terms: HinvT must be [nsub, C, C]")
    if z_nonzero.numel() != nsub:
        raise ValueError("gptqplus_terms: one z_nonzero flag per subgroup")
    for t, n in ((beta, "beta"), (Z, "Z"), (GHinv, "GHinv"), (GH0, "GH0"), (HinvT, "HinvT")):
        _cout(t, n)
    _cout(z_nonzero, "z_nonzero", torch.int32)
    nat.call("rq_gptqplus_terms", nat.ptr(G), G.stride(0), nat.ptr(hinv_diag), nat.ptr(Hinv), nat.ptr(HinvT),
             R_s, nsub, C, float(alpha_eff), float(reference_loss), int(beta_mode), nat.ptr(beta), nat.ptr(Z),
             nat.ptr(GHinv), Z.stride(0), nat.ptr(GH0), nat.ptr(z_nonzero), _stream(G))


def _surrogate(gmode, anchor, beta, R, C):
    if gmode not in (nat.RQ_GMODE_SURROGATE_BLOCK, nat.RQ_GMODE_SURROGATE_ONLINE):
        return 0
    if anchor is None or beta is None:
        raise ValueError("surrogate g_update modes need anchor and beta")
    if anchor.shape != (R, C) or anchor.stride(1) != 1 or beta.numel() != R or not beta.is_contiguous():
        raise ValueError("anchor must be row-major [R, C] and beta a contiguous [R] vector")
    if anchor.dtype != torch.float32 or beta.dtype != torch.float32:
        raise ValueError("anchor and beta must be float32")
    return anchor.stride(0)


def quant_block(Wp, Hinv_all, GH, Z, R_s, i1, count, qmode, scale, col_group, dyn_scale, maxq, sym,
                atomic, z_nonzero, codes, err, gmode=nat.RQ_GMODE_FROZEN, anchor=None, beta=None,
                second_order_scale=1.0):
    R, C = Wp.shape
    if Hinv_all.shape != (R // R_s, C, C):
        raise ValueError("quant_block: Hinv_all must be [G, C, C]")
    lda = _surrogate(gmode, anchor, beta, R, C)
    _cout(Wp, "Wp")
    for t, n in ((Hinv_all, "Hinv_all"), (GH, "GH"), (Z, "Z")):
        nat.require_gpu(t, n)
        if t.dtype != _f32:
            raise ValueError(f"{n} must be {_f32}")
    if not (Hinv_all.is_contiguous() and GH.stride(1) == 1 and Z.stride(1) == 1):
        raise ValueError("quant_block: Hinv_all must be contiguous, GH / Z row-major")
    nat.call("rq_quant_block", nat.ptr(Wp), Wp.stride(0), nat.ptr(Hinv_all), C, nat.ptr(GH), nat.ptr(Z),
             GH.stride(0), R, R_s, int(i1), int(count), int(qmode), nat.ptr(scale), nat.ptr(col_group),
             nat.ptr(dyn_scale), int(maxq), int(bool(sym)), int(bool(atomic)), nat.ptr(z_nonzero),
             nat.ptr(codes), nat.ptr(err), int(gmode), nat.ptr(anchor), lda, nat.ptr(beta),
             float(second_order_scale), _stream(Wp))


def quant_block_lookahead(Wp, Hinv_all, R_s, i1, count, err, count_next, qmode, scale, col_group, dyn_scale,
                          maxq, sym, atomic, codes, err_next):
    """Block k's trailing update (W-only: frozen mode, Z identically zero) and block k+1's
    quantisation in one launch; equal bit for bit to trailing_update(k) then quant_block(k+1)."""
    R, C = Wp.shape
    if Hinv_all.shape != (R // R_s, C, C) or not Hinv_all.is_contiguous():
        raise ValueError("quant_block_lookahead: Hinv_all must be contiguous [G, C, C]")
    _cout(Wp, "Wp"), _cout(err_next, "err_next")
    err = _cin(err, "err")
    if err.data_ptr() == err_next.data_ptr():
        raise ValueError("quant_block_lookahead: err and err_next must be different buffers")
    nat.call("rq_quant_block_lookahead", nat.ptr(Wp), Wp.stride(0), nat.ptr(Hinv_all), C, R, R_s, int(i1),
             int(count), nat.ptr(err), int(count_next), int(qmode), nat.ptr(scale), nat.ptr(col_group),
             nat.ptr(dyn_scale), int(maxq), int(bool(sym)), int(bool(atomic)), nat.ptr(codes),
             nat.ptr(err_next), _stream(Wp))


def trailing_update(Wp, GH, Z, Hinv_all, R_s, i1, count, err, z_nonzero, gmode=nat.RQ_GMODE_FROZEN,
                    anchor=None, beta=None, second_order_scale=1.0, z_zero=False):
    """z_zero=True states that Z (and GH) are identically zero, i.e. that z_nonzero holds 0; the
    frozen and block_gd modes then run the W-only kernel."""
    R, C = Wp.shape
    lda = _surrogate(gmode, anchor, beta, R, C)
    _cout(Wp, "Wp"), _cout(GH, "GH"), _cout(err, "err")
    if not (Hinv_all.is_contiguous() and Z.stride(1) == 1):
        raise ValueError("trailing_update: Hinv_all must be contiguous, Z row-major")
    nat.call("rq_trailing_update", nat.ptr(Wp), Wp.stride(0), nat.ptr(GH), nat.ptr(Z), GH.stride(0),
             nat.ptr(Hinv_all), C, R, R_s, int(i1), int(count), nat.ptr(err), nat.ptr(z_nonzero),
             int(bool(z_zero)), int(gmode), nat.ptr(anchor), lda, nat.ptr(beta), float(second_order_scale),
             _stream(Wp))


def writeback(codes, invperm, qmode, scale, col_group, dyn_scale, blocksize, q_out, w_int_out=None,
              scale_out=None, nan_flag=None):
    R, C = codes.shape
    nat.call("rq_writeback", nat.ptr(codes), R, C, nat.ptr(invperm), int(qmode), nat.ptr(scale),
             nat.ptr(col_group), nat.ptr(dyn_scale), int(blocksize), nat.ptr(q_out),
             nat.dtype_code(q_out.dtype), q_out.stride(0), nat.ptr(w_int_out), nat.ptr(scale_out),
             nat.ptr(nan_flag), _stream(codes))


def packed_words(C, nbits):
    n = nat.load().rq_packed_words_per_row(int(C), int(nbits))
    if n < 0:
        raise ValueError(f"packed_words: bad C={C} / nbits={nbits}")
    return int(n)


def pack_codes(codes, nbits, invperm=None, out=None, range_flag=None):
    """int16 codes [R, C] (permuted order when invperm is given) -> [R, ceil(C*nbits/32)] words
    (uint32 bit patterns held in an int32 tensor)."""
    nat.require_gpu(codes, "codes")
    if codes.dtype != torch.int16 or codes.dim() != 2 or codes.stride(1) != 1:
        raise ValueError("pack_codes: codes must be row-major int16 [R, C]")
    R, C = codes.shape
    words = packed_words(C, nbits)
    if out is None:
        out = torch.empty((R, words), dtype=torch.int32, device=codes.device)
    if out.dtype != torch.int32 or out.shape != (R, words) or out.stride(1) != 1:
        raise ValueError("pack_codes: out must be row-major int32 [R, words]")
    if invperm is not None:
        invperm = _cin(invperm, "invperm", torch.int64)
        if invperm.numel() != C:
            raise ValueError("pack_codes: invperm must be int64 [C]")
    nat.call("rq_pack_codes", nat.ptr(codes), R, C, codes.stride(0), nat.ptr(invperm), int(nbits),
             nat.ptr(out), out.stride(0), nat.ptr(range_flag), _stream(codes))
    return out


def unpack_dequant(packed, C, nbits, scales=None, g_idx=None, q_dtype=torch.float16, want_codes=False):
    """Inverse of pack_codes: returns (Q [R, C] in q_dtype or None, codes int16 [R, C] or None)."""
    nat.require_gpu(packed, "packed")
    R = packed.shape[0]
    if packed.dtype != torch.int32 or packed.stride(1) != 1 or packed.shape[1] < packed_words(C, nbits):
        raise ValueError("unpack_dequant: packed must be row-major int32 [R, >= words]")
    q = codes = None
    if scales is not None:
        scales = _cin(scales, "scales")
        if scales.dtype != torch.float32 or scales.dim() != 2 or scales.shape[1] != R:
            raise ValueError("unpack_dequant: scales must be float32 [ngroups, R]")
        if g_idx is not None:
            g_idx = _cin(g_idx, "g_idx", torch.int32)
            if g_idx.numel() != C:
                raise ValueError("unpack_dequant: g_idx must be int32 [C]")
            if int(g_idx.min()) < 0 or int(g_idx.max()) >= scales.shape[0]:
                raise ValueError("unpack_dequant: g_idx out of range of the scale table")
        elif scales.shape[0] != 1:
            raise ValueError("unpack_dequant: several scale groups need g_idx")
        q = torch.empty((R, C), dtype=q_dtype, device=packed.device)
    if want_codes:
        codes = torch.empty((R, C), dtype=torch.int16, device=packed.device)
    if q is None and codes is None:
        raise ValueError("unpack_dequant: nothing to produce")
    nat.call("rq_unpack_dequant", nat.ptr(packed), R, C, packed.stride(0), int(nbits), nat.ptr(scales),
             R, nat.ptr(g_idx), nat.ptr(q), nat.dtype_code(q_dtype) if q is not None else 0,
             C, nat.ptr(codes), _stream(packed))
    return q, codes


# --- refresh g_update modes (block_gd / block_backward) ---------------------------------
OPTIMIZERS = {"sgd": 0, "adam": 1, "h_adam": 2}
REGULARIZERS = {"none": 0, "l2": 1, "hessian": 2, "quant_error_gate": 3, "quant_error_gate_optimized": 4}


def current_weight(Wp, codes, i_q, qmode, scale, col_group, dyn_scale, blocksize, invperm=None,
                   sub_ref=None, out=None):
    """Quantized columns (permuted j < i_q) as fl32(scale * code), the rest from Wp; natural
    column order when invperm is given; minus sub_ref when given."""
    R, C = Wp.shape
    _rowmajor(Wp, "Wp")
    if codes.shape != (R, C) or codes.dtype != torch.int16 or not codes.is_contiguous():
        raise ValueError("current_weight: codes must be contiguous int16 [R, C]")
    if invperm is not None:
        invperm = _cin(invperm, "invperm", torch.int64)
    if sub_ref is not None:
        _rowmajor(sub_ref, "sub_ref")
    if out is None:
        out = torch.empty((R, C), dtype=torch.float32, device=Wp.device)
    _cout(out, "out")
    nat.call("rq_current_weight", nat.ptr(Wp), Wp.stride(0), nat.ptr(codes), R, C, int(i_q), int(qmode),
             nat.ptr(scale), nat.ptr(col_group), nat.ptr(dyn_scale), int(blocksize), nat.ptr(invperm),
             nat.ptr(sub_ref), sub_ref.stride(0) if sub_ref is not None else 0, nat.ptr(out),
             out.stride(0), _stream(Wp))
    return out


def gather_cols(src, perm, out=None):
    R, C = src.shape
    src = _cin(src, "src")
    if perm is not None:
        perm = _cin(perm, "perm", torch.int64)
    if out is None:
        out = torch.empty((R, C), dtype=torch.float32, device=src.device)
    _cout(out, "out")
    nat.call("rq_gather_cols", nat.ptr(src), src.stride(0), nat.ptr(perm), R, C, nat.ptr(out),
             out.stride(0), _stream(src))
    return out


def kfac_curvature(H_work, damping):
    G, C, _ = H_work.shape
    H_work = _cin(H_work, "H_work")
    curv = torch.empty((G, C), dtype=torch.float32, device=H_work.device)
    nat.call("rq_kfac_curvature", nat.ptr(H_work), C, G, float(damping), nat.ptr(curv), _stream(H_work))
    return curv


def hessian_reg_gemm(diff, H_reg, R_s, i2):
    R, C = diff.shape
    diff = _cin(diff, "diff")
    H_reg = _cin(H_reg, "H_reg")
    if H_reg.shape != (R // R_s, C, C):
        raise ValueError("hessian_reg_gemm: H_reg must be [G, C, C]")
    out = torch.empty((R, C - i2), dtype=torch.float32, device=diff.device)
    nat.call("rq_hessian_reg_gemm", nat.ptr(diff), diff.stride(0), nat.ptr(H_reg), C, R, R_s, int(i2),
             nat.ptr(out), out.stride(0), _stream(diff))
    return out


def block_gd_step(Wp, R_s, i2, grad, perm, optimizer, step, lr, grad_clip, exp_avg=None,
                  exp_avg_sq=None, curvature=None, reg="none", reg_lambda=0.0, w_fp=None, hreg=None,
                  gate_qmode=0, gate_scale=None, gate_zero=None, col_group=None, maxq=0, sym=True,
                  gate_floor=0.1, gate_sharpness=1.0, sine_amp=0.0, stats_parts=None):
    """One block_gd step on the trailing columns [i2, C); stats_parts (optional, contiguous
    float32 [4, R, C - i2]) receives the optimizer step, the applied update, the regularizer
    part and the sine part."""
    R, C = Wp.shape
    _cout(Wp, "Wp")
    grad = _cin(grad, "grad")
    if grad.shape != (R, C):
        raise ValueError("block_gd_step: grad must be [R, C]")
    if perm is not None:
        perm = _cin(perm, "perm", torch.int64)
    for t, n in ((exp_avg, "exp_avg"), (exp_avg_sq, "exp_avg_sq"), (w_fp, "w_fp")):
        if t is not None and (t.shape != (R, C) or not t.is_contiguous() or t.dtype != torch.float32):
            raise ValueError(f"block_gd_step: {n} must be contiguous float32 [R, C]")
    if curvature is not None and (curvature.shape != (R // R_s, C) or not curvature.is_contiguous()):
        raise ValueError("block_gd_step: curvature must be contiguous [G, C]")
    if hreg is not None and (hreg.shape != (R, C - i2) or hreg.stride(1) != 1):
        raise ValueError("block_gd_step: hreg must be row-major [R, C - i2]")
    if stats_parts is not None and stats_parts.shape != (4, R, C - i2):
        raise ValueError("block_gd_step: stats_parts must be [4, R, C - i2]")
    _cout(stats_parts, "stats_parts")
    nat.call("rq_block_gd_step", nat.ptr(Wp), Wp.stride(0), R, R_s, C, int(i2), nat.ptr(grad),
             grad.stride(0), nat.ptr(perm), OPTIMIZERS[optimizer], int(step), float(lr),
             float(grad_clip if grad_clip is not None else 0.0), nat.ptr(exp_avg), nat.ptr(exp_avg_sq),
             nat.ptr(curvature), REGULARIZERS[reg], float(reg_lambda), nat.ptr(w_fp),
             w_fp.stride(0) if w_fp is not None else 0, nat.ptr(hreg),
             hreg.stride(0) if hreg is not None else 0, int(gate_qmode), nat.ptr(gate_scale),
             nat.ptr(gate_zero), nat.ptr(col_group), int(maxq), int(bool(sym)), float(gate_floor),
             float(gate_sharpness), float(sine_amp), nat.ptr(stats_parts), _stream(Wp))
