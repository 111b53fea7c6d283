"""CPU-only checks of the native boundary: the library loads and exports every symbol the
header declares; the ctypes bindings cover them; host-side validation rejects bad calls
before any device work; the drop-in classes refuse non-GPU tensors loudly."""
import ctypes

import pytest
import torch

from gptq_plus_mp_quant_amd import _native as nat


def _lib():
    if not nat.LIB_PATH.exists():
        pytest.skip("library not built")
    return nat.load()


def test_header_symbols_are_exported_and_bound():
    lib = _lib()
    syms = nat.header_symbols()
    assert len(syms) >= 22
    for name in syms:
        assert hasattr(lib, name), f"{name} not exported"
        assert name in nat.SIGNATURES, f"{name} has no ctypes binding"
    assert set(nat.SIGNATURES) == set(syms)


def test_version_and_workspace_query():
    lib = _lib()
    assert lib.rq_version() == 100
    assert lib.rq_chol_workspace_bytes(64) == (2 * 64 * 64 + 64 * 64) * 8
    assert lib.rq_chol_workspace_bytes(0) < 0


def test_argument_validation_needs_no_device():
    lib = _lib()
    null = ctypes.c_void_p(0)
    assert lib.rq_hessian_accum(null, 0, 10, 8, 8, null, 1, 1, null, null, null, 0, null) == nat.RQ_EINVAL
    assert lib.rq_hessian_workspace_bytes(10, 0, 1, nat.RQ_F16) < 0
    assert lib.rq_find_params(null, 0, 4, 4, 4, -1, 7, 1, 1, null, null, null) == nat.RQ_EINVAL
    assert lib.rq_act_order_perm(null, 4, null, null, null) == nat.RQ_EINVAL
    damp = (ctypes.c_double * 1)(0.01)
    assert lib.rq_chol_hinv_attempt(null, 4, 1, damp, null, null, null, null, null, null) == nat.RQ_EINVAL
    assert lib.rq_chol_hinv_attempt(null, 4, 65, damp, null, null, null, null, null, null) == nat.RQ_EINVAL
    assert lib.rq_quant_block(null, 4, null, 4, null, null, 4, 4, 4, 0, 4, 0, null, null, null, 7, 1,
                              0, null, null, null, 0, null, 4, null, 1.0, null) == nat.RQ_EINVAL
    assert lib.rq_trailing_update(null, 4, null, null, 4, null, 4, 4, 4, 0, 4, null, null, 0, 0, null, 4,
                                  null, 1.0, null) == nat.RQ_EINVAL
    # a surrogate g_update mode without its anchor / beta is refused before any launch
    fake = ctypes.c_void_p(16)
    assert lib.rq_quant_block(fake, 4, fake, 4, fake, fake, 4, 4, 4, 0, 4, 0, fake, null, null, 7, 1,
                              0, fake, fake, fake, 1, null, 4, null, 1.0, null) == nat.RQ_EINVAL
    assert lib.rq_trailing_update(fake, 4, fake, fake, 4, fake, 4, 4, 4, 0, 2, fake, fake, 0, 2, fake, 4,
                                  null, 1.0, null) == nat.RQ_EINVAL
    assert lib.rq_trailing_update(fake, 4, fake, fake, 4, fake, 4, 4, 4, 0, 2, fake, fake, 0, 4, fake, 4,
                                  fake, 1.0, null) == nat.RQ_EINVAL
    # refresh-mode entry points: missing optimizer state / regularizer inputs are refused
    D = ctypes.c_double
    assert lib.rq_block_gd_step(fake, 8, 4, 4, 8, 4, fake, 8, null, 1, 1, D(1e-3), D(1.0), null, null,
                                null, 0, D(0.0), null, 0, null, 0, 0, null, null, null, 7, 1, D(0.1),
                                D(1.0), D(0.0), null, null) == nat.RQ_EINVAL
    assert lib.rq_block_gd_step(fake, 8, 4, 4, 8, 4, fake, 8, null, 0, 0, D(1e-3), D(1.0), null, null,
                                null, 2, D(0.1), null, 0, null, 0, 0, null, null, null, 7, 1, D(0.1),
                                D(1.0), D(0.0), null, null) == nat.RQ_EINVAL
    assert lib.rq_current_weight(fake, 8, fake, 4, 8, 4, 1, fake, null, null, 8, null, null, 0, fake, 8,
                                 null) == nat.RQ_EINVAL
    assert lib.rq_hessian_reg_gemm(fake, 8, fake, 8, 4, 3, 0, fake, 8, null) == nat.RQ_EINVAL
    assert lib.rq_writeback(null, 4, 4, null, 0, null, null, null, 4, null, 0, 4, null, null, null,
                            null) == nat.RQ_EINVAL
    # packed export: word count, and refusal of bad widths / short rows before any launch
    assert lib.rq_packed_words_per_row(33, 3) == 4 and lib.rq_packed_words_per_row(32, 4) == 4
    assert lib.rq_packed_words_per_row(8, 1) < 0
    fake = ctypes.c_void_p(16)
    assert lib.rq_pack_codes(fake, 2, 8, 8, null, 1, fake, 4, null, null) == nat.RQ_EINVAL
    assert lib.rq_pack_codes(fake, 2, 33, 33, null, 3, fake, 3, null, null) == nat.RQ_EINVAL
    assert lib.rq_unpack_dequant(fake, 2, 33, 4, 3, null, 2, null, null, 0, 33, null, null) == nat.RQ_EINVAL
    assert lib.rq_unpack_dequant(fake, 2, 33, 4, 3, null, 2, null, fake, 0, 33, null, null) == nat.RQ_EINVAL


def test_dropin_rejects_cpu_tensors():
    _lib()
    from gptq_plus_mp_quant_amd import GPTQPlus, WeightQuantizer
    layer = torch.nn.Linear(8, 4, bias=False)
    with pytest.raises(RuntimeError, match="GPU"):
        GPTQPlus(layer, torch.ones(1, 2, 1), torch.zeros(4, 8), 1, 0.0, 0.0)
    q = WeightQuantizer()
    q.configure(4, perchannel=True, sym=True)
    with pytest.raises(RuntimeError, match="GPU"):
        q.find_params(torch.ones(4, 8))
    q.configure(4, perchannel=True, sym=True, mse=True)
    with pytest.raises(RuntimeError, match="GPU"):
        q.find_params(torch.ones(4, 8))
    q.configure(4, perchannel=True, sym=True, weight_groupsize=4)
    with pytest.raises(RuntimeError, match="GPU"):
        q.find_params(torch.ones(4, 8))


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(nat, "LIB_PATH", tmp_path / "absent.so")
    monkeypatch.setattr(nat, "_lib", None)
    with pytest.raises(RuntimeError, match="not built"):
        nat.load()


def test_act_order_width_refused_before_device_work():
    """rq_act_order_perm sorts at most RQ_ACT_ORDER_MAXC columns; both fasterquant entry points
    refuse a wider act_order linear with NotImplementedError before any device work (the
    objects here carry CPU tensors only, so any launch would fail differently)."""
    lib = _lib()
    from gptq_plus_mp_quant_amd import GPTQ, GPTQPlus, WeightQuantizer
    from gptq_plus_mp_quant_amd import kernels as K
    fake = ctypes.c_void_p(16)
    assert lib.rq_act_order_perm(fake, nat.RQ_ACT_ORDER_MAXC + 1, fake, fake, None) == nat.RQ_EINVAL
    K.check_act_order_width(nat.RQ_ACT_ORDER_MAXC)
    with pytest.raises(NotImplementedError, match="at most 65536"):
        K.check_act_order_width(nat.RQ_ACT_ORDER_MAXC + 1)
    q = WeightQuantizer()
    q.configure(4, perchannel=True, sym=False)
    for cls in (GPTQPlus, GPTQ):
        g = object.__new__(cls)
        g.rows, g.columns, g.quantizer, g.profile_recorder, g._finalized = 4, nat.RQ_ACT_ORDER_MAXC + 1, q, None, True
        g.layer = torch.nn.Linear(4, 4, bias=False)
        with pytest.raises(NotImplementedError, match="at most 65536"):
            g.fasterquant(blocksize=128, actorder=True)
