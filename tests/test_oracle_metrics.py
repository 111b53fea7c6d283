"""Pin the oracle's refresh_full_metrics statistics (gptq_plus_utils.py:1448-1496, 1626-1817)
by relations its own formulas do not state: with sgd, no regularizer and no clipping the
optimizer step is lr * g, so its statistics are lr times those of the trailing gradient, the
applied update equals the step and the regularizer parts vanish; the trailing gradient is the
refreshed gradient (captured from the refresh function) in act_order, columns [i2, C)."""
import numpy as np
import pytest
import torch

from oracle.gptqplus_cpu import GPTQPlusOracle, make_quantizer
from tests.golden.fixtures import quadratic_refresh


def _setup(seed, R=16, C=64, G=2):
    r = np.random.Generator(np.random.PCG64(seed))
    X = torch.from_numpy(r.standard_normal((4, 32, C)).astype(np.float32))
    W = torch.from_numpy(r.standard_normal((R, C)).astype(np.float32) * 0.05)
    s = torch.from_numpy(r.lognormal(size=(4, 32, G)).astype(np.float32))
    g0 = torch.from_numpy(r.standard_normal((R, C)).astype(np.float32) * 0.1)
    o = GPTQPlusOracle(W, s, g0, G, 0.05, 100.0)
    o.quantizer = make_quantizer(4, True)
    o.add_batch(X)
    o.finalize_hessian()
    base = quadratic_refresh(X, W, g0)
    captured = []

    def fn(w, slide_alpha=None):
        g, meta = base(w, slide_alpha=slide_alpha)
        captured.append(g.clone())
        return g, meta
    return o, fn, captured


def _rel(a, b):
    return abs(a - b) / max(abs(b), 1e-30)


def test_block_gd_sgd_statistics():
    o, fn, captured = _setup(1)
    recs = []
    lr = 1e-3
    o.fasterquant(blocksize=16, actorder=True, static_groups=True, g_update_mode="block_gd",
                  gradient_refresh_fn=fn, grad_lr=lr, grad_optimizer="sgd", grad_clip=0.0,
                  block_observer=recs.append, refresh_full_metrics=True)
    perm = torch.argsort(o.act_square, descending=True)
    assert len(recs) == len(captured) == 64 // 16 - 1
    for rec, g in zip(recs, captured):
        i2 = rec["col_end"]
        gt = g[:, perm][:, i2:].double()
        assert rec["remaining_columns"] == 64 - i2
        assert _rel(rec["remaining_grad_abs_mean"], float(gt.abs().mean())) <= 1e-6
        assert _rel(rec["remaining_grad_mean_row_l2"], float(gt.norm(dim=1).mean())) <= 1e-6
        assert rec["remaining_grad_clipped_abs_mean"] == rec["remaining_grad_abs_mean"]
        assert _rel(rec["first_order_raw_abs_mean"], lr * rec["remaining_grad_abs_mean"]) <= 1e-6
        assert _rel(rec["first_order_raw_mean_row_l2"], lr * rec["remaining_grad_mean_row_l2"]) <= 1e-6
        assert rec["first_order_update_abs_mean"] == rec["first_order_raw_abs_mean"]
        assert _rel(rec["first_order_update_abs_max"], lr * float(gt.abs().max())) <= 1e-6
        q = float(torch.quantile(gt.abs().flatten(), 0.99))
        assert _rel(rec["first_order_update_abs_q99"], lr * q) <= 1e-5
        assert rec["regularizer_update_abs_mean"] == 0.0 and rec["sine_regularizer_update_abs_mean"] == 0.0
        assert rec["second_order_update_abs_mean"] > 0 and rec["second_order_update_abs_max"] >= \
            rec["second_order_update_abs_q99"] >= 0
        assert rec["mean_refresh_loss"] is not None and rec["slide_alpha"] is not None


def test_block_gd_clip_and_off_switch():
    o, fn, _ = _setup(2)
    recs = []
    o.fasterquant(blocksize=16, actorder=False, g_update_mode="block_gd", gradient_refresh_fn=fn,
                  grad_lr=1e-3, grad_optimizer="adam", grad_clip=0.01, block_observer=recs.append,
                  refresh_full_metrics=True)
    for rec in recs:
        assert rec["remaining_grad_clipped_abs_mean"] <= min(0.01, rec["remaining_grad_abs_mean"])
    o2, fn2, _ = _setup(2)
    recs2 = []
    o2.fasterquant(blocksize=16, actorder=False, g_update_mode="block_gd", gradient_refresh_fn=fn2,
                   grad_lr=1e-3, grad_optimizer="adam", grad_clip=0.01, block_observer=recs2.append)
    assert len(recs2) == len(recs)
    for rec in recs2:        # flag off: every statistic None, the refresh loss still reported
        assert all(v is None for k, v in rec.items() if k.endswith(("_mean", "_l2", "_max", "_q99"))
                   and "refresh_loss" not in k)
        assert rec["mean_refresh_loss"] is not None


def test_block_backward_statistics():
    o, fn, captured = _setup(3)
    recs = []
    o.fasterquant(blocksize=16, actorder=True, static_groups=True, g_update_mode="block_backward",
                  gradient_refresh_fn=fn, grad_clip=0.05, block_observer=recs.append,
                  refresh_full_metrics=True)
    perm = torch.argsort(o.act_square, descending=True)
    assert len(recs) == len(captured) == 64 // 16
    for rec, g in zip(recs, captured):
        i2 = rec["col_end"]
        if i2 == 64:
            assert rec["remaining_grad_abs_mean"] is None
            continue
        gt = g[:, perm][:, i2:].double()
        assert _rel(rec["remaining_grad_abs_mean"], float(gt.abs().mean())) <= 1e-6
        assert _rel(rec["remaining_grad_clipped_abs_mean"], float(gt.clamp(-0.05, 0.05).abs().mean())) <= 1e-6
        assert rec["first_order_raw_abs_mean"] is None and rec["second_order_update_abs_mean"] is None
