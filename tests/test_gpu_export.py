"""Packed export on the GPU: rq_pack_codes / rq_unpack_dequant against the format's CPU
definition (oracle/packing.py), and export_packed -> dequantize_packed reproducing the layer
weight fasterquant wrote, bit for bit."""
import numpy as np
import pytest
import torch

from gptq_plus_mp_quant_amd import (GPTQPlus, WeightQuantizer, dequantize_packed, export_packed,
                                    load_packed, save_packed)
from gptq_plus_mp_quant_amd import kernels as K
from gptq_plus_mp_quant_amd.export import unpack_codes
from oracle.packing import pack_rows
from tests._util import rng, synth

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@pytest.mark.parametrize("nbits", [2, 3, 4, 5, 8])
@pytest.mark.parametrize("C", [1, 33, 1000])
@pytest.mark.parametrize("permuted", [False, True])
def test_pack_codes_matches_format(nbits, C, permuted):
    r = rng(nbits * 7 + C)
    half = 1 << (nbits - 1)
    codes = r.integers(-half, half, size=(37, C)).astype(np.int16)
    want = pack_rows(codes, nbits)
    src = torch.from_numpy(codes)
    invperm = None
    if permuted:
        perm = torch.from_numpy(r.permutation(C))
        src = src[:, perm].contiguous()                   # codes in permuted column order
        invperm = torch.argsort(perm).to(DEV)
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    got = K.pack_codes(src.to(DEV), nbits, invperm=invperm, range_flag=flag)
    torch.cuda.synchronize()
    assert int(flag.item()) == 0
    assert np.array_equal(got.cpu().numpy().view(np.uint32), want)
    _, back = K.unpack_dequant(got, C, nbits, want_codes=True)
    assert np.array_equal(back.cpu().numpy(), codes)


def test_out_of_range_code_is_flagged():
    codes = torch.tensor([[0, 7, 8, -9, -32768]], dtype=torch.int16, device=DEV)
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    K.pack_codes(codes, 4, range_flag=flag)
    assert int(flag.item()) == 1


CASES = [
    dict(name="channel_sym", bits=4, sym=True, gs=-1, act=True, static=False),
    dict(name="channel_asym", bits=4, sym=False, gs=-1, act=True, static=False),
    dict(name="static_sym3", bits=3, sym=True, gs=64, act=True, static=True),
    dict(name="dynamic_asym", bits=4, sym=False, gs=64, act=False, static=False),
    dict(name="dynamic_act_sym", bits=4, sym=True, gs=64, act=True, static=False),
]


def _quantized(case, mse=False):
    R, C, G = 96, 320, 2
    X, W, s, grad = synth(5 + case["bits"], R, C, G, 4, 64)
    layer = torch.nn.Linear(C, R, bias=False).to(DEV, torch.float16)
    layer.weight.data.copy_(W.to(DEV))
    g = GPTQPlus(layer, saliency=s, gradient=grad, num_groups=G, alpha=0.0, reference_loss=0.0)
    g.quantizer = WeightQuantizer()
    g.quantizer.configure(case["bits"], perchannel=True, sym=case["sym"], mse=mse)
    for j in range(0, 4, 2):
        g.add_batch(X[j:j + 2].to(DEV), None)
    g.finalize_hessian()
    g.fasterquant(blocksize=64, percdamp=0.01, groupsize=case["gs"], actorder=case["act"],
                  static_groups=case["static"], export_to_et=True)
    return g, layer


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_export_reproduces_layer_weight(case, tmp_path):
    g, layer = _quantized(case)
    e = g.export_packed()
    nb = case["bits"] + (0 if case["sym"] else 1)
    assert e["nbits"] == nb and e["qweight"].shape == (96, (320 * nb + 31) // 32)
    q = dequantize_packed(e)
    torch.cuda.synchronize()
    assert q.dtype == layer.weight.dtype
    assert torch.equal(q.cpu(), layer.weight.data.cpu())                 # bit for bit
    codes = unpack_codes(e)
    assert torch.equal(codes.cpu(), g.codes.cpu())
    assert torch.equal(codes.float().cpu(), layer.int_weight.cpu())      # export_to_et codes
    per_elem = e["scales"][e["g_idx"].long(), :].T                       # [R, C]
    assert torch.equal(per_elem.cpu(), layer.scale.cpu())                # export_to_et scales
    # file round trip with the quantizers dict, loaded without executing anything
    path = str(tmp_path / "packed.safetensors")
    save_packed(path, {"model.layers.0.self_attn.q_proj": e},
                quantizers={"model.layers.0.self_attn.q_proj": g.quantizer})
    entries, quants = load_packed(path, device=DEV)
    e2 = entries["model.layers.0.self_attn.q_proj"]
    assert torch.equal(dequantize_packed(e2).cpu(), layer.weight.data.cpu())
    qs = quants["model.layers.0.self_attn.q_proj"]
    assert torch.equal(qs["scale"].cpu(), g.quantizer.scale.float().cpu())
    assert int(qs["maxq"]) == int(g.quantizer.maxq)


def test_export_after_free_fails_loudly():
    g, _ = _quantized(CASES[0])
    g.free()
    with pytest.raises(RuntimeError):
        export_packed(g)
