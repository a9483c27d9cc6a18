"""Golden vectors (tests/golden/golden.npz, written by make_golden.py).

CPU: the oracle and the product quantizer still reproduce every vector, and
the seeded layer inputs regenerate to the stored SHA-256.
GPU: the HIP path reproduces them through the C ABI -- packing, routing and
permutation bit for bit, the layer output within max-abs 1e-2 / rel-L2 1e-3.
"""

import os

import numpy as np
import pytest
import torch

from conftest import relative_error, to_np
from golden import make_golden as mg

GOLD = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz"))
BITS = (1, 2, 3, 4)


# ------------------------------------------------------------------- CPU
def test_oracle_reproduces_golden():
    fresh = mg.build()
    assert set(fresh) == set(GOLD.files)
    for key in GOLD.files:
        if key == "block_out":  # fp32 BLAS: summation order may differ between hosts
            np.testing.assert_allclose(fresh[key], GOLD[key], rtol=1e-5, atol=1e-6, err_msg=key)
        else:
            np.testing.assert_array_equal(fresh[key], GOLD[key], err_msg=key)


def test_hf_level2_golden_regenerates():
    """tests/golden/hf_level2.npz is what make_hf_level2.py writes: the seeded
    inputs bit for bit, the stock transformers blocks' float32 outputs within
    BLAS summation-order noise."""
    pytest.importorskip("transformers")
    from golden import make_hf_level2 as mk
    gold = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "hf_level2.npz"))
    for family in ("olmoe", "mixtral"):
        x = mk.inputs(family)
        np.testing.assert_array_equal(gold[f"{family}_x"], x.numpy())
        ref = mk.reference_block(family, mk.hf_block(family, mk.config(family)))
        with torch.no_grad():
            y = ref(x[:mk.T].float().reshape(1, mk.T, mk.H))
        y = (y[0] if isinstance(y, tuple) else y).reshape(mk.T, mk.H).numpy()
        np.testing.assert_allclose(y, gold[f"{family}_prefill"], rtol=1e-4, atol=1e-6)


def test_block_inputs_regenerate_bit_exact():
    gate, experts, x = mg.block_inputs()
    assert bytes(GOLD["block_sha256"]).hex() == mg.digest(gate, experts, x)


@pytest.mark.parametrize("nbits", BITS)
def test_product_quantizer_matches_golden(nbits):
    from robustgemq_amd.quantize import rtn_quantize
    t = rtn_quantize(torch.from_numpy(GOLD[f"rtn_b{nbits}_W"]), nbits, 64)
    for name, ref in (("Q", "Q"), ("scales", "s"), ("zeros", "z")):
        np.testing.assert_array_equal(getattr(t, name).numpy().view(np.uint16),
                                      GOLD[f"rtn_b{nbits}_{ref}"].view(np.uint16), err_msg=name)


# ------------------------------------------------------------------- GPU
@pytest.mark.gpu
@pytest.mark.parametrize("nbits", BITS)
def test_gpu_packing_matches_golden(device, nbits):
    from robustgemq_amd import ops
    from robustgemq_amd.experts import QuantProjection
    print(f"[golden pack] nbits={nbits}", flush=True)
    codes = torch.from_numpy(GOLD[f"pack_b{nbits}_codes"]).to(device)
    words, _ = ops.pack_weights_over_cols(codes, nbits)
    np.testing.assert_array_equal(to_np(words), GOLD[f"pack_b{nbits}_words"])
    w256, _ = ops.pack_weights_over_cols(codes[:, :256].contiguous(), nbits)
    s = torch.ones((256 // 64, 16), dtype=torch.float16, device=device)
    proj = QuantProjection([w256], [s], [torch.zeros_like(s)], [nbits], 256, 16, 64, 0)
    np.testing.assert_array_equal(to_np(proj.words).view(np.uint32).reshape(1, 2, 16, 4, nbits),
                                  GOLD[f"pack_b{nbits}_build"])


@pytest.mark.gpu
def test_gpu_routing_matches_golden(device):
    from robustgemq_amd import ops
    print("[golden route]", flush=True)
    x = torch.from_numpy(GOLD["route_x"]).to(device)
    for norm in (0, 1):
        lg, idx, w = ops.route(x, torch.from_numpy(GOLD["route_wg"]).to(device), 2, bool(norm))
        np.testing.assert_array_equal(to_np(lg).view(np.uint16), GOLD["route_logits"].view(np.uint16))
        np.testing.assert_array_equal(to_np(idx), GOLD[f"route_idx_n{norm}"])
        np.testing.assert_allclose(to_np(w), GOLD[f"route_w_n{norm}"], rtol=2e-6, atol=1e-7)
    perm = ops.permute(torch.from_numpy(GOLD["route_idx_n0"]).to(device), 8)
    for key in ("counts", "offsets", "row_token", "row_pair", "inv_perm"):
        np.testing.assert_array_equal(to_np(perm[key]), GOLD[f"route_perm_{key}"], err_msg=key)
    lg, idx, w = ops.route(x, torch.from_numpy(GOLD["route32_wg"]).to(device), 6, False)
    np.testing.assert_array_equal(to_np(lg).view(np.uint32), GOLD["route32_logits"].view(np.uint32))
    np.testing.assert_array_equal(to_np(idx), GOLD["route32_idx"])
    np.testing.assert_allclose(to_np(w), GOLD["route32_w"], rtol=2e-6, atol=1e-7)
    perm = ops.permute(idx, 16, n_shared=2)
    for key in ("counts", "offsets", "row_token", "row_pair", "inv_perm"):
        np.testing.assert_array_equal(to_np(perm[key]), GOLD[f"route32_perm_{key}"], err_msg=key)


@pytest.mark.gpu
def test_gpu_block_matches_golden(device):
    from robustgemq_amd.quantize import QuantTriplet
    from robustgemq_amd.synthetic import CONFIGS, build_block
    print("[golden block] H=F=512 E=8 k=2 g=128 T=16", flush=True)
    cfg = CONFIGS["ref_test"]
    gate, experts, x = mg.block_inputs()
    H, F, g = mg.BLOCK["H"], mg.BLOCK["F"], mg.BLOCK["g"]
    shapes = {"gate_proj": (F, H), "up_proj": (F, H), "down_proj": (H, F)}
    ex_t = [{name: QuantTriplet(*(torch.from_numpy(a) for a in ex[name]), mg.BLOCK["bits"][e], g, shapes[name])
             for name in shapes} for e, ex in enumerate(experts)]
    w = dict(bits=list(mg.BLOCK["bits"]), gate=torch.from_numpy(gate), experts=ex_t, shared=None, bias=None)
    block = build_block(cfg, w, device=device)
    layer = block._layer
    xd = torch.from_numpy(x).to(device)
    from robustgemq_amd import ops
    lg, idx, wt = ops.route(xd, layer.gate_w, layer.top_k, layer.norm_topk)
    np.testing.assert_array_equal(to_np(lg).view(np.uint16), GOLD["block_logits"].view(np.uint16))
    np.testing.assert_array_equal(to_np(idx), GOLD["block_idx"])
    out32, _ = layer.forward(xd, out_dtype=torch.float32, want_logits=False)
    got, ref = to_np(out32), GOLD["block_out"]
    err, mx = relative_error(got, ref), float(np.abs(got - ref).max())
    print(f"    rel-L2 {err:.3e} max-abs {mx:.3e}", flush=True)
    assert err <= 1e-3 and mx <= 1e-2
    y, router_logits = block(xd.reshape(1, 16, H))
    got16 = to_np(y.reshape(16, H)).astype(np.float32)
    assert relative_error(got16, ref) <= 1e-3 and float(np.abs(got16 - ref).max()) <= 1e-2
    np.testing.assert_array_equal(to_np(router_logits).view(np.uint16), GOLD["block_logits"].view(np.uint16))
