"""Dense quantized linear (QuantLinear, the E = 1 grouped GEMM) against the
oracle: y = x @ ((Q - z) * s)^T + b in fp32, the check of
tests/test_quant_linear_equiv.py:134-194 (GemLite linear vs fp16 matmul on the
dequantized weight) at the expert path's bar: max-abs 1e-2, rel-L2 1e-3."""

import numpy as np
import pytest
import torch

from conftest import relative_error, to_np
from oracle import quant as oq

pytestmark = pytest.mark.gpu

MAX_ABS = 1e-2
REL_L2 = 1e-3


def _weights(N, K, nbits, g, seed):
    from robustgemq_amd.quantize import rtn_quantize
    gen = torch.Generator().manual_seed(seed)
    W = (torch.randn(N, K, generator=gen) * 0.02).half()
    t = rtn_quantize(W, nbits, g)
    dense = oq.dequant_hqq(t.Q.numpy(), t.scales.numpy(), t.zeros.numpy()).reshape(N, K).astype(np.float32)
    return t, dense


@pytest.mark.parametrize("nbits", [1, 2, 3, 4])
@pytest.mark.parametrize("g", [64, 128])
@pytest.mark.parametrize("M", [1, 16, 300])
def test_quant_linear_matches_oracle(device, nbits, g, M):
    from robustgemq_amd.linear import QuantLinear
    print(f"[linear] nbits={nbits} g={g} M={M}", flush=True)
    N, K = 384, 1024
    t, dense = _weights(N, K, nbits, g, seed=nbits * 100 + g + M)
    bias = torch.from_numpy((np.random.default_rng(M).standard_normal(N) * 0.1).astype(np.float16))
    lin = QuantLinear.from_triplet(t.to(device), bias=bias)
    x = torch.from_numpy((np.random.default_rng(M + 1).standard_normal((M, K)) * 0.5).astype(np.float16))
    y = lin(x.to(device))
    assert y.shape == (M, N) and y.dtype == torch.float16
    ref = x.float().numpy() @ dense.T + bias.float().numpy()
    got = to_np(y).astype(np.float32)
    err, mx = relative_error(got, ref), float(np.abs(got - ref).max())
    print(f"    rel-L2 {err:.3e} max-abs {mx:.3e}", flush=True)
    assert err <= REL_L2 and mx <= MAX_ABS


def test_quant_linear_bf16_and_leading_dims(device):
    from robustgemq_amd.linear import QuantLinear
    print("[linear] bf16, [B, S, K] input", flush=True)
    N, K = 256, 512
    t, dense = _weights(N, K, 4, 64, seed=7)
    lin = QuantLinear.from_triplet(t.to(device), act_dtype=torch.bfloat16)
    x = (torch.randn(2, 24, K, generator=torch.Generator().manual_seed(3)) * 0.5).to(torch.bfloat16)
    y = lin(x.to(device))
    assert y.shape == (2, 24, N) and y.dtype == torch.bfloat16
    ref = x.float().numpy().reshape(-1, K) @ dense.T
    got = to_np(y.float()).reshape(-1, N)
    assert relative_error(got, ref) <= 1e-2 and float(np.abs(got - ref).max()) <= MAX_ABS


def test_quant_linear_from_hqq_layer_and_gemlite_views(device):
    """from_hqq_layer makes create_gemlite_from_hqq's reads (patch.py:27-50),
    including the cut of the 3-bit padding rows; the GemLite views are what
    from_hf reads, and dequantize as q * s + z'."""
    from robustgemq_amd.linear import QuantLinear
    from robustgemq_amd.moe_block import _is_packed_linear
    print("[linear] from_hqq_layer, 3-bit with padding rows", flush=True)
    N, K, g, nbits = 128, 768, 64, 3
    t, dense = _weights(N, K, nbits, g, seed=11)
    codes = t.codes()
    pad = torch.full((5, g), 7, dtype=torch.uint8)  # the padding rows a 3-bit HQQ unpack returns

    class FakeHQQ:
        W_q = torch.zeros(1, device=device)
        meta = {"shape": (N, K), "nbits": nbits, "group_size": g, "axis": 1,
                "scale": t.scales.to(device), "zero": t.zeros.to(device)}
        bias = None

        def unpack(self, reshape=False, dtype=torch.uint8):
            return torch.cat([codes.reshape(-1, g), pad]).to(device=device, dtype=dtype)

    lin = QuantLinear.from_hqq_layer(FakeHQQ())
    assert _is_packed_linear(lin)
    x = torch.from_numpy((np.random.default_rng(5).standard_normal((7, K)) * 0.5).astype(np.float16))
    got = to_np(lin(x.to(device))).astype(np.float32)
    ref = x.float().numpy() @ dense.T
    assert relative_error(got, ref) <= REL_L2 and float(np.abs(got - ref).max()) <= MAX_ABS
    np.testing.assert_array_equal(to_np(lin.W_q).view(np.uint32), oq.pack_cols(codes.numpy(), nbits).view(np.uint32))
    s = to_np(lin.scales).astype(np.float32)
    zp = to_np(lin.zeros).astype(np.float32)
    gi = np.arange(K) // g
    w_aff = codes.numpy().T.astype(np.float32) * s[gi] + zp[gi]  # [K, N]
    assert float(np.abs(w_aff - dense.T).max()) <= 2e-3 * float(np.abs(dense).max())


def test_replace_linear_recursive(device):
    from robustgemq_amd.linear import QuantLinear, replace_linear_recursive
    print("[linear] replace_linear_recursive", flush=True)
    N, K = 128, 256
    t, dense = _weights(N, K, 2, 64, seed=13)
    marker = torch.nn.Linear(K, N, bias=False)
    model = torch.nn.Sequential(torch.nn.Identity(), torch.nn.Sequential(torch.nn.Identity(), marker))
    replace_linear_recursive(model, lambda m: QuantLinear.from_triplet(t.to(device)) if m is marker else None)
    assert isinstance(model[1][1], QuantLinear)
    x = torch.randn(3, K, device=device).half()
    ref = x.float().cpu().numpy() @ dense.T
    assert relative_error(to_np(model(x)).astype(np.float32), ref) <= REL_L2


@pytest.mark.parametrize("nbits", [1, 2, 3, 4])
def test_hqq_checkpoint_linears(device, tmp_path, nbits):
    """HQQ layer states (packed as hqq's BitPack, scale/zero in the meta) saved
    to a file and loaded without hqq: the linears equal the dequantized
    weight's matmul at the expert path's bar, and the name filter applies."""
    from robustgemq_amd import hqq_format as hf
    print(f"[linear] HQQ checkpoint load, nbits={nbits}", flush=True)
    N, K, g = 256, 512, 64
    t, dense = _weights(N, K, nbits, g, seed=31 + nbits)
    bias = torch.from_numpy((np.random.default_rng(nbits).standard_normal(N) * 0.1).astype(np.float16))
    st = hf.HQQLinearState.from_quantized(t.Q, t.scales, t.zeros, t.shape, nbits, g, bias=bias)
    p = tmp_path / "qmodel.pt"
    torch.save({"layers.0.mlp.down_proj": {"W_q": st.W_q, "meta": st.meta, "bias": bias},
                "layers.0.input_layernorm": {"weight": torch.ones(K)}}, p)
    lins = hf.load_hqq_linears(p, device=device)
    assert list(lins) == ["layers.0.mlp.down_proj"]
    assert hf.load_hqq_linears(p, device=device, names=lambda n: "attn" in n) == {}
    x = torch.from_numpy((np.random.default_rng(7).standard_normal((5, K)) * 0.5).astype(np.float16))
    got = to_np(lins["layers.0.mlp.down_proj"](x.to(device))).astype(np.float32)
    ref = x.float().numpy() @ dense.T + bias.float().numpy()
    assert relative_error(got, ref) <= REL_L2 and float(np.abs(got - ref).max()) <= MAX_ABS
