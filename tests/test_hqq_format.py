"""HQQ bit-packing restated without hqq (robustgemq_amd/hqq_format.py): hand-
computed packed words, round trips for every width, the 3-bit zero padding
and its cut (gemq/inference/patch.py:37-39), and the layer-state readers.
Parity with hqq's own bytes is unpinned (no hqq, no checkpoint here)."""

import numpy as np
import pytest
import torch

from robustgemq_amd import hqq_format as hf


def test_hand_computed_words():
    # 4-bit: two half slices, the first in the high nibble
    Q = torch.tensor([[1, 2], [3, 4], [5, 6], [7, 8]])
    W = hf.pack(Q, 4)
    assert W.dtype == torch.uint8
    assert W.tolist() == [[0x15, 0x26], [0x37, 0x48]]
    # 2-bit: four quarters, 0b01_10_11_00
    assert hf.pack(torch.tensor([[1], [2], [3], [0]]), 2).tolist() == [[0b01101100]]
    # 1-bit: eight eighths, 0b1011_0010
    assert hf.pack(torch.tensor([[1], [0], [1], [1], [0], [0], [1], [0]]), 1).tolist() == [[0b10110010]]
    # 3-bit: 3 rows padded with zeros to 10, fields from bit 27 down
    W3 = hf.pack(torch.tensor([[5], [2], [7]]), 3)
    assert W3.dtype == torch.int32 and W3.tolist() == [[719323136]]  # 5<<27 | 2<<24 | 7<<21
    U = hf.unpack(W3, "3bit_32")
    assert U.shape == (10, 1) and U[:, 0].tolist() == [5, 2, 7, 0, 0, 0, 0, 0, 0, 0]
    # 8-bit is the identity
    assert hf.pack(torch.tensor([[200, 3]]), 8).tolist() == [[200, 3]]


@pytest.mark.parametrize("nbits", [1, 2, 3, 4, 8])
@pytest.mark.parametrize("rows", [40, 80, 123])
def test_round_trip(nbits, rows):
    S = {1: 8, 2: 4, 3: 10, 4: 2, 8: 1}[nbits]
    if nbits != 3 and rows % S:
        with pytest.raises(ValueError):
            hf.pack(torch.zeros(rows, 64, dtype=torch.int32), nbits)
        return
    g = torch.Generator().manual_seed(nbits * 1000 + rows)
    Q = torch.randint(0, 2 ** nbits, (rows, 64), generator=g)
    W = hf.pack(Q, nbits)
    assert W.shape[0] == -(-rows // S)
    U = hf.unpack(W, hf.BIT_TO_PACKING[nbits])
    assert torch.equal(U[:rows].long(), Q)
    assert not U[rows:].any()  # 3-bit padding rows are zero


@pytest.mark.parametrize("nbits", [1, 2, 3, 4])
def test_codes_cut_and_layer_state(nbits):
    """codes() == the [N, K] view create_gemlite_from_hqq makes; both
    state-dict forms read back."""
    from robustgemq_amd.quantize import rtn_quantize
    N, K, gs = 96, 256, 64
    W = (torch.randn(N, K, generator=torch.Generator().manual_seed(nbits)) * 0.02).half()
    t = rtn_quantize(W, nbits, gs)
    st = hf.HQQLinearState.from_quantized(t.Q, t.scales, t.zeros, t.shape, nbits, gs)
    assert st.meta["packing"] == hf.BIT_TO_PACKING[nbits]
    want = t.codes()
    assert torch.equal(hf.codes(st.W_q, st.meta), want)
    raw = st.unpack(reshape=False)
    assert raw.shape[0] >= N * K // gs
    assert torch.equal(raw[:N * K // gs].reshape(N, K), want)
    assert torch.equal(st.unpack(reshape=True), want)
    nested = hf.HQQLinearState.from_state_dict({"W_q": st.W_q, "meta": st.meta, "bias": None})
    flat = hf.HQQLinearState.from_state_dict({"W_q": st.W_q, **st.meta})
    for s2 in (nested, flat):
        assert torch.equal(hf.codes(s2.W_q, s2.meta), want)
        assert torch.equal(s2.meta["scale"], t.scales) and torch.equal(s2.meta["zero"], t.zeros)
    with pytest.raises(KeyError):
        hf.HQQLinearState.from_state_dict({"W_q": st.W_q, "nbits": nbits})


def test_out_of_range_codes_are_refused():
    with pytest.raises(ValueError):
        hf.pack(torch.tensor([[4], [0], [1], [2]]), 2)  # 4 does not fit 2 bits
    with pytest.raises(ValueError):
        hf.pack(torch.tensor([[-1], [0]]), 4)
    with pytest.raises(ValueError):
        hf.pack(torch.tensor([[0.5], [1.0]]), 4)


def test_axis_other_than_one_is_refused():
    st = hf.HQQLinearState.from_quantized(torch.zeros(8, 4), torch.ones(8, 1), torch.zeros(8, 1), (8, 4), 4, 4)
    st.meta["axis"] = 0
    with pytest.raises(ValueError):
        hf.codes(st.W_q, st.meta)


def test_file_round_trip_is_weights_only(tmp_path):
    """A {name: layer state} file written with torch.save reads back with
    torch.load(weights_only=True) (what load_hqq_linears uses)."""
    from robustgemq_amd.quantize import rtn_quantize
    t = rtn_quantize((torch.randn(32, 128) * 0.02).half(), 2, 64)
    st = hf.HQQLinearState.from_quantized(t.Q, t.scales, t.zeros, t.shape, 2, 64)
    p = tmp_path / "qmodel.pt"
    torch.save({"model.layers.0.mlp.experts.0.gate_proj": {"W_q": st.W_q, "meta": st.meta}}, p)
    back = torch.load(p, map_location="cpu", weights_only=True)
    s2 = hf.HQQLinearState.from_state_dict(back["model.layers.0.mlp.experts.0.gate_proj"])
    np.testing.assert_array_equal(hf.codes(s2.W_q, s2.meta).numpy(), t.codes().numpy())
