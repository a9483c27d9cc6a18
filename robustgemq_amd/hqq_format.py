"""HQQ quantized-linear format, read and written without the hqq package.

An HQQ linear -- what create_hqq_linear_from_quantized_weights builds
(gemq/utils/quant_utils.py:55-97) and what the reference's checkpoints hold
per layer (loaded by AutoHQQHFModel, gemq/utils/hf_loading.py:67-78) -- is

  W_q   the codes Q [N*K/g, g] (one row per group, grouped along K: axis 1),
        bit-packed along dim 0 in the format meta["packing"] names;
  meta  nbits, group_size, shape (N, K), scale and zero [N*K/g, 1], axis (1),
        packing, ... (the keys quant_utils.py:72-83 sets);
  bias  optional.

Packing formats (Quantizer.bit_to_packing per nbits; hqq's BitPack): the
rows are cut into S equal slices and slice i is shifted into bit field i of
one packed row, the first slice in the highest field:

  8bit_u8  S = 1   uint8 as is
  4bit_u8  S = 2   byte  = s0 << 4 | s1
  2bit_u8  S = 4   byte  = s0 << 6 | s1 << 4 | s2 << 2 | s3
  1bit_u8  S = 8   byte  = s0 << 7 | ... | s7
  3bit_32  S = 10  int32 = s0 << 27 | s1 << 24 | ... | s9, rows first
                   zero-padded to a multiple of 10 (so an unpack returns the
                   padding rows, which create_gemlite_from_hqq cuts off,
                   gemq/inference/patch.py:37-39)

The byte layout is restated from hqq's published BitPack algorithm; neither
the hqq package nor a checkpoint is available here, so parity with hqq's own
bytes is unpinned: the tests pin round trips, hand-computed vectors and the
3-bit padding cut.
"""

import math

import torch

BIT_TO_PACKING = {8: "8bit_u8", 4: "4bit_u8", 3: "3bit_32", 2: "2bit_u8", 1: "1bit_u8"}
# packing -> (slices per packed row, bits per field, packed dtype)
_FORMAT = {
    "8bit_u8": (1, 8, torch.uint8),
    "4bit_u8": (2, 4, torch.uint8),
    "2bit_u8": (4, 2, torch.uint8),
    "1bit_u8": (8, 1, torch.uint8),
    "3bit_32": (10, 3, torch.int32),
}


def pack(Q, nbits):
    """Codes Q [R, g] (integers in 0 .. 2**nbits - 1) -> packed W_q."""
    S, b, dt = _FORMAT[BIT_TO_PACKING[int(nbits)]]
    if Q.is_floating_point() and not torch.equal(Q, Q.round()):
        raise ValueError("codes must be integers")
    Q = Q.to(torch.int32)
    if Q.numel() and (int(Q.min()) < 0 or int(Q.max()) >= (1 << b)):
        raise ValueError(f"codes outside 0..{(1 << b) - 1} for {nbits}-bit packing")
    R = Q.shape[0]
    if dt == torch.int32:
        rows = S * math.ceil(R / S)
        if rows != R:
            Q = torch.cat([Q, Q.new_zeros((rows - R,) + tuple(Q.shape[1:]))])
    elif R % S:
        raise ValueError(f"{BIT_TO_PACKING[nbits]} needs a row count divisible by {S}, got {R}")
    step = Q.shape[0] // S
    out = torch.zeros((step,) + tuple(Q.shape[1:]), dtype=torch.int32, device=Q.device)
    for i in range(S):
        out |= Q[i * step:(i + 1) * step] << (b * (S - 1 - i))
    return out.to(dt)


def unpack(W_q, packing, dtype=torch.uint8):
    """Packed W_q -> codes [S * rows, g] (for 3bit_32 including the zero
    padding rows)."""
    S, b, _ = _FORMAT[packing]
    w = W_q.to(torch.int32)
    mask = (1 << b) - 1
    return torch.cat([(w >> (b * (S - 1 - i))) & mask for i in range(S)]).to(dtype)


def codes(W_q, meta):
    """The [N, K] codes of an HQQ linear: unpack, cut the 3-bit padding rows
    (patch.py:37-39), view as (out_features, in_features)."""
    N, K = (int(v) for v in meta["shape"])
    g = int(meta["group_size"])
    if int(meta.get("axis", 1)) != 1:
        raise ValueError("Only axis==1 is supported.")
    packing = meta.get("packing") or BIT_TO_PACKING[int(meta["nbits"])]
    Q = unpack(W_q, packing)
    return Q[:N * K // g].reshape(N, K)


class HQQLinearState:
    """An HQQ linear held as its tensors (W_q, meta, bias), with the
    `unpack(reshape=False, dtype)` read that create_gemlite_from_hqq makes
    (patch.py:35), so QuantLinear.from_hqq_layer takes it like an HQQLinear."""

    def __init__(self, W_q, meta, bias=None):
        self.W_q = W_q
        self.meta = dict(meta)
        self.meta.setdefault("packing", BIT_TO_PACKING[int(self.meta["nbits"])])
        self.meta.setdefault("axis", 1)
        self.bias = bias

    def unpack(self, reshape=False, dtype=torch.uint8):
        Q = unpack(self.W_q, self.meta["packing"], dtype=dtype)
        if reshape:
            N, K = (int(v) for v in self.meta["shape"])
            g = int(self.meta["group_size"])
            return Q[:N * K // g].reshape(N, K)
        return Q

    @classmethod
    def from_quantized(cls, Q, scale, zero, shape, nbits, group_size, bias=None):
        """What create_hqq_linear_from_quantized_weights stores
        (quant_utils.py:55-97): Q [N*K/g, g] packed, scale / zero kept as given."""
        meta = {"nbits": int(nbits), "group_size": int(group_size), "shape": tuple(int(v) for v in shape),
                "scale": scale, "zero": zero, "axis": 1, "packing": BIT_TO_PACKING[int(nbits)],
                "quant_scale": False, "quant_zero": False, "view_as_float": False}
        return cls(pack(Q, nbits), meta, bias)

    @classmethod
    def from_state_dict(cls, sd):
        """One layer's tensors: {"W_q", "meta": {...}, "bias"} or the same
        keys flattened into one dict ({"W_q", "nbits", "group_size", "shape",
        "scale", "zero", ...})."""
        if "meta" in sd:
            meta, bias = sd["meta"], sd.get("bias")
        else:
            meta = {k: v for k, v in sd.items() if k not in ("W_q", "bias")}
            bias = sd.get("bias")
        for k in ("nbits", "group_size", "shape", "scale", "zero"):
            if k not in meta:
                raise KeyError(f"HQQ layer state lacks {k!r}")
        shape = meta["shape"]
        meta = dict(meta)
        meta["shape"] = tuple(int(v) for v in (shape.tolist() if torch.is_tensor(shape) else shape))
        for k in ("nbits", "group_size", "axis"):
            if k in meta and torch.is_tensor(meta[k]):
                meta[k] = int(meta[k])
        return cls(sd["W_q"], meta, bias)


def load_hqq_linears(source, device="cuda", names=None):
    """{layer name: QuantLinear} from HQQ layer states: `source` is a mapping
    {name: layer state} or a file of one, read with torch.load(...,
    weights_only=True) (nothing in the file is executed).  `names` filters the
    layers (a callable on the name)."""
    from .linear import QuantLinear
    if isinstance(source, (str, bytes)) or hasattr(source, "__fspath__"):
        source = torch.load(source, map_location="cpu", weights_only=True)
    out = {}
    for name, sd in source.items():
        if names is not None and not names(name):
            continue
        if not isinstance(sd, dict) or "W_q" not in sd:
            continue
        st = HQQLinearState.from_state_dict(sd)
        st.W_q = st.W_q.to(device)
        out[name] = QuantLinear.from_hqq_layer(st, device=torch.device(device))
    return out


__all__ = ["BIT_TO_PACKING", "pack", "unpack", "codes", "HQQLinearState", "load_hqq_linears"]
