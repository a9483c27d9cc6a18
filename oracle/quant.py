"""Quantizer, dequantizer and packed-word layouts (CPU restatement).

Reference files restated:
  gemq/quantizers/rtn.py:15-61          RTNWeightQuantizer.quantize / dequantize
  tests/conftest.py:117-131             quantize_weight (fake-quant twin W_deq)
  gemq/triton_kernels/utils.py:33-113   pack_weights_over_cols (K7), packed layout
  gemq/triton_kernels/utils.py:192-212  dequantize (kernel read pattern, q*s+z')
  gemq/triton_kernels/dequant_group_gemm.py:118-130  word row k//eps, shift (k%eps)*b
"""

import numpy as np

from .fp import f32, h_add, h_div, h_mul, h_sub, to_f16


# ------------------------------------------------------------------ RTN (A13)
def rtn_quantize(W, nbits, group_size):
    """RTNWeightQuantizer.quantize, gemq/quantizers/rtn.py:15-55.

    W: fp16 [out_features, in_features]; groups of ``group_size`` run along
    the input dim (HQQ axis=1).  Returns fp16 (Q [G, g], scales [G, 1],
    zeros [G, 1]) with G = W.size // g, every op in fp16 as torch runs it.

    The 1-bit scale ``2 * mean(|W|)`` (rtn.py:38) is taken here as an exact
    (float64) sum, divided by g, rounded to fp32 then fp16; torch sums in fp32,
    which can differ in the last fp16 bit only when that fp32 sum lies within
    2^-24 of an fp16 rounding boundary.
    """
    W = np.asarray(W, dtype=np.float16)
    assert W.shape[-1] % group_size == 0, (W.shape, group_size)
    Wg = W.reshape(-1, group_size)
    G = Wg.shape[0]
    if nbits == 0:  # rtn.py:29-34
        return (np.zeros_like(Wg), np.ones((G, 1), np.float16), np.zeros((G, 1), np.float16))
    if nbits == 1:  # rtn.py:36-40
        Q = (Wg >= 0).astype(np.float16)
        mean = np.abs(Wg.astype(np.float64)).sum(axis=1, keepdims=True) / group_size
        s = h_mul(to_f16(mean.astype(np.float32)), np.float16(2.0))
        z = np.full((G, 1), 0.5, np.float16)
        return Q, s, z
    mx = Wg.max(axis=1, keepdims=True)  # rtn.py:42-43, exact
    mn = Wg.min(axis=1, keepdims=True)
    max_int = 2 ** nbits - 1  # rtn.py:45
    rng = h_sub(mx, mn)
    rng = np.maximum(rng, np.float16(1e-5))  # clamp(min=1e-5): the bound is cast to fp16 first
    s = h_div(rng, np.float16(max_int))  # rtn.py:47
    z = np.clip(-np.round(h_div(mn, s)), 0, max_int).astype(np.float16)  # rtn.py:48
    Q = np.clip(h_add(np.round(h_div(Wg, s)), z), 0, max_int).astype(np.float16)  # rtn.py:53
    return Q, s, z


def dequant_hqq(Q, s, z):
    """Fake-quant weight ``(Q - zeros) * scales`` in fp16, rtn.py:57-61 and
    tests/conftest.py:130.  Q [G, g], s/z [G, 1] broadcast.  Returns fp16."""
    return h_mul(h_sub(Q, z), s)


def dequant_affine(Q, s, zp):
    """GemLite-convention weight ``fma(fp16(q), s, z')`` with one rounding,
    gemq/triton_kernels/utils.py:206-210 (tl.fma on fp16 operands)."""
    exact = f32(Q).astype(np.float64) * f32(s).astype(np.float64) + f32(zp).astype(np.float64)
    # q*s and z' are multiples of 2^-24 (the fp16 quantum) below 2^21, so their
    # sum is exact in float64 and the direct float64->fp16 cast rounds once.
    return exact.astype(np.float16)


def codes_from_q(Q, N, K):
    """HQQ logical Q [N*K/g, g] (float codes) -> uint8 codes [N, K]."""
    return np.asarray(Q).reshape(N, K).astype(np.uint8)


def groups_to_nk(v, N, K, group_size):
    """Per-group values [N*K/g, 1] (row-major over (n, group)) -> [K/g, N],
    the layout the reference stacks (scales/zeros [sum K/g, N])."""
    return np.asarray(v).reshape(N, K // group_size).T.copy()


# ------------------------------------------------- reference word layout (A10)
def eps_of(nbits):
    return 32 // nbits


def pack_cols(codes, nbits):
    """pack_weights_over_cols_triton, gemq/triton_kernels/utils.py:74-113.

    codes uint8 [N, K] -> int32 [ceil(K/eps), N]: word (r, n) holds codes
    k = r*eps + i (i < eps) of column n at bits [i*b, i*b + b), LSB first; the
    tail of the last row and the dead bits (3-bit: 30..31) are zero.  The
    Triton wrapper returns the transposed view, which from_hf concatenates row
    wise (moe_block.py:725-733), so [rows, N] with N contiguous is the stacked
    layout."""
    codes = np.asarray(codes, dtype=np.uint32)
    N, K = codes.shape
    eps = eps_of(nbits)
    rows = -(-K // eps)
    c = np.zeros((N, rows * eps), np.uint32)
    c[:, :K] = codes
    c = c.reshape(N, rows, eps)
    shifts = (np.arange(eps, dtype=np.uint32) * nbits).astype(np.uint32)
    words = np.bitwise_or.reduce(c << shifts, axis=2)  # [N, rows]
    return np.ascontiguousarray(words.T).view(np.int32)


def unpack_cols(words, nbits, K):
    """The kernels' read of the packed layout: word row k // eps, shift
    (k % eps) * b, mask 2^b - 1 (dequant_group_gemm.py:118, :128-130;
    utils.py:206).  int32 [rows, N] -> uint8 codes [N, K]."""
    w = np.asarray(words).view(np.uint32)
    eps = eps_of(nbits)
    k = np.arange(K)
    vals = (w[k // eps, :] >> ((k % eps) * nbits).astype(np.uint32)[:, None]) & ((1 << nbits) - 1)
    return vals.T.astype(np.uint8)


# --------------------------------------------------- build layout (this repo)
# Codes of column n, reduction index k = 128*c + 32*kb + i (i = 8*t + 2*d + h)
# sit in the lane slice (c, n, kb), nbits words long, so that for MFMA step t
# and pair d the two codes (h = 0, 1) land at the same bit offset of the low
# and high 16-bit halves of one word.  Slices are stored panel-major: panel
# p = n // 16 holds chunk 0's slices of its 16 columns, then chunk 1's, ...
# (order [p][c][n % 16][kb][word]).
def _slice_bits(nbits):
    """For each i in 0..31 a list of (word, bit, code_shift, width) fields."""
    out = []
    for i in range(32):
        t, d, h = i // 8, (i % 8) // 2, i % 2
        if nbits == 4:
            out.append([(t, 16 * h + 4 * d, 0, 4)])
        elif nbits == 2:
            out.append([(t // 2, 16 * h + 2 * (4 * (t % 2) + d), 0, 2)])
        elif nbits == 1:
            out.append([(0, 16 * h + 4 * t + d, 0, 1)])
        elif nbits == 3:
            out.append([(t // 2, 16 * h + 2 * (4 * (t % 2) + d), 0, 2),
                        (2, 16 * h + 4 * t + d, 2, 1)])
        else:
            raise ValueError(nbits)
    return out


def repack_build(codes, nbits):
    """uint8 codes [N, K] -> uint32 build-layout words, shape
    [N/16, K/128, 16, 4, nbits] = [panel, c, n % 16, kb, word] (flattened in
    that order on the device)."""
    codes = np.asarray(codes, dtype=np.uint32)
    N, K = codes.shape
    assert K % 128 == 0 and N % 16 == 0
    C = K // 128
    q = codes.reshape(N // 16, 16, C, 4, 32).transpose(0, 2, 1, 3, 4)  # [p, c, n%16, kb, i]
    out = np.zeros((N // 16, C, 16, 4, nbits), np.uint32)
    for i, fields in enumerate(_slice_bits(nbits)):
        for (w, bit, cshift, width) in fields:
            v = (q[..., i] >> np.uint32(cshift)) & np.uint32((1 << width) - 1)
            out[..., w] |= (v << np.uint32(bit)).astype(np.uint32)
    return out


def unpack_build(words, nbits, N, K):
    """Inverse of repack_build: words [N/16, K/128, 16, 4, nbits] -> codes [N, K]."""
    w = np.asarray(words, dtype=np.uint32).reshape(N // 16, K // 128, 16, 4, nbits)
    q = np.zeros((N // 16, K // 128, 16, 4, 32), np.uint32)
    for i, fields in enumerate(_slice_bits(nbits)):
        for (wi, bit, cshift, width) in fields:
            q[..., i] |= ((w[..., wi] >> np.uint32(bit)) & np.uint32((1 << width) - 1)) << np.uint32(cshift)
    return q.transpose(0, 2, 1, 3, 4).reshape(N, K).astype(np.uint8)


def prep_scales(s, z, dq_mode):
    """Per-group (s, z) fp16 arrays [G, N] (one expert) -> uint32 half2 pairs
    in the panel-major build order [N/16, G, 16]:
    HQQ (mode 0): low half s, high half -z; AFFINE (mode 1): s, z';
    HQQ_INT (mode 2, integer z in 0..1023): s, -(1024 + z)."""
    sb = np.asarray(s, dtype=np.float16).view(np.uint16).astype(np.uint32)
    zz = np.asarray(z, dtype=np.float16)
    if dq_mode == 0:
        zz = -zz
    elif dq_mode == 2:
        assert np.all((zz == np.round(zz)) & (zz >= 0) & (zz <= 1023))
        zz = (-(1024.0 + zz.astype(np.float64))).astype(np.float16)
    zb = zz.astype(np.float16).view(np.uint16).astype(np.uint32)
    pairs = (sb | (zb << 16)).astype(np.uint32)
    G, N = pairs.shape
    assert N % 16 == 0
    return np.ascontiguousarray(pairs.reshape(G, N // 16, 16).transpose(1, 0, 2))


def kernel_dequant_hqq(codes, s_nk, z_nk, group_size):
    """Weight the kernels form in HQQ mode, w[k, n] = fp16(fp16(q - z) * s),
    written as the kernel evaluates it (q exact, one fp16 rounding for the
    subtraction, one for the product).  codes [N, K]; s/z [K/g, N] fp16.
    Returns fp16 [K, N].  Equal to dequant_hqq for every fp16 z (checked
    exhaustively in the tests), i.e. to the fake-quant weight."""
    q = np.asarray(codes).T.astype(np.float64)  # [K, N]
    g = np.arange(q.shape[0]) // group_size
    zz = f32(z_nk)[g, :].astype(np.float64)
    ss = f32(s_nk)[g, :]
    t = (q - zz).astype(np.float16)  # q - z is exact in float64; one rounding to fp16
    return h_mul(t, ss)
