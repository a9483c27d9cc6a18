"""Pins the CPU oracle before it is trusted as the parity reference.

The reference ships no golden vectors (its tests draw inputs live on CUDA), so
each oracle function is checked against what fixes it independently:
torch's own fp16 CPU arithmetic running the reference formulas, closed forms,
exact rational arithmetic, brute force on small inputs, and library routines.
"""

import itertools
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import fp, moe, quant, route


# ------------------------------------------------------------ fp16 semantics
def _all_finite_f16():
    bits = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    v = bits.view(np.float16)
    return v[np.isfinite(v)]


def test_kernel_subtraction_equals_torch_double_rounding_exhaustive():
    """The kernels form t = fp16(q - z) with ONE rounding; torch (and the
    fake-quant weight (Q - zeros) * scales, rtn.py:57-61) computes the
    difference in fp32 and then rounds to fp16.  For every code q in 0..15 and
    every finite fp16 z the two agree bit for bit."""
    z = _all_finite_f16()
    for q in range(16):
        one = (np.float64(q) - z.astype(np.float64)).astype(np.float16)  # exact -> one rounding
        two = fp.h_sub(np.float16(q), z)                                  # fp32 -> fp16
        np.testing.assert_array_equal(one.view(np.uint16), two.view(np.uint16), err_msg=f"q={q}")


def test_oracle_dequant_matches_torch_fp16_arithmetic():
    """oracle.quant.dequant_hqq == torch's fp16 (Q - z) * s on the CPU, for
    every code of 1..4-bit against a broad sample of fp16 (s, z)."""
    rng = np.random.default_rng(0)
    z = _all_finite_f16()
    z = z[np.abs(z.astype(np.float32)) < 64]
    s = rng.choice(_all_finite_f16(), size=z.size)
    s = s[np.isfinite(s)]
    n = min(z.size, s.size)
    z, s = z[:n, None], np.abs(s[:n, None])
    for nbits in (1, 2, 3, 4):
        Q = np.tile(np.arange(1 << nbits, dtype=np.float16), (n, 1))
        ours = quant.dequant_hqq(Q, s, z)
        ref = ((torch.from_numpy(Q) - torch.from_numpy(z)) * torch.from_numpy(s)).numpy()
        np.testing.assert_array_equal(ours.view(np.uint16), ref.view(np.uint16))
        # and the kernel's formulation (q exact, fp16(q - z), fp16(t * s))
        kern = quant.kernel_dequant_hqq(Q.astype(np.uint8), s.T.astype(np.float16), z.T.astype(np.float16),
                                        group_size=1 << nbits)
        np.testing.assert_array_equal(kern.T.view(np.uint16), ref.view(np.uint16))


def test_affine_dequant_single_rounding():
    """fma(q, s, z') rounds once: compare with exact rationals."""
    rng = np.random.default_rng(1)
    s = (rng.standard_normal(300) * 0.02).astype(np.float16)
    zp = (rng.standard_normal(300) * 0.05).astype(np.float16)
    for q in range(16):
        got = quant.dequant_affine(np.full(300, q, np.float16), s, zp)
        for i in range(0, 300, 7):
            exact = Fraction(q) * Fraction(float(s[i])) + Fraction(float(zp[i]))
            cand = np.float16(float(exact))
            lo, hi = np.nextafter(cand, np.float16(-np.inf)), np.nextafter(cand, np.float16(np.inf))
            best = min((lo, cand, hi), key=lambda c: (abs(Fraction(float(c)) - exact),
                                                      int(np.array(c).view(np.uint16)) & 1))
            assert got[i].view(np.uint16) == np.float16(best).view(np.uint16)


# ----------------------------------------------------------------- RTN (A13)
@pytest.mark.parametrize("nbits", [1, 2, 3, 4])
@pytest.mark.parametrize("group_size", [64, 128])
def test_rtn_against_torch_fp16_ops(nbits, group_size):
    """The oracle quantizer equals the reference formula (rtn.py:42-53) run with
    torch's fp16 CPU kernels, i.e. the arithmetic the reference uses."""
    g = torch.Generator().manual_seed(0)
    W = (torch.randn(64, 512, generator=g) * 0.02).half()
    Q, s, z = quant.rtn_quantize(W.numpy(), nbits, group_size)
    Wg = W.reshape(-1, group_size)
    if nbits == 1:
        Qt = torch.where(Wg >= 0, 1, 0).to(Wg.dtype)
        np.testing.assert_array_equal(Q, Qt.numpy())
        assert np.all(z == np.float16(0.5))
        st = (Wg.abs().double().mean(dim=1, keepdim=True).float().half() * 2).numpy()
        np.testing.assert_array_equal(s.view(np.uint16), st.view(np.uint16))
        return
    mx, mn = Wg.amax(dim=1, keepdim=True), Wg.amin(dim=1, keepdim=True)
    max_int = 2 ** nbits - 1
    st = (mx - mn).clamp(min=1e-5) / max_int
    zt = (-torch.round(mn / st)).clamp_(0, max_int)
    Qt = torch.clamp(torch.round(Wg / st) + zt, 0, max_int)
    np.testing.assert_array_equal(s.view(np.uint16), st.numpy().view(np.uint16))
    np.testing.assert_array_equal(z.view(np.uint16), zt.numpy().view(np.uint16))
    np.testing.assert_array_equal(Q.view(np.uint16), Qt.numpy().view(np.uint16))


@pytest.mark.parametrize("nbits", [2, 3, 4])
def test_rtn_recovers_codes_on_exact_grid(nbits):
    """Closed form: a group whose values are (q - z) * s on a power-of-two grid
    spanning the full code range quantizes back to exactly (q, z, s)."""
    rng = np.random.default_rng(nbits)
    max_int = 2 ** nbits - 1
    G, g = 40, 64
    s0 = np.float16(2.0 ** -6)
    z0 = rng.integers(0, max_int + 1, size=(G, 1)).astype(np.float16)
    q0 = rng.integers(0, max_int + 1, size=(G, g))
    q0[:, 0], q0[:, 1] = 0, max_int  # full range -> scale = s0 exactly
    W = ((q0 - z0.astype(np.float64)) * float(s0)).astype(np.float16)
    Q, s, z = quant.rtn_quantize(W, nbits, g)
    assert np.all(s == s0)
    np.testing.assert_array_equal(z, z0)
    np.testing.assert_array_equal(Q, q0.astype(np.float16))


def test_rtn_constant_group_and_bounds():
    """Constant groups take the 1e-5 clamp path (rtn.py:47); codes stay in
    range; non-clamped weights dequantize within half a step."""
    W = np.full((4, 64), 0.01, np.float16)
    Q, s, z = quant.rtn_quantize(W, 2, 64)
    assert np.all(s == fp.h_div(np.float16(1e-5), np.float16(3)))
    rng = np.random.default_rng(3)
    W = (rng.standard_normal((128, 256)) * 0.02).astype(np.float16)
    for b in (2, 3, 4):
        Q, s, z = quant.rtn_quantize(W, b, 64)
        assert Q.min() >= 0 and Q.max() <= 2 ** b - 1 and np.all(Q == np.round(Q))
        Wd = quant.dequant_hqq(Q, s, z).astype(np.float64).reshape(W.shape)
        err = np.abs(Wd - W.astype(np.float64)).reshape(-1, 64)
        assert np.all(err <= s.astype(np.float64) * 0.5 * 1.01 + 2e-4)


# ------------------------------------------------------------- packed layout
@pytest.mark.parametrize("nbits", [1, 2, 3, 4])
def test_pack_single_code_brute_force(nbits):
    """Setting one code to 2^b - 1 lights exactly bits [(k % eps) b, +b) of word
    (k // eps, n) (utils.py:33-71 layout, read at dequant_group_gemm.py:118)."""
    eps = 32 // nbits
    N, K = 3, 2 * eps + 3  # ragged tail
    for n, k in itertools.product(range(N), range(K)):
        codes = np.zeros((N, K), np.uint8)
        codes[n, k] = (1 << nbits) - 1
        w = quant.pack_cols(codes, nbits).view(np.uint32)
        assert w.shape == (-(-K // eps), N)
        expect = np.zeros_like(w)
        expect[k // eps, n] = ((1 << nbits) - 1) << ((k % eps) * nbits)
        np.testing.assert_array_equal(w, expect)
    if nbits == 3:  # dead bits 30..31 stay clear
        full = np.full((N, K), 7, np.uint8)
        assert np.all(quant.pack_cols(full, 3).view(np.uint32) >> 30 == 0)


@pytest.mark.parametrize("nbits", [1, 2, 3, 4])
def test_pack_unpack_round_trip(nbits):
    rng = np.random.default_rng(nbits)
    codes = rng.integers(0, 1 << nbits, size=(48, 640)).astype(np.uint8)
    np.testing.assert_array_equal(quant.unpack_cols(quant.pack_cols(codes, nbits), nbits, 640), codes)


@pytest.mark.parametrize("nbits", [1, 2, 3, 4])
def test_build_layout_round_trip_and_bit_positions(nbits):
    rng = np.random.default_rng(10 + nbits)
    N, K = 32, 256
    codes = rng.integers(0, 1 << nbits, size=(N, K)).astype(np.uint8)
    words = quant.repack_build(codes, nbits)
    assert words.shape == (N // 16, K // 128, 16, 4, nbits)
    np.testing.assert_array_equal(quant.unpack_build(words, nbits, N, K), codes)
    # single code: k = 128 c + 32 kb + 8 t + 2 d + h of column n lands in half h
    # of one word of panel n // 16, row n % 16
    for n, k in ((5, 0), (5, 1), (21, 9), (5, 37), (30, 127), (16, 200)):
        one = np.zeros((N, K), np.uint8)
        one[n, k] = 1
        w = quant.repack_build(one, nbits)
        c, kb, i = k // 128, (k % 128) // 32, k % 32
        t, d, h = i // 8, (i % 8) // 2, i % 2
        nz = np.argwhere(w)
        assert len(nz) == 1 and tuple(nz[0][:4]) == (n // 16, c, n % 16, kb)
        # flat word index as the kernels address it
        flat = np.flatnonzero(w.reshape(-1))[0]
        assert flat // nbits == ((n // 16 * (K // 128) + c) * 64 + (n % 16) * 4 + kb)
        bit = int(np.log2(int(w[tuple(nz[0])])))
        assert (bit >= 16) == bool(h)
        pos = {4: 4 * d, 2: 2 * (4 * (t % 2) + d), 1: 4 * t + d, 3: 2 * (4 * (t % 2) + d)}[nbits]
        assert bit - 16 * h == pos


def test_prep_scales_panel_order_and_values():
    """Pair (g, n) lands at dword (n // 16 * G + g) * 16 + n % 16, holding
    fp16 s in the low half and the mode's zero term in the high half."""
    rng = np.random.default_rng(3)
    G, N = 6, 48
    s = (rng.standard_normal((G, N)) * 0.01).astype(np.float16)
    z = rng.integers(0, 16, size=(G, N)).astype(np.float16)
    for mode, zterm in ((0, -z), (1, z), (2, -(1024.0 + z.astype(np.float64)))):
        flat = quant.prep_scales(s, z, mode).reshape(-1)
        for g, n in ((0, 0), (5, 47), (2, 17), (3, 31), (1, 16)):
            v = int(flat[(n // 16 * G + g) * 16 + n % 16])
            assert np.uint16(v & 0xFFFF) == s[g, n].view(np.uint16)
            assert np.uint16(v >> 16) == np.float16(zterm[g, n]).view(np.uint16)


# ----------------------------------------------------------------- routing
def test_router_logits_exact_on_integer_inputs():
    """With small integer inputs every partial sum is exact, so any summation
    order gives the exact dot product."""
    rng = np.random.default_rng(0)
    x = rng.integers(-8, 9, size=(5, 1024)).astype(np.float32)
    w = rng.integers(-8, 9, size=(12, 1024)).astype(np.float32)
    got = route.router_logits_fixed(x, w)
    np.testing.assert_array_equal(got, (x.astype(np.int64) @ w.T.astype(np.int64)).astype(np.float32))


def test_router_logits_one_hot_selects_column():
    rng = np.random.default_rng(1)
    w = rng.standard_normal((7, 2048)).astype(np.float32)
    x = np.zeros((3, 2048), np.float32)
    x[0, 5], x[1, 2047], x[2, 1000] = 1.0, 1.0, 1.0
    got = route.router_logits_fixed(x, w)
    np.testing.assert_array_equal(got, w[:, [5, 2047, 1000]].T)


def test_router_logits_error_bound_vs_exact():
    """|fixed-order fp32 - exact| <= gamma_n * sum |x w| for a length-H dot
    product (Higham); a dropped or repeated term would break it."""
    rng = np.random.default_rng(2)
    H = 1536  # not a multiple of 512: exercises the ragged last chunk
    x = rng.standard_normal((2, H)).astype(np.float16).astype(np.float32)
    w = (rng.standard_normal((3, H)) * 0.02).astype(np.float16).astype(np.float32)
    got = route.router_logits_fixed(x, w)
    u = 2.0 ** -24
    gamma = (H + 6) * u / (1 - (H + 6) * u)
    for t in range(2):
        for e in range(3):
            exact = sum(Fraction(float(a)) * Fraction(float(b)) for a, b in zip(x[t], w[e]))
            bound = gamma * float(np.sum(np.abs(x[t].astype(np.float64) * w[e])))
            assert abs(float(got[t, e]) - float(exact)) <= bound


def test_topk_brute_force_and_softmax():
    import scipy.special
    rng = np.random.default_rng(3)
    E, k = 6, 3
    lg = rng.integers(-3, 4, size=(200, E)).astype(np.float32)  # many ties
    idx, w = route.topk_route(lg, k, norm_topk=False)
    p = scipy.special.softmax(lg.astype(np.float64), axis=1)
    for t in range(lg.shape[0]):
        # the chosen set: k largest logits, ties broken towards lower index
        order = sorted(range(E), key=lambda e: (-lg[t, e], e))[:k]
        assert list(idx[t]) == order
        np.testing.assert_allclose(w[t], p[t, order], rtol=1e-6)
    _, wn = route.topk_route(lg, k, norm_topk=True)
    np.testing.assert_allclose(wn.sum(axis=1), 1.0, rtol=1e-6)


@pytest.mark.parametrize("dtype,tdt", [("bf16", torch.bfloat16), ("f16", torch.float16)])
def test_act_softmax_router_matches_torch_ops(dtype, tdt):
    """topk_route_act_softmax against torch's own CPU ops running the lines of
    Mixtral's forward_one_token (moe_block.py:281-283) on 16-bit scores.
    Probabilities and weights must agree bit for bit, and the selection
    wherever the k-th and (k+1)-th rounded probabilities differ (torch's tie
    order is unspecified).  Ranking logits instead of rounded probabilities,
    renormalising in fp32 or skipping the rounding of the sum each fail this:
    with 8 experts about one token in a hundred has a tie at the top-2
    boundary, and the sum's rounding changes most weights."""
    import torch.nn.functional as F
    rng = np.random.default_rng(11)
    T, E, k = 20000, 8, 2
    lg = route.round_to(rng.normal(0, 0.7, size=(T, E)).astype(np.float32), dtype)
    idx, w, p, fragile = route.topk_route_act_softmax(lg, k, dtype)
    scores = torch.from_numpy(lg).to(tdt)
    tp = F.softmax(scores, dim=-1)
    tw, ti = torch.topk(tp, k, dim=-1)
    tw /= tw.sum(dim=-1, keepdim=True)
    # probabilities differ only where an fp32 value sits on a rounding midpoint
    differ = (p != tp.float().numpy()).any(1)
    assert not (differ & ~fragile).any() and fragile.mean() < 2e-2, (differ.sum(), fragile.sum())
    keep = ~fragile
    idx, w, p, lg, tw, ti = idx[keep], w[keep], p[keep], lg[keep], tw[keep], ti[keep]
    srt = -np.sort(-p, axis=1)
    untied = srt[:, k - 1] != srt[:, k]
    ties = int((~untied).sum())
    assert (50 if dtype == "bf16" else 10) < ties < 1000, ties  # the sample does exercise the tie rule
    np.testing.assert_array_equal(np.sort(idx[untied], 1), np.sort(ti.numpy()[untied], 1))
    distinct = untied & (np.diff(srt[:, :k + 1], axis=1) != 0).all(1)  # no tie inside the top k either
    np.testing.assert_array_equal(idx[distinct], ti.numpy()[distinct])
    # where tied, both selections hold the same values, so the weights agree
    np.testing.assert_array_equal(w.view(np.uint32), tw.float().numpy().view(np.uint32))
    order = np.argsort(-p, axis=1, kind="stable")[:, :k]
    np.testing.assert_array_equal(idx, order)  # equal values: lower index first
    # the rounded sum differs from the fp32 one often enough to matter
    w32 = np.take_along_axis(p, idx.astype(np.int64), 1)
    w32 = route.round_to((w32 / w32.sum(1, keepdims=True)).astype(np.float32), dtype)
    assert (w32 != w).any()
    assert np.array_equal(idx, route.topk_route(lg, k, True)[0]) is False


def test_permute_matches_reference_loop():
    rng = np.random.default_rng(4)
    for T, k, E in ((1, 1, 1), (1, 8, 64), (37, 2, 8), (256, 8, 64), (300, 6, 64)):
        idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
        p = route.permute(idx, E)
        np.testing.assert_array_equal(p["row_pair"], route.permute_loop(idx, E))
        np.testing.assert_array_equal(np.sort(p["row_pair"]), np.arange(T * k))
        np.testing.assert_array_equal(p["inv_perm"][p["row_pair"]], np.arange(T * k))
        assert p["counts"].sum() == T * k and p["offsets"][-1] == T * k
        for e in range(E):
            lo, hi = p["offsets"][e], p["offsets"][e + 1]
            assert np.all(idx.reshape(-1)[p["row_pair"][lo:hi]] == e)
        np.testing.assert_array_equal(p["row_token"], p["row_pair"] // k)


# ------------------------------------------------------------- expert loop
def _rand_experts(rng, E, H, F):
    W1 = [(rng.standard_normal((F, H)) * 0.05).astype(np.float32) for _ in range(E)]
    W3 = [(rng.standard_normal((F, H)) * 0.05).astype(np.float32) for _ in range(E)]
    W2 = [(rng.standard_normal((H, F)) * 0.05).astype(np.float32) for _ in range(E)]
    return W1, W3, W2


def test_moe_loop_equals_dense_einsum_formulation():
    rng = np.random.default_rng(5)
    T, H, F, E, k = 23, 64, 48, 6, 2
    W1, W3, W2 = _rand_experts(rng, E, H, F)
    x = rng.standard_normal((T, H)).astype(np.float32)
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    w = rng.random((T, k)).astype(np.float32)
    a = moe.moe_from_routing(x, idx, w, W1, W3, W2)
    b = moe.moe_dense_einsum(x, idx, w, W1, W3, W2)
    np.testing.assert_allclose(a, b, rtol=2e-5, atol=2e-6)


def test_moe_single_expert_is_one_dense_mlp():
    """All tokens on one expert with weight one: a single SwiGLU MLP written
    with torch.matmul (library routine)."""
    rng = np.random.default_rng(6)
    T, H, F, E = 31, 64, 32, 4
    W1, W3, W2 = _rand_experts(rng, E, H, F)
    x = rng.standard_normal((T, H)).astype(np.float32)
    idx = np.full((T, 1), 2, np.int32)
    w = np.ones((T, 1), np.float32)
    out = moe.moe_from_routing(x, idx, w, W1, W3, W2)
    xt = torch.from_numpy(x)
    ref = torch.matmul(torch.nn.functional.silu(xt @ torch.from_numpy(W1[2]).T) * (xt @ torch.from_numpy(W3[2]).T),
                       torch.from_numpy(W2[2]).T)
    np.testing.assert_allclose(out, ref.numpy(), rtol=2e-5, atol=2e-6)


def test_moe_k_equals_e_is_dense_mixture():
    rng = np.random.default_rng(7)
    T, H, F, E = 9, 32, 16, 3
    W1, W3, W2 = _rand_experts(rng, E, H, F)
    x = rng.standard_normal((T, H)).astype(np.float32)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    idx, w = route.topk_route(lg, E, norm_topk=False)
    out = moe.moe_from_routing(x, idx, w, W1, W3, W2)
    import scipy.special
    p = scipy.special.softmax(lg.astype(np.float64), axis=1)
    ref = sum(p[:, [e]] * moe.expert_mlp(x, W1[e], W3[e], W2[e]) for e in range(E))
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-6)
