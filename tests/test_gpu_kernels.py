"""GPU parity of each stage of the HIP path against the CPU oracle.

Integer / index outputs (packed words, routing indices, the permutation, tile
schedule) must match bit for bit; router logits too (same pinned fp32 order);
fp results (routing weights, GEMMs) within stated tolerances.
"""

import numpy as np
import pytest
import torch

from conftest import relative_error, to_np
from oracle import quant as oq
from oracle import route as orr

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


# ----------------------------------------------------------------- layouts
@pytest.mark.parametrize("nbits", [1, 2, 3, 4])
def test_pack_and_repack_bit_exact(device, nbits):
    from robustgemq_amd import ops
    from robustgemq_amd.experts import QuantProjection
    _say(f"[pack/repack] nbits={nbits}")
    rng = np.random.default_rng(nbits)
    N, K = 96, 640  # K not a multiple of eps for 3-bit: exercises the tail
    codes = rng.integers(0, 1 << nbits, size=(N, K)).astype(np.uint8)
    words, eps = ops.pack_weights_over_cols(torch.from_numpy(codes).to(device), nbits)
    assert eps == 32 // nbits
    np.testing.assert_array_equal(to_np(words).view(np.uint32), oq.pack_cols(codes, nbits).view(np.uint32))
    back = ops.unpack_words(words, nbits, K)
    np.testing.assert_array_equal(to_np(back), codes)
    # build layout through QuantProjection (moeq_repack + moeq_prep_scales)
    G = K // 64
    s = (rng.standard_normal((G, N)) * 0.01).astype(np.float16)
    z = rng.integers(0, 1 << nbits, size=(G, N)).astype(np.float16)
    Kb = 512
    Gb = Kb // 64
    codes_b = codes[:, :Kb]
    wb, _ = ops.pack_weights_over_cols(torch.from_numpy(codes_b).to(device), nbits)
    # a second expert of other bits: each expert's block at its own offset
    bits2 = nbits % 4 + 1
    codes2 = rng.integers(0, 1 << bits2, size=(N, Kb)).astype(np.uint8)
    w2, _ = ops.pack_weights_over_cols(torch.from_numpy(codes2).to(device), bits2)
    s2 = (rng.standard_normal((Gb, N)) * 0.01).astype(np.float16)
    z2 = rng.integers(0, 1 << bits2, size=(Gb, N)).astype(np.float16)
    for zz, zz2, want_mode in ((z, z2, 2), (z + np.float16(0.25), z2, 0)):  # integer zeros: the integer mode
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)
        proj = QuantProjection([wb, w2], [t(s[:Gb]), t(s2)], [t(zz[:Gb]), t(zz2)], [nbits, bits2], Kb, N, 64, 0)
        assert proj.dq_mode == want_mode
        words = to_np(proj.words).view(np.uint32)
        n0 = N * Kb * nbits // 32
        np.testing.assert_array_equal(words[:n0].reshape(N // 16, Kb // 128, 16, 4, nbits),
                                      oq.repack_build(codes_b, nbits))
        np.testing.assert_array_equal(words[n0:].reshape(N // 16, Kb // 128, 16, 4, bits2),
                                      oq.repack_build(codes2, bits2))
        sz = to_np(proj.sz).view(np.uint32)
        np.testing.assert_array_equal(sz[:Gb * N].reshape(N // 16, Gb, 16),
                                      oq.prep_scales(s[:Gb], zz[:Gb], want_mode))
        np.testing.assert_array_equal(sz[Gb * N:].reshape(N // 16, Gb, 16),
                                      oq.prep_scales(s2, zz2, want_mode))


# ------------------------------------------------------------------ routing
@pytest.mark.parametrize("gate", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("T,H,E,k,norm", [(1, 2048, 64, 8, False), (333, 2048, 64, 8, False),
                                         (2048, 2048, 64, 8, False),
                                         (257, 2048, 128, 8, True), (64, 4096, 8, 2, True),
                                         (40, 1536, 64, 6, False), (16, 512, 8, 2, False),
                                         (300, 1000, 60, 4, True), (130, 768, 256, 8, False),
                                         (2100, 2560, 8, 2, True)])
def test_route_bit_exact(device, gate, T, H, E, k, norm):
    from robustgemq_amd import ops
    _say(f"[route] gate={gate} T={T} H={H} E={E} k={k}")
    g = torch.Generator().manual_seed(T + H + E)
    act = torch.bfloat16 if gate == "bf16" else torch.float16
    x = torch.randn(T, H, generator=g).to(act)
    wg = (torch.randn(E, H, generator=g) * 0.02).to(act)
    gw = wg.float() if gate == "f32" else wg
    lg, idx, w = ops.route(x.to(device), gw.to(device), k, norm)
    x32 = x.float().numpy()
    ref_lg = orr.router_logits(x32, wg.float().numpy(), gate)
    np.testing.assert_array_equal(lg.float().cpu().numpy().view(np.uint32), ref_lg.view(np.uint32))
    ref_idx, ref_w = orr.topk_route(ref_lg, k, norm)
    np.testing.assert_array_equal(to_np(idx), ref_idx)
    np.testing.assert_allclose(to_np(w), ref_w, rtol=2e-6, atol=1e-7)
    # same selection from the logits alone
    idx2, w2 = ops.route_from_logits(lg, k, norm)
    np.testing.assert_array_equal(to_np(idx2), ref_idx)
    np.testing.assert_allclose(to_np(w2), ref_w, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("T,H,E,k", [(1, 1024, 64, 6), (300, 1024, 64, 6), (2100, 2560, 8, 2)])
def test_route_fp32_activations(device, T, H, E, k):
    """fp32 activations with an fp32 gate, logits kept in fp32: T = 1 through
    logits_kernel, the others (T * E > 16384) through logits_topk_kernel,
    which reads fp32 rows straight from global memory (16-bit rows are
    staged in LDS)."""
    from robustgemq_amd import ops
    _say(f"[route] fp32 x T={T} H={H} E={E} k={k}")
    g = torch.Generator().manual_seed(T * 3 + E)
    x = torch.randn(T, H, generator=g)
    wg = torch.randn(E, H, generator=g) * 0.02
    lg, idx, w = ops.route(x.to(device), wg.to(device), k, True)
    ref_lg = orr.router_logits(x.numpy(), wg.numpy(), "f32")
    np.testing.assert_array_equal(lg.float().cpu().numpy().view(np.uint32), ref_lg.view(np.uint32))
    ref_idx, ref_w = orr.topk_route(ref_lg, k, True)
    np.testing.assert_array_equal(to_np(idx), ref_idx)
    np.testing.assert_allclose(to_np(w), ref_w, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("E,k", [(8, 2), (64, 8), (96, 16), (300, 6)])
def test_topk_special_values_and_ties(device, E, k):
    """Selection order on hand-made logit rows: a stable descending sort
    (equal values, +0 and -0 included, in index order), NaN ranked as -inf
    (after every finite value; equal to -inf, so in index order), +inf first.  Rows mix these with coarse values (many
    exact ties) and fine ones; E = 96 and 300 leave part of the last lane
    register empty."""
    from robustgemq_amd import ops
    _say(f"[topk] special values E={E} k={k}")
    rng = np.random.default_rng(E * 31 + k)
    T = 64
    lg = rng.integers(-3, 4, size=(T, E)).astype(np.float32) * 0.5  # many ties
    lg[1::4] = rng.standard_normal((len(range(1, T, 4)), E)).astype(np.float32)
    lg[2, :] = 0.0
    lg[2, ::3] = -0.0
    lg[3, :] = -np.inf
    for t in range(4, T, 5):  # NaN / -inf holes, at least k finite values left
        holes = rng.choice(E, size=E - k, replace=False)
        lg[t, holes[: len(holes) // 2]] = np.nan
        lg[t, holes[len(holes) // 2:]] = -np.inf
    lg[5, rng.choice(E, size=min(k, 2), replace=False)] = np.inf
    with np.errstate(invalid="ignore"):  # rows 3 and 5: non-finite weights, not compared
        ref_idx, ref_w = orr.topk_route(np.where(np.isnan(lg), -np.inf, lg), k, True)
    idx, w = ops.route_from_logits(torch.from_numpy(lg).to(device), k, True)
    np.testing.assert_array_equal(to_np(idx), ref_idx)
    finite = np.isfinite(ref_w).all(axis=1)
    np.testing.assert_allclose(to_np(w)[finite], ref_w[finite], rtol=2e-6, atol=1e-7)
    assert (to_np(idx)[3] == np.arange(k)).all()  # all -inf: index order


def test_route_bias_and_ties(device):
    from robustgemq_amd import ops
    _say("[route] bias + ties")
    T, H, E, k = 50, 512, 16, 4
    x = torch.zeros(T, H, dtype=torch.float16)
    wg = torch.zeros(E, H, dtype=torch.float16)
    bias = torch.tensor([0.5 if e % 3 == 0 else 0.0 for e in range(E)], dtype=torch.float32)
    lg, idx, w = ops.route(x.to(device), wg.float().to(device), k, True, logit_bias=bias.to(device))
    # all-zero logits plus bias: experts 0, 3, 6, 9 tie at 0.5 and win in index order
    assert (to_np(idx) == np.array([0, 3, 6, 9])).all()
    np.testing.assert_allclose(to_np(w), 0.25, rtol=1e-6)


@pytest.mark.parametrize("T,k,E,S,bm", [(1, 8, 64, 0, 16), (1, 6, 64, 2, 16), (700, 2, 8, 0, 64),
                                        (2048, 8, 64, 0, 128), (4096, 8, 128, 0, 128),
                                        (300, 6, 64, 2, 32), (5000, 1, 3, 0, 128), (5000, 8, 64, 2, 128),
                                        (9000, 8, 64, 0, 128), (3000, 4, 300, 0, 64),
                                        (128, 8, 64, 0, 64), (129, 8, 64, 0, 64), (512, 8, 64, 0, 64)])
def test_permute_bit_exact(device, T, k, E, S, bm):
    from robustgemq_amd import ops
    _say(f"[permute] T={T} k={k} E={E} shared={S} bm={bm}")
    rng = np.random.default_rng(T * 7 + E)
    p = np.exp(-2.0 * rng.random(E))
    p /= p.sum()
    idx = np.stack([rng.choice(E, size=k, replace=False, p=p) for _ in range(T)]).astype(np.int32)
    out = ops.permute(torch.from_numpy(idx).to(device), E, n_shared=S, bm=bm)
    ref = orr.permute(idx, E, n_shared=S)
    for key in ("counts", "offsets", "row_token", "row_pair", "inv_perm"):
        np.testing.assert_array_equal(to_np(out[key]), ref[key], err_msg=key)
    # tile schedule: covers each expert's rows exactly once, <= bm rows, in order
    nt = int(to_np(out["n_tiles"])[0])
    assert 0 < nt <= out["max_tiles"]
    tiles = to_np(out["tiles"])[:nt]
    covered = np.zeros(T * k + S * T, np.int32)
    cap = ops.L.lib().moeq_tile_rows(bm)
    for e, r0, rc, _ in tiles:
        assert 0 < rc <= cap
        assert ref["offsets"][e] <= r0 and r0 + rc <= ref["offsets"][e + 1]
        covered[r0:r0 + rc] += 1
    assert (covered == 1).all()
    # each expert's m rows in ceil(m / cap) tiles cut at 16-row boundaries,
    # as the host-side restatement split_rows cuts them
    from robustgemq_amd.linear import split_rows
    sizes = {}
    for e, r0, rc, _ in tiles:
        sizes.setdefault(int(e), []).append((int(r0 - ref["offsets"][e]), int(rc)))
    for e, m in enumerate(ref["counts"]):
        got = sizes.get(e, [])
        assert len(got) == -(-int(m) // cap), (e, m, got)
        assert got == (split_rows(int(m), bm) if m else []), (e, m, got)


# ------------------------------------------------------------- grouped GEMM
def _make_proj(device, rng, E, K, N, bits, g, mode):
    """mode: 'int' (integer HQQ zeros), 'frac' (fractional HQQ zeros, as GPTQ
    checkpoints have) or 'affine' (GemLite zeros z' = -z*s)."""
    from robustgemq_amd import _lib as L
    from robustgemq_amd.experts import QuantProjection, pack_codes
    codes, s_l, z_l, words = [], [], [], []
    for e in range(E):
        b = bits[e]
        c = rng.integers(0, 1 << b, size=(N, K)).astype(np.uint8)
        s = (np.abs(rng.standard_normal((K // g, N))) * 0.01 + 1e-3).astype(np.float16)
        if mode == "int":
            z = rng.integers(0, 1 << b, size=(K // g, N)).astype(np.float16)
        elif mode == "frac":
            z = (rng.random((K // g, N)) * ((1 << b) - 1)).astype(np.float16)
        else:
            z = (rng.standard_normal((K // g, N)) * 0.02).astype(np.float16)
        codes.append(c)
        s_l.append(s)
        z_l.append(z)
        words.append(pack_codes(torch.from_numpy(c).to(device), b))
    proj = QuantProjection(words, [torch.from_numpy(s).to(device) for s in s_l],
                           [torch.from_numpy(z).to(device) for z in z_l], bits, K, N, g,
                           L.DQ_AFFINE if mode == "affine" else L.DQ_HQQ)
    assert proj.dq_mode == {"int": L.DQ_HQQ_INT, "frac": L.DQ_HQQ, "affine": L.DQ_AFFINE}[mode]
    dense = []
    for c, s, z in zip(codes, s_l, z_l):
        if mode != "affine":
            W = oq.kernel_dequant_hqq(c, s, z, g)  # [K, N] fp16, == fake-quant weight
        else:
            gi = np.arange(K) // g
            W = oq.dequant_affine(c.T.astype(np.float16), s[gi, :], z[gi, :])
        dense.append(W.astype(np.float32))
    return proj, dense


@pytest.mark.parametrize("bm", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("mode", ["int", "frac", "affine"])
@pytest.mark.parametrize("g", [64, 128])
def test_grouped_gemm_store_matches_fp32(device, bm, mode, g):
    from robustgemq_amd import ops
    _say(f"[gemm/store] bm={bm} mode={mode} g={g}")
    rng = np.random.default_rng(bm + 10 * len(mode) + g)
    E, K, N = 5, 384, 160  # N not a multiple of the column tile
    bits = [1, 2, 3, 4, 2]
    proj, dense = _make_proj(device, rng, E, K, N, bits, g, mode)
    counts = [bm * 2 + 3, 1, 0, 17, bm - 5]
    rows = sum(counts)
    T = 61
    x = (rng.standard_normal((T, K)) * 0.5).astype(np.float16)
    row_src = rng.integers(0, T, size=rows).astype(np.int32)
    cap = ops.L.lib().moeq_tile_rows(bm)  # tiles as tall as the class holds
    tiles, r = [], 0
    for e, m in enumerate(counts):
        for j in range(0, m, cap):
            tiles.append((e, r + j, min(cap, m - j), 0))
        r += m
    tt = torch.tensor(tiles, dtype=torch.int32, device=device)
    n = torch.tensor([len(tiles)], dtype=torch.int32, device=device)
    out = ops.grouped_gemm(torch.from_numpy(x).to(device), rows, N, tt, n, len(tiles) + 3, bm, proj,
                           row_src=torch.from_numpy(row_src).to(device), out_dtype=torch.float32)
    ref = np.zeros((rows, N), np.float32)
    r = 0
    for e, m in enumerate(counts):
        ref[r:r + m] = x[row_src[r:r + m]].astype(np.float32) @ dense[e]
        r += m
    got = to_np(out)
    assert relative_error(got, ref) < 2e-6
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("K", [384, 1024, 1536, 3072, 5120])
def test_grouped_gemm_decode_k_split_depths(device, K):
    """16-row launches with few column blocks split K over the waves: one,
    two, up to four, up to eight chunks per wave fetched at once, and the
    4-deep ring beyond that; rows of 1..16 tokens and a zero-row expert."""
    from robustgemq_amd import ops
    _say(f"[gemm/decode k-split] K={K}")
    rng = np.random.default_rng(K)
    E, N = 4, 96
    bits = [2, 3, 4, 1]
    proj, dense = _make_proj(device, rng, E, K, N, bits, 64, "int")
    counts = [1, 16, 0, 5]
    rows = sum(counts)
    x = (rng.standard_normal((rows, K)) * 0.5).astype(np.float16)
    tiles, r = [], 0
    for e, m in enumerate(counts):
        for j in range(0, m, 16):
            tiles.append((e, r + j, min(16, m - j), 0))
        r += m
    tt = torch.tensor(tiles, dtype=torch.int32, device=device)
    n = torch.tensor([len(tiles)], dtype=torch.int32, device=device)
    out = ops.grouped_gemm(torch.from_numpy(x).to(device), rows, N, tt, n, len(tiles), 16, proj,
                           out_dtype=torch.float32)
    got = to_np(out)
    r = 0
    for e, m in enumerate(counts):
        ref = x[r:r + m].astype(np.float32) @ dense[e]
        np.testing.assert_allclose(got[r:r + m], ref, rtol=1e-4, atol=1e-4)
        r += m


@pytest.mark.parametrize("bm", [16, 128, 256])
@pytest.mark.parametrize("adt", [torch.float16, torch.bfloat16])
def test_grouped_gemm_silu_mul_and_splitk(device, bm, adt):
    from robustgemq_amd import ops
    _say(f"[gemm/silu+splitk] bm={bm} act={adt}")
    rng = np.random.default_rng(bm)
    E, K, N = 3, 512, 256
    bits = [2, 3, 4]
    p1, d1 = _make_proj(device, rng, E, K, N, bits, 64, "int")
    p3, d3 = _make_proj(device, rng, E, K, N, bits, 64, "int")
    counts = [40, 7, 130]
    rows = sum(counts)
    x = torch.from_numpy((rng.standard_normal((rows, K)) * 0.5).astype(np.float32)).to(adt)
    cap = ops.L.lib().moeq_tile_rows(bm)  # tiles as tall as the class holds
    tiles, r = [], 0
    for e, m in enumerate(counts):
        for j in range(0, m, cap):
            tiles.append((e, r + j, min(cap, m - j), 0))
        r += m
    tt = torch.tensor(tiles, dtype=torch.int32, device=device)
    n = torch.tensor([len(tiles)], dtype=torch.int32, device=device)
    h = ops.grouped_gemm(x.to(device), rows, N, tt, n, len(tiles), bm, p1, p1=p3)
    x32 = x.float().numpy()
    ref = np.zeros((rows, N), np.float32)
    r = 0
    for e, m in enumerate(counts):
        g_ = x32[r:r + m] @ d1[e]
        u = x32[r:r + m] @ d3[e]
        ref[r:r + m] = g_ / (1 + np.exp(-g_)) * u
        r += m
    assert relative_error(to_np(h).astype(np.float32), ref) < 1e-3
    # split-K store of the same first projection
    y = ops.grouped_gemm(x.to(device), rows, N, tt, n, len(tiles), bm, p1, out_dtype=torch.float32, splits=3)
    assert tuple(y.shape) == (3, rows, N)
    ys = to_np(y).sum(axis=0)
    r = 0
    for e, m in enumerate(counts):
        np.testing.assert_allclose(ys[r:r + m], x32[r:r + m] @ d1[e], rtol=1e-4, atol=1e-4)
        r += m


def test_combine_deterministic_order(device):
    from robustgemq_amd import ops
    _say("[combine]")
    rng = np.random.default_rng(0)
    T, k, S, H = 37, 3, 2, 256
    rows = T * k + S * T
    y = rng.standard_normal((2, rows, H)).astype(np.float32)
    perm = rng.permutation(T * k).astype(np.int32)
    w = rng.random((T, k)).astype(np.float32)
    out = ops.combine(torch.from_numpy(y).to(device), torch.from_numpy(perm).to(device),
                      torch.from_numpy(w).to(device), T, k, S, torch.float32)
    ys = y.sum(axis=0)
    ref = np.zeros((T, H), np.float32)
    for t in range(T):
        for s in range(k):
            ref[t] += w[t, s] * ys[perm[t * k + s]]
        for v in range(S):
            ref[t] += ys[T * k + v * T + t]
    np.testing.assert_allclose(to_np(out), ref, rtol=1e-5, atol=1e-5)
