"""Whole-layer parity of QuantFused*MoEBlock on the GPU against the oracle.

Bar: routing and permutation bit-exact; outputs within
max-abs 1e-2 and relative-L2 1e-3 of the fp32 reference (the oracle's
dequantize-then-matmul loop).  For bf16 activations the fp32 pre-cast output
is compared at that bar, and the bf16 output is checked against the fp32
reference at bf16 resolution (rel-L2 1e-2, since bf16 rounding alone is
~2e-3).
"""

import numpy as np
import pytest
import torch

from conftest import relative_error, to_np
from oracle import moe as om
from oracle import quant as oq
from oracle import route as orr

pytestmark = pytest.mark.gpu

MAX_ABS = 1e-2
REL_L2 = 1e-3


def _say(msg):
    print(msg, flush=True)


_CACHE = {}


def _layer(name, seed=0):
    """(cfg, weights (CPU), block (GPU), oracle dense weights) -- cached."""
    from robustgemq_amd.synthetic import CONFIGS, build_block, make_weights
    key = (name, seed)
    if key not in _CACHE:
        cfg = CONFIGS[name]
        w = make_weights(cfg, seed=seed)
        block = build_block(cfg, w, device="cuda")

        def dense(t):
            N, K = t.shape
            return oq.dequant_hqq(t.Q.numpy(), t.scales.numpy(), t.zeros.numpy()).reshape(N, K).astype(np.float32)

        W1 = [dense(e["gate_proj"]) for e in w["experts"]]
        W3 = [dense(e["up_proj"]) for e in w["experts"]]
        W2 = [dense(e["down_proj"]) for e in w["experts"]]
        shared = ()
        if w["shared"] is not None:
            shared = ((dense(w["shared"]["gate_proj"]), dense(w["shared"]["up_proj"]),
                       dense(w["shared"]["down_proj"])),)
        _CACHE.clear()
        _CACHE[key] = (cfg, w, block, (W1, W3, W2, shared))
    return _CACHE[key]


def _oracle(cfg, w, dense, x):
    W1, W3, W2, shared = dense
    gate = w["gate"].float().numpy()
    ldt = "f32" if cfg.family == "deepseekv2" else ("bf16" if cfg.act_dtype == torch.bfloat16 else "f16")
    if cfg.family != "deepseekv2" and cfg.act_dtype == torch.bfloat16:
        gate = w["gate"].to(torch.bfloat16).float().numpy()
    bias = None if w["bias"] is None else w["bias"].numpy()
    return om.moe_forward(x.float().numpy(), gate, ldt, cfg.top_k,
                          cfg.norm_topk or cfg.family == "mixtral", W1, W3, W2, shared, bias=bias)


def _check(cfg, block, w, dense, T, seed=5):
    from robustgemq_amd.synthetic import make_inputs
    x = make_inputs(cfg, T, seed=seed)
    ref, ref_lg, ref_idx, ref_w = _oracle(cfg, w, dense, x)
    xd = x.to("cuda")
    layer = block._layer
    # routing bit-exact: logits and the selected experts
    from robustgemq_amd import ops
    lg, idx, wt = ops.route(xd, layer.gate_w, layer.top_k, layer.norm_topk, logit_bias=layer.logit_bias)
    np.testing.assert_array_equal(lg.float().cpu().numpy().view(np.uint32), ref_lg.view(np.uint32))
    np.testing.assert_array_equal(to_np(idx), ref_idx)
    perm = ops.permute(idx, layer.n_experts, layer.n_shared)
    ref_perm = orr.permute(ref_idx, layer.n_experts, layer.n_shared)
    for key in ("counts", "offsets", "row_token", "row_pair", "inv_perm"):
        np.testing.assert_array_equal(to_np(perm[key]), ref_perm[key], err_msg=key)
    # outputs: fp32 pre-cast and activation dtype
    out32, _ = layer.forward(xd, out_dtype=torch.float32, want_logits=False)
    got32 = to_np(out32)
    err = relative_error(got32, ref)
    mx = float(np.abs(got32 - ref).max())
    _say(f"    {cfg.name} T={T}: rel-L2 {err:.3e} max-abs {mx:.3e} (|ref|max {np.abs(ref).max():.3e})")
    assert err <= REL_L2 and mx <= MAX_ABS
    out = block(xd.reshape(1, T, -1))
    out = out[0] if isinstance(out, tuple) else out
    got = to_np(out.reshape(T, -1)).astype(np.float32)
    if cfg.act_dtype == torch.float16:
        assert relative_error(got, ref) <= REL_L2 and float(np.abs(got - ref).max()) <= MAX_ABS
    else:
        assert relative_error(got, ref) <= 1e-2 and float(np.abs(got - ref).max()) <= MAX_ABS
    return got32


@pytest.mark.parametrize("name,T", [("ref_test", 16), ("ref_test", 1), ("olmoe_2bit", 128),
                                    ("olmoe_mixed", 512), ("olmoe_mixed", 1), ("olmoe_mixed", 8),
                                    ("olmoe_mixed", 32)])
def test_layer_matches_oracle_olmoe(device, name, T):
    _say(f"[layer] {name} T={T}")
    cfg, w, block, dense = _layer(name)
    _check(cfg, block, w, dense, T)


@pytest.mark.parametrize("T", [1, 64, 512])
def test_layer_matches_oracle_qwen3_bf16(device, T):
    _say(f"[layer] qwen3_mixed T={T}")
    cfg, w, block, dense = _layer("qwen3_mixed")
    _check(cfg, block, w, dense, T)


@pytest.mark.parametrize("T", [1, 16, 64, 300])
def test_layer_matches_oracle_mixtral_bf16(device, T):
    """Mixtral family: top-2 always renormalised (moe_block.py:245-249), w1/w3/w2
    naming, bf16 activations, a down projection with K = 3584."""
    _say(f"[layer] mixtral_small T={T}")
    cfg, w, block, dense = _layer("mixtral_small")
    _check(cfg, block, w, dense, T)


@pytest.mark.parametrize("T", [1, 300])
def test_layer_matches_oracle_deepseek_shared_zipf(device, T):
    _say(f"[layer] deepseek_v2_lite T={T}")
    cfg, w, block, dense = _layer("deepseek_v2_lite")
    out = block(make_x(cfg, T).to("cuda").reshape(1, T, -1))
    assert torch.is_tensor(out)  # DeepSeek returns a tensor (moe_block.py:578, :623)
    _check(cfg, block, w, dense, T)


@pytest.mark.parametrize("name", ["ref_test", "olmoe_mixed", "qwen3_mixed", "mixtral_small", "deepseek_v2_lite"])
def test_one_token_forward_routing(device, name):
    """A one-token forward routes and groups in a single launch (gate matrices
    of 512 KB and more: a logits launch over the GPU and a one-wave top-k,
    here qwen3_mixed and deepseek_v2_lite); the logits it returns and the
    selection, weights and permutation it leaves in its workspace equal the
    oracle's (and moeq_route's weights) bit for bit, and the output meets the
    layer bar."""
    from robustgemq_amd import ops
    _say(f"[layer] one-token forward routing: {name}")
    cfg, w, block, dense = _layer(name)
    x = make_x(cfg, 1, seed=11)
    ref, ref_lg, ref_idx, ref_w = _oracle(cfg, w, dense, x)
    layer = block._layer
    k, E, ns = layer.top_k, layer.n_experts, layer.n_shared
    if layer.one_token_act_softmax:  # Mixtral's forward_one_token router (moe_block.py:280-283)
        ref_idx, ref_w, _, fragile = orr.topk_route_act_softmax(ref_lg, k, "bf16")
        assert not fragile.any()
        ref = om.moe_from_routing(x.float().numpy(), ref_idx, ref_w, *dense[:3], dense[3])
    xd = x.to("cuda")
    out32, lg = layer.forward(xd, out_dtype=torch.float32, want_logits=True, one_token=True)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(lg.float().cpu().numpy().view(np.uint32), ref_lg.view(np.uint32))
    offs, ws = layer.workspace_layout(1), layer._ws

    def arr(i, n, dt=torch.int32):
        return ws[offs[i]:offs[i] + 4 * n].view(dt).cpu().numpy()

    np.testing.assert_array_equal(arr(0, k), ref_idx.reshape(-1))
    wt = arr(1, k, torch.float32)
    if layer.one_token_act_softmax:
        np.testing.assert_array_equal(wt.view(np.uint32), ref_w.reshape(-1).view(np.uint32))
    else:
        _, _, w2 = ops.route(xd, layer.gate_w, k, layer.norm_topk, logit_bias=layer.logit_bias)
        np.testing.assert_array_equal(wt.view(np.uint32), to_np(w2).reshape(-1).view(np.uint32))
        np.testing.assert_allclose(wt, ref_w.reshape(-1), rtol=2e-6, atol=1e-7)
    ref_perm = orr.permute(ref_idx, E, ns)
    rows = k + ns
    for i, key, n in ((2, "counts", E + ns), (3, "offsets", E + ns + 1), (4, "row_token", rows),
                      (5, "row_pair", k), (6, "inv_perm", k)):
        np.testing.assert_array_equal(arr(i, n), ref_perm[key], err_msg=key)
    nt = int(arr(8, 1)[0])
    assert nt == rows
    tiles = arr(7, 4 * nt).reshape(nt, 4)
    want = np.stack([np.concatenate([np.sort(ref_idx.reshape(-1)), E + np.arange(ns)]), np.arange(rows),
                     np.ones(rows), np.zeros(rows)], 1).astype(np.int32)
    np.testing.assert_array_equal(tiles, want)
    got = to_np(out32)
    assert relative_error(got, ref) <= REL_L2 and float(np.abs(got - ref).max()) <= MAX_ABS


def test_mixtral_one_token_routing_ties(device):
    """Mixtral's forward_one_token ranks bf16 softmax probabilities and
    renormalises in bf16 (moe_block.py:280-283).  1024 single-token forwards:
    the selection and weights the forward leaves in its workspace equal the
    oracle's restatement bit for bit (tokens whose fp32 softmax sits on a bf16
    rounding midpoint aside, where any fp32 softmax may round either way);
    the tokens whose 2nd and 3rd probabilities tie in bf16 are counted, and
    torch's own softmax/topk on the device is compared as a second reading
    (its tie order is unspecified, so it may differ only at ties)."""
    import torch.nn.functional as F
    cfg, w, block, dense = _layer("mixtral_small")
    layer = block._layer
    T, k = 1024, layer.top_k
    x = make_x(cfg, T, seed=13)
    gate = w["gate"].to(torch.bfloat16).float().numpy()
    ref_lg = orr.router_logits(x.float().numpy(), gate, "bf16")
    ref_idx, ref_w, p, fragile = orr.topk_route_act_softmax(ref_lg, k, "bf16")
    offs = layer.workspace_layout(1)
    xd = x.to("cuda")
    gi, gw = [], []
    for t in range(T):
        layer.forward(xd[t:t + 1], want_logits=False, one_token=True)
        ws = layer._ws
        gi.append(ws[offs[0]:offs[0] + 4 * k].view(torch.int32).clone())
        gw.append(ws[offs[1]:offs[1] + 4 * k].view(torch.float32).clone())
    got_idx = torch.stack(gi).cpu().numpy()
    got_w = torch.stack(gw).cpu().numpy()
    keep = ~fragile
    np.testing.assert_array_equal(got_idx[keep], ref_idx[keep])
    np.testing.assert_array_equal(got_w[keep].view(np.uint32), ref_w[keep].view(np.uint32))
    srt = -np.sort(-p, axis=1)
    tie = srt[:, k - 1] == srt[:, k]
    lg_rank = orr.topk_route(ref_lg, k, True)[0]
    changed = (np.sort(lg_rank, 1) != np.sort(ref_idx, 1)).any(1)
    tp = F.softmax(torch.from_numpy(ref_lg).to("cuda", torch.bfloat16), dim=-1)
    tw, ti = torch.topk(tp, k, dim=-1)
    agree = (np.sort(ti.cpu().numpy(), 1) == np.sort(got_idx, 1)).all(1)
    _say(f"    {T} tokens: {int(tie.sum())} bf16 ties at the top-{k} boundary, {int(changed.sum())} selections "
         f"differ from logit ranking, {int(fragile.sum())} near-midpoint tokens; torch.topk on the device "
         f"differs on {int((~agree).sum())} ({int((~agree & tie).sum())} of them at ties)")
    assert not (~agree & ~tie & ~fragile).any()
    assert not (changed & ~tie).any()  # logit ranking and probability ranking part only at ties


def test_forward_timed_matches_forward(device):
    """moeq_moe_forward_timed (benchmark introspection) gives the forward's
    output bit for bit and brackets the gate/up launch with its two events."""
    _say("[layer] forward_timed == forward")
    cfg, w, block, dense = _layer("olmoe_mixed")
    layer = block._layer
    x = make_x(cfg, 256, seed=3).to("cuda")
    ref, _ = layer.forward(x, want_logits=False)
    ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
    for e in ev:
        e.record()
    got, _ = layer.forward(x, want_logits=False, gate_up_events=ev)
    torch.cuda.synchronize()
    assert torch.equal(ref, got)
    assert ev[0].elapsed_time(ev[1]) > 0


def test_full_size_prefill_rows_match_oracle(device):
    """BASELINE configs[1] at its benchmark size, T = 2048: the logits and
    output rows of 64 sampled tokens against the oracle run on those tokens
    alone (a token's logits and output depend on that token only), and a
    second forward is bit-identical."""
    _say("[layer] olmoe_mixed T=2048 sampled rows vs oracle, determinism")
    cfg, w, block, dense = _layer("olmoe_mixed")
    layer = block._layer
    T = 2048
    x = make_x(cfg, T, seed=21)
    xd = x.to("cuda")
    out32, lg = layer.forward(xd, out_dtype=torch.float32, want_logits=True)
    sel = np.sort(np.random.default_rng(0).choice(T, 64, replace=False))
    ref, ref_lg, _, _ = _oracle(cfg, w, dense, x[torch.from_numpy(sel)])
    np.testing.assert_array_equal(lg.float().cpu().numpy()[sel].view(np.uint32), ref_lg.view(np.uint32))
    got = to_np(out32)[sel]
    err, mx = relative_error(got, ref), float(np.abs(got - ref).max())
    _say(f"    rel-L2 {err:.3e} max-abs {mx:.3e}")
    assert err <= REL_L2 and mx <= MAX_ABS
    again, _ = layer.forward(xd, out_dtype=torch.float32, want_logits=False)
    assert torch.equal(out32, again)


def make_x(cfg, T, seed=5):
    from robustgemq_amd.synthetic import make_inputs
    return make_inputs(cfg, T, seed=seed)


def test_decode_equals_prefill_and_is_deterministic(device):
    """forward_one_token == forward_n_tokens on the same token (reference test
    :395-416) and repeated calls are bit-identical even when the allocator
    hands back NaN-poisoned memory (tests/test_decode_nan_hunt.py:34-98)."""
    _say("[layer] decode==prefill, determinism, poisoned allocator")
    cfg, w, block, dense = _layer("ref_test")
    x = make_x(cfg, 1).to("cuda").reshape(1, 1, -1)
    one = block.forward_one_token(x)[0].clone()
    many = block.forward_n_tokens(x)[0].clone()
    assert torch.equal(one, many)
    outs = []
    for _ in range(5):
        junk = torch.full((64 * 1024 * 1024,), float("nan"), dtype=torch.float16, device="cuda")
        del junk
        block._layer._ws = None  # force a fresh (poisoned) workspace
        outs.append(block(x)[0].clone())
    assert not torch.isnan(outs[0]).any()
    assert all(torch.equal(outs[0], o) for o in outs[1:])
    xs = make_x(cfg, 48).to("cuda").reshape(1, 48, -1)
    a = block(xs)[0].clone()
    block._layer._ws = None
    torch.full((64 * 1024 * 1024,), float("nan"), dtype=torch.float16, device="cuda")
    b = block(xs)[0].clone()
    assert torch.equal(a, b) and not torch.isnan(a).any()


@pytest.mark.parametrize("T", [128, 512, 2048])
def test_prefill_classes_write_every_output(device, T):
    """The 48-, 96- and 160-row tile classes (OLMoE T = 128 / 512 / 2048,
    with partial last tiles and the mixed block-count schedule) write every
    row of h and y they later read: a workspace filled with NaN gives the
    same output, bit for bit, as one filled with zeros, and no NaN."""
    _say(f"[layer] poisoned workspace, olmoe_mixed T={T}")
    cfg, w, block, dense = _layer("olmoe_mixed")
    layer = block._layer
    x = make_x(cfg, T, seed=31).to("cuda")
    need = layer.workspace_size(T)
    outs = []
    for fill in (0.0, float("nan")):
        layer._ws = torch.full((need // 2 + 1,), fill, dtype=torch.float16, device="cuda").view(torch.uint8)
        outs.append(layer.forward(x, out_dtype=torch.float32, want_logits=False)[0].clone())
    layer._ws = None
    _say(f"    plan {layer.plan(T)}")
    assert not torch.isnan(outs[1]).any()
    assert torch.equal(outs[0], outs[1])


def test_bf16_activations_beyond_fp16_range(device):
    """bf16 layers feed the expert GEMMs fp16 activations and keep the
    intermediate products in fp16, as the reference's kernels emit fp16
    (dequant_group_gemm.py:138, :181; fused_dequant_bmm.py:152-153, :292).
    A token with an activation beyond 65504 therefore has a non-finite output
    row (the overflow shows; it is never a finite wrong value); its routing
    is still exact and every other token is unaffected and within the bar."""
    _say("[layer] bf16 activations beyond the fp16 range")
    cfg, w, block, dense = _layer("qwen3_mixed")
    layer = block._layer
    T, bad = 64, 5
    x = make_x(cfg, T, seed=9)
    x[bad, 7] = 1.0e5
    ref, ref_lg, ref_idx, ref_w = _oracle(cfg, w, dense, x)
    xd = x.to("cuda")
    out32, lg = layer.forward(xd, out_dtype=torch.float32, want_logits=True)
    np.testing.assert_array_equal(lg.float().cpu().numpy().view(np.uint32), ref_lg.view(np.uint32))
    got = to_np(out32)
    assert not np.isfinite(got[bad]).all()
    ok = np.arange(T) != bad
    assert np.isfinite(got[ok]).all()
    assert relative_error(got[ok], ref[ok]) <= REL_L2 and float(np.abs(got[ok] - ref[ok]).max()) <= MAX_ABS


def test_block_api_conventions(device):
    _say("[layer] API conventions")
    cfg, w, block, dense = _layer("ref_test")
    x = make_x(cfg, 7).to("cuda").reshape(1, 7, -1)
    out, logits = block(x)
    assert out.shape == x.shape and out.dtype == x.dtype
    assert logits.shape == (7, cfg.n_experts) and logits.dtype == torch.float16
    one = block(x[:, :1])
    assert one[1] is None
    assert torch.equal(block.w1_nbits.cpu(), torch.tensor(w["bits"], dtype=torch.int32))
    assert torch.equal(block.w1_nbits, block.w3_nbits) and torch.equal(block.w1_wq_strides, block.w3_wq_strides)
    assert block.block_group_size == cfg.group_size
    # the stacked reference tensors hold the GemLite/HQQ packed words
    t0 = w["experts"][0]["gate_proj"]
    rows = -(-cfg.hidden // (32 // w["bits"][0]))
    np.testing.assert_array_equal(to_np(block.w1_wq[:rows]).view(np.uint32),
                                  oq.pack_cols(t0.codes().numpy(), w["bits"][0]).view(np.uint32))


def test_reference_kernel_surface(device):
    """The reference operator signatures (GemLite convention w = q*s + z')
    against fp32 matmul on the dequantized weight."""
    from robustgemq_amd import ops
    _say("[ops] reference kernel-level surface")
    rng = np.random.default_rng(3)
    E, K, N, g = 4, 512, 256, 128
    bits = [1, 2, 3, 4]
    words, sc, ze, dense = [], [], [], []
    for b in bits:
        codes = rng.integers(0, 1 << b, size=(N, K)).astype(np.uint8)
        s = (np.abs(rng.standard_normal((K // g, N))) * 0.01 + 1e-3).astype(np.float16)
        zp = (rng.standard_normal((K // g, N)) * 0.01).astype(np.float16)
        words.append(torch.from_numpy(oq.pack_cols(codes, b)))
        sc.append(torch.from_numpy(s))
        ze.append(torch.from_numpy(zp))
        gi = np.arange(K) // g
        dense.append(oq.dequant_affine(codes.T.astype(np.float16), s[gi], zp[gi]).astype(np.float32))
    wq = torch.cat(words).cuda()
    scales, zeros = torch.cat(sc).cuda(), torch.cat(ze).cuda()
    nb = torch.tensor(bits, dtype=torch.int32, device="cuda")
    gs = torch.full((E,), g, dtype=torch.int32, device="cuda")
    wst = torch.tensor(np.cumsum([0] + [w.numel() for w in words])[:-1], dtype=torch.int32, device="cuda")
    zst = torch.tensor(np.cumsum([0] + [s.numel() for s in sc])[:-1], dtype=torch.int32, device="cuda")
    x = torch.from_numpy((rng.standard_normal((19, K)) * 0.5).astype(np.float16))
    ind = torch.tensor([3, 0, 2], dtype=torch.int32, device="cuda")
    out = ops.dequant_group_gemm(x.cuda(), ind, wq, scales, zeros, nb, gs, wst, zst)
    assert out.shape == (3, 19, N) and out.dtype == torch.float16
    for a, e in enumerate([3, 0, 2]):
        ref = x.float().numpy() @ dense[e]
        assert relative_error(to_np(out[a]).astype(np.float32), ref) < 1e-3
    x1, x3 = ops.fused_dequant_up_proj(x[:1].cuda(), ind, wq, wq, scales, zeros, scales, zeros, nb, wst, g)
    assert x1.shape == (1, 3 * N)
    for a, e in enumerate([3, 0, 2]):
        ref = x[:1].float().numpy() @ dense[e]
        assert relative_error(to_np(x1[0, a * N:(a + 1) * N]).astype(np.float32), ref[0]) < 1e-3
    # fused_dequant_down_proj: fp32 SiLU*mul of the up projection's outputs,
    # rounded to fp16 (fused_dequant_bmm.py:236-239), then the down GEMV
    x1s = torch.from_numpy((rng.standard_normal((1, 3 * K)) * 2).astype(np.float16))
    x3s = torch.from_numpy((rng.standard_normal((1, 3 * K)) * 2).astype(np.float16))
    x2 = ops.fused_dequant_down_proj(x1s.cuda(), x3s.cuda(), ind, wq, scales, zeros, nb, wst, g)
    assert x2.shape == (1, 3 * N) and x2.dtype == torch.float16
    a1, a3 = x1s.float().numpy()[0], x3s.float().numpy()[0]
    h = (a1 / (1.0 + np.exp(-a1)) * a3).astype(np.float16).astype(np.float32)
    for a, e in enumerate([3, 0, 2]):
        ref = h[a * K:(a + 1) * K] @ dense[e]
        assert relative_error(to_np(x2[0, a * N:(a + 1) * N]).astype(np.float32), ref) < 1e-3
    y = ops.dequant_gemm(x.cuda(), words[1].cuda(), sc[1].cuda(), ze[1].cuda(), 2, g)
    assert relative_error(to_np(y).astype(np.float32), x.float().numpy() @ dense[1]) < 1e-3
    v = ops.dequant_splitk_gemv(x[:1].cuda(), words[2].cuda(), sc[2].cuda(), ze[2].cuda(), 3, g)
    assert relative_error(to_np(v).astype(np.float32), x[:1].float().numpy() @ dense[2]) < 1e-3
    # the repacked-weight cache follows the tensors, not their addresses: new
    # weights of the same shape (the caching allocator hands back the freed
    # block) and an in-place change both take effect
    xd = x.cuda()
    for trial in range(3):
        codes = rng.integers(0, 4, size=(N, K)).astype(np.uint8)
        wt = torch.from_numpy(oq.pack_cols(codes, 2)).cuda()
        st, zt = sc[1].cuda(), ze[1].cuda()
        gi = np.arange(K) // g
        dn = oq.dequant_affine(codes.T.astype(np.float16), sc[1].numpy()[gi], ze[1].numpy()[gi]).astype(np.float32)
        yt = ops.dequant_gemm(xd, wt, st, zt, 2, g)
        assert relative_error(to_np(yt).astype(np.float32), x.float().numpy() @ dn) < 1e-3, trial
        del wt, st, zt, yt
    st, zt = sc[1].cuda(), ze[1].cuda()
    wt = words[1].cuda()
    before = ops.dequant_gemm(xd, wt, st, zt, 2, g).clone()
    st.mul_(2)  # in place: the version counter moves
    after = ops.dequant_gemm(xd, wt, st, zt, 2, g)
    fresh = ops.dequant_gemm(xd, wt.clone(), st.clone(), zt.clone(), 2, g)  # new tensors: built anew
    assert torch.equal(after, fresh) and not torch.equal(after, before)


# ------------------------------------------------------------- from_hf
class _PackedLinear:
    """Stand-in for a GemLite-converted linear: the five attributes from_hf
    reads (moe_block.py:720-733) -- W_q [ceil(K/eps), N] int32 words,
    scales / zeros [K/g, N] fp16 with zeros = z' (w = q*s + z')."""

    def __init__(self, rng, N, K, bits, g, device):
        self.codes = rng.integers(0, 1 << bits, size=(N, K)).astype(np.uint8)
        s = (np.abs(rng.standard_normal((K // g, N))) * 0.004 + 5e-4).astype(np.float16)
        zp = (rng.standard_normal((K // g, N)) * 0.004).astype(np.float16)
        self.W_q = torch.from_numpy(oq.pack_cols(self.codes, bits)).to(device)
        self.scales = torch.from_numpy(s).to(device)
        self.zeros = torch.from_numpy(zp).to(device)
        self.W_nbits, self.group_size = bits, g
        gi = np.arange(K) // g
        self.dense = oq.dequant_affine(self.codes.T.astype(np.float16), s[gi], zp[gi]).astype(np.float32).T.copy()


class _Expert:
    def __init__(self, rng, H, F, bits, g, device):
        self.gate_proj = _PackedLinear(rng, F, H, bits, g, device)
        self.up_proj = _PackedLinear(rng, F, H, bits, g, device)
        self.down_proj = _PackedLinear(rng, H, F, bits, g, device)


class _HFBlock(torch.nn.Module):
    def __init__(self, rng, H, F, E, bits, g, n_shared, device):
        super().__init__()
        self.gate = torch.nn.Linear(H, E, bias=False).to(device=device, dtype=torch.float16)
        with torch.no_grad():
            self.gate.weight.copy_(torch.from_numpy((rng.standard_normal((E, H)) * 0.05).astype(np.float16)))
        self.experts = [_Expert(rng, H, F, bits[e], g, device) for e in range(E)]
        self.shared_experts = _Expert(rng, H, n_shared * F, 4, g, device) if n_shared else None


@pytest.mark.parametrize("family,T", [("olmoe", 24), ("olmoe", 1), ("deepseekv2", 40), ("deepseekv2", 1)])
def test_from_hf_gemlite_linears(device, family, T):
    """from_hf, the constructor replace_moe_blocks calls (patch.py:86-162),
    on GemLite-style expert linears: the stacked reference attributes and the
    output against the oracle on q*s + z' weights."""
    from robustgemq_amd.moe_block import BLOCKS
    from robustgemq_amd.synthetic import _Cfg
    _say(f"[from_hf] {family} T={T}")
    rng = np.random.default_rng(11)
    H, F, E, k, g = 512, 256, 8, 2, 64
    bits = [1, 2, 3, 4, 2, 3, 4, 2]
    n_sh = 2 if family == "deepseekv2" else 0
    hf = _HFBlock(rng, H, F, E, bits, g, n_sh, "cuda")
    common = dict(hidden_size=H, num_experts_per_tok=k, norm_topk_prob=False)
    if family == "olmoe":
        cfg = _Cfg(intermediate_size=F, num_experts=E, **common)
    else:
        cfg = _Cfg(moe_intermediate_size=F, n_routed_experts=E, n_shared_experts=n_sh, topk_method="greedy",
                   scoring_func="softmax", routed_scaling_factor=1.0, **common)
    block = BLOCKS[family].from_hf(cfg, hf)
    # stacked reference attributes (moe_block.py:725-758)
    assert torch.equal(block.w1_nbits.cpu(), torch.tensor(bits, dtype=torch.int32))
    assert block.block_group_size == g
    rows = [-(-H // (32 // b)) for b in bits]
    assert block.w1_wq_strides.cpu().tolist() == list(np.cumsum([0] + [r * F for r in rows])[:-1])
    assert torch.equal(block.w1_wq[:rows[0]], hf.experts[0].gate_proj.W_q)
    if n_sh:
        assert block.shared_nbits == 4 and block.shared_group_size == g
    x = torch.from_numpy((rng.standard_normal((T, H)) * 0.5).astype(np.float16))
    W1 = [e.gate_proj.dense for e in hf.experts]
    W3 = [e.up_proj.dense for e in hf.experts]
    W2 = [e.down_proj.dense for e in hf.experts]
    shared = ()
    if n_sh:
        sh = hf.shared_experts
        shared = ((sh.gate_proj.dense, sh.up_proj.dense, sh.down_proj.dense),)
    gate = hf.gate.weight.detach().float().cpu().numpy()
    ldt = "f32" if n_sh else "f16"
    ref, ref_lg, ref_idx, _ = om.moe_forward(x.float().numpy(), gate, ldt, k, False, W1, W3, W2, shared)
    res = block(x.cuda().reshape(1, T, H))
    assert isinstance(res, tuple) == (family == "olmoe")
    out = res[0] if isinstance(res, tuple) else res
    got = to_np(out.reshape(T, H)).astype(np.float32)
    out32, _ = block._layer.forward(x.cuda(), out_dtype=torch.float32, want_logits=False)
    got32 = to_np(out32)
    err, mx = relative_error(got32, ref), float(np.abs(got32 - ref).max())
    _say(f"    rel-L2 {err:.3e} max-abs {mx:.3e} (|ref|max {np.abs(ref).max():.3e})")
    assert err <= REL_L2 and mx <= MAX_ABS
    assert relative_error(got, ref) <= REL_L2 and float(np.abs(got - ref).max()) <= MAX_ABS
    if family == "olmoe" and T > 1:
        np.testing.assert_array_equal(to_np(res[1]).astype(np.float32).view(np.uint32), ref_lg.view(np.uint32))
