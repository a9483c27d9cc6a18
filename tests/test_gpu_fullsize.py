"""Full-size parity of the BASELINE workloads on the GPU against the oracle.

Each workload runs through the layer forward at the size the benchmark
reports it:

  * OLMoE uniform 2-bit, prefill T = 2048 (the north-star layer),
  * Qwen3-30B-A3B shaped (bf16, 128 experts, g = 128), prefill T = 4096,
  * DeepSeek-V2-Lite shaped with Zipf-skewed routing and two shared
    experts, prefill T = 2048,
  * Mixtral-8x7B shaped (H = 4096, F = 14336: a 112-chunk down projection),
    decode B = 1 / 16 / 64 and a 2-layer slice of the T = 1024 stack.

What is checked, following the reference's per-family block checks
(tests/test_moe_block_equiv.py:336-392):

  * routing on the WHOLE batch bit for bit: the logits the forward returns,
    and the selection, weights, grouping (counts, offsets, rows, inverse
    permutation) and tile schedule it leaves in its workspace, against the
    oracle's router (router_exact.c), top-k and permutation;
  * sampled output rows within max-abs 1e-2 / rel-L2 1e-3 of the oracle's
    fp32 dequantize-then-matmul loop run on those tokens alone (a token's
    output depends on that token only); the oracle dequantizes only the
    experts the sample hits;
  * a second forward is bit-identical to the first.
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


class _Layer:
    """A synthetic layer on the GPU and the oracle's view of it (dense fp32
    fake-quant weights, dequantized per expert on first use)."""

    def __init__(self, name, seed=0):
        from robustgemq_amd.synthetic import CONFIGS, build_block, make_weights
        self.cfg = CONFIGS[name]
        self.w = make_weights(self.cfg, seed=seed, quant_device="cuda")
        self.block = build_block(self.cfg, self.w, device="cuda")
        self.layer = self.block._layer
        self._dense = {}

    @staticmethod
    def _deq(t):
        N, K = t.shape
        return oq.dequant_hqq(t.Q.cpu().numpy(), t.scales.cpu().numpy(),
                              t.zeros.cpu().numpy()).reshape(N, K).astype(np.float32)

    def expert(self, e):
        if e not in self._dense:
            ex = self.w["experts"][e]
            self._dense[e] = tuple(self._deq(ex[n]) for n in ("gate_proj", "up_proj", "down_proj"))
        return self._dense[e]

    def shared(self):
        if self.w["shared"] is None:
            return ()
        if "shared" not in self._dense:
            sh = self.w["shared"]
            self._dense["shared"] = tuple(self._deq(sh[n]) for n in ("gate_proj", "up_proj", "down_proj"))
        return (self._dense["shared"],)

    @property
    def logits_dtype(self):
        if self.cfg.family == "deepseekv2":
            return "f32"
        return "bf16" if self.cfg.act_dtype == torch.bfloat16 else "f16"

    def gate32(self):
        g = self.w["gate"]
        if self.cfg.family != "deepseekv2" and self.cfg.act_dtype == torch.bfloat16:
            g = g.to(torch.bfloat16)
        return g.float().numpy()

    def bias(self):
        return None if self.w["bias"] is None else self.w["bias"].numpy()

    def renorm(self):
        return self.cfg.norm_topk or self.cfg.family == "mixtral"

    def oracle_rows(self, x32, idx, wts):
        """Oracle output of the tokens x32 [n, H] routed as (idx, wts)."""
        hit = sorted(set(np.asarray(idx).reshape(-1).tolist()))
        E = self.cfg.n_experts
        W1, W3, W2 = [None] * E, [None] * E, [None] * E
        for e in hit:
            W1[e], W3[e], W2[e] = self.expert(e)
        return om.moe_from_routing(x32, idx, wts, W1, W3, W2, self.shared())


def _check_routing_in_workspace(L, T, x32, lg):
    """Logits, selection, weights, grouping and tile schedule of a T-token
    forward against the oracle, bit for bit; returns (ref_idx, ref_w)."""
    from robustgemq_amd.linear import split_rows
    layer = L.layer
    ref_lg = orr.router_logits(x32, L.gate32(), L.logits_dtype, L.bias())
    np.testing.assert_array_equal(lg.float().cpu().numpy().view(np.uint32), ref_lg.view(np.uint32))
    k, E, S = layer.top_k, layer.n_experts, layer.n_shared
    ref_idx, ref_w = orr.topk_route(ref_lg, k, L.renorm())
    offs, ws = layer.workspace_layout(T), layer._ws
    plan = layer.plan(T)

    def arr(i, n, dt=torch.int32):
        return ws[offs[i]:offs[i] + 4 * n].view(dt).cpu().numpy()

    np.testing.assert_array_equal(arr(0, T * k).reshape(T, k), ref_idx)
    np.testing.assert_allclose(arr(1, T * k, torch.float32).reshape(T, k), ref_w, rtol=2e-6, atol=1e-7)
    ref_perm = orr.permute(ref_idx, E, S)
    rows = T * k + S * T
    for i, key, n in ((2, "counts", E + S), (3, "offsets", E + S + 1), (4, "row_token", rows),
                      (5, "row_pair", T * k), (6, "inv_perm", T * k)):
        np.testing.assert_array_equal(arr(i, n), ref_perm[key], err_msg=key)
    nt = int(arr(8, 1)[0])
    assert 0 < nt <= plan["max_tiles"]
    tiles = arr(7, 4 * nt).reshape(nt, 4)
    want = [(e, int(ref_perm["offsets"][e]) + r0, rc, 0)
            for e in range(E + S) for r0, rc in (split_rows(int(ref_perm["counts"][e]), plan["bm"])
                                                  if ref_perm["counts"][e] else [])]
    # listed by the kernel variant of each expert's first (largest) tile,
    # largest first: more than s2 16-row blocks, then more than the variant
    # below s2, then the rest; experts in order within each group and an
    # expert's tiles together (a stable sort on the expert's key)
    s2 = {16: 1, 32: 2, 64: 4, 128: 8, 256: 10}[plan["bm"]]
    below = {64: 2, 128: 4, 256: 8}.get(plan["bm"], 0)
    blocks = lambda rc: -(-rc // 16)
    cls = lambda rc: 0 if blocks(rc) > s2 else 1 if blocks(rc) > below else 2
    first = {}
    for t in want:
        first.setdefault(t[0], cls(t[2]))
    want.sort(key=lambda t: first[t[0]])
    np.testing.assert_array_equal(tiles, np.array(want, np.int32).reshape(-1, 4))
    return ref_idx, ref_w


def _prefill(L, T, n_sample=48, seed=21):
    from robustgemq_amd.synthetic import make_inputs
    cfg, layer = L.cfg, L.layer
    x = make_inputs(cfg, T, seed=seed)
    x32 = x.float().numpy()
    xd = x.to("cuda")
    out32, lg = layer.forward(xd, out_dtype=torch.float32, want_logits=True)
    torch.cuda.synchronize()
    _say(f"    {cfg.name} T={T}: plan {layer.plan(T)}")
    ref_idx, ref_w = _check_routing_in_workspace(L, T, x32, lg)
    counts = np.bincount(ref_idx.reshape(-1), minlength=cfg.n_experts)
    _say(f"    routing bit-exact; rows per expert min {counts.min()} max {counts.max()}")
    sel = np.sort(np.random.default_rng(0).choice(T, n_sample, replace=False))
    ref = L.oracle_rows(x32[sel], ref_idx[sel], ref_w[sel])
    got = to_np(out32)[sel]
    err, mx = relative_error(got, ref), float(np.abs(got - ref).max())
    _say(f"    {n_sample} sampled rows: rel-L2 {err:.3e} max-abs {mx:.3e}")
    assert err <= REL_L2 and mx <= MAX_ABS
    again, _ = layer.forward(xd, out_dtype=torch.float32, want_logits=False)
    assert torch.equal(out32, again)
    return x, out32


def test_olmoe_2bit_prefill_T2048(device):
    """configs[0]'s layer at the north-star size (the OLMoE
    2-bit layer at 2048-token prefill)."""
    _say("[fullsize] olmoe_2bit T=2048")
    _prefill(_Layer("olmoe_2bit"), 2048)


def test_qwen3_prefill_T4096(device):
    """bf16 activations, 128 experts, g = 128, T = 4096."""
    _say("[fullsize] qwen3_mixed T=4096")
    _prefill(_Layer("qwen3_mixed"), 4096)


def test_deepseek_zipf_prefill_T2048(device):
    """Zipf-skewed routing (the hottest expert spans many
    160-row tiles) plus two always-on shared experts, T = 2048."""
    _say("[fullsize] deepseek_v2_lite (Zipf) T=2048")
    L = _Layer("deepseek_v2_lite")
    _prefill(L, 2048)


@pytest.fixture(scope="module")
def mixtral(device):
    _say("[fullsize] building mixtral_mixed (H=4096, F=14336, 8 experts)")
    L = _Layer("mixtral_mixed")
    yield L
    del L
    torch.cuda.empty_cache()


@pytest.mark.parametrize("B", [1, 16, 64])
def test_mixtral_decode(mixtral, B):
    """configs[4] decode at its real shape: every row of the batch against the
    oracle.  B = 1 goes through forward_one_token (bf16 softmax probabilities,
    moe_block.py:280-283), larger batches through forward_n_tokens."""
    from robustgemq_amd.synthetic import make_inputs
    L = mixtral
    cfg, layer = L.cfg, L.layer
    _say(f"[fullsize] mixtral_mixed decode B={B}: plan {layer.plan(B)}")
    x = make_inputs(cfg, B, seed=2)
    x32 = x.float().numpy()
    xd = x.to("cuda")
    ref_lg = orr.router_logits(x32, L.gate32(), "bf16")
    if B == 1:
        ref_idx, ref_w, _, fragile = orr.topk_route_act_softmax(ref_lg, cfg.top_k, "bf16")
        assert not fragile.any()
        out32, lg = layer.forward(xd, out_dtype=torch.float32, want_logits=True, one_token=True)
        np.testing.assert_array_equal(lg.float().cpu().numpy().view(np.uint32), ref_lg.view(np.uint32))
        offs, ws = layer.workspace_layout(1), layer._ws
        np.testing.assert_array_equal(ws[offs[0]:offs[0] + 8].view(torch.int32).cpu().numpy(), ref_idx[0])
        np.testing.assert_array_equal(ws[offs[1]:offs[1] + 8].view(torch.float32).cpu().numpy().view(np.uint32),
                                      ref_w[0].view(np.uint32))
        blk = L.block(xd.reshape(1, 1, -1))[0].reshape(1, -1)
        assert torch.equal(blk, out32.to(torch.bfloat16))
    else:
        out32, lg = layer.forward(xd, out_dtype=torch.float32, want_logits=True)
        ref_idx, ref_w = _check_routing_in_workspace(L, B, x32, lg)
    ref = L.oracle_rows(x32, ref_idx, ref_w)
    got = to_np(out32)
    err, mx = relative_error(got, ref), float(np.abs(got - ref).max())
    _say(f"    B={B}: rel-L2 {err:.3e} max-abs {mx:.3e}")
    assert err <= REL_L2 and mx <= MAX_ABS
    again, _ = layer.forward(xd, out_dtype=torch.float32, want_logits=False, one_token=B == 1)
    assert torch.equal(out32, again)


def test_mixtral_stack_slice_T1024(mixtral):
    """Two layers of the T = 1024 stack (the benchmark's stack reuses one
    layer's weights): each layer's routing on the whole batch bit for bit and
    sampled rows against the oracle fed with that layer's actual input.
    Layer 2 reads layer 1's output scaled to unit RMS per token, as the
    RMSNorm in front of every MoE block of these models leaves it (raw
    outputs are several times larger, and the fp16 intermediates' absolute
    error grows with them while the relative error stays put)."""
    L = mixtral
    cfg, layer = L.cfg, L.layer
    _say("[fullsize] mixtral_mixed 2-layer slice, T=1024")
    x, out1 = _prefill(L, 1024, n_sample=32, seed=4)
    rms = out1.pow(2).mean(dim=1, keepdim=True).sqrt()
    h = (out1 / rms).to(torch.bfloat16)  # the stack passes bf16 activations on
    out2, lg2 = layer.forward(h, out_dtype=torch.float32, want_logits=True)
    torch.cuda.synchronize()
    h32 = h.float().cpu().numpy()
    ref_idx, ref_w = _check_routing_in_workspace(L, 1024, h32, lg2)
    sel = np.sort(np.random.default_rng(1).choice(1024, 32, replace=False))
    ref = L.oracle_rows(h32[sel], ref_idx[sel], ref_w[sel])
    got = to_np(out2)[sel]
    err, mx = relative_error(got, ref), float(np.abs(got - ref).max())
    _say(f"    layer 2: rel-L2 {err:.3e} max-abs {mx:.3e}")
    assert err <= REL_L2 and mx <= MAX_ABS
