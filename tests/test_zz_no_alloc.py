"""moeq_moe_forward_static, the forward that allocates nothing (its scratch is
a static device array per GPU), against moeq_moe_forward with a caller
workspace: bit-identical outputs and logits on two calls in a row, the second
with fewer tokens (the array keeps the first call's contents), and a size
beyond the array refused before any launch."""


import pytest
import torch

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def test_static_scratch_forward_matches_workspace_forward(device):
    from robustgemq_amd import _lib as L
    from robustgemq_amd.synthetic import CONFIGS, build_block, make_inputs, make_weights
    lib = L.lib()
    for name, sizes in (("olmoe_mixed", (512, 24)), ("qwen3_mixed", (64, 1))):
        cfg = CONFIGS[name]
        block = build_block(cfg, make_weights(cfg, seed=0), device="cuda")
        layer = block._layer
        for T in sizes:
            _say(f"[static scratch] {name} T={T}")
            x = make_inputs(cfg, T, seed=T).to("cuda")
            ref, ref_lg = layer.forward(x, want_logits=True)
            out = torch.empty_like(ref)
            lg = torch.empty_like(ref_lg)
            rc = lib.moeq_moe_forward_static(layer.desc, L.ptr(x), T, L.ptr(out), L.dtype_code(out.dtype),
                                             L.ptr(lg), L.stream_handle(x.device))
            L.check(rc, "moeq_moe_forward_static")
            torch.cuda.synchronize()
            assert torch.equal(out, ref) and torch.equal(lg, ref_lg), (name, T)
        # more tokens than the static array holds: refused, nothing launched
        big = 1
        while layer.workspace_size(big) <= (64 << 20):
            big *= 2
        # full-size buffers, so a launch would stay in bounds if the check failed
        xb = torch.zeros((big, cfg.hidden), dtype=cfg.act_dtype, device="cuda")
        ob = torch.empty_like(xb)
        rc = lib.moeq_moe_forward_static(layer.desc, L.ptr(xb), big, L.ptr(ob), L.dtype_code(xb.dtype), None,
                                         L.stream_handle(xb.device))
        assert rc == -3 and b"static array" in lib.moeq_last_error()
        del block, layer
        torch.cuda.empty_cache()
