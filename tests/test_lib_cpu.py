"""CPU-side checks of the native library: it loads, exports every symbol the
header declares, rejects bad arguments without launching anything, and its
host-only planning functions behave.  No kernel is launched here."""

import ctypes
import os
import re

import numpy as np
import pytest
import torch

from robustgemq_amd import _lib as L
from robustgemq_amd.quantize import rtn_quantize
from oracle import quant as oq

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "moeq.h")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(moeq_[a-z_0-9]+)\s*\(", src, flags=re.M)))


def test_header_symbols_exported():
    names = declared_functions()
    assert len(names) >= 15, names
    lib = L.lib()
    for n in names:
        assert hasattr(lib, n), f"libmoeq.so does not export {n}"
        assert n in L.SIGNATURES, f"_lib.SIGNATURES lacks {n}"
    assert set(L.SIGNATURES) == set(names)
    assert lib.moeq_version() >= 1


def test_struct_layouts_match_header(tmp_path):
    """ctypes mirrors of the C structs agree with the C compiler's sizeof and
    offsetof for every field of include/moeq.h."""
    import subprocess
    structs = {"moeq_proj": L.MoeqProj, "moeq_moe": L.MoeqMoe, "moeq_gemm": L.MoeqGemm}
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void) {"]
    for cname, cls in structs.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for fname, _ in cls._fields_:
            lines.append(f'printf("{cname} {fname} %zu\\n", offsetof({cname}, {fname}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-o", str(exe), str(src)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    seen = 0
    for line in filter(None, out):
        cname, field, val = line.split()
        cls = structs[cname]
        want = ctypes.sizeof(cls) if field == "size" else getattr(cls, field).offset
        assert int(val) == want, (cname, field, val, want)
        seen += 1
    assert seen == sum(len(c._fields_) + 1 for c in structs.values())


def _err(rc):
    return rc, L.lib().moeq_last_error().decode()


def test_invalid_arguments_are_rejected_before_launch():
    lib = L.lib()
    fake = ctypes.c_void_p(0x1000)
    rc, msg = _err(lib.moeq_pack_cols(None, 4, 8, 2, fake, None))
    assert rc == -1 and "null" in msg
    rc, msg = _err(lib.moeq_pack_cols(fake, 4, 8, 5, fake, None))
    assert rc == -1 and "nbits" in msg
    rc, msg = _err(lib.moeq_repack(fake, 100, 16, 2, fake, None))
    assert rc == -1 and "128" in msg
    rc, msg = _err(lib.moeq_repack(fake, 128, 24, 2, fake, None))
    assert rc == -1 and "16" in msg
    rc, msg = _err(lib.moeq_prep_scales(fake, fake, 1, 2, 16, 7, fake, None))
    assert rc == -1 and "dq_mode" in msg
    rc, msg = _err(lib.moeq_prep_scales(fake, fake, 1, 2, 24, 0, fake, None))
    assert rc == -1 and "multiple of 16" in msg
    # route: top_k > E, unsupported hidden size
    rc, msg = _err(lib.moeq_route(fake, L.F16, 4, 2048, fake, L.F16, None, 8, 9, 0, None, fake, fake, None, 0, None))
    assert rc == -1 and "top_k" in msg
    rc, msg = _err(lib.moeq_route(fake, L.F16, 4, 8192, fake, L.F16, None, 8, 2, 0, None, fake, fake, None, 0, None))
    assert rc == -2
    rc, msg = _err(lib.moeq_route(fake, L.F16, 4, 2048, fake, L.F16, None, 8, 2, 0, None, fake, fake, fake,
                                  lib.moeq_route_workspace_size(4, 8) - 1, None))
    assert rc == -3 and "workspace" in msg
    # permute: workspace too small
    need = lib.moeq_permute_workspace_size(16, 2, 8, 0)
    rc, msg = _err(lib.moeq_permute(fake, 16, 2, 8, 0, 16, fake, fake, fake, fake, fake, fake, fake, fake,
                                    need - 1, None))
    assert rc == -3 and "workspace" in msg
    rc, msg = _err(lib.moeq_permute(fake, 16, 2, 8, 0, 24, fake, fake, fake, fake, fake, fake, fake, fake,
                                    need, None))
    assert rc == -1 and "bm" in msg


def _proj(K, N, g=64, mode=0):
    f = 0x1000
    return L.MoeqProj(words=f, word_off=f, sz=f, sz_off=f, nbits=f, K=K, N=N, group_size=g, dq_mode=mode)


def test_grouped_gemm_argument_checks():
    lib = L.lib()
    f = 0x1000
    g = L.MoeqGemm(a=f, a_dtype=L.F16, lda=2048, row_src=None, tiles=f, n_tiles=f, max_tiles=4, bm=16,
                   epilogue=L.EPI_SILU_MUL, out=f, out_dtype=L.F16, ldo=1024, splits=1, split_stride=0)
    rc, msg = _err(lib.moeq_grouped_gemm(g, _proj(2048, 1024), _proj(2048, 512), None))
    assert rc == -1 and "differ" in msg
    rc, msg = _err(lib.moeq_grouped_gemm(g, _proj(2000, 1024), _proj(2000, 1024), None))
    assert rc == -2 and "128" in msg
    g.epilogue = L.EPI_STORE
    rc, msg = _err(lib.moeq_grouped_gemm(g, _proj(2048, 1024), _proj(2048, 1024), None))
    assert rc == -1 and "one projection" in msg
    g.splits, g.out_dtype = 2, L.F16
    rc, msg = _err(lib.moeq_grouped_gemm(g, _proj(2048, 1024), None, None))
    assert rc == -1 and "F32" in msg
    g.splits, g.bm = 1, 48
    rc, msg = _err(lib.moeq_grouped_gemm(g, _proj(2048, 1024), None, None))
    assert rc == -1 and "bm" in msg


def test_silu_mul_argument_checks():
    lib = L.lib()
    f = ctypes.c_void_p(0x1000)
    rc, msg = _err(lib.moeq_silu_mul(f, f, 12, f, None))
    assert rc == -1 and "multiple of 8" in msg
    rc, msg = _err(lib.moeq_silu_mul(None, f, 16, f, None))
    assert rc == -1 and "null" in msg


def test_activation_rows_2gib_guard():
    """Every row tile addresses activation rows with 32-bit offsets: the
    operator refuses activations whose rows end past 2 GiB, whatever the tile
    class, and QuantLinear slices its rows so every slice fits."""
    from types import SimpleNamespace

    from robustgemq_amd import ops

    def fake(rows, stride, esize=2):
        return SimpleNamespace(shape=(rows, stride), stride=lambda i: stride, element_size=lambda: esize)

    K = 4096
    fit = (1 << 31) // (K * 2)
    assert ops.a_rows_addressable(fake(fit, K), 128)
    assert not ops.a_rows_addressable(fake(fit + 1, K), 128)
    assert not ops.a_rows_addressable(fake(fit + 1, K), 32)
    assert not ops.a_rows_addressable(fake(fit + 1, K), 16)
    assert ops.a_rows_addressable(fake(fit, K), 16)
    for K in (128, 2048, 4096, 14336, 1 << 20):
        rows_max = max(16, (ops.A_ROWS_MAX_BYTES // (K * 2)) // 16 * 16)  # QuantLinear's slice
        assert ops.a_rows_addressable(fake(rows_max, K), 128) or rows_max == 16


def test_max_tiles_bounds_every_routing():
    """The host bound on row tiles must cover any routing the device can see."""
    lib = L.lib()
    rng = np.random.default_rng(0)
    from oracle.route import permute
    for T, k, E, S, bm in ((1, 8, 64, 0, 16), (7, 2, 8, 0, 16), (2048, 8, 64, 0, 128), (2048, 6, 64, 2, 128),
                           (300, 6, 64, 2, 32), (33, 8, 64, 0, 64)):
        bound = lib.moeq_max_tiles(T, k, E, S, bm)
        cap = lib.moeq_tile_rows(bm)
        assert cap >= bm
        for skew in (0.0, 3.0):
            p = np.exp(-skew * np.arange(E) / E)
            p /= p.sum()
            idx = np.stack([rng.choice(E, size=k, replace=False, p=p) for _ in range(T)])
            counts = list(np.bincount(idx.reshape(-1), minlength=E)) + [T] * S
            tiles = 0
            for m in counts:
                tiles += -(-m // cap)
            assert tiles <= bound, (T, k, E, S, bm, tiles, bound)
        assert permute  # imported for parity of the tile rule with the oracle grouping


def test_tile_rows_classes():
    lib = L.lib()
    assert [lib.moeq_tile_rows(b) for b in (16, 32, 64, 128, 256)] == [32, 48, 96, 160, 256]
    assert lib.moeq_tile_rows(48) == 0 and lib.moeq_tile_rows(0) == 0


def test_tile_split_rule():
    """Tiles cover an expert's rows once, in ceil(m / cap) tiles of at most cap
    rows at 16-row boundaries, and never run more 16-row blocks (rounded up to
    the kernel's variants) than an even split of the rows would."""
    from robustgemq_amd.linear import split_rows
    variants = {16: (1, 2), 32: (2, 3), 64: (2, 4, 6), 128: (2, 4, 8, 10), 256: (2, 4, 8, 10, 16)}

    def run_blocks(rows, bm):
        b = -(-rows // 16)
        return min(v for v in variants[bm] if v >= b)

    lib = L.lib()
    for bm in (16, 32, 64, 128, 256):
        cap = lib.moeq_tile_rows(bm)
        for m in range(1, 3000):
            t = split_rows(m, bm)
            assert len(t) == -(-m // cap)
            assert [r0 for r0, _ in t] == [sum(rc for _, rc in t[:j]) for j in range(len(t))]
            assert sum(rc for _, rc in t) == m and all(0 < rc <= cap for _, rc in t)
            assert all(rc % 16 == 0 for _, rc in t[:-1])
            nt = len(t)
            even = [m * (j + 1) // nt - m * j // nt for j in range(nt)]
            assert sum(run_blocks(rc, bm) for _, rc in t) <= sum(run_blocks(rc, bm) for rc in even), (bm, m, t)
    # an expert of 17 blocks in the 128-row class runs 10 + 8 blocks, not 10 + 10
    assert split_rows(260, 128) == [(0, 160), (160, 100)]


def test_layer_plan_and_workspace():
    lib = L.lib()
    f = 0x1000
    m = L.MoeqMoe(hidden=2048, inter=1024, n_experts=64, top_k=8, n_shared=0, act_dtype=L.F16,
                  gate_dtype=L.F16, norm_topk=0, gate_w=f, w1=_proj(2048, 1024), w3=_proj(2048, 1024),
                  w2=_proj(1024, 2048), logit_bias=None)
    plan = (ctypes.c_int32 * 4)()
    assert lib.moeq_moe_plan(m, 2048, plan) == 0
    assert plan[0] == 128 and plan[1] == 1
    assert lib.moeq_moe_plan(m, 1, plan) == 0
    assert plan[0] == 16 and plan[1] >= 1
    # 16 rows per expert: 64 small experts take the 48-row class (each expert's
    # weights streamed once), 8 large ones (Mixtral) keep the 16-row kernel
    assert lib.moeq_moe_plan(m, 128, plan) == 0 and plan[0] == 32
    assert lib.moeq_moe_plan(m, 64, plan) == 0 and plan[0] == 16
    mx = L.MoeqMoe(hidden=4096, inter=14336, n_experts=8, top_k=2, n_shared=0, act_dtype=L.BF16,
                   gate_dtype=L.BF16, norm_topk=1, gate_w=f, w1=_proj(4096, 14336), w3=_proj(4096, 14336),
                   w2=_proj(14336, 4096), logit_bias=None)
    assert lib.moeq_moe_plan(mx, 64, plan) == 0 and plan[0] == 16
    ws = lib.moeq_moe_workspace_size(m, 2048)
    # at least h [T*k, F] fp16 and y [T*k, H] fp16
    assert ws >= 2048 * 8 * (1024 + 2048) * 2
    m.w2 = _proj(1024, 1024)
    assert lib.moeq_moe_workspace_size(m, 2048) == 0  # invalid layer -> 0
    assert lib.moeq_gemm_tile_n(128, L.EPI_SILU_MUL) > 0 and lib.moeq_gemm_tile_n(48, 0) == 0
    assert lib.moeq_gemm_tile_n(256, L.EPI_SILU_MUL) == 128 and lib.moeq_gemm_tile_n(256, L.EPI_STORE) == 256


@pytest.mark.parametrize("nbits", [1, 2, 3, 4])
def test_product_quantizer_matches_oracle(nbits):
    g = torch.Generator().manual_seed(nbits)
    W = (torch.randn(96, 256, generator=g) * 0.02).half()
    t = rtn_quantize(W, nbits, 64)
    Q, s, z = oq.rtn_quantize(W.numpy(), nbits, 64)
    np.testing.assert_array_equal(t.Q.numpy().view(np.uint16), Q.view(np.uint16))
    np.testing.assert_array_equal(t.scales.numpy().view(np.uint16), s.view(np.uint16))
    np.testing.assert_array_equal(t.zeros.numpy().view(np.uint16), z.view(np.uint16))
    np.testing.assert_array_equal(t.dequantize().numpy().view(np.uint16),
                                  oq.dequant_hqq(Q, s, z).reshape(W.shape).view(np.uint16))
