"""ctypes binding of libmoeq.so (C ABI declared in include/moeq.h).

The library is loaded after torch so that both share one HIP runtime (torch
ships libamdhip64.so.7 and the loader reuses it).  There is no fallback: if
the library is missing or fails to load, importing the ops raises.
"""

import ctypes
import os

import torch  # noqa: F401  (loads the HIP runtime first)

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmoeq.so")

MOEQ_OK = 0
F16, BF16, F32 = 0, 1, 2
DQ_HQQ, DQ_AFFINE, DQ_HQQ_INT = 0, 1, 2
EPI_STORE, EPI_SILU_MUL = 0, 1

c_void_p = ctypes.c_void_p
c_int = ctypes.c_int
c_int32 = ctypes.c_int32
c_int64 = ctypes.c_int64
c_size_t = ctypes.c_size_t


class MoeqProj(ctypes.Structure):
    _fields_ = [
        ("words", c_void_p),
        ("word_off", c_void_p),
        ("sz", c_void_p),
        ("sz_off", c_void_p),
        ("nbits", c_void_p),
        ("K", c_int32),
        ("N", c_int32),
        ("group_size", c_int32),
        ("dq_mode", c_int32),
    ]


class MoeqMoe(ctypes.Structure):
    _fields_ = [
        ("hidden", c_int32),
        ("inter", c_int32),
        ("n_experts", c_int32),
        ("top_k", c_int32),
        ("n_shared", c_int32),
        ("act_dtype", c_int32),
        ("gate_dtype", c_int32),
        ("norm_topk", c_int32),
        ("gate_w", c_void_p),
        ("w1", MoeqProj),
        ("w3", MoeqProj),
        ("w2", MoeqProj),
        ("logit_bias", c_void_p),
        ("one_token_act_softmax", c_int32),
    ]


class MoeqGemm(ctypes.Structure):
    _fields_ = [
        ("a", c_void_p),
        ("a_dtype", c_int32),
        ("lda", c_int64),
        ("row_src", c_void_p),
        ("tiles", c_void_p),
        ("n_tiles", c_void_p),
        ("max_tiles", c_int32),
        ("bm", c_int32),
        ("epilogue", c_int32),
        ("out", c_void_p),
        ("out_dtype", c_int32),
        ("ldo", c_int64),
        ("splits", c_int32),
        ("split_stride", c_int64),
    ]


# name -> (restype, argtypes); every symbol include/moeq.h declares
SIGNATURES = {
    "moeq_last_error": (ctypes.c_char_p, []),
    "moeq_version": (c_int, []),
    "moeq_pack_cols": (c_int, [c_void_p, c_int64, c_int64, c_int, c_void_p, c_void_p]),
    "moeq_repack": (c_int, [c_void_p, c_int64, c_int64, c_int, c_void_p, c_void_p]),
    "moeq_prep_scales": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int, c_void_p, c_void_p]),
    "moeq_route_workspace_size": (c_size_t, [c_int64, c_int]),
    "moeq_route": (c_int, [c_void_p, c_int, c_int64, c_int, c_void_p, c_int, c_void_p, c_int, c_int, c_int,
                           c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    "moeq_route_from_logits": (c_int, [c_void_p, c_int, c_int64, c_int, c_int, c_int, c_void_p,
                                       c_void_p, c_void_p]),
    "moeq_max_tiles": (c_int, [c_int64, c_int, c_int, c_int, c_int]),
    "moeq_tile_rows": (c_int, [c_int]),
    "moeq_permute_workspace_size": (c_size_t, [c_int64, c_int, c_int, c_int]),
    "moeq_permute": (c_int, [c_void_p, c_int64, c_int, c_int, c_int, c_int, c_void_p, c_void_p,
                             c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t,
                             c_void_p]),
    "moeq_grouped_gemm": (c_int, [ctypes.POINTER(MoeqGemm), ctypes.POINTER(MoeqProj),
                                  ctypes.POINTER(MoeqProj), c_void_p]),
    "moeq_combine": (c_int, [c_void_p, c_int, c_int, c_int64, c_int64, c_void_p, c_void_p, c_int64,
                             c_int, c_int, c_int, c_void_p, c_int, c_void_p]),
    "moeq_silu_mul": (c_int, [c_void_p, c_void_p, c_int64, c_void_p, c_void_p]),
    "moeq_moe_workspace_size": (c_size_t, [ctypes.POINTER(MoeqMoe), c_int64]),
    "moeq_moe_forward": (c_int, [ctypes.POINTER(MoeqMoe), c_void_p, c_int64, c_void_p, c_int,
                                 c_void_p, c_void_p, c_size_t, c_void_p]),
    "moeq_moe_forward_static": (c_int, [ctypes.POINTER(MoeqMoe), c_void_p, c_int64, c_void_p, c_int,
                                        c_void_p, c_void_p]),
    "moeq_gemm_tile_n": (c_int, [c_int, c_int]),
    "moeq_moe_plan": (c_int, [ctypes.POINTER(MoeqMoe), c_int64, c_void_p]),
    "moeq_moe_workspace_layout": (c_int, [ctypes.POINTER(MoeqMoe), c_int64, c_void_p]),
    "moeq_moe_forward_timed": (c_int, [ctypes.POINTER(MoeqMoe), c_void_p, c_int64, c_void_p, c_int,
                                       c_void_p, c_void_p, c_size_t, c_void_p, c_void_p, c_void_p]),
}

_lib = None


class MoeqError(RuntimeError):
    pass


def lib():
    """The loaded library; raises if libmoeq.so is absent or incomplete."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise MoeqError(
                f"{LIB_PATH} is missing: build it with `python -m robustgemq_amd.build` "
                "(there is no CPU or PyTorch fallback for the MoE expert path)")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(rc, what):
    if rc != MOEQ_OK:
        msg = lib().moeq_last_error().decode(errors="replace")
        raise MoeqError(f"{what} failed ({rc}): {msg}")


def ptr(t):
    """Device (or host) address of a tensor, or None."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_handle(device=None):
    """hipStream_t of torch's current stream on `device`."""
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def dtype_code(dt):
    if dt == torch.float16:
        return F16
    if dt == torch.bfloat16:
        return BF16
    if dt == torch.float32:
        return F32
    raise ValueError(f"unsupported dtype {dt}")
