"""ctypes binding of libdspark_hip.so (include/dspark_hip.h).

The library is the only compute path: there is no CPU fallback. Importing this module on a
machine without the built library raises ImportError; calling an entry point without a GPU
raises RuntimeError from the HIP runtime through dsk_last_error().
"""

from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

_LIB_PATH = Path(os.environ.get("DSPARK_HIP_LIB", Path(__file__).with_name("libdspark_hip.so")))

c_void_p, c_int, c_int64, c_float, c_size_t, c_uint64, c_uint32 = (
    C.c_void_p, C.c_int, C.c_int64, C.c_float, C.c_size_t, C.c_uint64, C.c_uint32)

# name -> (restype, argtypes); mirrors include/dspark_hip.h
SIGNATURES: dict[str, tuple] = {
    "dsk_last_error": (C.c_char_p, []),
    "dsk_abi_version": (c_int, []),
    "dsk_w8_quantize": (c_int, [c_void_p, c_int, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p]),
    "dsk_w8_repack": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int, c_void_p, c_void_p,
                              c_void_p]),
    "dsk_w4_quantize": (c_int, [c_void_p, c_int, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p]),
    "dsk_w4_repack": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int, c_void_p, c_void_p,
                              c_void_p]),
    "dsk_w4_gemm": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int64, c_int64, c_int, c_void_p, c_int, c_int64,
                            c_void_p, c_int64, c_float, c_void_p]),
    "dsk_act_pack_bytes": (c_size_t, [c_int, c_int64]),
    "dsk_act_pack": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_int, c_int64, c_void_p,
                             c_float, c_void_p, c_void_p]),
    "dsk_act_pack_scaled": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_int, c_int64,
                                    c_void_p, c_float, c_float, c_void_p, c_void_p]),
    "dsk_w8_gemm_splits": (c_int, [c_int, c_int64, c_int64]),
    "dsk_w4_gemm_splits": (c_int, [c_int, c_int64, c_int64]),
    "dsk_w8_gemm": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int64, c_int64, c_int, c_void_p, c_int, c_int64,
                            c_void_p, c_int64, c_float, c_void_p]),
    "dsk_act_pack_rn": (c_int, [c_void_p, c_int, c_void_p, c_int64, c_void_p, c_int64, c_int, c_int64, c_void_p,
                                c_void_p, c_void_p, c_void_p]),
    "dsk_w8_gemm_rn": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int64, c_int64, c_int, c_void_p, c_int,
                               c_int64, c_float, c_void_p, c_int, c_float, c_void_p, c_int64, c_void_p, c_int64,
                               c_void_p, c_void_p, c_void_p]),
    "dsk_w8_gemm_plan": (c_int, [c_int, c_int64, c_int64, c_int, c_int, c_void_p]),
    "dsk_w8_gemm_rn_planned": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int64, c_int64, c_int, c_void_p,
                                       c_int, c_int64, c_float, c_void_p, c_int, c_float, c_void_p, c_int64, c_void_p,
                                       c_int64, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p]),
    "dsk_w8_dequant_rows": (c_int, [c_void_p, c_void_p, c_int, c_int64, c_int64, c_int, c_void_p, c_void_p]),
    "dsk_rows_rmsnorm": (c_int, [c_void_p, c_int64, c_void_p, c_float, c_int64, c_int64, c_void_p, c_int64, c_void_p]),
    "dsk_rows_gated": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_int, c_void_p, c_int64, c_void_p]),
    "dsk_w8_embed": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_float,
                             c_void_p, c_int64, c_void_p]),
    "dsk_qkv_rope_append": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_float,
                                    c_void_p, c_void_p, c_int, c_void_p, c_int, c_int, c_int, c_void_p, c_void_p,
                                    c_void_p, c_void_p, c_void_p, c_void_p]),
    "dsk_qkv_norm_rope_append": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_int, c_int, c_void_p, c_void_p,
                                         c_void_p, c_float, c_void_p, c_void_p, c_int, c_void_p, c_int, c_int, c_int,
                                         c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "dsk_qkv_rope_append_rn": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_float,
                                       c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_void_p, c_void_p,
                                       c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_float, c_void_p]),
    "dsk_attn_ws_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "dsk_attention": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_int, c_float, c_int, c_int, c_float,
                              c_void_p, c_int, c_void_p, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p,
                              c_void_p, c_void_p, c_int, c_void_p, c_size_t, c_void_p]),
    "dsk_qkv_attention": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_float,
                                  c_void_p, c_float, c_int, c_int, c_float, c_void_p, c_int, c_void_p, c_int, c_int,
                                  c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_size_t,
                                  c_void_p]),
    "dsk_accept_greedy": (c_int, [c_void_p, c_int, c_int64, c_int, c_int, c_int64, c_void_p, c_void_p,
                                  c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    "dsk_accept_greedy_static": (c_int, [c_void_p, c_int, c_int64, c_int, c_int, c_int64, c_void_p, c_void_p,
                                         c_void_p, c_void_p, c_void_p, c_void_p]),
    "dsk_accept_ws_bytes": (c_size_t, [c_int, c_int, c_int64]),
    "dsk_accept_ws_init": (c_int, [c_void_p, c_size_t, c_void_p]),
    "dsk_accept_sample": (c_int, [c_void_p, c_void_p, c_int64, c_int, c_int, c_void_p, c_float, c_float, c_int,
                                  c_int, c_uint64, c_uint32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                  c_void_p, c_size_t, c_void_p, c_void_p]),
    "dsk_sample_ws_bytes": (c_size_t, [c_int, c_int64]),
    "dsk_sample_rows": (c_int, [c_void_p, c_int64, c_int, c_float, c_float, c_int, c_int, c_uint64, c_uint32,
                                c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    "dsk_argmax_ws_bytes": (c_size_t, [c_int]),
    "dsk_argmax_rows": (c_int, [c_void_p, c_int, c_int64, c_int64, c_int, c_void_p, c_void_p, c_size_t, c_void_p]),
    "dsk_lens_add": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p]),
    "dsk_prefetch": (c_int, [c_void_p, c_size_t, c_int, c_void_p, c_void_p]),
    "dsk_markov_ws_bytes": (c_size_t, [c_int, c_int64, c_int]),
    "dsk_markov_block": (c_int, [c_void_p, c_int64, c_int, c_int, c_int64, c_int, c_void_p, c_void_p, c_void_p,
                                 c_void_p, c_void_p, c_void_p, c_float, c_float, c_int, c_uint64, c_uint32, c_int,
                                 c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    "dsk_row_logprobs": (c_int, [c_void_p, c_int64, c_int, c_int64, c_void_p, c_int, c_void_p, c_void_p, c_void_p,
                                 c_void_p]),
    "dsk_logits_penalize": (c_int, [c_void_p, c_int64, c_int, c_void_p, c_void_p, c_void_p, c_void_p]),
}

DSK_F32, DSK_BF16 = 0, 1
DSK_KV_BF16, DSK_KV_U8 = 0, 1
DSK_EPI_STORE, DSK_EPI_SWIGLU, DSK_EPI_GEGLU, DSK_EPI_PARTIAL, DSK_EPI_RESIDUAL = 0, 1, 2, 3, 4


def _load():
    if not _LIB_PATH.exists():
        raise ImportError(
            f"libdspark_hip.so not found at {_LIB_PATH}: build it with "
            f"`python mlx-dspark_amd/build.py` (there is no CPU fallback)")
    lib = C.CDLL(str(_LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


class HipError(RuntimeError):
    pass


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        msg = lib.dsk_last_error().decode(errors="replace")
        raise HipError(f"{what or 'dsk call'} failed ({rc}): {msg}")


def call(name: str, *args) -> None:
    check(getattr(lib, name)(*args), name)


def stream_ptr():
    """The current torch (HIP) stream as a raw hipStream_t."""
    import torch

    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def ptr(t) -> C.c_void_p:
    """Device pointer of a torch tensor (None -> NULL)."""
    return C.c_void_p(0 if t is None else t.data_ptr())


def exported_symbols() -> list[str]:
    return sorted(SIGNATURES)
