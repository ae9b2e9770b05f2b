"""ctypes binding of ``libt2i_hip.so`` (the C ABI in ``include/t2i_hip.h``).

The library is built in-tree by ``torch2iron_amd.build``.  Loading fails
loudly (``RuntimeError``) when it is missing: there is no CPU fallback.
``torch`` is imported first so that the process uses torch's HIP runtime; the
library's ``libamdhip64.so.7`` dependency then resolves to that same runtime.
"""

from __future__ import annotations

import ctypes
from ctypes import c_float, c_int32, c_size_t, c_void_p
from pathlib import Path

import torch  # noqa: F401  (must precede the library load, see module docstring)

LIB_PATH = Path(__file__).resolve().parent / "libt2i_hip.so"

T2I_ERR_NULL = -1
T2I_ERR_SHAPE = -2
T2I_ERR_ALIGN = -3
T2I_ERR_GROUP = -4
T2I_ERR_WORKSPACE = -5
T2I_ERR_VALUE = -6
T2I_TILES_STORE = 0
T2I_TILES_SWIGLU = 1
T2I_TILES_PAIRED = 2

# name -> (restype, argtypes); mirrors include/t2i_hip.h
SIGNATURES = {
    "t2i_abi_version": (c_int32, []),
    "t2i_strerror": (ctypes.c_char_p, [c_int32]),
    "t2i_last_error": (ctypes.c_char_p, []),
    "t2i_w4a16_dequant_f32": (c_int32, [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_void_p, c_void_p]),
    "t2i_w4a16_linear": (c_int32, [c_void_p, c_int32, c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32,
                                   c_void_p, c_void_p, c_void_p]),
    "t2i_w4a16_gate_up": (c_int32, [c_void_p, c_int32, c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32,
                                    c_int32, c_void_p, c_void_p, c_void_p]),
    "t2i_w4a16_rmsnorm_linear": (c_int32, [c_void_p, c_int32, c_void_p, c_float, c_void_p, c_void_p, c_void_p,
                                           c_int32, c_int32, c_int32, c_void_p, c_void_p]),
    "t2i_w4a16_rmsnorm_gate_up": (c_int32, [c_void_p, c_int32, c_void_p, c_float, c_void_p, c_void_p, c_void_p,
                                            c_int32, c_int32, c_int32, c_int32, c_void_p, c_void_p, c_void_p]),
    "t2i_w4a16_tile_qweight": (c_int32, [c_void_p, c_int32, c_int32, c_void_p, c_void_p]),
    "t2i_w4a16_linear_tiles": (c_int32, [c_void_p, c_int32, c_void_p, c_float, c_void_p, c_void_p, c_void_p,
                                         c_void_p, c_int32, c_int32, c_int32, c_int32, c_void_p, c_void_p,
                                         c_void_p, c_void_p]),
    "t2i_w4a16_linear_tiles_chain": (c_int32, [c_void_p, c_int32, c_void_p, c_float, c_void_p, c_void_p, c_void_p,
                                               c_void_p, c_int32, c_int32, c_int32, c_int32, c_void_p, c_void_p,
                                               c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "t2i_w4a16_chain_supported": (c_int32, [c_int32, c_int32, c_int32, c_int32]),
    "t2i_rmsnorm": (c_int32, [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_void_p, c_float, c_void_p,
                              c_void_p, c_void_p, c_void_p]),
    "t2i_decode_attention_workspace_bytes": (c_size_t, [c_int32, c_int32, c_int32, c_int32]),
    "t2i_decode_attention": (c_int32, [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32, c_void_p, c_void_p,
                                       c_float, c_void_p, c_int32, c_void_p, c_void_p, c_int32, c_void_p, c_void_p,
                                       c_size_t, c_void_p]),
    "t2i_decode_attention_noalloc": (c_int32, [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32, c_void_p,
                                               c_void_p, c_float, c_void_p, c_int32, c_void_p, c_void_p, c_int32,
                                               c_void_p, c_void_p]),
    "t2i_decode_attention_prepared": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32,
                                                c_int32, c_void_p, c_void_p, c_int32, c_void_p, c_void_p, c_size_t,
                                                c_void_p]),
    "t2i_rmsnorm_rope": (c_int32, [c_void_p, c_int32, c_int32, c_void_p, c_void_p, c_int32, c_float, c_int32,
                                   c_void_p, c_void_p]),
    "t2i_silu_mul": (c_int32, [c_void_p, c_void_p, ctypes.c_int64, c_void_p, c_void_p]),
    "t2i_residual_add_rmsnorm": (c_int32, [c_void_p, c_void_p, c_int32, c_int32, c_void_p, c_float, c_void_p,
                                           c_void_p, c_void_p]),
    "t2i_qkv_attention_workspace_bytes": (c_size_t, [c_int32, c_int32, c_int32]),
    "t2i_qkv_attention_error_offset": (c_size_t, [c_int32, c_int32, c_int32]),
    "t2i_qkv_attention": (c_int32, [c_void_p, c_int32, c_void_p, c_float, c_void_p, c_void_p, c_void_p, c_int32,
                                    c_int32, c_void_p, c_int32, c_int32, c_int32, c_void_p, c_void_p, c_void_p,
                                    c_int32, c_void_p, c_void_p, c_int32, c_void_p, c_void_p, c_size_t, c_void_p]),
    "t2i_decode_step_workspace_bytes": (c_size_t, [c_int32, c_int32, c_int32, c_int32, c_int32, c_int32]),
    "t2i_decode_step_offset": (c_size_t, [c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32]),
    "t2i_decode_step": (c_int32, [c_void_p, c_int32, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32, c_int32,
                                  c_int32, c_int32, c_void_p, c_void_p, c_int32, c_int32, c_float, c_void_p, c_size_t,
                                  c_void_p]),
    "t2i_prefill_qk_rope_kv": (c_int32, [c_void_p, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32,
                                         c_void_p, c_void_p, c_float, c_void_p, c_int32, c_void_p, c_void_p,
                                         c_void_p, c_int32, c_void_p]),
    "t2i_prefill_attention": (c_int32, [c_void_p, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32,
                                        c_void_p, c_void_p, c_int32, c_void_p, c_void_p]),
    "t2i_prefill_qkv_rope_kv": (c_int32, [c_void_p, c_int32, c_int32, c_int32, c_void_p, c_void_p, c_void_p, c_int32,
                                          c_int32, c_int32, c_int32, c_int32, c_void_p, c_void_p, c_float, c_void_p,
                                          c_int32, c_void_p, c_void_p, c_void_p, c_int32, c_void_p]),
    "t2i_rmsnorm_sums": (c_int32, [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_void_p, c_float, c_void_p,
                                   c_void_p, c_void_p, c_void_p]),
    "t2i_prefill_attention_sums": (c_int32, [c_void_p, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32,
                                             c_void_p, c_void_p, c_int32, c_void_p, c_void_p, c_void_p]),
    "t2i_w4a16_linear_sums": (c_int32, [c_void_p, c_void_p, c_int32, c_int32, c_void_p, c_void_p, c_void_p, c_int32,
                                        c_int32, c_int32, c_void_p, c_void_p, c_void_p]),
    "t2i_w4a16_gate_up_sums": (c_int32, [c_void_p, c_void_p, c_int32, c_int32, c_void_p, c_void_p, c_void_p,
                                         c_int32, c_int32, c_int32, c_int32, c_void_p, c_void_p, c_void_p,
                                         c_void_p]),
    "t2i_prefill_qkv_rope_kv_sums": (c_int32, [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_void_p, c_void_p,
                                               c_void_p, c_int32, c_int32, c_int32, c_int32, c_int32, c_void_p,
                                               c_void_p, c_float, c_void_p, c_int32, c_void_p, c_void_p, c_void_p,
                                               c_int32, c_void_p]),
    "t2i_lm_head_argmax": (c_int32, [c_void_p, c_int32, c_void_p, c_int32, c_int32, c_void_p, c_void_p, c_void_p]),
    "t2i_rmsnorm_lm_head_argmax": (c_int32, [c_void_p, c_int32, c_void_p, c_float, c_void_p, c_int32, c_int32,
                                             c_void_p, c_void_p, c_void_p]),
    "t2i_greedy_advance": (c_int32, [c_void_p, c_int32, c_void_p, c_void_p, c_void_p, c_int32, c_void_p, c_void_p]),
    "t2i_prompt_advance": (c_int32, [c_void_p, c_int32, c_int32, c_void_p, c_void_p, c_void_p]),
    "t2i_stream_read_out_words": (ctypes.c_int64, [c_size_t, c_int32]),
    "t2i_stream_read": (c_int32, [c_void_p, c_size_t, c_int32, c_void_p, c_void_p]),
}

_LIB = None


def load() -> ctypes.CDLL:
    """Load the library once; raise RuntimeError if it is not built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -m torch2iron_amd.build` "
            "(the W4A16 path has no CPU fallback)")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def check(rc: int, what: str) -> None:
    """Map ABI return codes to the reference's exception types.

    Negative codes are argument errors -> ``ValueError`` (as the reference's
    operator ``__post_init__`` checks, e.g. ``w4a16_gemm/op.py:55-74``);
    positive codes are HIP errors -> ``RuntimeError`` (as a failed XRT run,
    ``fusion.py:724-726``).
    """
    if rc == 0:
        return
    lib = load()
    msg = lib.t2i_last_error().decode(errors="replace")
    if rc < 0:
        raise ValueError(f"{what}: {lib.t2i_strerror(rc).decode()}: {msg}")
    raise RuntimeError(f"{what}: HIP error {rc}: {msg}")


def ptr(t) -> int | None:
    """Device address of a tensor (``None`` for ``None``)."""
    return None if t is None else t.data_ptr()


def stream_handle(device=None) -> int:
    """hipStream_t of torch's current stream on ``device``."""
    return torch.cuda.current_stream(device).cuda_stream
