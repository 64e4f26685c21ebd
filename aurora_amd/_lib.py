"""ctypes binding of libaurora_hip.so (the C ABI declared in include/aurora_hip.h).

Loading fails loudly: there is no CPU fallback for any entry point.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libaurora_hip.so"

_c_ctx = C.c_void_p
_f = C.c_void_p  # device pointers travel as integers
_u32 = C.c_uint32
_i32 = C.c_int

# name -> (restype, argtypes); mirrors include/aurora_hip.h one to one.
SIGNATURES: dict[str, tuple] = {
    "aur_init": (_i32, [_i32, C.POINTER(C.c_void_p)]),
    "aur_destroy": (_i32, [_c_ctx]),
    "aur_last_error": (C.c_char_p, [_c_ctx]),
    "aur_stream": (C.c_void_p, [_c_ctx]),
    "aur_device_info": (_i32, [_c_ctx, C.c_char_p, C.c_size_t, C.POINTER(_i32)]),
    "aur_malloc": (_i32, [_c_ctx, C.c_size_t, C.POINTER(C.c_void_p)]),
    "aur_free": (_i32, [_c_ctx, C.c_void_p]),
    "aur_h2d": (_i32, [_c_ctx, C.c_void_p, C.c_void_p, C.c_size_t]),
    "aur_d2h": (_i32, [_c_ctx, C.c_void_p, C.c_void_p, C.c_size_t]),
    "aur_d2d": (_i32, [_c_ctx, C.c_void_p, C.c_void_p, C.c_size_t]),
    "aur_memset0": (_i32, [_c_ctx, C.c_void_p, C.c_size_t]),
    "aur_sync": (_i32, [_c_ctx]),
    "aur_event_create": (_i32, [_c_ctx, C.POINTER(C.c_void_p)]),
    "aur_event_record": (_i32, [_c_ctx, C.c_void_p]),
    "aur_event_elapsed_ms": (_i32, [_c_ctx, C.c_void_p, C.c_void_p, C.POINTER(C.c_float)]),
    "aur_event_destroy": (_i32, [_c_ctx, C.c_void_p]),
    "aur_gemm_nn": (_i32, [_c_ctx, _f, _f, _f, _u32, _u32, _u32]),
    "aur_gemm_nt": (_i32, [_c_ctx, _f, _f, _f, _u32, _u32, _u32]),
    "aur_outer_accum": (_i32, [_c_ctx, _f, _f, _f, _u32, _u32, _u32]),
    "aur_outer_accum_noalloc": (_i32, [_c_ctx, _f, _f, _f, _u32, _u32, _u32]),
    "aur_gemm_ex": (_i32, [_c_ctx, _i32, _i32, _f, _u32, _f, _u32, _f, _u32,
                           _u32, _u32, _u32, _i32]),
    "aur_mha_fwd": (_i32, [_c_ctx, _f, _f, _f, _f, _f, _u32, _u32, _u32, _u32]),
    "aur_mha_bwd_ws_bytes": (C.c_size_t, [_u32, _u32, _u32]),
    "aur_mha_bwd": (_i32, [_c_ctx, _f, _f, _f, _f, _f, _f, _f, _f, _f, _f,
                           _u32, _u32, _u32, _u32]),
    "aur_mha_fwd_ex": (_i32, [_c_ctx, _f, _f, _f, _u32, _f, _u32, _f,
                              _u32, _u32, _u32, _u32]),
    "aur_mha_bwd_ex": (_i32, [_c_ctx, _f, _f, _f, _u32, _f, _f, _u32, _f,
                              _f, _f, _f, _u32, _f, _u32, _u32, _u32, _u32]),
    "aur_mha_kv_ws_bytes": (C.c_size_t, [_u32, _u32, _u32]),
    "aur_mha_kv_step": (_i32, [_c_ctx, _f, _f, _f, _f, _f, _u32, _u32, _u32, _u32]),
    "aur_mha_kv_step_batched": (_i32, [_c_ctx, _f, _f, _f, _f, _f, _f, _u32,
                                       _u32, _u32, _u32, _u32]),
    "aur_model_create": (_i32, [_c_ctx, C.c_void_p, _u32, C.POINTER(C.c_void_p)]),
    "aur_model_destroy": (_i32, [C.c_void_p]),
    "aur_model_tensor": (_i32, [C.c_void_p, C.c_char_p, C.c_int32, C.c_int32,
                                C.POINTER(C.c_void_p), C.POINTER(C.c_size_t)]),
    "aur_model_zero_grad": (_i32, [C.c_void_p]),
    "aur_model_step_muon_hybrid": (_i32, [C.c_void_p, C.c_float, C.c_float, C.c_int32, C.c_float,
                                          _u32, C.c_float, C.c_float, C.c_float, C.c_float,
                                          C.c_float]),
    "aur_model_clip_grads_adamw_subset": (_i32, [C.c_void_p, C.c_float, C.POINTER(C.c_float)]),
    "aur_checkpoint_peek": (_i32, [C.c_char_p, C.c_void_p, C.POINTER(_u32), C.POINTER(_u32),
                                   C.POINTER(C.c_uint64)]),
    "aur_model_load_checkpoint": (_i32, [C.c_void_p, C.c_char_p, C.POINTER(_u32),
                                         C.POINTER(C.c_uint64)]),
    "aur_model_save_checkpoint": (_i32, [C.c_void_p, C.c_char_p, _u32, C.c_uint64]),
    "aur_model_train_step_batch": (_i32, [C.c_void_p, C.c_void_p, C.c_void_p, _u32, _u32,
                                          C.POINTER(C.c_float)]),
    "aur_model_train_step_batch_ex": (_i32, [C.c_void_p, C.c_void_p, C.c_void_p, _u32, _u32, _u32,
                                             C.POINTER(C.c_float)]),
    "aur_model_grad_norm": (_i32, [C.c_void_p, C.POINTER(C.c_float)]),
    "aur_model_state_bytes": (_i32, [C.c_void_p, C.POINTER(C.c_size_t)]),
    "aur_model_state_save": (_i32, [C.c_void_p, C.c_void_p, C.c_size_t, C.POINTER(C.c_uint64)]),
    "aur_model_state_load": (_i32, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_uint64]),
    "aur_model_forward": (_i32, [C.c_void_p, C.c_void_p, _u32, _u32, C.c_void_p]),
    "aur_model_eval_step_batch": (_i32, [C.c_void_p, C.c_void_p, C.c_void_p, _u32, _u32,
                                         C.c_void_p]),
    "aur_model_clip_grads": (_i32, [C.c_void_p, C.c_float, C.POINTER(C.c_float)]),
    "aur_model_step_adamw": (_i32, [C.c_void_p, C.c_float, C.c_float, C.c_float, C.c_float,
                                    C.c_float]),
    "aur_model_clip_step_adamw": (_i32, [C.c_void_p, C.c_float, C.c_float, C.c_float, C.c_float,
                                         C.c_float, C.c_float, C.POINTER(C.c_float)]),
    "aur_kv_cache_create": (_i32, [C.c_void_p, _u32, _u32, C.POINTER(C.c_void_p)]),
    "aur_kv_cache_reset": (_i32, [C.c_void_p]),
    "aur_kv_cache_destroy": (_i32, [C.c_void_p]),
    "aur_kv_cache_len": (_i32, [C.c_void_p, C.POINTER(_u32)]),
    "aur_kv_cache_history": (_i32, [C.c_void_p, _u32, C.POINTER(C.c_void_p),
                                    C.POINTER(C.c_void_p)]),
    "aur_model_prefill_kv": (_i32, [C.c_void_p, C.c_void_p, C.c_void_p, _u32, _u32, C.c_void_p]),
    "aur_model_generate_step": (_i32, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                       C.c_void_p]),
    "aur_model_generate_greedy": (_i32, [C.c_void_p, C.c_void_p, _u32, C.c_void_p]),
}


class AuroraError(RuntimeError):
    """A non-zero return code of the C ABI, with aur_last_error's message."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed with code {code}: {msg}")
        self.code = code


_lib = None


def load() -> C.CDLL:
    """Load libaurora_hip.so once and attach the prototypes."""
    global _lib
    if _lib is not None:
        return _lib
    # AUR_LIB: another build of the same library (A/B timing of two builds).
    path = Path(os.environ["AUR_LIB"]) if os.environ.get("AUR_LIB") else LIB_PATH
    if not path.exists():
        raise ImportError(
            f"{path} is missing: build it first (python -c "
            "'import __graft_entry__ as g; g.build()'); there is no CPU fallback")
    lib = C.CDLL(str(path))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def call(ctx_ptr, name: str, *args) -> None:
    """Call an int-returning entry point; raise AuroraError on failure."""
    lib = load()
    rc = getattr(lib, name)(ctx_ptr, *args)
    if rc != 0:
        msg = lib.aur_last_error(ctx_ptr)
        raise AuroraError(name, rc, msg.decode() if msg else "")
