"""ctypes binding of libatma_hip.so (the C ABI declared in include/atma_hip.h).

torch is imported first on purpose: the library's HIP runtime dependency
(libamdhip64.so.7) then resolves to the copy torch already loaded, so device
pointers and streams are shared with torch.
"""

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (must precede loading the library; see module docstring)

LIB_PATH = Path(__file__).resolve().parent / "libatma_hip.so"
HEADER = Path(__file__).resolve().parent.parent / "include" / "atma_hip.h"

ATMA_F32, ATMA_BF16, ATMA_F16 = 0, 1, 2
DTYPE_CODE = {torch.float32: ATMA_F32, torch.bfloat16: ATMA_BF16, torch.float16: ATMA_F16}

_p, _i64, _i32, _f32, _sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_size_t

# name -> (restype, argtypes); must match include/atma_hip.h
SIGNATURES = {
    "atma_abi_version": (_i32, []),
    "atma_last_error": (ctypes.c_char_p, []),
    "atma_store_kvcache": (_i32, [_p, _i64, _p, _i64, _p, _p, _p, _i64, _i64, _i64, _i32, _p]),
    "atma_polar_attention_fwd": (_i32, [
        _p, _i64, _i64, _i64, _p, _i64, _i64, _i64, _p, _i64, _i64, _i64,
        _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p,
        _i64, _i64, _i64, _i64, _i64, _i64, _i32, _i32, _i64, _i32, _f32, _p]),
    "atma_polar_attention_bwd_prep": (_i32, [_p] * 17 + [_i64, _i64, _i64, _i64, _i32, _i64, _i32, _f32, _p]),
    "atma_polar_bwd_group_sum": (_i32, [_p, _i32, _p, _i64, _i64, _i64, _i32, _p]),
    "atma_polar_bwd_param_grads_workspace_bytes": (_sz, [_i64, _i64]),
    "atma_polar_bwd_param_grads": (_i32, [_p] * 8 + [_i64] * 5 + [_i32, _p, _sz, _p]),
    "atma_polar_attention_bwd": (_i32, [
        _p, _i64, _i64, _i64, _p, _i64, _i64, _i64, _p, _i64, _i64, _i64, _p, _i64, _i64, _i64,
        _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _i32, _i64,
        _p]),
    "atma_polar_attention_packed_fwd": (_i32, [
        _p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _p, _p, _p, _i64,
        _p, _p, _p, _p, _p, _p, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _i64,
        _f32, _p]),
    "atma_polar_decode_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64, _i64, _i64, _i32]),
    "atma_polar_attention_decode": (_i32, [
        _p, _i64, _i64, _p, _p, _i64, _i64, _i64, _p, _i64, _i64, _p,
        _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i32, _i64, _f32, _p, _sz, _p]),
    "atma_polar_decode_noalloc_max_bytes": (_sz, []),
    "atma_polar_attention_decode_noalloc": (_i32, [
        _p, _i64, _i64, _p, _p, _i64, _i64, _i64, _p, _i64, _i64, _p,
        _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i32, _i64, _f32, _p]),
    "atma_gated_delta_decode_step": (_i32, [
        _p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _p, _p, _p, _i64, _p, _p,
        _i64, _i64, _i64, _i64, _i64, _i32, _f32, _p]),
    "atma_global_decode_step_supported": (_i32, [_i64, _i64, _i64, _i64, _i64, _i64, _i32]),
    "atma_global_decode_step": (_i32, [
        _p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _p, _p, _i64, _i64, _i64, _p, _p, _i64, _i64,
        _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _p, _p, _i64, _i64, _i64, _i32, _i64,
        _f32, _f32, _p, _sz, _p]),
    "atma_gated_delta_bwd_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64, _i64]),
    "atma_gated_delta_bwd": (_i32, [_p] * 14 + [_i64] * 5 + [_p, _sz, _p]),
    "atma_gated_delta_bwd16_prep": (_i32, [_p] * 17 + [_i64] * 4 + [_f32, _i32, _i32, _p]),
    "atma_gated_delta_bwd16_chain": (_i32, [_p] * 17 + [_i64] * 3 + [_i32, _p]),
    "atma_gated_delta_bwd16_local": (_i32, [_p] * 18 + [_i64] * 4 + [_i32, _p]),
    "atma_squared_relu_gate": (_i32, [_p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _i32, _p]),
    "atma_softcap_logits": (_i32, [_p, _p, _i64, _i32, _p]),
    "atma_softcap_argmax": (_i32, [_p, _i64, _p, _i64, _p, _i64, _i64, _i32, _p]),
    "atma_linear_tokens_supported": (_i32, [_i64, _i64, _i64, _i32]),
    "atma_linear_tokens": (_i32, [_p, _i64, _p, _i64, _p, _p, _i64, _i64, _i64, _i64, _i32, _p]),
    "atma_linear_tokens_multi": (_i32, [_p, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _p, _p, _i32, _p]),
    "atma_linear_tokens_gated": (_i32, [_p, _i64, _p, _i64, _p, _p, _i64, _i64, _i64, _i64, _i32, _p]),
    "atma_linear_gated": (_i32, [_p, _i64, _p, _i64, _p, _p, _i64, _i64, _i64, _i64, _i32, _p]),
    "atma_linear_tokens_conv": (_i32, [_p, _i64, _p, _i64, _p, _p, _i64, _p, _p, _i64, _i64, _p, _i64, _i64, _i64,
                                       _i64, _i32, _p]),
    "atma_linear_tokens_chunks": (_i32, [_p, _i64, _i64, _i64, _i64, _p, _p, _i64, _p, _i32, _p]),
    "atma_residual_rms_norm": (_i32, [_p, _i64, _p, _i64, _p, _i64, _p, _i64, _p, _i64, _p, _i64, _p, _i64,
                                      _p, _p, _i64, _i64, _i64, _f32, _i32, _p]),
    "atma_lfm2_conv_step": (_i32, [_p, _i64, _p, _i64, _p, _p, _i64, _i64, _p, _i64, _i64, _i64, _i32, _p]),
    "atma_global_decode_prep": (_i32, [_p, _i64, _i64, _i64, _i64, _i64, _p, _p, _p, _i64, _p, _i64, _p, _i64,
                                       _p, _i64, _i64, _p, _p, _p, _p, _p, _p, _f32, _f32, _f32, _i64, _i64,
                                       _i64, _i64, _i32, _p]),
    "atma_global_decode_gate": (_i32, [_p, _p, _p, _i64, _i64, _p, _i64, _f32, _i64, _i64, _i64, _i32, _p]),
    "atma_head_rms_norm": (_i32, [_p, _i64, _i64, _p, _i64, _i64, _i64, _f32, _i32, _p]),
    "atma_global_gate": (_i32, [_p, _i64, _i64, _i64, _i64, _p, _i64, _i64, _p, _i64, _i32, _p, _i64, _p, _i64,
                                _p, _i64, _i64, _i64, _i64, _f32, _i32, _p]),
    "atma_lfm2_conv_packed": (_i32, [_p, _i64, _p, _i64, _p, _i64, _p, _i64, _i64, _p, _p, _p, _i64, _i64,
                                     _i32, _p]),
    "atma_packed_causal_conv1d": (_i32, [
        _p, _i64, _i64, _p, _i64, _i64, _p, _p, _i64, _i64, _i64, _i64, _p, _p, _p, _i64, _i64, _i64,
        _i32, _i32, _p]),
    "atma_causal_conv1d_decode_step": (_i32, [
        _p, _i64, _p, _i64, _i64, _p, _p, _i64, _i64, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i32,
        _i32, _p]),
    "atma_gated_delta_gates": (_i32, [_p, _p, _f32, _f32, _p, _p, _i64, _i32, _p]),
    "atma_chunk_gated_delta_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64, _i64, _i64, _i32]),
    "atma_chunk_gated_delta_rule": (_i32, [
        _p, _i64, _i64, _i64, _p, _i64, _i64, _i64, _p, _i64, _i64, _i64,
        _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _f32, _i32, _i32, _f32, _f32,
        _i64, _p, _sz, _p, _i32, _p]),
    "atma_wait_start_flag": (_i32, [_p, _i32, _i64, _p]),
}

_lock = threading.Lock()
_lib = None


class HipLibraryMissing(ImportError, RuntimeError):
    """libatma_hip.so is not built (or failed to load).

    An ImportError, so that importing the ops package without the library fails the
    way a missing kernel backend fails in the reference (its callers guard the import
    with ``try/except`` and take their eager path); also a RuntimeError for callers
    that load the library lazily."""


def load():
    """Load (once) and return the ctypes handle; raise if the library is absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise HipLibraryMissing(
                    f"{LIB_PATH} is not built; run `python -m atma_amd._build` (hipcc, gfx950)")
            try:
                lib = ctypes.CDLL(str(LIB_PATH))
            except OSError as e:
                raise HipLibraryMissing(f"failed to load {LIB_PATH}: {e}") from e
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def available() -> bool:
    try:
        load()
        return True
    except HipLibraryMissing:
        return False


def check(rc: int, what: str):
    if rc != 0:
        msg = load().atma_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (code {rc}): {msg}")


def ptr(t):
    """Device address of a tensor (None -> NULL)."""
    return None if t is None else t.data_ptr()


def stream_handle(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def dtype_code(dtype) -> int:
    try:
        return DTYPE_CODE[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype} (float32, bfloat16, float16)") from None
