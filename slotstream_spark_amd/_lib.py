"""ctypes binding of libssmoe.so (the C ABI declared in include/ssmoe.h).

The library is built in-tree by slotstream_spark_amd.build. There is no fallback: a missing or stale library raises
at the first call, so nothing can silently run another code path.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libssmoe.so"
ABI_VERSION = 1

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_F = ctypes.c_float

# name -> (restype, argtypes); the exact export list of include/ssmoe.h.
SIGNATURES = {
    "ssmoe_last_error": (ctypes.c_char_p, []),
    "ssmoe_version": (_I, []),
    "ssmoe_device_error": (_I, [_P, _I]),
    "ssmoe_set_trace": (_I, [_P, _I64]),
    "ssmoe_record_layout": (_I, [_I, _I, _P]),
    "ssmoe_moe_decode": (_I, [_P, _I, _P, _P, _I, _P, _I64, _P, _I64, _P, _P, _P, _I, _I, _I, _I, _I, _P]),
    "ssmoe_topk_stable": (_I, [_P, _P, _P, _P, _I, _I, _I, _P]),
    "ssmoe_dense_gemv_bf16": (_I, [_P, _P, _P, _I, _I, _I, _P]),
    "ssmoe_dense_gemm": (_I, [_P, _I64, _P, _I64, _P, _I64, _I, _I, _I, _P]),
    "ssmoe_router": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "ssmoe_router_topk": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _P]),
    "ssmoe_verify_workspace_bytes": (_I64, [_I, _I, _I, _I, _I, _I]),
    "ssmoe_moe_verify_layer": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _P, _I64, _P, _I64, _P, _I64,
                                    _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P]),
    "ssmoe_moe_verify_layer_chain": (_I, [_P, _P, _F, _P, _P, _P, _P, _P, _P, _I, _P, _I64, _P, _I64, _P, _I64,
                                          _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P]),
    "ssmoe_moe_verify_layer_q4s": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _P, _I64, _P, _I64, _P, _I64,
                                        _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P]),
    "ssmoe_moe_verify_layer_chain_q4s": (_I, [_P, _P, _F, _P, _P, _P, _P, _P, _P, _P, _I, _P, _I64, _P, _I64, _P,
                                              _I64, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P]),
    "ssmoe_verify_chain_workspace_bytes": (_I64, [_I, _I, _I, _I, _I, _I]),
    "ssmoe_moe_verify_chain": (_I, [_P, _F, _P, _P, _I, _P, _I64, _P, _I64, _P, _I64, _I, _I, _I, _I, _I, _I, _P]),
    "ssmoe_moe_verify_layer_noalloc": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _P, _I64, _P, _I64,
                                            _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P]),
    "ssmoe_accept_workspace_bytes": (_I64, [_I, _I]),
    "ssmoe_accept_greedy": (_I, [_P, _P, _I, _I, _P, _I64, _P, _P]),
    "ssmoe_accept_pq": (_I, [_P, _P, _P, _P, _I, _I, _F, _P, _I64, _P, _P]),
    "ssmoe_padded_rows": (_I64, [_I64, _I, _I]),
    "ssmoe_moe_align_workspace_bytes": (_I64, [_I64, _I]),
    "ssmoe_moe_align": (_I, [_P, _I64, _I, _I, _P, _I64, _P, _P, _P, _P]),
    "ssmoe_fused_moe_affine": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _P, _P, _I64, _I, _I, _I, _P]),
    "ssmoe_combine_rank_order": (_I, [_P, _I, _I, _I, _P, _P]),
    "ssmoe_moe_prefill_workspace_bytes": (_I64, [_I64, _I, _I]),
    "ssmoe_moe_prefill": (_I, [_P, _P, _P, _I, _P, _I64, _P, _I64, _P, _I64, _P, _P, _P, _I64, _I, _I, _I, _I, _P]),
    "ssmoe_shared_hs": (_I, [_P, _I64, _I, _I, _P, _P, _P]),
    "ssmoe_combine_shared": (_I, [_P, _P, _P, _P, _I, _I, _P]),
    "ssmoe_residual_rmsnorm": (_I, [_P, _P, _P, ctypes.c_float, _I, _I, _P, _P, _P]),
    "ssmoe_sample_workspace_bytes": (_I64, [_I]),
    "ssmoe_sample": (_I, [_P, _I, _P, _I, _F, _F, _I, _F, _F, _P, _P, _I64, _P, _P]),
    "ssmoe_accept_sampled_workspace_bytes": (_I64, [_I, _I]),
    "ssmoe_sample_rows_workspace_bytes": (_I64, [_I, _I]),
    "ssmoe_bench_stream_read": (_I, [_P, _I64, _P, _I, _P]),
    "ssmoe_bench_mfma_bf16": (_I, [_P, _I, _P, _I, _P]),
    "ssmoe_bf16_round": (_I, [_P, _P, _I64, _P]),
    "ssmoe_sample_rows": (_I, [_P, _I, _I, _F, _P, _P, _I64, _P, _P]),
    "ssmoe_pool_open": (_I, [ctypes.c_char_p, _I, _I, _I64, _I, _I64, _P, _P, ctypes.POINTER(_P)]),
    "ssmoe_pool_close": (_I, [_P]),
    "ssmoe_pool_set_reader": (_I, [_P, _I, _I]),
    "ssmoe_pool_resize": (_I, [_P, _I]),
    "ssmoe_pool_ensure": (_I, [_P, _I, _P, _I, ctypes.c_uint64, _P, _P]),
    "ssmoe_pool_retire_below": (_I, [_P, ctypes.c_uint64]),
    "ssmoe_pool_stats": (_I, [_P, _P]),
    "ssmoe_pool_set_progress": (_I, [_P, _P]),
    "ssmoe_pool_copy_slot": (_I, [_P, _I, _P, _I64]),
    "ssmoe_gemv_affine4": (_I, [_P, _I, _I, _I, _P, _P, _P, _I, _P, _P]),
    "ssmoe_lm_head_greedy_workspace_bytes": (_I64, [_I, _I]),
    "ssmoe_lm_head_greedy": (_I, [_P, _I, _I, _I, _P, _P, _P, _I, _P, _P, _I64, _P, _P, _P]),
    "ssmoe_accept_sampled": (_I, [_P, _P, _I, _I, _P, _I, _F, _F, _I, _F, _F, _P, _P, _I64, _P, _P]),
    "ssmoe_lm_head_pq_workspace_bytes": (_I64, [_I, _I]),
    "ssmoe_lm_head_pq": (_I, [_P, _I, _I, _I, _P, _P, _P, _I, _P, _P, _P, _F, _P, _I64, _P, _P, _P]),
    "ssmoe_lm_head_argmax_workspace_bytes": (_I64, [_I, _I]),
    "ssmoe_lm_head_argmax": (_I, [_P, _I, _I, _I, _P, _P, _P, _I, _I, _P, _I64, _P, _P, _P]),
    "ssmoe_rmsnorm": (_I, [_P, _P, _F, _I, _I, _I, _P, _P]),
    "ssmoe_dense_gemv_epi": (_I, [_P, _I, _I, _P, _I, _I, _I, _P, _I, _P, _P]),
    "ssmoe_hc_mean": (_I, [_P, _P, _I, _I, _I, _P, _P]),
    "ssmoe_head_gemv": (_I, [_P, _P]),
    "ssmoe_hc_inject": (_I, [_P, _P, _P, _I, _I, _I, _P, _P]),
    "ssmoe_gather_rows": (_I, [_P, _I64, _I64, _P, _I, _I, _P, _P]),
}

_lib = None


class SsmoeError(RuntimeError):
    pass


SSMOE_EXHAUSTED, SSMOE_EIO = 3, 4


class Exhausted(SsmoeError):
    """The pool has too few unpinned slots for the request (slotio.Exhausted); nothing changed."""


class IoError(SsmoeError):
    """A record could not be read (slotio.IoError); nothing was published."""


def lib() -> ctypes.CDLL:
    """The loaded library (raises when it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m slotstream_spark_amd.build`")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        if L.ssmoe_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} has ABI {L.ssmoe_version()}, expected {ABI_VERSION}: rebuild it")
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        msg = lib().ssmoe_last_error().decode(errors="replace")
        cls = {SSMOE_EXHAUSTED: Exhausted, SSMOE_EIO: IoError}.get(rc, SsmoeError)
        raise cls(f"ssmoe status {rc}: {msg}")


def ptr(t) -> int | None:
    """Device (or host) address of a tensor, None for None."""
    return None if t is None else t.data_ptr()


def stream_of(t) -> int:
    """The current torch stream on the tensor's device, as a hipStream_t handle."""
    import torch

    return torch.cuda.current_stream(t.device).cuda_stream


def device_error(clear: bool = True) -> int:
    """Status bits raised by kernels on the current device since the last clear (synchronises)."""
    flags = ctypes.c_int(0)
    check(lib().ssmoe_device_error(ctypes.byref(flags), 1 if clear else 0))
    return flags.value


def record_layout(H: int, I: int) -> tuple[list[int], int]:
    """(nine piece offsets, record bytes) of an affine-4bit expert record for hidden H and intermediate I."""
    off = (ctypes.c_int64 * 10)()
    check(lib().ssmoe_record_layout(H, I, off))
    return list(off[:9]), int(off[9])
