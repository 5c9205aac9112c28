"""Dense operations of the MTP draft head on gfx950 (the `lin` / norm / hyper-connection calls of
slotstream_spark/engine/mtp.py:184-227 and model/layers.py:190-198, attention excluded).

Each op is one launch of libssmoe.so with a fixed fp32 reduction order and torch's bf16 rounding points, row by row,
so an S-row call equals S one-row calls bit for bit:

  rmsnorm(x, w, eps, group)      R.rmsnorm (model/reference_torch.py:30-38), per group of `group` elements
  lin_epi(x, w, epi, ...)        lin on a bf16 weight (model/layers.py:62-76) with the op after it fused
  hc_mean(m, hn, hc)             (m * hn.unflatten(-1, (hc, H))).mean(dim=-2)       (model/layers.py:195)
  hc_inject(hyp, y, inj)         hyp + (y.unsqueeze(-2) * inj.unsqueeze(-1)).flatten(-2)  (engine/mtp.py:226)
  gather_rows(src, idx, add)     src[idx + add] with the index read on the device (embed([tok]), engine/mtp.py:274)
"""
from __future__ import annotations

import ctypes

import torch

from .. import _lib

EPI_NONE, EPI_ADD, EPI_SILU_DIV, EPI_SIGMOID, EPI_INJECT = range(5)


def _bf16(name: str, t: torch.Tensor, shape=None) -> None:
    if t.dtype != torch.bfloat16 or not t.is_contiguous() or not t.is_cuda:
        raise ValueError(f"{name} must be a contiguous bf16 GPU tensor")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must be {tuple(shape)}, got {tuple(t.shape)}")


def rmsnorm(x: torch.Tensor, w: torch.Tensor | None, eps: float, group: int | None = None,
            out: torch.Tensor | None = None) -> torch.Tensor:
    """x bf16 [R, n] -> bf16((x * r) * w), r per group of `group` (default n) elements of a row."""
    _bf16("x", x)
    if x.dim() != 2:
        raise ValueError("x must be 2-D")
    R, n = x.shape
    g = n if group is None else int(group)
    if w is not None:
        _bf16("w", w)
        if w.numel() != n:
            raise ValueError(f"w must hold {n} elements")
    out = torch.empty_like(x) if out is None else out
    _bf16("out", out, (R, n))
    _lib.check(_lib.lib().ssmoe_rmsnorm(x.data_ptr(), _lib.ptr(w), float(eps), R, n, g, out.data_ptr(),
                                        _lib.stream_of(x)))
    return out


def lin_epi(x: torch.Tensor, w: torch.Tensor, epi: int = EPI_NONE, hc: int = 1, add: torch.Tensor | None = None,
            add_div: int = 1, out: torch.Tensor | None = None) -> torch.Tensor:
    """x bf16 [R, K] @ w bf16 [N, K]^T rounded to bf16, then the EPI_* op -> bf16 [R, N]."""
    _bf16("x", x)
    _bf16("w", w)
    if x.dim() != 2 or w.dim() != 2 or x.shape[1] != w.shape[1]:
        raise ValueError("x [R, K] and w [N, K] must share K")
    R, N = x.shape[0], w.shape[0]
    if epi == EPI_ADD:
        if add is None:
            raise ValueError("EPI_ADD needs `add`")
        _bf16("add", add, ((R + add_div - 1) // add_div, N))
    out = torch.empty((R, N), dtype=torch.bfloat16, device=x.device) if out is None else out
    _bf16("out", out, (R, N))
    _lib.check(_lib.lib().ssmoe_dense_gemv_epi(x.data_ptr(), R, x.shape[1], w.data_ptr(), N, int(epi), int(hc),
                                               _lib.ptr(add), int(add_div), out.data_ptr(), _lib.stream_of(x)))
    return out


class _HeadGemvArgs(ctypes.Structure):
    _fields_ = [("src", ctypes.c_void_p), ("src_idx", ctypes.c_void_p), ("n_src", ctypes.c_int64),
                ("inj_y", ctypes.c_void_p), ("inj", ctypes.c_void_p), ("inj_hc", ctypes.c_int),
                ("norm_w", ctypes.c_void_p), ("eps", ctypes.c_float), ("group", ctypes.c_int), ("S", ctypes.c_int),
                ("n", ctypes.c_int), ("K", ctypes.c_int), ("w", ctypes.c_void_p), ("N", ctypes.c_int),
                ("epi", ctypes.c_int), ("hc", ctypes.c_int), ("add", ctypes.c_void_p), ("add_div", ctypes.c_int),
                ("out", ctypes.c_void_p), ("w2", ctypes.c_void_p), ("N2", ctypes.c_int), ("epi2", ctypes.c_int),
                ("out2", ctypes.c_void_p), ("h_out", ctypes.c_void_p), ("x_out", ctypes.c_void_p),
                ("mean_hn", ctypes.c_void_p), ("mean_out", ctypes.c_void_p)]


def head_gemv(src: torch.Tensor, w: torch.Tensor, out: torch.Tensor, *, S: int, n: int, K: int,
              src_idx: torch.Tensor | None = None, inj: torch.Tensor | None = None, inj_y: torch.Tensor | None = None,
              inj_hc: int = 1, norm_w: torch.Tensor | None = None, eps: float = 1e-6, group: int = 0,
              epi: int = EPI_NONE, hc: int = 1, add: torch.Tensor | None = None, add_div: int = 1,
              w2: torch.Tensor | None = None, out2: torch.Tensor | None = None, epi2: int = EPI_NONE,
              h_out: torch.Tensor | None = None, x_out: torch.Tensor | None = None,
              mean_hn: torch.Tensor | None = None, mean_out: torch.Tensor | None = None) -> torch.Tensor:
    """One launch of the head's fused dense step (ssmoe_head_gemv): S source rows of n (src [S, n], or rows
    src_idx of the table src), optionally injected (hc_inject) and normalized (rmsnorm over groups of `group`), then
    the GEMV over them viewed as [S n / K, K] with w (and w2 for extra rows into out2), or with the branch mean
    (hc_mean with mean_hn) into mean_out. Bit for bit the separate calls."""
    for name, t in (("src", src), ("w", w), ("out", out)):
        _bf16(name, t)
    for name, t in (("inj_y", inj_y), ("norm_w", norm_w), ("add", add), ("w2", w2), ("out2", out2),
                    ("h_out", h_out), ("x_out", x_out), ("mean_hn", mean_hn), ("mean_out", mean_out), ("inj", inj)):
        if t is not None:
            _bf16(name, t)
    if src_idx is not None and (src_idx.dtype != torch.int32 or not src_idx.is_cuda or src_idx.numel() < S):
        raise ValueError(f"src_idx must be a GPU int32 tensor of at least {S} entries")
    a = _HeadGemvArgs(src.data_ptr(), _lib.ptr(src_idx), src.shape[0] if src_idx is not None else 0,
                      _lib.ptr(inj_y), _lib.ptr(inj), int(inj_hc), _lib.ptr(norm_w), float(eps), int(group), int(S),
                      int(n), int(K), w.data_ptr(), w.shape[0], int(epi), int(hc), _lib.ptr(add), int(add_div),
                      out.data_ptr(), _lib.ptr(w2), w2.shape[0] if w2 is not None else 0, int(epi2), _lib.ptr(out2),
                      _lib.ptr(h_out), _lib.ptr(x_out), _lib.ptr(mean_hn), _lib.ptr(mean_out))
    _lib.check(_lib.lib().ssmoe_head_gemv(ctypes.byref(a), _lib.stream_of(src)))
    return out


def hc_mean(m: torch.Tensor, hn: torch.Tensor, hc: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """m, hn bf16 [S, hc H] -> bf16 [S, H]: the mean over the hc branches of bf16(m * hn)."""
    _bf16("m", m)
    _bf16("hn", hn, m.shape)
    S, n = m.shape
    if n % hc:
        raise ValueError(f"row width {n} is not a multiple of hc={hc}")
    H = n // hc
    out = torch.empty((S, H), dtype=torch.bfloat16, device=m.device) if out is None else out
    _bf16("out", out, (S, H))
    _lib.check(_lib.lib().ssmoe_hc_mean(m.data_ptr(), hn.data_ptr(), S, hc, H, out.data_ptr(), _lib.stream_of(m)))
    return out


def hc_inject(hyp: torch.Tensor, y: torch.Tensor, inj: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """hyp bf16 [S, hc H] + (y [S, H] per branch scaled by inj [S, hc]) -> bf16 [S, hc H] (out may be hyp)."""
    _bf16("hyp", hyp)
    S, hc = inj.shape
    H = y.shape[1]
    _bf16("y", y, (S, H))
    _bf16("inj", inj, (S, hc))
    if tuple(hyp.shape) != (S, hc * H):
        raise ValueError(f"hyp must be [{S}, {hc * H}]")
    out = torch.empty_like(hyp) if out is None else out
    _bf16("out", out, hyp.shape)
    _lib.check(_lib.lib().ssmoe_hc_inject(hyp.data_ptr(), y.data_ptr(), inj.data_ptr(), S, hc, H, out.data_ptr(),
                                          _lib.stream_of(hyp)))
    return out


def gather_rows(src: torch.Tensor, idx: torch.Tensor, idx_add: int = 0, out: torch.Tensor | None = None) -> torch.Tensor:
    """src [N, ...] rows idx[i] + idx_add (idx int32 on the device, read by the kernel) -> [len(idx), ...]. An index
    outside [0, N) gives a zero row and raises SSMOE_ERR_TOKEN in the device status."""
    if not src.is_cuda or not src.is_contiguous() or not idx.is_cuda or idx.dtype != torch.int32:
        raise ValueError("src must be a contiguous GPU tensor and idx a GPU int32 tensor")
    if not idx.is_contiguous():
        raise ValueError("idx must be contiguous")
    n = idx.numel()
    row_bytes = src[0].numel() * src.element_size()
    out = torch.empty((n, *src.shape[1:]), dtype=src.dtype, device=src.device) if out is None else out
    if out.dtype != src.dtype or tuple(out.shape[1:]) != tuple(src.shape[1:]) or out.shape[0] != n \
            or not out.is_contiguous():
        raise ValueError(f"out must be contiguous {src.dtype} {(n, *src.shape[1:])}")
    _lib.check(_lib.lib().ssmoe_gather_rows(src.data_ptr(), src.shape[0], row_bytes, idx.data_ptr(), n, int(idx_add),
                                            out.data_ptr(), _lib.stream_of(src)))
    return out
