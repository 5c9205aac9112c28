"""Grouped affine 4-bit MoE for prefill on gfx950 (drop-in for slotstream_spark/kernels/fused_moe_affine.py).

Two launches over an aligned plan (BLOCK_M = 128): gate/up writes h = silu(x Wg^T) * (x Wu^T) as bf16 [R, I]; down
writes y = (h Wd^T) * w as fp32 [R, H] into `out_rows`. Each block takes 128 sorted rows of one expert and 256 of
its weight rows: the weights are dequantized to bf16(q*s + b) (the reference's _wtile rounding) straight into MFMA
registers, the activation rows are staged in LDS, and bf16 MFMA 16x16x32 accumulates in fp32; the loads of the next
K steps overlap the MFMAs of the current one. Tiles are constants (128 x 256 x 64), never functions of R, so a
row's bits depend on that row and that record only. The reference's BLOCK_M is 64; a plan here is aligned to 128
(align_rows produces it), which only changes the padding, never a row's result.

Differences from the reference interface: the shape is read from the tensors (the reference fixes H 2560, I 640)
and a group may hold up to 4096 experts, because every expert of a layer is resident in HBM and one plan covers
them all (the reference stages groups of at most 32 records from NVMe).
"""
from __future__ import annotations

import torch

from .. import _lib
from .moe_align import moe_align

BLOCK_M = 128
GROUP_MAX = 4096


def align_rows(row_expert: torch.Tensor, expert_map: torch.Tensor, num_local: int):
    """Local expert of every row through `expert_map` (-1 outside the group), aligned to BLOCK_M
    (fused_moe_affine.py:130-133)."""
    local = expert_map[row_expert.long()].to(torch.int32)
    return moe_align(local, num_local, BLOCK_M)


def fused_moe_affine(x, row_token, row_weight, expert_map, group_ptr, out_rows, *, row_expert, h_buf=None,
                     aligned=None, inter: int | None = None):
    """x bf16 [T,H] · row_token int32 [R] · row_weight fp32 [R] · expert_map int32 [E] (local index or -1) ·
    group_ptr int64 [G] record base addresses · out_rows fp32 [R,H] (rows outside the group are left alone) -> None.
    `row_expert` int32 [R] is the global expert of each row; `aligned` may carry an align_rows result and `h_buf`
    a bf16 [R, I] buffer; I comes from h_buf or `inter` (fused_moe_affine.py:136-161)."""
    r = row_token.numel()
    if x.dtype != torch.bfloat16 or x.dim() != 2 or not x.is_contiguous():
        raise ValueError("x must be a contiguous bf16 [T, H] tensor")
    hid = x.shape[1]
    if row_token.dtype != torch.int32 or row_weight.dtype != torch.float32 or row_weight.numel() != r:
        raise ValueError("row_token must be int32 [R] and row_weight fp32 [R]")
    if row_expert.dtype != torch.int32 or row_expert.numel() != r:
        raise ValueError("row_expert must be int32 [R]")
    if expert_map.dtype != torch.int32 or group_ptr.dtype != torch.int64:
        raise ValueError("expert_map must be int32 and group_ptr int64")
    if not 1 <= group_ptr.numel() <= GROUP_MAX:
        raise ValueError(f"a group holds 1..{GROUP_MAX} experts")
    if tuple(out_rows.shape) != (r, hid) or out_rows.dtype != torch.float32 or not out_rows.is_contiguous():
        raise ValueError(f"out_rows must be contiguous fp32 [R, {hid}]")
    if h_buf is None:
        if inter is None:
            raise ValueError("pass h_buf or inter")
        h_buf = torch.empty((r, inter), dtype=torch.bfloat16, device=x.device)
    elif h_buf.dim() != 2 or h_buf.shape[0] != r or h_buf.dtype != torch.bfloat16 or not h_buf.is_contiguous():
        raise ValueError("h_buf must be contiguous bf16 [R, I]")
    if not all(t.is_cuda for t in (x, row_token, row_weight, expert_map, group_ptr, out_rows, h_buf)):
        raise ValueError("all tensors must be on the GPU")
    if aligned is None:
        aligned = align_rows(row_expert, expert_map, group_ptr.numel())
    sorted_rows, block_expert, num_padded = aligned
    _lib.check(_lib.lib().ssmoe_fused_moe_affine(
        x.data_ptr(), row_token.contiguous().data_ptr(), row_weight.contiguous().data_ptr(), sorted_rows.data_ptr(),
        block_expert.data_ptr(), num_padded.data_ptr(), group_ptr.contiguous().data_ptr(), group_ptr.numel(),
        h_buf.data_ptr(), out_rows.data_ptr(), r, x.shape[0], hid, h_buf.shape[1], _lib.stream_of(x)))


def combine_rank_order(out_rows: torch.Tensor, T: int, K: int = 10, out: torch.Tensor | None = None):
    """out_rows fp32 [T*K, H], row = token*K + rank -> fp32 [T, H], summed in router rank order (sequential fp32)
    (fused_moe_affine.py:164-172)."""
    if out_rows.shape[0] != T * K:
        raise ValueError("out_rows must have T*K rows")
    if out_rows.dtype != torch.float32 or out_rows.dim() != 2 or not out_rows.is_contiguous() or not out_rows.is_cuda:
        raise ValueError("out_rows must be a contiguous fp32 GPU tensor")
    hid = out_rows.shape[1]
    if out is None:
        out = torch.empty((T, hid), dtype=torch.float32, device=out_rows.device)
    _lib.check(_lib.lib().ssmoe_combine_rank_order(out_rows.data_ptr(), T, K, hid, out.data_ptr(),
                                                   _lib.stream_of(out_rows)))
    return out
