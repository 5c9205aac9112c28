"""Decode / verify MoE for one step, MLX affine 4-bit gs64 (q*s + b, fp32 accumulate), on gfx950.

Drop-in for slotstream_spark/kernels/moe_gemv_affine.py: same function, arguments, buffers and ValueError
conventions, parametrised by the shape instead of the reference's fixed (2560, 640, 10). The expert record of e
is read at slot_ptr[map[layer * E + e]] in the reference piece layout (gate.w gate.s gate.b up.w up.s up.b down.w
down.s down.b). h_buf receives h = silu(Wg x) * (Wu x), o_buf the weighted expert outputs (Wd h) * w, out their
router-rank-order sum; no atomics, so a T-row call equals T one-row calls bit for bit and moving a record between
slots changes no bit (moe_gemv_affine.py:1-13).

The persistent kernel (csrc/ss_verify.hip, decode mode) streams each weight row with 16-byte loads, turns nibbles
into bf16 1 + q/16 in registers and runs bf16 MFMA 16x16x32 with the per-group scale and bias applied to the fp32
partials (w x = 16 s (sum (1 + q/16) x) + (b - 16 s) sum x); there are no tunable tiles, so `cfg` is validated like
the reference's and otherwise ignored.
"""
from __future__ import annotations

import torch

from .. import _lib

HID, INTER, TOPK = 2048, 512, 10          # BASELINE shape (the reference model uses 2560, 640, 10)
GS = 64
EXPERTS_PER_LAYER = 512


def record_layout(hidden: int = HID, inter: int = INTER):
    """(offsets of the nine pieces, record bytes); 1,769,472 B at (2048, 512)."""
    return _lib.record_layout(hidden, inter)


def __getattr__(name):
    # Lazily expose the reference's layout constants (RECORD_BYTES, O_GATE_W, ...) at the BASELINE shape.
    names = ("O_GATE_W", "O_GATE_S", "O_GATE_B", "O_UP_W", "O_UP_S", "O_UP_B", "O_DOWN_W", "O_DOWN_S", "O_DOWN_B")
    if name == "RECORD_BYTES" or name in names:
        offs, total = record_layout()
        if name == "RECORD_BYTES":
            return total
        return offs[names.index(name)]
    raise AttributeError(name)


def moe_decode(x, expert_ids, weights, layer: int, map_t, slot_ptr_t, h_buf, o_buf, out, cfg=None, *,
               experts_per_layer: int = EXPERTS_PER_LAYER):
    """x [R,H] bf16|fp32 · expert_ids int32 [R,K] (device) · weights fp32 [R,K] · map_t int32 [L*E] ·
    slot_ptr_t int64 [n_slots] · h_buf [R,K,I] f32 · o_buf [R,K,H] f32 · out [R,H] f32 -> out.
    (slotstream_spark/kernels/moe_gemv_affine.py:113-147)"""
    if x.dim() != 2 or not x.is_contiguous() or x.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("x must be a contiguous [R, H] bf16 or fp32 tensor")
    r, hid = x.shape
    if expert_ids.dim() != 2 or expert_ids.shape[0] != r or expert_ids.dtype != torch.int32 \
            or not expert_ids.is_contiguous():
        raise ValueError("expert_ids must be contiguous int32 [R, K]")
    topk = expert_ids.shape[1]
    if tuple(weights.shape) != (r, topk) or weights.dtype != torch.float32 or not weights.is_contiguous():
        raise ValueError(f"weights must be contiguous fp32 [R, {topk}]")
    if map_t.dtype != torch.int32 or slot_ptr_t.dtype != torch.int64:
        raise ValueError("map_t must be int32 and slot_ptr_t int64")
    if h_buf.dim() != 3:
        raise ValueError(f"buffer must be contiguous fp32 ({r}, {topk}, I)")
    inter = h_buf.shape[2]
    for t, shape in ((h_buf, (r, topk, inter)), (o_buf, (r, topk, hid)), (out, (r, hid))):
        if tuple(t.shape) != shape or t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError(f"buffer must be contiguous fp32 {shape}")
    if cfg is not None:
        c = dict(cfg)
        if c.get("bk", 64) % 64 or c.get("bkd", 64) % 64:
            raise ValueError("bk and bkd must be multiples of 64")
    tensors = (x, expert_ids, weights, map_t, slot_ptr_t, h_buf, o_buf, out)
    if not all(t.is_cuda for t in tensors) or len({t.device for t in tensors}) != 1:
        raise ValueError("all tensors must be on the same GPU")
    L = _lib.lib()
    _lib.check(L.ssmoe_moe_decode(
        x.data_ptr(), 1 if x.dtype == torch.float32 else 0, expert_ids.data_ptr(), weights.data_ptr(), int(layer),
        map_t.data_ptr(), map_t.numel(), slot_ptr_t.data_ptr(), slot_ptr_t.numel(), h_buf.data_ptr(),
        o_buf.data_ptr(), out.data_ptr(), r, hid, inter, topk, int(experts_per_layer), _lib.stream_of(x)))
    return out
