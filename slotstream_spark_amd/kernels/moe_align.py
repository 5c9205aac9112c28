"""Row alignment for the grouped MoE kernel (drop-in for slotstream_spark/kernels/moe_align.py).

Rows are sorted by local expert (stable: inside an expert the order is the row order), each expert's rows are padded
to `block_m` with the sentinel R, and every block of `block_m` positions belongs to one expert. The gfx950 version
(csrc/ss_prefill.hip) ranks rows inside 256-row chunks by comparison and offsets the chunks with a sequential scan
per expert, so it uses no order-dependent atomics; every output size depends only on (R, num_local, block_m).
"""
from __future__ import annotations

import torch

from .. import _lib


def padded_rows(r: int, num_local: int, block_m: int) -> int:
    """Upper bound of the padded length, rounded up to a whole number of blocks (moe_align.py:11-14)."""
    n = r + num_local * (block_m - 1)
    return (n + block_m - 1) // block_m * block_m


def moe_align(local_expert: torch.Tensor, num_local: int, block_m: int, *, workspace: torch.Tensor | None = None):
    """local_expert int32 [R] (-1 = not in the current group) -> (sorted_rows int32 [P], block_expert int32 [P // block_m],
    num_padded int32 [1]) (moe_align.py:17-48)."""
    if local_expert.dtype != torch.int32 or local_expert.dim() != 1:
        raise ValueError("local_expert must be int32 [R]")
    if num_local < 1 or block_m < 1:
        raise ValueError("num_local and block_m must be positive")
    if not local_expert.is_cuda:
        raise ValueError("local_expert must be on the GPU")
    r = local_expert.numel()
    dev = local_expert.device
    p = padded_rows(r, num_local, block_m)
    sorted_rows = torch.empty(p, dtype=torch.int32, device=dev)
    block_expert = torch.empty(p // block_m, dtype=torch.int32, device=dev)
    num_padded = torch.empty(1, dtype=torch.int32, device=dev)
    L = _lib.lib()
    nb = L.ssmoe_moe_align_workspace_bytes(r, num_local)
    if workspace is None or workspace.numel() < nb:
        workspace = torch.empty(max(int(nb), 4), dtype=torch.uint8, device=dev)
    _lib.check(L.ssmoe_moe_align(local_expert.contiguous().data_ptr(), r, int(num_local), int(block_m),
                                 workspace.data_ptr(), workspace.numel(), sorted_rows.data_ptr(),
                                 block_expert.data_ptr(), num_padded.data_ptr(), _lib.stream_of(local_expert)))
    return sorted_rows, block_expert, num_padded
