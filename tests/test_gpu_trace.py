"""The diagnostics switch (ssmoe_set_trace) changes no result: the prefill GEMM pair with per-block stamps on gives the
same bits as with them off, and the stamps describe the launch (one entry per block of the plan, start before end,
valid rows and expert ids those of the plan)."""
import numpy as np
import pytest
import torch

from slotstream_spark_amd import _lib
from slotstream_spark_amd.engine.prefill import MoEPrefillLayer
from slotstream_spark_amd.kernels.fused_moe_affine import BLOCK_M
from slotstream_spark_amd.memory.synth import LayerWeights, normal_bf16
from tests.gpu_util import make_pool, rand_ids, rand_weights

pytestmark = pytest.mark.gpu


def test_prefill_trace_changes_no_bits_and_stamps_the_plan():
    T, K, E, H, I = 300, 4, 8, 256, 128  # several 128-row blocks per expert, 1 gate/up and 1 down N tile
    print(f"[trace] T={T} K={K} E={E} H={H} I={I}", flush=True)
    pool = make_pool(E, H, I, seed=41)
    x = normal_bf16((T, H), 1.0, 42)
    ids = rand_ids(T, K, E, 43).cuda()
    w = rand_weights(T, K, 44).cuda()
    lw = LayerWeights(H, E, 64, seed=45)
    layer = MoEPrefillLayer(pool, 0, lw.router_w, lw.sh_gate, lw.sh_up, lw.sh_down, lw.sh_g, top_k=K, max_tokens=T)
    off = layer.routed_experts(x, ids, w).clone()
    h_off, rows_off = layer.h_buf[:T * K].clone(), layer.out_rows[:T * K].clone()
    buf = torch.zeros(16384, dtype=torch.int64, device="cuda")
    _lib.check(_lib.lib().ssmoe_set_trace(buf.data_ptr(), buf.numel()))
    try:
        on = layer.routed_experts(x, ids, w)
        torch.cuda.synchronize()
    finally:
        _lib.check(_lib.lib().ssmoe_set_trace(None, 0))
    assert torch.equal(on, off)
    assert torch.equal(layer.h_buf[:T * K], h_off) and torch.equal(layer.out_rows[:T * K], rows_off)
    # the plan: rows per expert, padded to whole blocks
    counts = np.bincount(ids.reshape(-1).cpu().numpy(), minlength=E)
    blocks = [(e, min(BLOCK_M, int(c) - BLOCK_M * b)) for e, c in enumerate(counts) for b in range((int(c) + BLOCK_M - 1) // BLOCK_M)]
    tr = buf.cpu().numpy().view(np.uint64)
    for name, base in (("gate/up", 0), ("down", 8192)):
        t = tr[base:base + 8192].reshape(-1, 4)
        t = t[t[:, 0] > 0]
        assert len(t) == len(blocks), name  # one N tile per block at these shapes
        assert np.all(t[:, 1] >= t[:, 0]), name
        got = sorted(((int(v >> np.uint64(32)), int(v & np.uint64(0xFFFFFFFF))) for v in t[:, 2]))
        assert got == sorted(blocks), name
