"""ssmoe_moe_verify_layer_noalloc (the verify layer on the library's static device scratch) against
ssmoe_moe_verify_layer (the same layer on a caller workspace), both called through the C ABI: ids, weights, y and
the routed sum bit for bit on consecutive calls, each later one with fewer tokens than the one before; shapes beyond
the static scratch are refused before anything is launched."""
import numpy as np
import pytest
import torch

from slotstream_spark_amd import _lib
from slotstream_spark_amd.memory.synth import LayerWeights, normal_bf16, zipf_bias
from tests.gpu_util import make_pool

pytestmark = pytest.mark.gpu

H, I, IS, E, K = 2048, 512, 512, 512, 10


def _outputs(T, dev="cuda"):
    return (torch.full((T, K), -7, dtype=torch.int32, device=dev), torch.full((T, K), -7.0, device=dev),
            torch.zeros((T, H), dtype=torch.bfloat16, device=dev), torch.full((T, H), -7.0, device=dev))


def _args(pool, lw, bias, x):
    return (x.data_ptr(), lw.router_w.data_ptr(), bias.data_ptr(), lw.sh_gate.data_ptr(), lw.sh_up.data_ptr(),
            lw.sh_down.data_ptr(), lw.sh_g.data_ptr(), 0, pool.map.data_ptr(), pool.map.numel(),
            pool.slot_ptr.data_ptr(), pool.slot_ptr.numel())


def test_noalloc_verify_layer_equals_workspace_entry_point():
    L = _lib.lib()
    pool = make_pool(E, H, I, seed=81)
    lw = LayerWeights(H, E, IS, seed=82)
    bias = zipf_bias(E, 1.1, 83)
    ws_bytes = L.ssmoe_verify_workspace_bytes(4, H, I, IS, K, E)
    ws = torch.zeros(int(ws_bytes), dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    for T, seed in ((4, 84), (2, 85), (1, 86)):
        print(f"[noalloc] T={T} E={E} K={K}", flush=True)
        x = normal_bf16((T, H), 1.0, seed)
        ids_a, w_a, y_a, r_a = _outputs(T)
        ids_b, w_b, y_b, r_b = _outputs(T)
        _lib.check(L.ssmoe_moe_verify_layer(*_args(pool, lw, bias, x), ws.data_ptr(), ws.numel(), ids_a.data_ptr(),
                                            w_a.data_ptr(), y_a.data_ptr(), r_a.data_ptr(), T, H, I, IS, K, E, stream))
        _lib.check(L.ssmoe_moe_verify_layer_noalloc(*_args(pool, lw, bias, x), ids_b.data_ptr(), w_b.data_ptr(),
                                                    y_b.data_ptr(), r_b.data_ptr(), T, H, I, IS, K, E, stream))
        torch.cuda.synchronize()
        assert _lib.device_error() == 0
        assert torch.equal(ids_a, ids_b)
        assert np.array_equal(w_a.cpu().numpy().view(np.uint32), w_b.cpu().numpy().view(np.uint32))
        assert torch.equal(y_a.view(torch.int16), y_b.view(torch.int16))
        assert np.array_equal(r_a.cpu().numpy().view(np.uint32), r_b.cpu().numpy().view(np.uint32))
        assert (ids_b >= 0).all() and torch.isfinite(y_b.float()).all()


def test_noalloc_refuses_shapes_beyond_its_scratch():
    L = _lib.lib()
    tables = [None] * 7 + [0, None, 0, None, 0]      # weights, layer, map, map_len, slot_ptr, n_slots
    # I 1024 x K 16 needs about 330 KiB of scratch, more than the 192 KiB the library holds
    rc = L.ssmoe_moe_verify_layer_noalloc(*tables, None, None, None, None, 4, 2048, 1024, 512, 16, 512, None)
    assert rc == 1 and b"no-alloc entry point holds" in L.ssmoe_last_error()
