"""The fused MoE verify layer (router + routed experts + shared expert) on the GPU at BASELINE configs 0 and 1,
against the oracle: router ids and weights bit for bit, y within the north-star bound (2e-2 relative on bf16),
and against the torch CPU restatement of the reference's moe_ref."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from slotstream_spark_amd.engine.verify import MoEVerifyLayer
from slotstream_spark_amd.memory.synth import LayerWeights, normal_bf16, zipf_bias
from tests.gpu_util import DenseCache, bits, make_pool

pytestmark = pytest.mark.gpu

REL_Y = 2e-2      # MoE outputs within 2e-2 relative on bf16


def _layer(experts, k, seed, bias):
    pool = make_pool(experts, 2048, 512, seed=seed)
    lw = LayerWeights(2048, experts, 512, seed=seed)
    b = zipf_bias(experts, 1.1, 1731) if bias else None
    return pool, lw, MoEVerifyLayer(pool, 0, lw.router_w, lw.sh_gate, lw.sh_up, lw.sh_down, lw.sh_g, top_k=k,
                                    router_bias=b), b


def _oracle_y(pool, lw, x, k, bias):
    xb = bits(x)
    _, _, ids, w = O.router(xb, bits(lw.router_w), k, None if bias is None else bias.cpu().numpy())
    routed = O.moe_routed_fp64(O.bf16_to_f32(xb), ids, w, DenseCache(pool)).astype(np.float32)
    sh, sgl = O.shared_expert(xb, bits(lw.sh_gate), bits(lw.sh_up), bits(lw.sh_down), bits(lw.sh_g))
    return ids, w, routed, O.combine_shared(routed, sh, sgl)


@pytest.mark.parametrize("experts,k,bias,t", [(64, 4, False, 2), (512, 10, True, 2), (512, 10, True, 4),
                                             (512, 10, False, 1)])
def test_verify_layer_vs_oracle(experts, k, bias, t):
    print(f"[verify] E={experts} K={k} bias={bias} T={t}", flush=True)
    pool, lw, layer, b = _layer(experts, k, 1729 + experts, bias)
    x = normal_bf16((t, 2048), 1.0, 1730 + t)
    routed = torch.empty((t, 2048), dtype=torch.float32, device="cuda")
    y, ids, w = layer(x, routed=routed)
    torch.cuda.synchronize()
    rids, rw, rrouted, ry = _oracle_y(pool, lw, x, k, b)
    assert np.array_equal(ids.cpu().numpy(), rids)
    assert np.array_equal(w.cpu().numpy().view(np.uint32), rw.view(np.uint32))
    err_r = O.rel_l2(routed.cpu().numpy(), rrouted)
    err_y = O.rel_l2(O.bf16_to_f32(bits(y)), O.bf16_to_f32(ry))
    same = float(np.mean(bits(y) == ry))
    print(f"routed rel_l2 {err_r:.3e}; y rel_l2 {err_y:.3e}; y bf16 bits equal {same:.4f}")
    assert err_r <= 1e-4
    assert err_y <= REL_Y


def test_verify_layer_vs_torch_moe_ref():
    """Against the torch CPU restatement of reference_torch.moe_ref (config 0 shape, no bias)."""
    pool, lw, layer, _ = _layer(64, 4, 99, False)
    x = normal_bf16((2, 2048), 1.0, 5)
    y, ids, w = layer(x)
    torch.cuda.synchronize()
    dense = DenseCache(pool)

    def expert(e):
        return tuple(torch.from_numpy(d.astype(np.float32)) for d in dense(e))

    yr, ti, tv = O.moe_ref(x.cpu(), lw.router_w.cpu(), 4, expert, lw.sh_gate.cpu(), lw.sh_up.cpu(),
                           lw.sh_down.cpu(), lw.sh_g.cpu())
    assert np.array_equal(ids.cpu().numpy(), ti.numpy().astype(np.int32))
    err = O.rel_l2(y.float().cpu().numpy(), yr.float().numpy())
    print(f"y vs torch moe_ref rel_l2 {err:.3e}")
    assert err <= REL_Y


def test_verify_rows_independent():
    """A 2-token call equals two 1-token calls bit for bit (graphs.py 3-row == 3 x 1-row, tests/gates/test_h3.py)."""
    _, _, layer, _ = _layer(512, 10, 7, True)
    x = normal_bf16((2, 2048), 1.0, 8)
    y2, i2, w2 = layer(x)
    for t in range(2):
        y1, i1, w1 = layer(x[t:t + 1].contiguous())
        assert torch.equal(y1[0], y2[t]) and torch.equal(i1[0], i2[t]) and torch.equal(w1[0], w2[t])
