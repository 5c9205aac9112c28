"""Prefill path on the GPU (BASELINE config 3 semantics) against the oracle: moe_align bit for bit, the grouped
gate/up/down within the bf16 rounding of h, the rank-order combine bit for bit, and the routed output within the
north-star bound against the fp64 exact-dequant reference."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from slotstream_spark_amd import _lib
from slotstream_spark_amd.engine.prefill import MoEPrefillLayer
from slotstream_spark_amd.kernels.fused_moe_affine import BLOCK_M, align_rows, combine_rank_order, fused_moe_affine
from slotstream_spark_amd.kernels.moe_align import moe_align
from slotstream_spark_amd.kernels.router import gemm_bf16
from slotstream_spark_amd.memory.synth import LayerWeights, normal_bf16, zipf_bias
from tests.gpu_util import DenseCache, bits, make_pool, rand_ids, rand_weights

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("R,nl,bm,seed", [(0, 4, 64, 0), (1, 1, 64, 1), (37, 5, 4, 2), (1000, 32, 64, 3),
                                          (4099, 7, 16, 4), (20480, 512, 64, 5)])
def test_moe_align_matches_oracle(R, nl, bm, seed):
    print(f"[align] R={R} nl={nl} bm={bm}", flush=True)
    rng = np.random.default_rng(seed)
    le = rng.integers(-1, nl + 1, size=R).astype(np.int32)  # includes -1 and out-of-range entries
    if R > 10000:  # skewed, as Zipf routing makes it
        le = np.minimum(rng.zipf(1.3, size=R) - 1, nl - 1).astype(np.int32)
    s, b, n = moe_align(torch.from_numpy(le).cuda(), nl, bm)
    torch.cuda.synchronize()
    rs, rb, rn = O.moe_align(le, nl, bm)
    assert int(n.item()) == rn
    assert np.array_equal(s.cpu().numpy(), rs)
    assert np.array_equal(b.cpu().numpy(), rb)


def _prefill_case(T, K, E, H, I, seed):
    pool = make_pool(E, H, I, seed=seed)
    x = normal_bf16((T, H), 1.0, seed + 1)
    ids = rand_ids(T, K, E, seed + 2).cuda()
    w = rand_weights(T, K, seed + 3).cuda()
    return pool, x, ids, w


def _oracle_rows(pool, x, ids, w, bf16_weights=True):
    H, I = pool.hidden, pool.inter
    cache = DenseCache(pool)
    dense = {}

    def weights_of(e):
        if e not in dense:
            rec = cache.record(e)
            dense[e] = O.expert_bf16(rec, H, I) if bf16_weights else O.expert_dense(rec, H, I, np.float64)
        return dense[e]
    T, K = ids.shape
    R = T * K
    return O.prefill_rows(O.bf16_to_f32(bits(x)), np.arange(R) // K, w.cpu().numpy().reshape(-1),
                          ids.cpu().numpy().reshape(-1), weights_of)


@pytest.mark.parametrize("T,K,E,H,I", [(50, 4, 16, 256, 128), (64, 10, 512, 2048, 512), (130, 10, 64, 2048, 512)])
def test_moe_prefill_matches_oracle(T, K, E, H, I):
    print(f"[prefill] T={T} K={K} E={E} H={H} I={I}", flush=True)
    pool, x, ids, w = _prefill_case(T, K, E, H, I, 1729 + T)
    lw = LayerWeights(H, E, 64, seed=7)
    layer = MoEPrefillLayer(pool, 0, lw.router_w, lw.sh_gate, lw.sh_up, lw.sh_down, lw.sh_g, top_k=K, max_tokens=T)
    routed = layer.routed_experts(x, ids, w)
    torch.cuda.synchronize()
    assert _lib.device_error() == 0
    h_ref, rows_ref = _oracle_rows(pool, x, ids, w)
    R = T * K
    h = layer.h_buf[:R].float().cpu().numpy()
    rows = layer.out_rows[:R].cpu().numpy()
    same_h = float(np.mean(h == h_ref))
    err_rows = O.rel_l2(rows, rows_ref)
    print(f"h bf16 equal {same_h:.4f}; out_rows rel_l2 {err_rows:.2e}")
    assert same_h > 0.98            # h differs only where fp32 vs fp64 accumulation crosses a bf16 rounding edge
    assert err_rows < 2e-3
    # the combine is the sequential fp32 rank-order sum of the GPU's own rows, bit for bit
    assert np.array_equal(routed.cpu().numpy(), O.combine_rank_order(rows, T, K))
    # north star: within 2e-2 of the fp64 exact-dequant routed output
    _, rows64 = _oracle_rows(pool, x, ids, w, bf16_weights=False)
    err = O.rel_l2(routed.cpu().numpy(), O.combine_rank_order(rows64, T, K))
    print(f"routed vs exact-dequant fp64 rel_l2 {err:.2e}")
    assert err < 2e-2


def test_prefill_rows_independent_of_batch():
    """A row's output depends on that row and its record only (fused_moe_affine.py:1-20 contract)."""
    T, K, E, H, I = 96, 4, 8, 256, 128
    pool, x, ids, w = _prefill_case(T, K, E, H, I, 99)
    lw = LayerWeights(H, E, 64, seed=3)
    layer = MoEPrefillLayer(pool, 0, lw.router_w, lw.sh_gate, lw.sh_up, lw.sh_down, lw.sh_g, top_k=K, max_tokens=T)
    layer.routed_experts(x, ids, w)
    full = layer.out_rows[:T * K].clone()
    half = T // 3
    layer.routed_experts(x[:half].contiguous(), ids[:half].contiguous(), w[:half].contiguous())
    torch.cuda.synchronize()
    assert torch.equal(layer.out_rows[:half * K], full[:half * K])


def test_fused_moe_affine_group_semantics():
    """The reference interface: a group of local experts through expert_map; rows outside it are left alone."""
    T, K, E, H, I = 40, 4, 12, 256, 128
    pool, x, ids, w = _prefill_case(T, K, E, H, I, 5)
    group = [1, 4, 7, 9]
    emap = torch.full((E,), -1, dtype=torch.int32)
    emap[group] = torch.arange(len(group), dtype=torch.int32)
    slots = pool.map.cpu()
    gptr = torch.tensor([int(pool.slot_ptr[int(slots[e])]) for e in group], dtype=torch.int64).cuda()
    R = T * K
    row_expert = ids.reshape(-1).contiguous()
    row_token = (torch.arange(R, device="cuda") // K).to(torch.int32)
    row_weight = w.reshape(-1).contiguous()
    out_rows = torch.full((R, H), 7.0, device="cuda")
    fused_moe_affine(x, row_token, row_weight, emap.cuda(), gptr, out_rows, row_expert=row_expert, inter=I)
    torch.cuda.synchronize()
    _, rows_ref = _oracle_rows(pool, x, ids, w)
    in_group = np.isin(row_expert.cpu().numpy(), group)
    got = out_rows.cpu().numpy()
    assert np.all(got[~in_group] == 7.0)
    assert O.rel_l2(got[in_group], rows_ref[in_group]) < 2e-3
    s, b, n = align_rows(row_expert, emap.cuda(), len(group))
    rs, rb, rn = O.moe_align(np.where(in_group, emap.numpy()[row_expert.cpu().numpy()], -1), len(group), BLOCK_M)
    assert np.array_equal(s.cpu().numpy(), rs) and int(n.item()) == rn


def test_combine_rank_order_bitwise():
    T, K, H = 33, 10, 2048
    g = torch.Generator(device="cuda").manual_seed(1)
    rows = torch.randn((T * K, H), generator=g, device="cuda") * 3
    out = combine_rank_order(rows, T, K)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), O.combine_rank_order(rows.cpu().numpy(), T, K))


def test_prefill_unmapped_expert_flagged():
    T, K, E, H, I = 8, 2, 8, 256, 128
    pool, x, ids, w = _prefill_case(T, K, E, H, I, 11)
    lw = LayerWeights(H, E, 64, seed=2)
    layer = MoEPrefillLayer(pool, 0, lw.router_w, lw.sh_gate, lw.sh_up, lw.sh_down, lw.sh_g, top_k=K, max_tokens=T)
    ids = ids.clone()
    ids[3, 1] = E + 5
    _lib.device_error()
    routed = layer.routed_experts(x, ids, w)
    torch.cuda.synchronize()
    assert _lib.device_error() & 1
    ids_c = ids.cpu().numpy().reshape(-1)
    _, rows_ref = _oracle_rows(pool, x, torch.from_numpy(np.where(ids_c < E, ids_c, -1).reshape(T, K)), w)
    ref = O.combine_rank_order(rows_ref, T, K)
    assert O.rel_l2(routed.cpu().numpy(), ref) < 2e-3


def test_prefill_layer_end_to_end():
    """Router (bf16 MFMA GEMM + device top-k) + routed experts + shared expert at the config-3 shape on a short chunk;
    the GEMMs themselves are checked in test_gpu_dense_gemm.py."""
    T, K, E, H, I = 128, 10, 512, 2048, 512
    pool = make_pool(E, H, I, seed=31)
    lw = LayerWeights(H, E, 512, seed=32)
    bias = zipf_bias(E, 1.1, 1731)
    layer = MoEPrefillLayer(pool, 0, lw.router_w, lw.sh_gate, lw.sh_up, lw.sh_down, lw.sh_g, top_k=K,
                            router_bias=bias, max_tokens=T)
    x = normal_bf16((T, H), 1.0, 33)
    y, ids, w, routed = layer(x)
    torch.cuda.synchronize()
    # routing against the oracle's router tail applied to the GEMM's own logits
    logits = gemm_bf16(x, lw.router_w)
    _, rids, rw = O.router_topk(bits(logits), K, bias.cpu().numpy())
    assert np.array_equal(ids.cpu().numpy(), rids)
    assert np.array_equal(w.cpu().numpy().view(np.uint32), rw.view(np.uint32))
    _, rows_ref = _oracle_rows(pool, x, ids, w)
    assert O.rel_l2(routed.cpu().numpy(), O.combine_rank_order(rows_ref, T, K)) < 2e-3
    # the shared expert's elementwise chain and y, bit for bit, from the GEMMs' own bf16 outputs
    proj = gemm_bf16(x, layer.sh_cat)
    Is = lw.sh_gate.shape[0]
    pb = bits(proj)
    hs_ref = O.shared_hs(pb[:, :Is], pb[:, Is:2 * Is])
    sh = gemm_bf16(torch.from_numpy(hs_ref.view(np.int16)).view(torch.bfloat16).cuda(), lw.sh_down)
    y_ref = O.combine_shared(routed.cpu().numpy(), bits(sh), pb[:, 2 * Is].copy())
    assert np.array_equal(bits(y), y_ref)
    assert torch.isfinite(y.float()).all()


@pytest.mark.parametrize("T,Is,ld", [(1, 8, 17), (37, 512, 1032), (300, 640, 1288)])
def test_shared_hs_bitwise(T, Is, ld):
    g = torch.Generator(device="cuda").manual_seed(T)
    proj = (torch.randn((T, ld), generator=g, device="cuda") * 4).to(torch.bfloat16)
    hs = torch.empty((T, Is), dtype=torch.bfloat16, device="cuda")
    sgl = torch.empty((T,), dtype=torch.bfloat16, device="cuda")
    _lib.check(_lib.lib().ssmoe_shared_hs(proj.data_ptr(), ld, T, Is, hs.data_ptr(), sgl.data_ptr(), 0))
    torch.cuda.synchronize()
    pb = bits(proj)
    assert np.array_equal(bits(hs), O.shared_hs(pb[:, :Is], pb[:, Is:2 * Is]))
    assert np.array_equal(bits(sgl), pb[:, 2 * Is])


@pytest.mark.parametrize("T,H", [(1, 4), (33, 2048), (129, 2560)])
def test_combine_shared_bitwise(T, H):
    g = torch.Generator(device="cuda").manual_seed(H + T)
    routed = torch.randn((T, H), generator=g, device="cuda") * 3
    sh = (torch.randn((T, H), generator=g, device="cuda")).to(torch.bfloat16)
    sgl = (torch.randn((T,), generator=g, device="cuda") * 5).to(torch.bfloat16)
    y = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    _lib.check(_lib.lib().ssmoe_combine_shared(routed.data_ptr(), sh.data_ptr(), sgl.data_ptr(), y.data_ptr(), T, H, 0))
    torch.cuda.synchronize()
    assert np.array_equal(bits(y), O.combine_shared(routed.cpu().numpy(), bits(sh), bits(sgl)))


def test_moe_prefill_config3_full_size():
    """BASELINE config 3 at its own size: 2048 tokens through the config-1 layer (E=512, top-10), routed by the
    oracle's router with the Zipf(1.1) bias, so the head experts hold many 128-row M blocks each (reached through
    block_expert and the XCD-contiguous tile order) and the tail experts a few rows. Every routed row against the
    oracle (fused_moe_affine.py:136-172, moe_sweep.py:80-176 semantics), the combine bit for bit, the routed output
    within the north-star bound of the fp64 exact-dequant reference."""
    T, K, E, H, I = 2048, 10, 512, 2048, 512
    print(f"[prefill config3] T={T} K={K} E={E}", flush=True)
    pool = make_pool(E, H, I, seed=2048)
    lw = LayerWeights(H, E, 512, seed=2049)
    bias = zipf_bias(E, 1.1, 1731)
    x = normal_bf16((T, H), 1.0, 2050)
    _, _, rids, rwt = O.router(bits(x), bits(lw.router_w), K, bias.cpu().numpy())
    counts = np.bincount(rids.reshape(-1), minlength=E)
    print(f"experts touched {int((counts > 0).sum())}, rows of the largest {int(counts.max())}", flush=True)
    assert counts.max() >= 4 * BLOCK_M                       # an expert spanning at least four M blocks
    assert ((counts > 0) & (counts < BLOCK_M)).sum() >= 10   # and many single-block experts
    layer = MoEPrefillLayer(pool, 0, lw.router_w, lw.sh_gate, lw.sh_up, lw.sh_down, lw.sh_g, top_k=K,
                            router_bias=bias, max_tokens=T)
    ids, w = torch.from_numpy(rids).cuda(), torch.from_numpy(rwt).cuda()
    routed = layer.routed_experts(x, ids, w)
    torch.cuda.synchronize()
    assert _lib.device_error() == 0
    cache = DenseCache(pool)
    R = T * K
    xf = O.bf16_to_f32(bits(x))
    h_ref, rows_ref = O.prefill_rows(xf, np.arange(R) // K, rwt.reshape(-1), rids.reshape(-1),
                                     lambda e: O.expert_bf16(cache.record(e), H, I))
    h = layer.h_buf[:R].float().cpu().numpy()
    rows = layer.out_rows[:R].cpu().numpy()
    same_h = float(np.mean(h == h_ref))
    err_rows = O.rel_l2(rows, rows_ref)
    worst = max(O.rel_l2(rows[rids.reshape(-1) == e], rows_ref[rids.reshape(-1) == e]) for e in np.nonzero(counts)[0])
    print(f"h bf16 equal {same_h:.4f}; out_rows rel_l2 {err_rows:.2e}, worst expert {worst:.2e}", flush=True)
    assert same_h > 0.98
    assert err_rows < 2e-3 and worst < 4e-3
    assert np.array_equal(routed.cpu().numpy(), O.combine_rank_order(rows, T, K))
    del h_ref, rows_ref
    _, rows64 = O.prefill_rows(xf, np.arange(R) // K, rwt.reshape(-1), rids.reshape(-1),
                               lambda e: O.expert_dense(cache.record(e), H, I, np.float64))
    err = O.rel_l2(routed.cpu().numpy(), O.combine_rank_order(rows64, T, K))
    print(f"routed vs exact-dequant fp64 rel_l2 {err:.2e}")
    assert err < 2e-2
