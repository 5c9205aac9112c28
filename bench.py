#!/usr/bin/env python3
"""Benchmark of the MTP verify MoE path on one MI355X (BASELINE.json metric, config 1).

One step = a T=2 verify through `--layers` distinct full-size MoE layers (hidden 2048, 512 routed experts top-10,
moe_intermediate 512, shared expert 512, affine-4bit gs64, Zipf(1.1) routing bias, experts in a 512-slot pool
per layer behind a random slot permutation), chained as in a verify step: a residual stream with an RMSNorm before
every MoE layer (no attention), all layers in one persistent launch (ssmoe_moe_verify_chain), a fresh input each
step. With 16 layers the touched bytes (about 33 MB per layer) exceed the 256 MB Infinity Cache, so each layer is
read cold from HBM.

Reported: value = microseconds per layer of the step (lower is better). The dominant kernel is the chain kernel (one
launch per step), so `roofline` is its algorithmic bytes per launch (the sum over its layers of each layer's bytes at
its measured unique-expert count) over its average launch time, both from HIP events around each replay on the
launch's stream. Also reported: the same layers as 16 independent single-layer launches on one input (`isolated`),
the routed-only moe_decode launch (`--legs` decode), measured achievable peaks (device copy, read stream, bf16 GEMM)
beside the spec peaks, and the CPU baseline: the torch-CPU restatement of the reference's moe_ref (oracle.moe_ref),
checked against the reference's fixtures first, timed on this host at config 0 and the config-1 shape.
`--copy-calib` first runs three 256 MiB device-to-device copies, the known-size kernel that scales rocprofv3's
FETCH_SIZE / WRITE_SIZE counters into bytes.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "µs per T=2 MTP verify step per MoE layer + HBM GB/s; prefill TFLOP/s at 2048 tok"
HBM_PEAK_GBS = 8000.0
H, I, E, K, IS = 2048, 512, 512, 10, 512


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def layer_bytes(u: int, t: int) -> int:
    """Algorithmic HBM bytes of one verify layer: u unique experts' affine 4-bit records (1,769,472 B each at H 2048
    / I 512), the router (512 x 2048 bf16), the shared expert's three projections (bf16), the shared gate row and
    the T rows of x read and y written."""
    return u * 1_769_472 + 2_097_152 + 6_291_456 + 4_096 + t * H * 4


PREFILL_T = 2048
# FLOP of one prefill layer (2 per multiply-add): routed gate/up/down over T*K rows, the shared expert's three
# projections and the router, 2 T (K 3 H I + 3 H Is + H E).
PREFILL_ROUTED_FLOP = 2 * PREFILL_T * K * 3 * H * I
PREFILL_FLOP = 2 * PREFILL_T * (K * 3 * H * I + 3 * H * IS + H * E)
MFMA_BF16_PEAK_TFLOPS = 2500.0


def timed_graph(fn, steps, warmup, stream):
    """Capture fn() in a HIP graph, replay it `warmup` times, then time `steps` replays with HIP events recorded on
    the graph's stream. Returns ms per replay."""
    import torch

    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        fn()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        fn()
    with torch.cuda.stream(stream):
        for _ in range(warmup):
            g.replay()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record(stream)
        for _ in range(steps):
            g.replay()
        ev1.record(stream)
    torch.cuda.synchronize()
    return ev0.elapsed_time(ev1) / steps


def prefill_leg(pool, weights, biases, nl, steps, warmup, dev):
    """2048 bf16 tokens through `nl` config-1 layers (each a full prefill layer: router GEMM,
    device top-k, moe_align, grouped gate/up and down, rank-order combine, shared expert), one HIP graph; and the
    grouped GEMM pair alone (ssmoe_fused_moe_affine over each layer's aligned plan), the MFMA-bound kernels."""
    import torch

    from slotstream_spark_amd.engine.prefill import MoEPrefillLayer
    from slotstream_spark_amd.kernels.fused_moe_affine import align_rows, fused_moe_affine
    from slotstream_spark_amd.memory.synth import normal_bf16

    TP = PREFILL_T
    layers = [MoEPrefillLayer(pool, l, w.router_w, w.sh_gate, w.sh_up, w.sh_down, w.sh_g, top_k=K,
                              router_bias=b, max_tokens=TP) for l, (w, b) in enumerate(zip(weights[:nl], biases[:nl]))]
    xp = normal_bf16((TP, H), 1.0, 1733, dev)
    outs = [None] * nl

    def full():
        for l in range(nl):
            outs[l] = layers[l](xp)

    s = torch.cuda.Stream(device=dev)
    ms = timed_graph(full, steps, warmup, s)
    us_layer = ms * 1000.0 / nl
    # the same layers' routing, aligned once, for the GEMM-pair leg
    R = TP * K
    row_token = (torch.arange(R, device=dev) // K).to(torch.int32)
    plans = []
    for l in range(nl):
        ids, w = outs[l][1], outs[l][2]
        row_expert = ids.reshape(-1).contiguous()
        emap = torch.arange(E, dtype=torch.int32, device=dev)
        gptr = pool.slot_ptr[pool.map[l * E:(l + 1) * E].long()].contiguous()
        plans.append((row_expert, w.reshape(-1).contiguous(), emap, gptr, align_rows(row_expert, emap, E)))
    uniq = [int(torch.unique(p[0]).numel()) for p in plans]
    padded = [int(p[4][2].item()) for p in plans]

    def gemms():
        for l in range(nl):
            row_expert, rw, emap, gptr, al = plans[l]
            fused_moe_affine(xp, row_token, rw, emap, gptr, layers[l].out_rows, row_expert=row_expert,
                             h_buf=layers[l].h_buf, aligned=al)

    ms_g = timed_graph(gemms, steps, warmup, s)
    us_g = ms_g * 1000.0 / nl
    tflops = PREFILL_FLOP / (us_layer * 1e-6) / 1e12
    g_tflops = PREFILL_ROUTED_FLOP / (us_g * 1e-6) / 1e12
    wbytes = sum(uniq) / nl * 1_769_472
    log(f"prefill layer {us_layer:.1f} us ({tflops:.1f} TFLOP/s); grouped GEMM pair {us_g:.1f} us "
        f"({g_tflops:.1f} TFLOP/s routed); unique experts {uniq}; padded rows {padded}")
    return {"tokens": TP, "layers": nl, "us_per_layer": round(us_layer, 2), "tflops": round(tflops, 2),
            "flop_per_layer": PREFILL_FLOP, "unique_experts_mean": sum(uniq) / nl,
            "padded_rows_mean": sum(padded) / nl,
            "roofline": {"bound": "mfma", "kernel": "prefill_gemm_kernel<true> + prefill_gemm_kernel<false> (grouped gate/up + down GEMM pair)",
                         "achieved": round(g_tflops, 2), "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(g_tflops / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": traffic_of("prefill_gemm"),
                         "us_per_launch": round(us_g, 2), "flop_per_launch": PREFILL_ROUTED_FLOP,
                         "expert_bytes_per_launch": int(wbytes),
                         "expert_stream_gbs": round(wbytes / (us_g * 1e-6) / 1e9, 1)}}


def verify_chain_leg(pool, weights, biases, nl, t, steps, warmup, dev):
    """BASELINE config 1 as a verify step: T tokens through `nl` chained config-1 layers in one persistent launch
    (ssmoe_moe_verify_chain; each layer on the RMSNorm of the residual stream, the stream += y after it), a new input
    copied in before each step (outside the timed interval). HIP events bracket each replay of the launch's graph on
    its stream. Returns the timing, the layers' unique-expert counts and bytes."""
    import torch

    from slotstream_spark_amd.engine.step import MoEWeights, MTPStepGraph
    from slotstream_spark_amd.memory.synth import normal_bf16

    mw = [MoEWeights(w.router_w, w.sh_gate, w.sh_up, w.sh_down, w.sh_g, b) for w, b in zip(weights[:nl], biases[:nl])]
    sg = MTPStepGraph(pool, mw, None, depth=t - 1, top_k=K, device=dev)
    if sg.chain is None:
        raise RuntimeError("no chain kernel for the config-1 shape on this device")
    xs = normal_bf16((8, t, H), 1.0, 1730, dev)
    s = sg.stream
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        sg.chain.run(sg.streams[0])
    s.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        sg.chain.run(sg.streams[0])
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    snaps = []
    with torch.cuda.stream(s):
        for st in range(warmup):
            sg.x_in.copy_(xs[st % 8])
            g.replay()
        for st in range(steps):
            sg.x_in.copy_(xs[st % 8])
            evs[st][0].record(s)
            g.replay()
            evs[st][1].record(s)
            if st < 8:
                snaps.append(sg.ids.clone())
    torch.cuda.synchronize()
    ms = sum(a.elapsed_time(b) for a, b in evs)
    us_step = ms * 1000.0 / steps
    uniq = [[len(set(sn[l].cpu().flatten().tolist())) for l in range(nl)] for sn in snaps]
    bytes_launch = sum(sum(layer_bytes(u, t) for u in row) for row in uniq) / len(uniq)
    u_mean = sum(map(sum, uniq)) / (len(uniq) * nl)
    gbs = bytes_launch / (us_step * 1e-6) / 1e9
    finite = bool(torch.isfinite(sg.streams[nl].float()).all().item())
    log(f"verify chain: {nl} layers in one launch, {us_step:.1f} us per step = {us_step / nl:.2f} us per layer "
        f"({gbs:.0f} GB/s algorithmic), mean unique experts {u_mean:.1f}, stream finite {finite}")
    del g, sg
    return {"us_per_step": us_step, "us_per_layer": us_step / nl, "bytes_per_launch": bytes_launch,
            "achieved_gbs": gbs, "unique_experts_mean": u_mean, "unique_experts_first_step": uniq[0],
            "stream_finite": finite}


def ref_chain_leg(steps, warmup, dev, nl=16):
    """The verify step at the reference model's MoE layer (model/config.py:8-21: H 2560, 512 experts top-10,
    moe_intermediate 640, shared 640 as affine 4-bit gs64 like the checkpoint's shared_expert projections, bf16 router
    and shared_expert_gate, Zipf 1.1 routing bias), `nl` distinct layers, T = 2 and T = 3 (the reference's verify
    width, 1 + DEPTH): one persistent launch for all layers (ssmoe_moe_verify_chain) against one launch per layer
    (ssmoe_moe_verify_layer_chain), each replayed as a HIP graph with a new input per step."""
    import torch

    from slotstream_spark_amd.engine.step import MoEWeights, MTPStepGraph
    from slotstream_spark_amd.memory.slot_pool import SlotPool
    from slotstream_spark_amd.memory.synth import LayerWeights, normal_bf16, zipf_bias

    HR, IR, ER = 2560, 640, 512
    pool = SlotPool(nl, ER, HR, IR, device=dev)
    pool.fill_random(5101)
    pool.place_permuted(5102)
    mw = []
    for l in range(nl):
        w = LayerWeights(HR, ER, IR, seed=5103 + l, device=dev, shared_q4=True)
        mw.append(MoEWeights(w.router_w, w.sh_gate, w.sh_up, w.sh_down, w.sh_g, zipf_bias(ER, 1.1, 5200 + l,
                                                                                              device=dev)))
    res = {"shape": "H 2560, E 512 top-10, I 640, shared 640 affine 4-bit gs64 (records of 2,764,800 B)",
           "layers": nl}
    for t in (2, 3):
        xs = normal_bf16((8, t, HR), 1.0, 5300 + t, dev)
        out = {}
        for name, single in (("single_launch", True), ("per_layer", False)):
            sg = MTPStepGraph(pool, mw, None, depth=t - 1, top_k=K, single_launch=single, device=dev)
            if single and sg.chain is None:
                raise RuntimeError("no chain kernel at the reference shape on this device")
            for i in range(warmup):
                sg.step(xs[i % 8])
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for i in range(steps):
                sg.step(xs[i % 8])
            e1.record()
            torch.cuda.synchronize()
            out[name] = round(e0.elapsed_time(e1) * 1000.0 / steps / nl, 3)
            del sg
        out["speedup"] = round(out["per_layer"] / out["single_launch"], 3)
        res[f"T{t}_us_per_layer"] = out
        log(f"reference-shape chain T={t}: single launch {out['single_launch']} us/layer, one launch per layer "
            f"{out['per_layer']} us/layer")
    del pool
    torch.cuda.empty_cache()
    return res


def peaks_leg(dev):
    """Measured achievable peaks beside the spec ones: a 1 GiB device copy (2 GiB moved), a 1 GiB fp32 sum (read
    stream) and an 8192^3 bf16 GEMM on the platform BLAS; best of 10 launches each, HIP events."""
    import torch

    def best(fn, reps=10):
        fn()
        torch.cuda.synchronize()
        out = []
        for _ in range(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            torch.cuda.synchronize()
            out.append(e0.elapsed_time(e1) * 1e-3)
        return min(out)

    nb = 1 << 30
    a = torch.empty(nb, dtype=torch.uint8, device=dev).fill_(1)
    b = torch.empty_like(a)
    t_copy = best(lambda: b.copy_(a))
    del a, b
    x = torch.ones(nb // 4, dtype=torch.float32, device=dev)
    t_sum = best(lambda: x.sum())
    del x
    n = 8192
    ga = torch.randn((n, n), device=dev, dtype=torch.bfloat16)
    gb = torch.randn((n, n), device=dev, dtype=torch.bfloat16)
    t_mm = best(lambda: torch.matmul(ga, gb), reps=5)
    del ga, gb
    torch.cuda.empty_cache()
    # this build's own ceilings (ssmoe_bench_stream_read / ssmoe_bench_mfma_bf16, csrc/ss_peaks.hip)
    from slotstream_spark_amd import _lib

    L = _lib.lib()
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    rb = 4 << 30
    buf = torch.ones(rb // 4, dtype=torch.int32, device=dev)
    outw = torch.zeros(cus * 8, dtype=torch.int32, device=dev)
    st = torch.cuda.current_stream(dev).cuda_stream
    t_rd = best(lambda: _lib.check(L.ssmoe_bench_stream_read(buf.data_ptr(), rb, outw.data_ptr(), cus * 8, st)))
    del buf
    seed = torch.tensor([0x3F803F80, 0x3F813F82, 0x3F833F84, 0x3F853F86, 0x3F873F88, 0x3F893F8A, 0x3F8B3F8C,
                         0x3F8D3F8E], dtype=torch.int64, device=dev).to(torch.int32)
    iters, grid = 20000, cus * 2
    outm = torch.zeros(grid * 4, dtype=torch.float32, device=dev)
    t_mf = best(lambda: _lib.check(L.ssmoe_bench_mfma_bf16(seed.data_ptr(), iters, outm.data_ptr(), grid, st)), reps=5)
    mf_flop = grid * 4 * 8 * iters * 2 * 16 * 16 * 32
    res = {"copy_gbs": round(2 * nb / t_copy / 1e9, 1), "read_gbs": round(nb / t_sum / 1e9, 1),
           "bf16_gemm_tflops": round(2 * n ** 3 / t_mm / 1e12, 1), "spec_hbm_gbs": HBM_PEAK_GBS,
           "spec_bf16_tflops": MFMA_BF16_PEAK_TFLOPS,
           "stream_read_gbs": round(rb / t_rd / 1e9, 1), "mfma_bf16_tflops": round(mf_flop / t_mf / 1e12, 1),
           "method": "best of 10 (GEMM and MFMA loop: 5) launches, HIP events: 1 GiB copy_ (read + write counted), "
                     "1 GiB fp32 sum, 8192^3 bf16 torch.matmul; this build's own kernels: a 4 GiB streaming read "
                     "(16-byte loads, 8 workgroups per CU) and a loop of independent v_mfma_f32_16x16x32_bf16 "
                     "(2 workgroups of 4 waves per CU, 8 accumulators per wave)"}
    log(f"measured peaks: {res}")
    return res


def config2_leg(pool, weights, biases, steps, dev, n_layers=8):
    """an MTP chain of depth 3 (T=4 verify) through config-1 layers, then acceptance over vocab
    151,936 on 1000 seeded steps of synthetic fp32 logits (target N(0,3), draft correlated rho=0.8): greedy
    argmax-match with the draft rows' argmax as drafts (the greedy proposal), p/q at temperature 0.7 with drafts
    drawn from q = softmax(draft / 0.7) on the device (ssmoe_sample_rows, the proposal Leviathan et al. Alg. 1
    needs), and (beside the step, as the reference's own sampled round) the reference sampler at temperature 0.7 with
    its default top-p 0.95 / top-k 40. Uniforms come from the sampler's splitmix64 stream seeded per step: the first
    D draw the drafts, the next D + 1 feed the p/q round. The verify layer is cold: each step has its own input rows
    and the steps rotate over `n_layers` distinct layers (8 x 906 MB of records, above the 256 MB Infinity Cache).
    Every step's inputs are resident in HBM before the timed region; the steps are captured as HIP graphs (100
    steps each) and replayed once, timed with HIP events."""
    import numpy as np
    import torch

    from slotstream_spark_amd.engine.accept import Acceptor, AcceptResult, RoundStats, UniformStream
    from slotstream_spark_amd.engine.sampler import SampleParams
    from slotstream_spark_amd.engine.verify import MoEVerifyLayer
    from slotstream_spark_amd.memory.synth import normal_bf16, verify_logits

    D, V, TEMP, T = 3, 151936, 0.7, 4
    sp = SampleParams(temperature=TEMP)
    layers = [MoEVerifyLayer(pool, l, weights[l].router_w, weights[l].sh_gate, weights[l].sh_up, weights[l].sh_down,
                             weights[l].sh_g, top_k=K, router_bias=biases[l], max_tokens=4) for l in range(n_layers)]
    xs = normal_bf16((steps, T, H), 1.0, 1734, dev)
    y = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
    ids = torch.empty((T, K), dtype=torch.int32, device=dev)
    wts = torch.empty((T, K), dtype=torch.float32, device=dev)
    tgt = torch.empty((steps, D + 1, V), device=dev)
    drf = torch.empty((steps, D, V), device=dev)
    for st in range(steps):
        tgt[st], drf[st] = verify_logits(D, V, 10_000 + st, device=dev)
    drafts_g = drf.argmax(dim=2).to(torch.int32).contiguous()
    un = np.stack([UniformStream(20_000 + st).peek(2 * D + 1) for st in range(steps)])
    u_draw = torch.from_numpy(np.ascontiguousarray(un[:, :D])).to(dev)
    u_acc = torch.from_numpy(np.ascontiguousarray(un[:, D:])).to(dev)
    u_smp = torch.from_numpy(np.ascontiguousarray(un[:, :D + 1])).to(dev)
    drafts_q = torch.empty((steps, D), dtype=torch.int32, device=dev)
    acc = Acceptor(D, V, device=dev)
    out_g = torch.empty((steps, D + 5), dtype=torch.int32, device=dev)
    out_p = torch.empty((steps, D + 5), dtype=torch.int32, device=dev)
    out_s = torch.empty((steps, D + 5), dtype=torch.int32, device=dev)
    acc_s = Acceptor(D, V, device=dev)
    chunk = 100

    def run(lo, hi, verify=True, greedy=False, draw=False, pq=False, sampled=False):
        for st in range(lo, hi):
            if verify:
                layers[st % n_layers](xs[st], y=y, ids=ids, weights=wts)
            if greedy:
                out_g[st].copy_(acc.greedy_async(tgt[st], drafts_g[st]))
            if draw:
                acc.draw_drafts_async(drf[st], u_draw[st], TEMP, out=drafts_q[st])
            if pq:
                out_p[st].copy_(acc.pq_async(tgt[st], drf[st], drafts_q[st], u_acc[st], TEMP))
            if sampled:
                out_s[st].copy_(acc_s.sampled_async(tgt[st], drafts_g[st], sp, (), u_smp[st]))

    s_ = torch.cuda.Stream(device=dev)
    res = {}
    legs = (("step_greedy", dict(greedy=True)), ("step_pq", dict(draw=True, pq=True)), ("verify", {}),
            ("greedy", dict(verify=False, greedy=True)), ("draw", dict(verify=False, draw=True)),
            ("pq", dict(verify=False, pq=True)), ("sampled", dict(verify=False, sampled=True)))
    for name, kw in legs:
        total = 0.0
        for lo in range(0, steps, chunk):
            total += timed_graph(lambda: run(lo, min(steps, lo + chunk), **kw), 1, 0, s_) * 1000.0
        res[name] = total / steps
    g = [AcceptResult.from_out(o) for o in out_g.cpu()]
    q = [AcceptResult.from_out(o) for o in out_p.cpu()]
    sm = [AcceptResult.from_out(o) for o in out_s.cpu()]
    stats = {}
    for name, rs in (("greedy", g), ("pq", q), ("sampled", sm)):
        st = RoundStats()
        for r in rs:
            st.add(D, r)
        stats[name] = {"acceptance_length": round(st.acceptance_length, 4),
                       "accepted_by_depth": st.accepted_by_depth, "attempts_by_depth": st.attempts_by_depth}
    # the acceptance rate Alg. 1 predicts for row 0 with sampled drafts: sum_x min(p(x), q(x)), from the first steps
    pred = []
    for st in range(min(steps, 32)):
        p0 = torch.softmax(tgt[st, 0].double() / TEMP, 0)
        q0 = torch.softmax(drf[st, 0].double() / TEMP, 0)
        pred.append(float(torch.minimum(p0, q0).sum()))
    stats["pq"]["predicted_accept_rate_row0"] = round(sum(pred) / len(pred), 4)
    stats["pq"]["measured_accept_rate_row0"] = round(stats["pq"]["accepted_by_depth"][0] / steps, 4)
    tok_s = stats["pq"]["acceptance_length"] / (res["step_pq"] * 1e-6)
    tok_g = stats["greedy"]["acceptance_length"] / (res["step_greedy"] * 1e-6)
    log(f"config2: step greedy {res['step_greedy']:.1f} us, step p/q {res['step_pq']:.1f} us (verify T=4 cold "
        f"{res['verify']:.1f}, greedy {res['greedy']:.1f}, draft draw {res['draw']:.1f}, p/q {res['pq']:.1f}; "
        f"sampled round {res['sampled']:.1f}); acceptance length greedy {stats['greedy']['acceptance_length']}, "
        f"p/q {stats['pq']['acceptance_length']} (row-0 accept {stats['pq']['measured_accept_rate_row0']} vs "
        f"predicted {stats['pq']['predicted_accept_rate_row0']}), sampled {stats['sampled']['acceptance_length']}")
    return {"steps": steps, "depth": D, "vocab": V, "temperature": TEMP, "verify_layers": n_layers,
            "us_per_step_greedy": round(res["step_greedy"], 2), "us_per_step_pq": round(res["step_pq"], 2),
            "us_verify_T4": round(res["verify"], 2), "us_accept_greedy": round(res["greedy"], 2),
            "us_draw_drafts": round(res["draw"], 2), "us_accept_pq": round(res["pq"], 2),
            "tokens_per_s_pq": round(tok_s, 1), "tokens_per_s_greedy": round(tok_g, 1),
            "greedy": stats["greedy"], "pq": stats["pq"],
            "us_accept_sampled": round(res["sampled"], 2),
            "sampled": dict(stats["sampled"], params="temperature 0.7, top_p 0.95, top_k 40 (SampleParams defaults)"),
            "timing": "HIP graphs of 100 steps, events on the graph stream; step_greedy = cold T=4 verify layer + "
                      "greedy round; step_pq = cold T=4 verify layer + draft draw from q + p/q round; the parts "
                      "and the sampled round in graphs of their own"}


def lm_head_leg(steps, dev):
    """The lm_head as the reference builds it (affine 4-bit gs64, 248,320 x 2560: gemv, kernels/gemv_affine.py:214-262)
    over R = 1, 2 and 4 verify rows, and over the 4 rows of a depth-3 round fused with the greedy acceptance
    (LMHeadGreedy). Two copies of the weights alternate so that every call streams its 358 MB from HBM (together
    they exceed the 256 MB Infinity Cache). Algorithmic bytes per call = N (K/2 + 4 K/64) + R K 2 + R N 4 (logits)."""
    import torch

    from slotstream_spark_amd.kernels.gemv_affine import AffineWeight, LMHeadGreedy, gemv
    from slotstream_spark_amd.memory.synth import normal_bf16

    N, KH = 248320, 2560
    g = torch.Generator(device=dev).manual_seed(2718)
    ws = []
    for c in range(2):
        q = torch.randint(-2**31, 2**31 - 1, (N, KH // 8), generator=g, device=dev, dtype=torch.int32)
        sc = (torch.randn((N, KH // 64), generator=g, device=dev) * 0.02).abs().to(torch.bfloat16)
        ws.append(AffineWeight(q, sc, (-8 * sc.float()).to(torch.bfloat16), 4, 64, N, KH))
    wbytes = N * (KH // 2 + 4 * (KH // 64))
    s_ = torch.cuda.Stream(device=dev)
    res = {}
    for R in (1, 2, 4):
        x = normal_bf16((R, KH), 1.0, 2719, dev)
        outs = [torch.empty((R, N), device=dev) for _ in range(2)]
        ms = timed_graph(lambda: [gemv(x, ws[i % 2], out=outs[i % 2]) for i in range(10)], steps, 2, s_)
        us = ms * 1000.0 / 10
        nbytes = wbytes + R * KH * 2 + R * N * 4
        res[f"R{R}"] = {"us_per_call": round(us, 2), "bytes_per_call": nbytes, "gbs": round(nbytes / (us * 1e-6) / 1e9, 1)}
    D = 3
    x4 = normal_bf16((D + 1, KH), 1.0, 2720, dev)
    heads = [LMHeadGreedy(w, D, device=dev) for w in ws]
    drafts = torch.zeros(D, dtype=torch.int32, device=dev)
    ms = timed_graph(lambda: [heads[i % 2].run_async(x4, drafts) for i in range(10)], steps, 2, s_)
    us = ms * 1000.0 / 10
    fbytes = wbytes + (D + 1) * KH * 2
    res["greedy_round_D3"] = {"us_per_call": round(us, 2), "bytes_per_call": fbytes,
                              "gbs": round(fbytes / (us * 1e-6) / 1e9, 1)}
    r4 = res["R4"]
    res["roofline"] = {"bound": "hbm", "kernel": "gemv_affine4_kernel (R = 4)", "achieved": r4["gbs"],
                       "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(r4["gbs"] / HBM_PEAK_GBS, 4),
                       "traffic": traffic_of("lm_head_gemv"), "us_per_launch": r4["us_per_call"],
                       "bytes_per_launch": r4["bytes_per_call"]}
    res["shape"] = "N 248320 x K 2560, affine 4-bit gs64 (357.6 MB of weights), bf16 x"
    res["reference_gb10_gbs"] = 232.95  # the reference's lm_head GEMV (tuning_gb10.json `248320x2560x4x64`)
    res["speedup_vs_reference_gb10"] = round(r4["gbs"] / 232.95, 2)
    log(f"lm_head: R1 {res['R1']['us_per_call']} us, R2 {res['R2']['us_per_call']} us, R4 {r4['us_per_call']} us "
        f"({r4['gbs']} GB/s), fused greedy round D=3 {res['greedy_round_D3']['us_per_call']} us")
    return res


def ref_decode_leg(steps, dev):
    """The reference's own published moe_decode benchmark, at its shape: hidden 2560, moe_intermediate 640, affine
    4-bit gs64 records of 2,764,800 B, 1 row x 10 experts (27,648,000 B per step), cold (152.23 us / 181.6 GB/s on
    GB10, slotstream_spark/kernels/tuning_gb10.json `moe`; records in pinned host memory there, in HBM here). Cold
    here: 16 layers of 64 experts, each call on its own layer with 10 distinct experts, 442 MB per graph replay
    (above the 256 MB Infinity Cache)."""
    import torch

    from slotstream_spark_amd.kernels.moe_gemv_affine import moe_decode
    from slotstream_spark_amd.memory.slot_pool import SlotPool
    from slotstream_spark_amd.memory.synth import normal_bf16

    HR, IR, ER, NLR, KR = 2560, 640, 64, 16, 10
    pool = SlotPool(NLR, ER, HR, IR, device=dev)
    pool.fill_random(4242)
    pool.place_permuted(4243)
    g = torch.Generator().manual_seed(4244)
    ids = [torch.randperm(ER, generator=g)[:KR].to(torch.int32).reshape(1, KR).to(dev) for _ in range(NLR)]
    wts = [torch.softmax(torch.randn(1, KR, generator=g), dim=-1).to(dev) for _ in range(NLR)]
    x = normal_bf16((1, HR), 1.0, 4245, dev)
    hb = [torch.empty((1, KR, IR), device=dev) for _ in range(NLR)]
    ob = [torch.empty((1, KR, HR), device=dev) for _ in range(NLR)]
    outs = [torch.empty((1, HR), device=dev) for _ in range(NLR)]

    def run():
        for l in range(NLR):
            moe_decode(x, ids[l], wts[l], l, pool.map, pool.slot_ptr, hb[l], ob[l], outs[l], experts_per_layer=ER)

    ms = timed_graph(run, steps, 3, torch.cuda.Stream(device=dev))
    us = ms * 1000.0 / NLR
    nbytes = KR * 2_764_800
    res = {"shape": "H 2560, I 640, 1 row x 10 experts, affine 4-bit gs64 (the reference model's)",
           "us_per_step": round(us, 2), "bytes_per_step": nbytes, "gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
           "reference_gb10_us_per_step": 152.23, "reference_gb10_gbs": 181.63,
           "speedup_vs_reference_gb10": round(152.23 / us, 2)}
    log(f"reference-shape moe_decode: {us:.2f} us per step ({res['gbs']} GB/s); GB10 reference 152.23 us")
    del pool
    return res


def step_leg(pool, weights, biases, steps, dev):
    """The whole verify round in one HIP graph (engine/step.py MTPStepGraph) at full size: 48 chained
    config-1 layers (residual + RMSNorm between them), the 248,320 x 2048 affine 4-bit lm_head fused with the greedy
    round, and the MTP head's MoE (map layer 48), for depth 1 (T = 2), depth 2 (T = 3, the reference's own verify
    width, engine/mtp.py:48) and depth 3 (T = 4). Timed with HIP events
    around `steps` replays; one int32 result vector per round is the only thing the host would read back."""
    import torch

    from slotstream_spark_amd.engine.step import MoEWeights, MTPStepGraph
    from slotstream_spark_amd.kernels.gemv_affine import AffineWeight
    from slotstream_spark_amd.memory.synth import normal_bf16

    N, NL = 248320, 48
    g = torch.Generator(device=dev).manual_seed(2721)
    q = torch.randint(-2**31, 2**31 - 1, (N, H // 8), generator=g, device=dev, dtype=torch.int32)
    sc = (torch.randn((N, H // 64), generator=g, device=dev) * 0.02).abs().to(torch.bfloat16)
    lm = AffineWeight(q, sc, (-8 * sc.float()).to(torch.bfloat16), 4, 64, N, H)
    mw = [MoEWeights(w.router_w, w.sh_gate, w.sh_up, w.sh_down, w.sh_g, b) for w, b in zip(weights, biases)]
    res = {"layers": NL, "head_layer": NL, "lm_head": f"{N} x {H} affine 4-bit gs64"}
    for depth in (1, 2, 3):
        sg = MTPStepGraph(pool, mw[:NL], lm, depth, head=mw[NL], top_k=K, device=dev)
        sg.step(normal_bf16((depth + 1, H), 1.0, 2722, dev), torch.zeros(depth, dtype=torch.int32, device=dev))
        for _ in range(2):
            sg.step()
        torch.cuda.synchronize()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record()
        for _ in range(steps):
            sg.step()
        ev1.record()
        torch.cuda.synchronize()
        us = ev0.elapsed_time(ev1) * 1000.0 / steps
        uniq = [len(set(sg.ids[l].cpu().flatten().tolist())) for l in range(NL)]
        res[f"T{depth + 1}"] = {"us_per_round": round(us, 1), "us_per_layer_incl_norm": round(us / NL, 2),
                                "unique_experts_mean": round(sum(uniq) / NL, 2),
                                "finite": bool(torch.isfinite(sg.mixed[NL].float()).all().item())}
        log(f"step graph T={depth + 1}: {us:.1f} us per round ({NL} layers + head MoE + lm_head greedy), "
            f"mean unique experts {sum(uniq) / NL:.1f}")
        del sg
    # the T=4 round with p/q acceptance fused behind the lm_head (temperature 0.7; the draft head's logits of the
    # round are an input, synthetic here, and the drafts are drawn from q = softmax(draft / 0.7) on the device, the
    # proposal the p/q rule needs)
    from slotstream_spark_amd.engine.accept import Acceptor

    sg = MTPStepGraph(pool, mw[:NL], lm, 3, head=mw[NL], top_k=K, accept="pq", temperature=0.7, device=dev)
    g2 = torch.Generator(device=dev).manual_seed(2723)
    sg.draft_logits.copy_(torch.randn(sg.draft_logits.shape, generator=g2, device=dev) * 3)
    sg.uniforms.copy_(torch.rand(4, generator=g2, device=dev))
    drafts = Acceptor(3, N, device=dev).draw_drafts_async(sg.draft_logits, torch.rand(3, generator=g2, device=dev),
                                                          0.7)
    sg.step(normal_bf16((4, H), 1.0, 2722, dev), drafts)
    for _ in range(2):
        sg.step()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(steps):
        sg.step()
    ev1.record()
    torch.cuda.synchronize()
    us = ev0.elapsed_time(ev1) * 1000.0 / steps
    res["T4_pq"] = {"us_per_round": round(us, 1), "temperature": 0.7, "result": sg.out.cpu().tolist()[:4],
                    "note": "lm_head GEMV writes logits and chunk maxima; the p/q round reads the logits once; "
                            "drafts drawn from q (ssmoe_sample_rows) before the round, outside the timing"}
    log(f"step graph T=4 with fused p/q: {us:.1f} us per round")
    del sg
    return res


def _lm_head_weight(dev, n=248320, seed=2721):
    import torch

    from slotstream_spark_amd.kernels.gemv_affine import AffineWeight

    g = torch.Generator(device=dev).manual_seed(seed)
    q = torch.randint(-2**31, 2**31 - 1, (n, H // 8), generator=g, device=dev, dtype=torch.int32)
    sc = (torch.randn((n, H // 64), generator=g, device=dev) * 0.02).abs().to(torch.bfloat16)
    return AffineWeight(q, sc, (-8 * sc.float()).to(torch.bfloat16), 4, 64, n, H)


def draft_leg(pool, weights, biases, steps, dev):
    """The MTP head's draft chain (engine/mtp.py, attention excluded) at the config-1
    shape: hc 4 hyper-connection branches of H 2048 with a 320-wide low rank, the head MoE on map layer 48 (E512
    top-10, shared 512), the 248,320 x 2048 affine 4-bit lm_head argmax; depth 2 (the reference's DEPTH) and 3, one
    HIP graph per chain, timed with HIP events around `steps` replays. Then the greedy speculative loop
    (engine/generate.py mtp_decode) over a 48-layer MoE stack with that head (hc 1 on the stack's one stream): wall
    time per emitted token with the host's per-round reads included."""
    import time

    import torch

    from slotstream_spark_amd.engine.generate import MoEStack, mtp_decode
    from slotstream_spark_amd.engine.mtp import DraftGraph, MTPHead
    from slotstream_spark_amd.engine.step import MoEWeights
    from slotstream_spark_amd.engine.verify import MoEVerifyLayer
    from slotstream_spark_amd.memory.synth import head_weights, normal_bf16

    NL = 48
    lm = _lm_head_weight(dev)
    hw_ = weights[NL]
    moe = MoEVerifyLayer(pool, NL, hw_.router_w, hw_.sh_gate, hw_.sh_up, hw_.sh_down, hw_.sh_g, top_k=K,
                         router_bias=biases[NL], max_tokens=4)
    head = MTPHead(head_weights(H, 4, 320, lm.n, seed=2730, device=dev), moe, lm, hc=4)
    res = {"hc": 4, "lowrank": 320, "head_layer": NL, "lm_head": f"{lm.n} x {H} affine 4-bit gs64"}
    for k in (2, 3):
        dg = DraftGraph(head, k)
        dg.token.fill_(12345)
        dg.multi.copy_(normal_bf16((1, 4 * H), 1.0, 2731, dev))
        dg.capture()
        for _ in range(3):
            dg.graph.replay()
        torch.cuda.synchronize()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record()
        for _ in range(steps):
            dg.graph.replay()
        ev1.record()
        torch.cuda.synchronize()
        us = ev0.elapsed_time(ev1) * 1000.0 / steps
        res[f"depth{k}"] = {"us_per_chain": round(us, 1), "us_per_draft": round(us / k, 1),
                            "drafts": dg.out.cpu().tolist()}
        log(f"draft chain depth {k}: {us:.1f} us ({us / k:.1f} us per drafted token)")
        del dg
    del head, moe
    # the speculative loop over the 48-layer stack
    mw = [MoEWeights(w.router_w, w.sh_gate, w.sh_up, w.sh_down, w.sh_g, b) for w, b in zip(weights[:NL], biases[:NL])]
    emb = head_weights(H, 1, 320, lm.n, seed=2732, device=dev)
    stack = MoEStack(pool, mw, lm, emb.embed, depth=2, top_k=K, device=dev)
    moe1 = MoEVerifyLayer(pool, NL, hw_.router_w, hw_.sh_gate, hw_.sh_up, hw_.sh_down, hw_.sh_g, top_k=K,
                          router_bias=biases[NL], max_tokens=4)
    head1 = MTPHead(emb, moe1, lm, hc=1)
    mtp_decode(stack, head1, [11, 12, 13], 8)  # captures the round graph, warms up
    stack.reset()
    head1.reset()
    n_tok = 64
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    out, _nan, secs, st = mtp_decode(stack, head1, [21, 22, 23], n_tok)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    res["loop"] = {"layers": NL, "depth": 2, "tokens": len(out), "rounds": st["rounds"], "accepted": st["accepted"],
                   "drafted": st["drafted"], "ms_per_round": round(1000 * sum(secs) / max(len(secs), 1), 3),
                   "tokens_per_s": round(len(out) / wall, 1),
                   "note": "random-init head and stack: drafts rarely match, so about one token per round"}
    log(f"speculative loop: {len(out)} tokens in {wall * 1000:.1f} ms, {st['rounds']} rounds, "
        f"{st['accepted']}/{st['drafted']} drafts accepted, {1000 * sum(secs) / max(len(secs), 1):.2f} ms per round")
    return res


def pool_leg(dev, calls=4):
    """The slot pool loading records from experts.bin (ExpertPool / ssmoe_pool_*): 256 records of the reference's
    2,764,800-byte layout (hidden 2560, moe_intermediate 640) in a 2 x 128 file, a 128-slot pool, and ensures of a
    whole layer (128 misses each, every call after the first evicting the other layer) with 1, 4 and 8 reader
    lanes, buffered (the file was just written, so reads come from the page cache) and, where the file system
    takes it, O_DIRECT. Also the hit path: an ensure of 10 resident experts, the per-layer call of a decode step."""
    import shutil
    import tempfile

    import numpy as np

    from slotstream_spark_amd import _lib
    from slotstream_spark_amd.memory.expert_pool import ExpertPool

    rec, layers, experts = 2_764_800, 2, 128
    d = Path(tempfile.mkdtemp(prefix="ssmoe-pool-"))
    res = {"record_bytes": rec, "records": layers * experts, "slots": experts}
    try:
        (d / "experts.bin").write_bytes(np.random.default_rng(5).bytes(layers * experts * rec))
        (d / "experts.manifest.json").write_text(json.dumps(
            {"record_bytes": rec, "layers": layers, "experts": experts, "alignment": 4096}))
        ids = np.arange(experts, dtype=np.int32)
        for lanes, direct in ((1, False), (4, False), (8, False), (8, True)):
            try:
                ep = ExpertPool(d, experts, lanes=lanes, direct=direct, device=dev)
            except _lib.IoError as e:
                res["direct"] = f"unsupported here: {e}"
                continue
            key = f"{'direct' if direct else 'buffered'}_lanes{lanes}"
            try:
                ep.ensure(0, ids, gen=1)
                t0 = time.perf_counter()
                for c in range(calls):
                    ep.retire_below(c + 2)
                    ep.ensure((c + 1) % 2, ids, gen=c + 2)
                dt = time.perf_counter() - t0
            except _lib.IoError as e:
                res[key] = f"read failed: {e}"
                log(f"pool {key}: {e}")
                ep.close()
                continue
            gbs = calls * experts * rec / dt / 1e9
            res[key] = {"gbs": round(gbs, 2), "ms_per_layer": round(dt * 1000 / calls, 2),
                        "read_ms_last": round(ep.last_timing["read_ns"] / 1e6, 2)}
            log(f"pool {key}: {gbs:.2f} GB/s, {dt * 1000 / calls:.1f} ms per 128-record layer")
            if lanes == 8 and not direct:
                rng = np.random.default_rng(6)
                picks = [rng.choice(experts, 10, replace=False).astype(np.int32) for _ in range(1000)]
                layer = calls % 2
                for i in range(50):
                    ep.ensure(layer, picks[i])
                t0 = time.perf_counter()
                for p in picks:
                    ep.ensure(layer, p)
                res["hit_us_per_ensure_10"] = round((time.perf_counter() - t0) * 1e6 / len(picks), 2)
                log(f"pool hit path: {res['hit_us_per_ensure_10']} us per ensure of 10 resident experts")
            ep.close()
    finally:
        shutil.rmtree(d, ignore_errors=True)
    return res


def config4_leg(pool, weights, biases, steps, dev):
    """a 48-layer routed-MoE stack (config-1 shape, all experts resident) run as an MTP loop of
    `steps` decode steps at T=2: per step, the 48 verify layers chained in one HIP graph (engine/step.py with the
    lm_head left out: each launch stages the RMSNorm of the residual stream and writes the next stream, so the chain
    keeps its scale and its routing stays well defined), then greedy acceptance (D=1) on that step's synthetic fp32
    logits (vocab 151,936, rho=0.8 draft). Effective tokens/s = emitted tokens / wall time of the whole loop,
    attention excluded."""
    import torch

    from slotstream_spark_amd.engine.accept import Acceptor, AcceptResult, RoundStats
    from slotstream_spark_amd.engine.step import MoEWeights, MTPStepGraph
    from slotstream_spark_amd.memory.synth import normal_bf16, verify_logits

    NL4, D, V, T = len(weights), 1, 151936, 2
    mw = [MoEWeights(w.router_w, w.sh_gate, w.sh_up, w.sh_down, w.sh_g, b) for w, b in zip(weights, biases)]
    sg = MTPStepGraph(pool, mw, None, depth=D, top_k=K, device=dev)
    # every step verifies new rows (in the real loop: the embeddings of the tokens accepted so far), so the routing,
    # and with it the experts each layer reads, changes from step to step
    x_steps = normal_bf16((steps + 2, T, H), 1.0, 1735, dev)
    sg.x_in.copy_(x_steps[0])
    tgt = torch.empty((steps, D + 1, V), device=dev)
    drf = torch.empty((steps, D, V), device=dev)
    for st in range(steps):
        tgt[st], drf[st] = verify_logits(D, V, 30_000 + st, device=dev)
    drafts = drf.argmax(dim=2).to(torch.int32).contiguous()
    acc = Acceptor(D, V, device=dev)
    out_g = torch.empty((steps, D + 5), dtype=torch.int32, device=dev)
    sg.capture()
    s_ = sg.stream
    with torch.cuda.stream(s_):
        for w_ in range(2):
            sg.x_in.copy_(x_steps[steps + w_])
            sg.graph.replay()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        uniq_steps = []
        ev0.record(s_)
        for st in range(steps):
            sg.x_in.copy_(x_steps[st])
            sg.graph.replay()
            out_g[st].copy_(acc.greedy_async(tgt[st], drafts[st]))
            if st % 64 == 63:
                uniq_steps.append(sg.ids.clone())
        ev1.record(s_)
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1)
    rs = RoundStats()
    for o in out_g.cpu():
        rs.add(D, AcceptResult.from_out(o))
    emitted = sum(rs.emitted_by_round)
    tok_s = emitted / (ms * 1e-3)
    if not uniq_steps:
        uniq_steps.append(sg.ids.clone())
    uniq = [len(set(u[l].cpu().flatten().tolist())) for u in uniq_steps for l in range(NL4)]
    same_route = sum(bool(torch.equal(uniq_steps[0][l], uniq_steps[1][l])) for l in range(NL4)) if len(uniq_steps) > 1 else None
    finite = bool(torch.isfinite(sg.streams[NL4].float()).all().item())
    log(f"config4: {NL4} layers x {steps} steps in {ms:.1f} ms ({ms * 1000 / steps:.1f} us/step, "
        f"{ms * 1000 / steps / NL4:.2f} us/layer); {emitted} tokens emitted, {tok_s:.0f} tokens/s; "
        f"mean unique experts {sum(uniq) / len(uniq):.1f}, stream finite {finite}, layers routed alike in two "
        f"sampled steps {same_route}")
    return {"layers": NL4, "steps": steps, "tokens": T, "ms_total": round(ms, 3),
            "us_per_step": round(ms * 1000 / steps, 2), "us_per_layer": round(ms * 1000 / steps / NL4, 3),
            "emitted_tokens": emitted, "acceptance_length": round(rs.acceptance_length, 4),
            "effective_tokens_per_s": round(tok_s, 1), "unique_experts_mean": round(sum(uniq) / len(uniq), 2),
            "layers_routed_alike_in_two_sampled_steps": same_route,
            "stream_finite": finite, "resident_expert_bytes": NL4 * E * 1_769_472,
            "timing": "per step: a copy of that step's input rows, one HIP graph of the 48 chained layers (norm and "
                      "residual add inside each verify launch), the greedy acceptance launches; events around the "
                      "whole loop"}


def traffic_of(kernel: str):
    """HBM bytes per launch of `kernel` measured with rocprofv3 FETCH_SIZE + WRITE_SIZE (scaled by a known-size copy),
    as recorded in profiles/traffic.json next to the command that produced it; None when not measured."""
    f = ROOT / "profiles" / "traffic.json"
    if not f.exists():
        return None
    rec = json.loads(f.read_text()).get(kernel)
    return None if rec is None else rec.get("bytes_per_launch")


def cpu_baseline(layer_w, bias, pool, x, layer_idx, budget_s):
    """The reference's CPU path for this layer, restated on torch CPU (oracle.moe_ref, model/reference_torch.py:118-134),
    timed on this host. First checked against the fixtures written from the reference's own moe_ref (ids and y bit for
    bit). Then, within about `budget_s` seconds: the config-1 shape (this bench's layer 0, Zipf bias) with
    dequantized fp32 experts cached (how the reference CPU path receives experts) at n threads (every CPU of the
    process's affinity, capped by this host's CPU share in OMP_NUM_THREADS) and at 1 thread, the dequant-per-call
    variant at n threads, and BASELINE config 0 (64 experts, top-4) at n and 1 threads. Medians of >= 15 steps where
    the budget allows."""
    import json as _json

    import numpy as np
    import torch

    from oracle import oracle as O
    from tests.golden import gen

    # 1. the restatement against the reference's fixtures
    Z = np.load(ROOT / "tests" / "golden" / "moe_ref_cases.npz")
    cases = _json.loads(bytes(Z["meta"]).decode())["cases"]
    checked = []
    for c in cases:
        if c["seed"] not in (0, 4):
            continue
        s_, T_, H_, E_, K_, I_, Is_ = (c[k] for k in ("seed", "T", "H", "E", "K", "I", "Is"))
        xb, rw, sg, su, sd, sgg = (torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)
                                   for a in gen.layer_inputs(s_, T_, H_, E_, Is_))
        ex = {}

        def fx(e, s_=s_, H_=H_, I_=I_, ex=ex):
            if e not in ex:
                ex[e] = tuple(torch.from_numpy(d) for d in O.expert_dense(gen.record(s_, e, H_, I_), H_, I_, np.float32))
            return ex[e]

        y, ti, _ = O.moe_ref(xb, rw, K_, fx, sg, su, sd, sgg)
        # The fixtures carry the bits of the CPU that wrote them: torch's CPU bf16 GEMM rounds in an order that
        # depends on the instruction set it dispatches to, so on another host a logit (and a y entry) can move by a
        # bf16 step. Bit for bit on the fixture host (tests/test_oracle_pins.py); here: the same ids and y within the
        # north-star bound.
        yb = y.view(torch.int16).numpy().view(np.uint16)
        same_ids = np.array_equal(ti.numpy().astype(np.int32), Z[f"s{s_}_ids"])
        err = O.rel_l2(O.bf16_to_f32(yb), O.bf16_to_f32(Z[f"s{s_}_y"]))
        if not same_ids or not err <= 2e-2:
            raise RuntimeError(f"oracle.moe_ref differs from the reference fixture s{s_}: ids equal {same_ids}, "
                               f"y rel_l2 {err:.3e}")
        checked.append(f"s{s_} (E={E_}, top-{K_}: ids equal, y rel_l2 {err:.1e}, "
                       f"{100.0 * float(np.mean(yb == Z[f's{s_}_y'])):.2f} % of y bit-identical)")

    n_aff = len(os.sched_getaffinity(0))
    share = int(os.environ.get("OMP_NUM_THREADS", n_aff) or n_aff)
    n = max(1, min(n_aff, share))

    def time_steps(fn, threads, seconds, min_steps=15, max_steps=200):
        torch.set_num_threads(threads)
        fn()
        times = []
        t_end = time.perf_counter() + seconds
        while (time.perf_counter() < t_end or len(times) < 3) and len(times) < max_steps:
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
            if len(times) >= min_steps and time.perf_counter() > t_end:
                break
        return sorted(times)[len(times) // 2] * 1e6, len(times)

    # 2. the config-1 shape: this bench's layer
    xc = x.cpu()
    rw, sg, su, sd, sgw = (t.cpu() for t in (layer_w.router_w, layer_w.sh_gate, layer_w.sh_up, layer_w.sh_down,
                                             layer_w.sh_g))
    bc = bias.cpu() if bias is not None else None
    mp = pool.map[layer_idx * E:(layer_idx + 1) * E].cpu().numpy()
    records = {}

    def record(e):
        if e not in records:
            records[e] = pool.record(int(mp[e])).cpu().numpy()
        return records[e]

    def dequant(e):
        return tuple(torch.from_numpy(d) for d in O.expert_dense(record(e), H, I, np.float32))

    cache = {}

    def cached(e):
        if e not in cache:
            cache[e] = dequant(e)
        return cache[e]

    c1 = lambda: O.moe_ref(xc, rw, K, cached, sg, su, sd, sgw, bc)  # noqa: E731
    c1_pc = lambda: O.moe_ref(xc, rw, K, dequant, sg, su, sd, sgw, bc)  # noqa: E731
    v1_n, s1_n = time_steps(c1, n, budget_s * 0.3)
    v1_1, s1_1 = time_steps(c1, 1, budget_s * 0.25, min_steps=5)
    vpc_n, spc_n = time_steps(c1_pc, n, budget_s * 0.15, min_steps=3)

    # 3. 64 experts, top-4 (the fixture generator's seed-0 layer)
    x0, rw0, sg0, su0, sd0, sgg0 = (torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)
                                    for a in gen.layer_inputs(0, 2, H, 64, IS))
    ex0 = {e: tuple(torch.from_numpy(d) for d in O.expert_dense(gen.record(0, e, H, I), H, I, np.float32))
           for e in range(64)}
    c0 = lambda: O.moe_ref(x0, rw0, 4, ex0.__getitem__, sg0, su0, sd0, sgg0)  # noqa: E731
    v0_n, s0_n = time_steps(c0, n, budget_s * 0.15)
    v0_1, s0_1 = time_steps(c0, 1, budget_s * 0.15, min_steps=5)
    torch.set_num_threads(n)
    res = {"value": round(v1_n, 1), "unit": "us per T=2 verify step per MoE layer", "cores": n, "kind": "port",
           "sample": f"torch-CPU moe_ref restatement (checked against the reference fixtures "
                     f"{', '.join(checked)}), config-1 layer (512 experts top-10, Zipf bias), T=2, dequantized fp32 "
                     f"experts cached, median of {s1_n} steps at {n} threads",
           "cores_affinity": n_aff, "cpu_share": share,
           "config1_1thread_us": round(v1_1, 1), "config1_1thread_steps": s1_1,
           "config1_dequant_per_call_us": round(vpc_n, 1), "config1_dequant_per_call_steps": spc_n,
           "config0_us": round(v0_n, 1), "config0_steps": s0_n,
           "config0_1thread_us": round(v0_1, 1), "config0_1thread_steps": s0_1,
           "tokens_per_s_config1": round(2 / (v1_n * 1e-6), 1)}
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--layers", type=int, default=16)
    ap.add_argument("--tokens", type=int, default=2)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--legs", default="isolated,decode,prefill,config2,config4,lm_head,step,draft,pool,ref_decode,"
                                      "ref_chain,peaks",
                    help="comma list of legs besides the headline chain: isolated, decode, prefill, config2, "
                         "config4, lm_head, step, draft, pool, ref_decode, ref_chain, peaks (chain alone: chain)")
    ap.add_argument("--prefill-layers", type=int, default=4)
    ap.add_argument("--config2-steps", type=int, default=1000)
    ap.add_argument("--config4-layers", type=int, default=48)
    ap.add_argument("--config4-steps", type=int, default=256)
    ap.add_argument("--copy-calib", action="store_true", help="run 3 x 256 MiB device copies first (PMC scaling)")
    args = ap.parse_args()
    known = {"isolated", "decode", "prefill", "config2", "config4", "lm_head", "step", "draft", "pool", "ref_decode",
             "ref_chain", "peaks", "chain"}  # "chain": the headline leg alone (it always runs)
    unknown = sorted(set(args.legs.split(",")) - known - {""})
    if unknown:
        ap.error(f"unknown legs {unknown}; known: {sorted(known)}")
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU: every GPU box here has one; sharding the path "
                                   "over several GPUs is designed but not built"}))
        sys.exit(2)

    import torch

    from slotstream_spark_amd.engine.verify import MoEVerifyLayer
    from slotstream_spark_amd.kernels.moe_gemv_affine import moe_decode
    from slotstream_spark_amd.memory.slot_pool import SlotPool
    from slotstream_spark_amd.memory.synth import LayerWeights, normal_bf16, zipf_bias

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    legs = set(args.legs.split(","))
    if args.copy_calib:
        a = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        del a, b
        log("copy calibration: 3 x 268435456-byte device copies done")
    NL, T = args.layers, args.tokens
    # The records are placed by a permutation over every slot, so the pool's size fixes which weights each expert
    # gets: config4 and the step graph both allocate one layer past config4's stack (the MTP layer), whichever legs
    # run, so that their routing and unique-expert counts do not depend on the leg list.
    NP = max(NL, args.config4_layers + 1 if "config4" in legs else 0, 49 if legs & {"step", "draft"} else 0)
    log(f"allocating {NP} layers x {E} experts ({NP * E * 1_769_472 / 2**30:.1f} GiB of records)")
    pool = SlotPool(NP, E, H, I, device=dev)
    pool.fill_random(1729)
    pool.place_permuted(1732)
    weights = [LayerWeights(H, E, IS, seed=1729 + l, device=dev) for l in range(NP)]
    biases = [zipf_bias(E, 1.1, 1731 + l, device=dev) for l in range(NP)]
    layers = [MoEVerifyLayer(pool, l, w.router_w, w.sh_gate, w.sh_up, w.sh_down, w.sh_g, top_k=K,
                             router_bias=b, max_tokens=max(T, 4)) for l, (w, b) in enumerate(zip(weights[:NL], biases[:NL]))]
    x = normal_bf16((T, H), 1.0, 1730, dev)
    ys = [torch.empty((T, H), dtype=torch.bfloat16, device=dev) for _ in range(NL)]
    ids = [torch.empty((T, K), dtype=torch.int32, device=dev) for _ in range(NL)]
    wts = [torch.empty((T, K), dtype=torch.float32, device=dev) for _ in range(NL)]

    # the headline: the chained verify step, every layer in one launch
    chain = verify_chain_leg(pool, weights, biases, NL, T, args.steps, args.warmup, dev)
    us_layer = chain["us_per_layer"]
    ms_step = chain["us_per_step"] / 1000.0
    layer_gbs = chain["achieved_gbs"]

    def step():
        for l in range(NL):
            layers[l](x, y=ys[l], ids=ids[l], weights=wts[l])

    s = torch.cuda.Stream(device=dev)
    iso = None
    uniq = None
    if "isolated" in legs or "decode" in legs:
        # the same layers as independent single-layer launches on one input (verify_kernel, one launch per layer)
        ms_iso = timed_graph(step, args.steps, args.warmup, s)
        uniq = [len(set(ids[l].cpu().flatten().tolist())) for l in range(NL)]
        bytes_iso = sum(layer_bytes(u, T) for u in uniq)
        iso = {"us_per_layer": round(ms_iso * 1000.0 / NL, 3),
               "achieved_gbs": round(bytes_iso / (ms_iso * 1e-3) / 1e9, 1), "unique_experts": uniq,
               "kernel": "verify_kernel, one launch per layer, every layer on the same input, in one HIP graph"}
        log(f"isolated layers: {iso['us_per_layer']:.2f} us per layer ({iso['achieved_gbs']:.0f} GB/s), "
            f"unique experts {uniq}")

    us_moe = moe_gbs = moe_bytes = None
    if "decode" in legs:
        # Routed experts only (moe_decode, decode mode of the same kernel) on the routing of the step, one graph of
        # NL calls.
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        hb = [torch.empty((T, K, I), device=dev) for _ in range(NL)]
        ob = [torch.empty((T, K, H), device=dev) for _ in range(NL)]
        outb = [torch.empty((T, H), device=dev) for _ in range(NL)]

        def routed():
            for l in range(NL):
                moe_decode(x, ids[l], wts[l], l, pool.map, pool.slot_ptr, hb[l], ob[l], outb[l], experts_per_layer=E)

        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            routed()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g2 = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g2):
            routed()
        for _ in range(args.warmup):
            g2.replay()
        torch.cuda.synchronize()
        ev0.record()
        for _ in range(args.steps):
            g2.replay()
        ev1.record()
        torch.cuda.synchronize()
        us_moe = ev0.elapsed_time(ev1) * 1000.0 / (args.steps * NL)
        moe_bytes = sum(u * 1_769_472 + T * H * 6 for u in uniq) / NL
        moe_gbs = moe_bytes / (us_moe * 1e-6) / 1e9
        log(f"moe_decode {us_moe:.2f} us per launch pair, {moe_gbs:.0f} GB/s algorithmic")


    prefill = None
    if "prefill" in legs:
        prefill = prefill_leg(pool, weights, biases, min(args.prefill_layers, NL), max(args.steps // 5, 3),
                              max(args.warmup // 5, 1), dev)

    c2 = c4 = None
    if "config2" in legs:
        c2 = config2_leg(pool, weights, biases, args.config2_steps, dev, n_layers=min(8, NP))
    if "config4" in legs:
        c4 = config4_leg(pool, weights[:args.config4_layers], biases[:args.config4_layers], args.config4_steps, dev)

    lmh = None
    if "lm_head" in legs:
        lmh = lm_head_leg(max(args.steps // 5, 3), dev)

    stp = None
    if "step" in legs:
        stp = step_leg(pool, weights, biases, max(args.steps // 5, 5), dev)

    drf = None
    if "draft" in legs:
        drf = draft_leg(pool, weights, biases, max(args.steps // 5, 5), dev)

    rd = None
    if "ref_decode" in legs:
        rd = ref_decode_leg(max(args.steps // 2, 10), dev)

    pl = None
    if "pool" in legs:
        pl = pool_leg(dev)

    rc_ = None
    if "ref_chain" in legs:
        rc_ = ref_chain_leg(max(args.steps // 2, 10), 3, dev)

    peaks = peaks_leg(dev) if "peaks" in legs else None
    if peaks is not None:
        # the same achieved figures against this build's own ceilings
        if prefill is not None:
            r = prefill["roofline"]
            r["measured_peak"] = peaks["mfma_bf16_tflops"]
            r["frac_of_measured_peak"] = round(r["achieved"] / peaks["mfma_bf16_tflops"], 4)

    cpu = None
    if not args.no_cpu:
        log("timing the CPU baseline")
        cpu = cpu_baseline(weights[0], biases[0], pool, x, 0, args.cpu_seconds)
        log(f"cpu {cpu}")

    line = {
        "metric": METRIC,
        "value": round(us_layer, 3),
        "unit": "us per T=2 verify step per MoE layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded random affine-4bit experts and bf16 router/shared weights; no checkpoint)",
        "config": {"workload": f"config1: T={T} verify through the config-1 MoE layer (H2048, E512 top-10, I512, "
                               f"shared 512, affine-4bit gs64, Zipf 1.1), {NL} distinct layers chained per step "
                               f"(RMSNorm + residual between them) in one launch, a new input each step",
                   "layers_per_step": NL, "tokens": T, "unique_experts_mean": round(chain["unique_experts_mean"], 2),
                   "parallelism": "single GPU"},
        "hbm_gbs_layer": round(layer_gbs, 1),
        "tokens_per_s_layer": round(T / (us_layer * 1e-6), 1),
        "roofline": {"bound": "hbm", "kernel": f"chain_kernel ({NL} layers per launch: norm, router, routed and "
                                               f"shared experts, combine, residual)",
                     "achieved": round(layer_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(layer_gbs / HBM_PEAK_GBS, 4), "traffic": traffic_of("chain_kernel"),
                     "us_per_launch": round(chain["us_per_step"], 2), "bytes_per_launch": int(chain["bytes_per_launch"]),
                     "bytes_per_layer": int(chain["bytes_per_launch"] / NL)},
        "isolated": iso,
        "measured_peaks": peaks,
        "roofline_vs_measured_read_peak": None if peaks is None else {
            "peak": peaks["stream_read_gbs"], "unit": "GB/s", "frac": round(layer_gbs / peaks["stream_read_gbs"], 4)},
        "moe_decode": None if us_moe is None else {
            "us_per_launch": round(us_moe, 3), "bytes_per_launch": int(moe_bytes), "achieved_gbs": round(moe_gbs, 1)},
        "prefill": prefill,
        "config2": c2,
        "config4": c4,
        "lm_head": lmh,
        "step_graph": stp,
        "draft_head": drf,
        "reference_shape_moe_decode": rd,
        "reference_shape_chain": rc_,
        "pool": pl,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
