"""CPU oracle of the MTP-verify MoE path. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module, and only to check or
time against it; the product package (slotstream_spark_amd) never imports it.

Two layers:
  * the C restatement (ssmoe_oracle.c, built into _build/liboracle.so) for everything the kernels must match bit
    for bit: bf16 rounding, the exp, router logits/softmax/top-k/renorm, topk_stable, greedy and p/q acceptance,
    the shared-expert bf16 chain;
  * numpy / torch-CPU restatements for the tolerance-checked MoE math: affine unpack/dequant
    (kernels/affine_ref.py:10-30), the fp64 exact-dequant expert reference (tests/t0/test_moe_gemv_affine.py:71-82)
    and the reference's torch CPU layer moe_ref (model/reference_torch.py:118-134).

Pins: see the header of ssmoe_oracle.c and tests/test_oracle.py, tests/test_golden.py.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "liboracle.so"

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-B", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        P = ctypes.c_void_p
        i32, i64, f32 = ctypes.c_int, ctypes.c_int64, ctypes.c_float
        L.or_expf.argtypes, L.or_expf.restype = [f32], f32
        L.or_expf_vec.argtypes, L.or_expf_vec.restype = [P, P, i64], None
        L.or_dense_rows.argtypes, L.or_dense_rows.restype = [P, P, P, i32, i32, i32], None
        L.or_router_topk.argtypes, L.or_router_topk.restype = [P, P, P, P, P, i32, i32, i32, P], None
        L.or_topk_stable.argtypes, L.or_topk_stable.restype = [P, P, P, P, i32, i32, i32, P], None
        L.or_accept_greedy.argtypes, L.or_accept_greedy.restype = [P, P, i32, i32, P], None
        L.or_accept_pq.argtypes, L.or_accept_pq.restype = [P, P, P, P, i32, i32, f32, P, P], None
        L.or_draw_rows.argtypes, L.or_draw_rows.restype = [P, i32, i32, f32, P, P], None
        L.or_row_z.argtypes, L.or_row_z.restype = [P, i32, f32], f32
        L.or_shared_hs.argtypes, L.or_shared_hs.restype = [P, P, P, i32], None
        L.or_dense_rows_q4.argtypes, L.or_dense_rows_q4.restype = [P, P, P, P, P, i32, i32, i32], None
        L.or_combine_shared.argtypes, L.or_combine_shared.restype = [P, P, P, P, i32, i32], None
        L.or_residual_rmsnorm.argtypes = [P, P, P, f32, i32, i32, P, P]
        L.or_residual_rmsnorm.restype = None
        L.or_sample.argtypes = [P, i32, P, i32, f32, f32, i32, f32, f32, f32, P, P]
        L.or_sample.restype = None
        L.or_rmsnorm_groups.argtypes, L.or_rmsnorm_groups.restype = [P, P, f32, i32, i32, i32, P], None
        L.or_dense_epi.argtypes, L.or_dense_epi.restype = [P, i32, i32, P, i32, i32, i32, P, i32, P], None
        L.or_hc_mean.argtypes, L.or_hc_mean.restype = [P, P, i32, i32, i32, P], None
        L.or_hc_inject.argtypes, L.or_hc_inject.restype = [P, P, P, i32, i32, i32, P], None
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---------------------------------------------------------------- bf16 (numpy, independent of the C code)
def f32_to_bf16(a) -> np.ndarray:
    """fp32 -> bf16 bits (uint16), round to nearest even, NaN -> quiet NaN."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    q = ((u >> 16) | 0x40) & 0xFFFF
    return np.where(nan, q, r).astype(np.uint16)


def bf16_to_f32(b) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------- C restatement wrappers
def expf(x) -> np.ndarray:
    x = _c(x, np.float32)
    y = np.empty_like(x)
    lib().or_expf_vec(_p(x), _p(y), x.size)
    return y


def dense_rows(x_bits, w_bits) -> np.ndarray:
    """bf16 [T, H] x bf16 [N, H]^T -> bf16 bits [T, N] in the kernel's fixed order."""
    x, w = _c(x_bits, np.uint16), _c(w_bits, np.uint16)
    T, H = x.shape
    N = w.shape[0]
    out = np.empty((T, N), dtype=np.uint16)
    lib().or_dense_rows(_p(x), _p(w), _p(out), T, H, N)
    return out


def router_topk(logits_bits, K, bias=None):
    """bf16 logits [T, E] (+ fp32 bias [E]) -> (probs fp32 [T, E], ids int32 [T, K], weights fp32 [T, K])."""
    lg = _c(logits_bits, np.uint16)
    T, E = lg.shape
    probs = np.empty((T, E), np.float32)
    ids = np.empty((T, K), np.int32)
    w = np.empty((T, K), np.float32)
    scratch = np.empty(2 * E, np.float32)
    b = _c(bias, np.float32) if bias is not None else None
    lib().or_router_topk(_p(lg), _p(b), _p(probs), _p(ids), _p(w), T, E, K, _p(scratch))
    return probs, ids, w


def router(x_bits, w_bits, K, bias=None):
    """Full router: (logits bf16 bits, probs, ids, weights)."""
    logits = dense_rows(x_bits, w_bits)
    probs, ids, w = router_topk(logits, K, bias)
    return logits, probs, ids, w


def topk_stable(scores, k, n_valid=None):
    s = _c(scores, np.float32)
    R, N = s.shape
    idx = np.empty((R, k), np.int32)
    val = np.empty((R, k), np.float32)
    nv = _c(n_valid, np.int32) if n_valid is not None else None
    taken = np.empty(N, np.uint8)
    lib().or_topk_stable(_p(s), _p(nv), _p(idx), _p(val), R, N, k, _p(taken))
    return idx, val


def accept_greedy(target, drafts) -> np.ndarray:
    t = _c(target, np.float32)
    d = _c(drafts, np.int32)
    D = d.size
    out = np.empty(D + 5, np.int32)
    lib().or_accept_greedy(_p(t), _p(d), D, t.shape[1], _p(out))
    return out


def accept_pq(target, draft, drafts, uniforms, temperature) -> np.ndarray:
    t = _c(target, np.float32)
    q = _c(draft, np.float32)
    d = _c(drafts, np.int32)
    u = _c(uniforms, np.float32)
    D, V = d.size, t.shape[1]
    out = np.empty(D + 5, np.int32)
    nch = (V + 1023) // 1024
    work = np.empty(nch * 65 + 64, np.float32)
    lib().or_accept_pq(_p(t), _p(q), _p(d), _p(u), D, V, float(temperature), _p(out), _p(work))
    return out


def draw_rows(logits, temperature, uniforms) -> np.ndarray:
    """x_r ~ softmax(logits[r] / temperature) with uniforms[r]: the proposal draw of the p/q round (or_draw_rows)."""
    x = _c(logits, np.float32)
    u = _c(uniforms, np.float32)
    R, V = x.shape
    out = np.empty(R, np.int32)
    lib().or_draw_rows(_p(x), R, V, float(temperature), _p(u), _p(out))
    return out


def row_z(x, temperature) -> float:
    x = _c(x, np.float32)
    return float(lib().or_row_z(_p(x), x.size, float(temperature)))


def dense_rows_q4(x_bits, words, s_bits, b_bits) -> np.ndarray:
    """bf16 [T, K] x affine 4-bit (gs 64) [N, K]^T -> bf16 bits [T, N] (or_dense_rows_q4: the or_dense_rows order,
    each weight q * s + b in fp32 first). words uint32/int32 [N, K/8], s, b bf16 bits [N, K/64]."""
    x = _c(x_bits, np.uint16)
    wd = np.ascontiguousarray(words).view(np.uint32)
    sb, bb = _c(s_bits, np.uint16), _c(b_bits, np.uint16)
    T, K = x.shape
    N = wd.shape[0]
    if wd.shape[1] * 8 != K or sb.shape != (N, K // 64) or bb.shape != (N, K // 64):
        raise ValueError("words [N, K/8], s and b [N, K/64]")
    out = np.empty((T, N), dtype=np.uint16)
    lib().or_dense_rows_q4(_p(x), _p(wd), _p(sb), _p(bb), _p(out), T, K, N)
    return out


def shared_expert_q4(x_bits, gate, up, down, sg_bits):
    """The shared expert's bf16 chain with affine 4-bit gate/up/down projections (each a (words, s bits, b bits)
    triple; the gate logit row sg stays bf16) -> (sh bf16 bits [T, H], gate projection bf16 bits [T])."""
    g = dense_rows_q4(x_bits, *gate)
    u = dense_rows_q4(x_bits, *up)
    hs = np.empty_like(g)
    lib().or_shared_hs(_p(g), _p(u), _p(hs), g.size)
    sh = dense_rows_q4(hs, *down)
    sgl = dense_rows(x_bits, sg_bits)[:, 0].copy()
    return sh, sgl


def shared_expert(x_bits, gate_bits, up_bits, down_bits, sg_bits):
    """bf16 chain of the shared expert -> (sh bf16 bits [T, H], gate projection bf16 bits [T])."""
    g = dense_rows(x_bits, gate_bits)
    u = dense_rows(x_bits, up_bits)
    hs = np.empty_like(g)
    lib().or_shared_hs(_p(g), _p(u), _p(hs), g.size)
    sh = dense_rows(hs, down_bits)
    sgl = dense_rows(x_bits, sg_bits)[:, 0].copy()
    return sh, sgl


def sample(logits, generated, temperature, top_p, top_k, min_p, presence_penalty, u):
    """The device sampler's definition (Sampler.next, engine/sampler.py:76-108, with this build's sum order and
    exp): (token, flags). Parameters must already be sanitized; `generated` is any iterable of token ids."""
    x = _c(logits, np.float32)
    g = np.array(sorted(set(int(t) for t in generated)), dtype=np.int32)
    out = np.zeros(2, np.int32)
    work = np.empty(2 * x.size, np.float32)
    lib().or_sample(_p(x), x.size, _p(g) if g.size else None, int(g.size), float(temperature), float(top_p),
                    int(top_k), float(min_p), float(presence_penalty), float(u), _p(out), _p(work))
    return int(out[0]), int(out[1])


def accept_sampled(target, drafts, seen, temperature, top_p, top_k, min_p, presence_penalty, uniforms):
    """The sampled verify round (engine/generate.py:208-229): row i stops the round if it holds a non-finite logit
    (:210-212), else draws with `sample` (uniforms[i], penalty set seen + tokens emitted so far, :213-214) and the
    round continues while the token equals drafts[i]. Returns int32 [D+5]: n_accept, n_emit, n_uniform, flags
    (1 non-finite row, 2 draft out of range, 8 argmax fallback), tokens (-1 past n_emit)."""
    t = _c(target, np.float32)
    D, V = t.shape[0] - 1, t.shape[1]
    out = np.zeros(D + 5, np.int32)
    out[4:] = -1
    gen = set(int(v) for v in seen)
    for i in range(D + 1):
        if not np.isfinite(t[i]).all():
            out[3] |= 1
            break
        tok, fb = sample(t[i], gen, temperature, top_p, top_k, min_p, presence_penalty, uniforms[i])
        out[4 + i] = tok
        out[1] = i + 1
        if temperature > 0:
            out[2] = i + 1
        out[3] |= 8 if fb else 0
        gen.add(tok)
        if i < D:
            d = int(drafts[i])
            if d < 0 or d >= V:
                out[3] |= 2
            if tok == d:
                out[0] = i + 1
                continue
        break
    return out


def shared_hs(g_bits, u_bits) -> np.ndarray:
    """hs = bf16(bf16(silu(g)) * u) elementwise on bf16 bits (the shared expert's F.silu and product)."""
    g = _c(g_bits, np.uint16)
    u = _c(u_bits, np.uint16)
    hs = np.empty_like(g)
    lib().or_shared_hs(_p(g), _p(u), _p(hs), g.size)
    return hs


def combine_shared(routed, sh_bits, sgl_bits) -> np.ndarray:
    r = _c(routed, np.float32)
    sh = _c(sh_bits, np.uint16)
    sg = _c(sgl_bits, np.uint16)
    T, H = r.shape
    y = np.empty((T, H), np.uint16)
    lib().or_combine_shared(_p(r), _p(sh), _p(sg), _p(y), T, H)
    return y


def residual_rmsnorm(resid_bits, y_bits=None, w_bits=None, eps=1e-6):
    """(stream_out, mixed) uint16 bf16 bits [R, H]: s = bf16(resid + y), mixed = bf16((s r) w) (or_residual_rmsnorm)."""
    x = _c(resid_bits, np.uint16)
    R, H = x.shape
    y = None if y_bits is None else _c(y_bits, np.uint16)
    w = None if w_bits is None else _c(w_bits, np.uint16)
    so = np.empty((R, H), np.uint16)
    mx = np.empty((R, H), np.uint16)
    lib().or_residual_rmsnorm(_p(x), None if y is None else _p(y), None if w is None else _p(w), eps, R, H, _p(so),
                              _p(mx))
    return so, mx


# ---------------------------------------------------------------- MTP head, dense part (or_* in ssmoe_oracle.c)
EPI_NONE, EPI_ADD, EPI_SILU_DIV, EPI_SIGMOID, EPI_INJECT = range(5)


def rmsnorm_groups(x_bits, w_bits=None, eps=1e-6, group=None):
    """bf16 bits [R, n] -> bf16 bits [R, n]: rmsnorm per group of `group` (default n) elements (or_rmsnorm_groups)."""
    x = _c(x_bits, np.uint16)
    x2 = x.reshape(-1, x.shape[-1])
    R, n = x2.shape
    G = n if group is None else int(group)
    w = None if w_bits is None else _c(w_bits, np.uint16)
    out = np.empty_like(x2)
    lib().or_rmsnorm_groups(_p(x2), _p(w), float(eps), R, n, G, _p(out))
    return out.reshape(x.shape)


def dense_epi(x_bits, w_bits, epi=EPI_NONE, hc=1, add_bits=None, add_div=1):
    """lin on a bf16 weight with the op after it fused (or_dense_epi): x [R, K], w [N, K] -> bf16 bits [R, N]."""
    x = _c(x_bits, np.uint16)
    w = _c(w_bits, np.uint16)
    R, K = x.shape
    N = w.shape[0]
    add = None if add_bits is None else _c(add_bits, np.uint16)
    out = np.empty((R, N), np.uint16)
    lib().or_dense_epi(_p(x), R, K, _p(w), N, int(epi), int(hc), _p(add), int(add_div), _p(out))
    return out


def hc_mean(m_bits, hn_bits, hc):
    """[S, hc H] x2 -> [S, H]: bf16(sum_c bf16(m hn) / hc) (or_hc_mean)."""
    m = _c(m_bits, np.uint16)
    hn = _c(hn_bits, np.uint16)
    S = m.shape[0]
    H = m.shape[1] // hc
    out = np.empty((S, H), np.uint16)
    lib().or_hc_mean(_p(m), _p(hn), S, hc, H, _p(out))
    return out


def hc_inject(hyp_bits, y_bits, inj_bits):
    """hyp [S, hc H], y [S, H], inj [S, hc] -> bf16(hyp + bf16(y inj)) (or_hc_inject)."""
    h = _c(hyp_bits, np.uint16)
    y = _c(y_bits, np.uint16)
    inj = _c(inj_bits, np.uint16)
    S, hc = inj.shape
    H = y.shape[1]
    out = np.empty_like(h)
    lib().or_hc_inject(_p(h), _p(y), _p(inj), S, hc, H, _p(out))
    return out


def argmax_bf16(logits) -> np.ndarray:
    """torch.argmax(bf16 logits .float()) per row (engine/mtp.py:275): the first maximal index, NaN counting as the
    maximum (np.argmax and torch.argmax agree on both)."""
    v = bf16_to_f32(f32_to_bf16(np.asarray(logits, np.float32)))
    return np.argmax(v.reshape(-1, v.shape[-1]), axis=-1).astype(np.int32)


# ---------------------------------------------------------------- affine 4-bit (kernels/affine_ref.py:10-30)
def unpack4(q) -> np.ndarray:
    """int32/uint32 [N, K/8] -> uint8 [N, K]; element i at bits [4i, 4i+4) of the little-endian stream."""
    b = np.ascontiguousarray(q).view(np.uint8)
    out = np.empty(b.shape[:-1] + (b.shape[-1] * 2,), dtype=np.uint8)
    out[..., 0::2] = b & 15
    out[..., 1::2] = b >> 4
    return out


def dequant(q, s_bits, b_bits, gs=64, dtype=np.float32) -> np.ndarray:
    """w = q * s + b per group of gs (fp32 like affine_ref.dequant, or fp64 for the exact reference)."""
    u = unpack4(q).astype(dtype)
    s = bf16_to_f32(s_bits).astype(dtype)
    b = bf16_to_f32(b_bits).astype(dtype)
    n, k = u.shape
    if k % gs or s.shape != (n, k // gs) or b.shape != (n, k // gs):
        raise ValueError(f"shape mismatch: q {u.shape} s {s.shape} gs {gs}")
    return u * np.repeat(s, gs, axis=1) + np.repeat(b, gs, axis=1)


def gemv_affine4_fp64(x, q, s_bits, b_bits, gs=64):
    """gemv (kernels/gemv_affine.py:214-262) in fp64 on the exactly dequantized weights: (y [R, N], bound [R, N])
    with bound = sum_k |x_k w_k|, the scale a fp32 accumulation error is measured against."""
    w = dequant(q, s_bits, b_bits, gs, np.float64)
    x64 = np.asarray(x, dtype=np.float64)
    return x64 @ w.T, np.abs(x64) @ np.abs(w).T


def record_offsets(H, I):
    """Piece offsets of one record (reference order, kernels/moe_gemv_affine.py:22-25 scaled to (H, I))."""
    w_gu, sb_gu = I * H // 2, I * (H // 64) * 2
    w_d, sb_d = H * I // 2, H * (I // 64) * 2
    offs, o = [], 0
    for size in (w_gu, sb_gu, sb_gu, w_gu, sb_gu, sb_gu, w_d, sb_d, sb_d):
        offs.append(o)
        o += size
    return offs, o


def unpack_record(rec: np.ndarray, H, I):
    """uint8 record -> ((q, s, b) gate, up, down) numpy arrays; the oracle's own reading of the layout."""
    offs, total = record_offsets(H, I)
    rec = np.ascontiguousarray(rec, dtype=np.uint8)
    if rec.size != total:
        raise ValueError(f"record has {rec.size} bytes, expected {total}")
    shapes = [((I, H // 8), (I, H // 64)), ((I, H // 8), (I, H // 64)), ((H, I // 8), (H, I // 64))]
    pieces = []
    for p, ((qn, qk), (sn, sk)) in enumerate(shapes):
        ow, os_, ob = offs[3 * p: 3 * p + 3]
        q = rec[ow: ow + qn * qk * 4].view(np.uint32).reshape(qn, qk)
        s = rec[os_: os_ + sn * sk * 2].view(np.uint16).reshape(sn, sk)
        b = rec[ob: ob + sn * sk * 2].view(np.uint16).reshape(sn, sk)
        pieces.append((q, s, b))
    return pieces


def expert_dense(rec, H, I, dtype=np.float64):
    """(gate [I, H], up [I, H], down [H, I]) dequantized from a record."""
    return tuple(dequant(q, s, b, 64, dtype) for (q, s, b) in unpack_record(rec, H, I))


def silu64(v):
    return v / (1.0 + np.exp(-v))


def moe_routed_fp64(x, ids, w, dense_of):
    """fp64 exact-dequant routed output (tests/t0/test_moe_gemv_affine.py:71-82): x [T, H] (any float dtype),
    ids [T, K], w [T, K], dense_of(e) -> (gate, up, down) fp64. Returns fp64 [T, H]."""
    x = np.asarray(x, dtype=np.float64)
    T, H = x.shape
    out = np.zeros((T, H), np.float64)
    for t in range(T):
        for k in range(ids.shape[1]):
            g, u, d = dense_of(int(ids[t, k]))
            h = silu64(g @ x[t]) * (u @ x[t])
            out[t] += float(w[t, k]) * (d @ h)
    return out


def rel_l2(a, ref) -> float:
    a = np.asarray(a, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(a - ref) / np.linalg.norm(ref))


# ---------------------------------------------------------------- torch CPU restatement of moe_ref
def moe_ref(x, router_w, topk, expert, sh_gate, sh_up, sh_down, sh_g, bias=None):
    """model/reference_torch.py:118-134 restated on torch CPU: bf16 router F.linear, fp32 softmax, torch.topk,
    renormalise, per token and rank fp32 expert matvecs summed in rank order, cast to the input dtype, plus the
    sigmoid-gated shared expert in the input dtype. `expert(e) -> (gate [I,H], up [I,H], down [H,I])` dense fp32.
    `bias` (fp32 [E], not in the reference) is added to the logits in fp32 before the softmax.
    Returns (y, ids, renormalised weights)."""
    import torch
    import torch.nn.functional as F

    logits = F.linear(x, router_w)
    scores = logits.float() + bias if bias is not None else logits
    probs = F.softmax(scores, dtype=torch.float, dim=-1)
    tv, ti = torch.topk(probs, topk, dim=-1)
    tv = tv / tv.sum(-1, keepdim=True)
    out = torch.zeros(x.shape[0], x.shape[1], dtype=torch.float32)
    for t in range(x.shape[0]):
        xt = x[t].float()
        for r in range(topk):
            gw, uw, dw = expert(int(ti[t, r]))
            h = F.silu(gw.float() @ xt) * (uw.float() @ xt)
            out[t] += tv[t, r] * (dw.float() @ h)
    sh = F.linear(F.silu(F.linear(x, sh_gate)) * F.linear(x, sh_up), sh_down)
    sh = torch.sigmoid(F.linear(x, sh_g)) * sh
    return out.to(x.dtype) + sh, ti, tv


# ---------------------------------------------------------------- splitmix64 uniforms (engine/sampler.py:20-24, :101-102)
_M64 = (1 << 64) - 1


def splitmix(v: int) -> int:
    v = (v + 0x9E3779B97F4A7C15) & _M64
    v = ((v ^ (v >> 30)) * 0xBF58476D1CE4E5B9) & _M64
    v = ((v ^ (v >> 27)) * 0x94D049BB133111EB) & _M64
    return v ^ (v >> 31)


def uniforms(seed: int, n: int) -> np.ndarray:
    """n draws of the sampler's stream: state = splitmix(state + 1); u = f32((state >> 11) / 2^53)."""
    st = seed if seed != 0 else 0xDEADBEEF
    out = np.empty(n, np.float32)
    for i in range(n):
        st = splitmix((st + 1) & _M64)
        out[i] = np.float32((st >> 11) / float(1 << 53))
    return out


# ---------------------------------------------------------------- prefill (kernels/moe_align.py, fused_moe_affine.py)
def padded_rows(r: int, num_local: int, block_m: int) -> int:
    n = r + num_local * (block_m - 1)
    return (n + block_m - 1) // block_m * block_m


def moe_align(local_expert, num_local: int, block_m: int):
    """kernels/moe_align.py:17-48 restated in numpy: (sorted_rows, block_expert, num_padded)."""
    le = np.asarray(local_expert, dtype=np.int64)
    r = le.size
    p = padded_rows(r, num_local, block_m)
    key = np.where((le >= 0) & (le < num_local), le, num_local)
    order = np.argsort(key, kind="stable")
    counts = np.bincount(key, minlength=num_local + 1)[:num_local]
    padded = (counts + block_m - 1) // block_m * block_m
    pad_end = np.cumsum(padded)
    pad_start = pad_end - padded
    start = np.cumsum(counts) - counts
    sorted_rows = np.full(p, r, dtype=np.int32)
    ks = key[order]
    for j, (row, k) in enumerate(zip(order, ks)):
        if k < num_local:
            sorted_rows[pad_start[k] + j - start[k]] = row
    nb = p // block_m
    pos = np.arange(nb, dtype=np.int64) * block_m
    idx = np.searchsorted(pad_end, pos, side="right")
    block_expert = np.where(idx < num_local, idx, -1).astype(np.int32)
    num_padded = int(pad_end[-1]) if num_local else 0
    return sorted_rows, block_expert, num_padded


def dequant_bf16(q, s_bits, b_bits, gs=64) -> np.ndarray:
    """bf16(q * s + b) as float32 (the reference's _wtile, fused_moe_affine.py:39-50): q*s is exact in fp32, so the
    fp32 value of q*s + b has one rounding whether or not it is fused."""
    w = dequant(q, s_bits, b_bits, gs, np.float32)
    return bf16_to_f32(f32_to_bf16(w))


def expert_bf16(rec, H, I):
    """(gate [I, H], up [I, H], down [H, I]) as float64 arrays of the bf16-rounded dequantized weights."""
    return tuple(dequant_bf16(q, s, b).astype(np.float64) for (q, s, b) in unpack_record(rec, H, I))


def prefill_rows(x, row_token, row_weight, row_expert, weights_of):
    """fused_moe_affine semantics per row (fp64 accumulation of bf16 operands): h = bf16(silu(g) * u), then
    out_rows[r] = fp32((Wd h) * w). x float array [T, H] holding bf16 values; weights_of(e) -> expert_bf16 tuple.
    Rows whose expert is negative are zero. Returns (h float32 [R, I] of bf16 values, out_rows float32 [R, H])."""
    x = np.asarray(x, np.float64)
    row_expert = np.asarray(row_expert)
    R = row_expert.size
    H = x.shape[1]
    I = None
    out = np.zeros((R, H), np.float32)
    hs = None
    for e in np.unique(row_expert):
        if e < 0:
            continue
        rows = np.nonzero(row_expert == e)[0]
        g_w, u_w, d_w = weights_of(int(e))
        if hs is None:
            I = g_w.shape[0]
            hs = np.zeros((R, I), np.float32)
        xr = x[np.asarray(row_token)[rows]]
        g = xr @ g_w.T
        u = xr @ u_w.T
        h = bf16_to_f32(f32_to_bf16((g / (1.0 + np.exp(-g)) * u).astype(np.float32)))
        hs[rows] = h
        o = (h.astype(np.float64) @ d_w.T) * np.asarray(row_weight, np.float64)[rows, None]
        out[rows] = o.astype(np.float32)
    return hs, out


def combine_rank_order(out_rows, T, K):
    """Sequential fp32 sum of each token's K rows in rank order (fused_moe_affine.py:164-172)."""
    v = np.asarray(out_rows, np.float32).reshape(T, K, -1)
    acc = v[:, 0].copy()
    for k in range(1, K):
        acc = (acc + v[:, k]).astype(np.float32)
    return acc
