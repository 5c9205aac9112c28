"""The C ABI without a GPU: libssmoe.so loads, exports exactly what include/ssmoe.h declares, computes its host-side
answers (record layout, workspace sizes) and rejects bad arguments with SSMOE_EINVAL before touching a device.
The Python mirrors raise the reference's ValueErrors and refuse CPU tensors instead of falling back."""
import ctypes
import re
from pathlib import Path

import pytest
import torch

from slotstream_spark_amd import _lib
from slotstream_spark_amd.kernels import moe_gemv_affine as mga
from slotstream_spark_amd.kernels.topk_stable import topk_stable

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "ssmoe.h"
EINVAL = 1


def _declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(ssmoe_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def L():
    if not _lib.LIB_PATH.exists():
        pytest.skip("libssmoe.so not built (python -m slotstream_spark_amd.build)")
    return _lib.lib()


def test_exports_every_declared_symbol(L):
    names = _declared()
    assert len(names) >= 14
    for n in names:
        assert hasattr(L, n), n
    assert sorted(_lib.SIGNATURES) == names  # the ctypes table binds exactly the header's list


def test_status_bits_match_the_kernels():
    """The status bits include/ssmoe.h publishes are the values the kernels raise (csrc/ss_common.hpp)."""
    hdr = dict((k, int(v)) for k, v in re.findall(r"#define SSMOE_ERR_(\w+)\s+(\d+)", HEADER.read_text()))
    src = (ROOT / "slotstream_spark_amd" / "csrc" / "ss_common.hpp").read_text()
    dev = dict((k, int(v)) for k, v in re.findall(r"\bSS_ERR_(\w+)\s*=\s*(\d+)", src))
    assert dev and hdr == dev
    assert all(v & (v - 1) == 0 for v in hdr.values())  # one bit each


def test_version_and_error_text(L):
    assert L.ssmoe_version() == _lib.ABI_VERSION
    assert L.ssmoe_record_layout(100, 512, (ctypes.c_int64 * 10)()) == EINVAL
    assert b"multiples of 64" in L.ssmoe_last_error()


def test_record_layout(L):
    offs, total = _lib.record_layout(2048, 512)
    assert offs == [0, 524288, 557056, 589824, 1114112, 1146880, 1179648, 1703936, 1736704]
    assert total == 1769472
    offs, total = _lib.record_layout(2560, 640)  # the reference constants (moe_gemv_affine.py:22-25)
    assert offs == [0, 819200, 870400, 921600, 1740800, 1792000, 1843200, 2662400, 2713600]
    assert total == 2764800
    assert mga.RECORD_BYTES == 1769472 and mga.O_DOWN_B == 1736704
    assert L.ssmoe_record_layout(2048, 512, None) == EINVAL


def test_workspace_sizes(L):
    assert L.ssmoe_verify_workspace_bytes(2, 2048, 512, 512, 10, 512) > 0
    assert L.ssmoe_verify_workspace_bytes(0, 2048, 512, 512, 10, 512) == -1
    assert L.ssmoe_accept_workspace_bytes(3, 151936) >= 4 * ((151936 + 1023) // 1024)
    assert L.ssmoe_accept_workspace_bytes(-1, 10) == -1


def test_trace_switch(L):
    assert L.ssmoe_set_trace(None, 0) == 0
    assert L.ssmoe_set_trace(ctypes.c_void_p(256), 10) == EINVAL


NONNULL = ctypes.c_void_p(4096)  # aligned dummy address; never dereferenced on an EINVAL path


@pytest.mark.parametrize("R,H,I,K,E,msg", [
    (0, 2048, 512, 10, 512, b"R must be"),
    (2, 2000, 512, 10, 512, b"H must be"),
    (2, 2048, 500, 10, 512, b"I must be"),
    (2, 2048, 512, 17, 512, b"K must be"),
])
def test_moe_decode_rejects_shapes(L, R, H, I, K, E, msg):
    p = NONNULL
    rc = L.ssmoe_moe_decode(p, 0, p, p, 0, p, 512, p, 512, p, p, p, R, H, I, K, E, None)
    assert rc == EINVAL and msg in L.ssmoe_last_error()


def test_moe_decode_rejects_tables(L):
    p = NONNULL
    assert L.ssmoe_moe_decode(None, 0, p, p, 0, p, 512, p, 512, p, p, p, 2, 2048, 512, 10, 512, None) == EINVAL
    assert L.ssmoe_moe_decode(p, 0, p, p, 1, p, 512, p, 512, p, p, p, 2, 2048, 512, 10, 512, None) == EINVAL
    assert b"map holds 512 entries" in L.ssmoe_last_error()
    assert L.ssmoe_moe_decode(ctypes.c_void_p(4100), 0, p, p, 0, p, 512, p, 512, p, p, p, 2, 2048, 512, 10, 512,
                              None) == EINVAL


def test_verify_layer_rejects(L):
    p = NONNULL
    args = lambda E, Is, ws: (p, p, None, p, p, p, p, 0, p, E, p, E, p, ws, p, p, p, None, 2, 2048, 512, Is, 10, E,
                              None)
    need = L.ssmoe_verify_workspace_bytes(2, 2048, 512, 512, 10, 512)
    assert L.ssmoe_moe_verify_layer(*args(1024, 512, need)) == EINVAL
    assert L.ssmoe_moe_verify_layer(*args(512, 500, need)) == EINVAL
    assert L.ssmoe_moe_verify_layer(*args(512, 512, need - 1)) == EINVAL
    assert b"workspace holds" in L.ssmoe_last_error()


def test_topk_router_accept_reject(L):
    p = NONNULL
    assert L.ssmoe_topk_stable(p, None, p, None, 1, 70000, 10, None) == EINVAL
    assert L.ssmoe_topk_stable(p, None, p, None, 1, 64, 65, None) == EINVAL
    assert L.ssmoe_router(p, p, None, p, None, p, p, 1, 2048, 512, 17, None) == EINVAL
    assert L.ssmoe_dense_gemv_bf16(p, p, p, 1, 2047, 8, None) == EINVAL
    ws = L.ssmoe_accept_workspace_bytes(3, 1000)
    assert L.ssmoe_accept_greedy(p, p, 61, 1000, p, ws, p, None) == EINVAL
    assert L.ssmoe_accept_greedy(p, p, 3, 1000, p, ws - 4, p, None) == EINVAL
    assert L.ssmoe_accept_pq(p, p, p, p, 3, 1000, 0.0, p, ws, p, None) == EINVAL
    assert b"temperature" in L.ssmoe_last_error()
    assert L.ssmoe_accept_greedy(p, p, 3, (1 << 20) + 1, p, 1 << 40, p, None) == EINVAL
    assert b"1048576" in L.ssmoe_last_error()


# ---------------------------------------------------------------- Python mirrors
def _decode_args(R=2, H=256, I=128, K=4, E=8, dtype=torch.bfloat16):
    return dict(x=torch.zeros(R, H, dtype=dtype), expert_ids=torch.zeros(R, K, dtype=torch.int32),
                weights=torch.zeros(R, K), layer=0, map_t=torch.zeros(E, dtype=torch.int32),
                slot_ptr_t=torch.zeros(E, dtype=torch.int64), h_buf=torch.zeros(R, K, I),
                o_buf=torch.zeros(R, K, H), out=torch.zeros(R, H))


@pytest.mark.parametrize("field,bad,msg", [
    ("x", torch.zeros(2, 256, dtype=torch.float16), "x must be"),
    ("expert_ids", torch.zeros(2, 4, dtype=torch.int64), "expert_ids must be"),
    ("weights", torch.zeros(2, 3), "weights must be"),
    ("map_t", torch.zeros(8, dtype=torch.int64), "map_t must be int32"),
    ("o_buf", torch.zeros(2, 4, 255), "buffer must be"),
    ("out", torch.zeros(2, 256, dtype=torch.float64), "buffer must be"),
])
def test_moe_decode_value_errors(field, bad, msg):
    a = _decode_args()
    a[field] = bad
    with pytest.raises(ValueError, match=msg):
        mga.moe_decode(**a)


def test_moe_decode_refuses_cpu_tensors():
    with pytest.raises(ValueError, match="same GPU"):
        mga.moe_decode(**_decode_args())
    with pytest.raises(ValueError, match="multiples of 64"):
        mga.moe_decode(**_decode_args(), cfg={"bk": 96})


def test_topk_value_errors():
    with pytest.raises(ValueError):
        topk_stable(torch.zeros(2, 8, dtype=torch.float64), 2)
    with pytest.raises(ValueError):
        topk_stable(torch.zeros(2, 8), 9)
    with pytest.raises(ValueError, match="GPU"):
        topk_stable(torch.zeros(2, 8), 2)


def test_shared_entry_points_reject_bad_arguments(L):
    p = ctypes.c_void_p(4096)
    assert L.ssmoe_shared_hs(p, 16, 4, 8, p, p, None) == EINVAL  # ld < 2 Is + 1
    assert b"ld >= 2 Is + 1" in L.ssmoe_last_error()
    assert L.ssmoe_shared_hs(None, 17, 4, 8, p, p, None) == EINVAL
    assert L.ssmoe_shared_hs(None, 17, 0, 8, None, None, None) == 0  # nothing to do
    assert L.ssmoe_combine_shared(p, p, p, p, 2, 6, None) == EINVAL  # H % 4
    assert L.ssmoe_combine_shared(ctypes.c_void_p(4100), p, p, p, 2, 8, None) == EINVAL  # routed alignment
    assert b"16-byte aligned" in L.ssmoe_last_error()
    assert L.ssmoe_combine_shared(None, None, None, None, 0, 8, None) == 0



def test_sample_rejects_bad_arguments(L):
    p = ctypes.c_void_p(4096)
    ws = L.ssmoe_sample_workspace_bytes(1000)
    assert ws > 2 * 1000 * 4 and L.ssmoe_sample_workspace_bytes(0) == -1
    assert L.ssmoe_sample_workspace_bytes((1 << 20) + 1) == -1
    good = dict(t=0.8, tp=0.9, tk=40, mp=0.0, pp=0.0)

    def call(V=1000, n=0, g=None, t=0.8, tp=0.9, tk=40, mp=0.0, pp=0.0, w=ws):
        return L.ssmoe_sample(p, V, g, n, t, tp, tk, mp, pp, p, ctypes.c_void_p(4096), w, p, None)
    assert call(t=-1.0) == EINVAL and b"temperature" in L.ssmoe_last_error()
    assert call(t=float("nan")) == EINVAL
    assert call(tp=0.0) == EINVAL and b"top_p" in L.ssmoe_last_error()
    assert call(tp=1.5) == EINVAL
    assert call(mp=-0.1) == EINVAL and b"min_p" in L.ssmoe_last_error()
    assert call(tk=-1) == EINVAL and b"top_k" in L.ssmoe_last_error()
    assert call(pp=float("inf")) == EINVAL
    assert call(n=3) == EINVAL and b"generated" in L.ssmoe_last_error()
    assert call(w=ws - 1) == EINVAL and b"workspace holds" in L.ssmoe_last_error()
    assert call(V=0) == EINVAL


def test_accept_sampled_rejects_bad_arguments(L):
    p = ctypes.c_void_p(4096)
    ws = L.ssmoe_accept_sampled_workspace_bytes(3, 1000)
    assert ws == 4 * L.ssmoe_sample_workspace_bytes(1000) and L.ssmoe_accept_sampled_workspace_bytes(61, 1000) == -1

    def call(D=3, V=1000, drafts=p, t=0.8, tp=0.9, w=ws):
        return L.ssmoe_accept_sampled(p, drafts, D, V, None, 0, t, tp, 40, 0.0, 0.0, p, ctypes.c_void_p(4096), w,
                                      p, None)
    assert call(D=61) == EINVAL and b"D must be" in L.ssmoe_last_error()
    assert call(D=-1) == EINVAL
    assert call(drafts=None) == EINVAL and b"non-null" in L.ssmoe_last_error()
    assert call(t=-0.5) == EINVAL and b"temperature" in L.ssmoe_last_error()
    assert call(tp=2.0) == EINVAL
    assert call(w=ws - 256) == EINVAL and b"workspace holds" in L.ssmoe_last_error()
    assert call(V=(1 << 20) + 1) == EINVAL


def test_gemv_rejects_bad_arguments(L):
    p = ctypes.c_void_p(4096)

    def call(R=2, K=2560, N=100, x=p, y=p, s=p):
        return L.ssmoe_gemv_affine4(x, 0, R, K, p, s, p, N, y, None)
    assert call(K=3000) == EINVAL and b"K must be" in L.ssmoe_last_error()
    assert call(N=0) == EINVAL and b"N must be" in L.ssmoe_last_error()
    assert call(R=-1) == EINVAL
    assert call(x=None) == EINVAL and b"non-null" in L.ssmoe_last_error()
    assert call(x=ctypes.c_void_p(4096 + 8)) == EINVAL and b"16-byte" in L.ssmoe_last_error()
    assert call(s=ctypes.c_void_p(4096 + 2)) == EINVAL and b"4-byte" in L.ssmoe_last_error()
    assert call(R=0) == 0  # nothing to do, no launch
    ws = L.ssmoe_lm_head_greedy_workspace_bytes(3, 248320)
    assert ws >= 4 * 12 and L.ssmoe_lm_head_greedy_workspace_bytes(61, 10) == -1

    def head(D=3, w=ws, drafts=p):
        return L.ssmoe_lm_head_greedy(p, 0, D, 2560, p, p, p, 248320, drafts, ctypes.c_void_p(4096), w, None, p, None)
    assert head(D=61) == EINVAL and b"D must be" in L.ssmoe_last_error()
    assert head(w=ws - 1) == EINVAL and b"workspace holds" in L.ssmoe_last_error()
    assert head(drafts=None) == EINVAL


def test_residual_rmsnorm_rejects_bad_arguments(L):
    p = ctypes.c_void_p(4096)
    rr = L.ssmoe_residual_rmsnorm
    assert rr(None, None, None, ctypes.c_float(1e-6), 2, 2048, None, p, None) == EINVAL
    assert rr(p, p, None, ctypes.c_float(1e-6), 2, 2048, None, ctypes.c_void_p(8192), None) == EINVAL  # y, no stream_out
    assert rr(p, None, None, ctypes.c_float(1e-6), 2, 2044, None, ctypes.c_void_p(8192), None) == EINVAL
    assert rr(p, None, None, ctypes.c_float(-1.0), 2, 2048, None, ctypes.c_void_p(8192), None) == EINVAL
    assert rr(p, None, None, ctypes.c_float(1e-6), 2, 2048, None, p, None) == EINVAL              # mixed aliases resid
    assert rr(ctypes.c_void_p(4098), None, None, ctypes.c_float(1e-6), 2, 2048, None, p, None) == EINVAL  # misaligned
    from slotstream_spark_amd.engine.step import residual_rmsnorm
    x = torch.zeros(2, 2048, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU"):
        residual_rmsnorm(x, None, torch.zeros_like(x))


def test_verify_chain_rejects_bad_arguments(L):
    p = ctypes.c_void_p(1 << 20)
    f = ctypes.c_float
    args = lambda H, eps, so: (p, None, f(eps), p, None, p, p, p, p, 0, p, 512, p, 512, p, 1 << 24, p, p, p, so, None,
                               2, H, 512, 512, 10, 512, None)
    assert L.ssmoe_moe_verify_layer_chain(*args(2304, 1e-6, None)) == EINVAL          # H not a multiple of 512
    assert b"multiple of 512" in L.ssmoe_last_error()
    assert L.ssmoe_moe_verify_layer_chain(*args(2048, -1.0, None)) == EINVAL
    assert L.ssmoe_moe_verify_layer_chain(*args(2048, 1e-6, p)) == EINVAL             # stream_out aliases stream_in
    assert b"alias" in L.ssmoe_last_error()
