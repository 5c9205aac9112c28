"""The self-speculative greedy loop (engine/generate.py mtp_decode over MoEStack and the MTP head) on the GPU.

Without attention each row of the MoE stack depends on its own token only, so the greedy sequence after a prompt is
the chain t -> f(t) of one-row steps, whatever the drafts: the loop must emit exactly that chain with the head's own
drafts, with drafts that are all right (every round keeps 1 + DEPTH rows), all wrong (keeps 1) or mixed, and leave
the position, the token list and the head's alignment as the reference's rollback and consume do
(engine/generate.py:152-238, engine/rollback.py:26-41). Also: StepRecord.restore_async with the keep read on the device.
"""
import pytest
import torch

from slotstream_spark_amd.engine import rollback as rb
from slotstream_spark_amd.engine.generate import MoEStack, mtp_decode
from slotstream_spark_amd.engine.mtp import MTPHead
from slotstream_spark_amd.engine.step import MoEWeights
from slotstream_spark_amd.engine.verify import MoEVerifyLayer
from slotstream_spark_amd.kernels.gemv_affine import AffineWeight
from slotstream_spark_amd.memory.synth import LayerWeights, head_weights, normal_bf16
from tests.gpu_util import make_pool

pytestmark = pytest.mark.gpu

H, I, E, K, NL, V, D = 2048, 512, 64, 4, 2, 4096, 2


def _lm_head(seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randint(-2**31, 2**31 - 1, (V, H // 8), generator=g, device="cuda", dtype=torch.int32)
    sc = (torch.randn((V, H // 64), generator=g, device="cuda") * 0.02).abs().to(torch.bfloat16)
    return AffineWeight(q, sc, (-8 * sc.float()).to(torch.bfloat16), 4, 64, V, H)


def _build(E, K):
    print(f"[generate] NL={NL} E={E} K={K} V={V} depth={D}", flush=True)
    pool = make_pool(E, H, I, seed=800, layers=NL + 1)
    lws = [LayerWeights(H, E, 512, seed=801 + l) for l in range(NL + 1)]
    mw = [MoEWeights(w.router_w, w.sh_gate, w.sh_up, w.sh_down, w.sh_g) for w in lws[:NL]]
    norms = [normal_bf16((H,), 0.1, 810 + l).float().add(1).to(torch.bfloat16) for l in range(NL + 1)]
    lm = _lm_head(820)
    hw = head_weights(H, 1, 32, V, seed=821)
    f = {}

    def make(max_ctx=64):
        stack = MoEStack(pool, mw, lm, hw.embed, depth=D, norm_weights=norms, top_k=K, max_ctx=max_ctx)
        moe = MoEVerifyLayer(pool, NL, lws[NL].router_w, lws[NL].sh_gate, lws[NL].sh_up, lws[NL].sh_down,
                             lws[NL].sh_g, top_k=K, max_tokens=4)
        return stack, MTPHead(hw, moe, lm, hc=1, max_ctx=max_ctx)

    probe, _ = make(1 << 20)

    def nxt(t):
        if t not in f:
            f[t] = probe.forward([t])[0][0]
        return f[t]

    return make, nxt


@pytest.fixture(scope="module")
def model():
    return _build(E, K)


@pytest.fixture(scope="module")
def model512():
    """The BASELINE layer shape (512 experts, top-10): the round's layers run as one ssmoe_moe_verify_chain launch."""
    return _build(512, 10)


def _chain(nxt, first, n):
    seq = [first]
    while len(seq) < n:
        seq.append(nxt(seq[-1]))
    return seq


@pytest.mark.parametrize("mode", ["head", "right", "wrong", "mixed"])
def test_loop_emits_the_plain_greedy_chain(model, mode):
    make, nxt = model
    print(f"[generate] drafts={mode}", flush=True)
    stack, head = make()
    prompt, n = [5, 17, 300], 14
    first = nxt(prompt[-1])
    want = _chain(nxt, first, n)
    calls = []

    def draft_fn(pending, depth, n_out):
        calls.append(n_out)
        right = _chain(nxt, nxt(pending), depth)
        if mode == "right" or (mode == "mixed" and len(calls) % 2):
            return right
        if mode == "mixed":
            return [right[0], (right[1] + 1) % V]
        return [(t + 1) % V for t in right]

    out, nan, secs, st = mtp_decode(stack, head, prompt, n, draft_fn=None if mode == "head" else draft_fn)
    assert out == want and not nan
    assert st["rounds"] == len(st["emitted_by_round"]) and sum(st["emitted_by_round"]) == len(out) - 1
    if mode == "right":
        assert all(e == D + 1 for e in st["emitted_by_round"][:-1]) and st["accepted"] >= st["drafted"] - D
    if mode == "wrong":
        assert st["accepted"] == 0 and all(e == 1 for e in st["emitted_by_round"])
    if mode == "mixed":
        assert 0 < st["accepted"] < st["drafted"]
    # Position and tokens: the prompt plus every kept row; the head stays aligned (pos == consumed - 1).
    assert stack.st.tokens[:len(prompt)] == prompt
    assert stack.st.pos == len(stack.st.tokens) == len(prompt) + len(out) - 1
    assert stack.st.tokens[len(prompt):] == out[:-1]
    assert head.state.aligned(head.consumed) and head.consumed == stack.st.pos
    assert stack.record.outstanding == 0


@pytest.mark.parametrize("mode", ["head", "mixed"])
def test_loop_through_the_single_launch_chain(model512, mode):
    """At E 512 / K 10 the verify rounds (rows = DEPTH + 1 = 3, the reference's width) go through the chain kernel
    and the loop still emits the plain greedy chain of one-row steps."""
    make, nxt = model512
    print(f"[generate] E=512 chain drafts={mode}", flush=True)
    stack, head = make()
    assert stack.graph.chain is not None, "the E 512 stack must run its rounds through ssmoe_moe_verify_chain"
    prompt, n = [7, 1234], 12
    want = _chain(nxt, nxt(prompt[-1]), n)
    calls = []

    def draft_fn(pending, depth, n_out):
        calls.append(n_out)
        right = _chain(nxt, nxt(pending), depth)
        return right if len(calls) % 2 else [right[0], (right[1] + 1) % V]

    out, nan, _, st = mtp_decode(stack, head, prompt, n, draft_fn=None if mode == "head" else draft_fn)
    assert out == want and not nan
    assert st["rounds"] > 0 and sum(st["emitted_by_round"]) == len(out) - 1
    if mode == "mixed":
        assert 0 < st["accepted"] < st["drafted"]
    assert stack.st.pos == len(prompt) + len(out) - 1
    assert head.state.aligned(head.consumed) and head.consumed == stack.st.pos


def test_loop_switches_to_plain_steps_near_the_context_end(model):
    make, nxt = model
    stack, head = make(max_ctx=9)
    prompt = [42]
    out, nan, _, st = mtp_decode(stack, head, prompt, 30)
    assert out == _chain(nxt, nxt(42), len(out))
    assert st["plain_steps"] > 0 and stack.st.pos <= 9


def test_step_record_restore_async():
    st = rb.SeqState(state={"multi": torch.zeros(2, 64, dtype=torch.bfloat16, device="cuda")})
    rec = rb.StepRecord(st, rows=3)
    for i in range(3):
        rec.ring["multi"][i].fill_(float(i + 1))
    for keep in (2, 3, 1):
        rec.begin()
        rec.restore_async(st, torch.tensor([keep], dtype=torch.int32, device="cuda"))
        torch.cuda.synchronize()
        assert torch.equal(st.state["multi"], torch.full((2, 64), float(keep), dtype=torch.bfloat16, device="cuda"))
    assert rec.outstanding == 0
