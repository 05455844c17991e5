"""The persistent layer pass (LS_PASS=1): every layer of a one-tile pass in one launch of one
workgroup per CU, the stages handing tagged units to each other through the exchange area
instead of through counters. It runs the plans of the layer stack, so it must give the stack's
bits: logits, acceptance and positions, over prompts, single steps, blocks and verify steps, for
every weight format and the 0.5B shape. Its failure path obeys the same host-set error word, and
its debug timeline stamps every unit of every layer in order."""
import numpy as np
import pytest

import layerstream_amd as LS
from test_gpu import bits, env, gpu_model, qwen05b, say

pytestmark = pytest.mark.gpu

BLOCK = [8, 9, 400, 33, 120, 5, 77, 301, 2]


def pass_and_stack(m, max_ctx):
    """The stack and the pass; the pass keeps a timeline, which shows that it ran."""
    with env("LS_PASS", "0"):
        a = gpu_model(m, max_ctx=max_ctx)
    with env("LS_PASS", "1"), env("LS_PASS_TIMELINE", "1"):
        b = gpu_model(m, max_ctx=max_ctx)
    assert b.debug_timeline() is not None, "the pass does not fit this model"
    return a, b


def pass_ran(b):
    return int((b.debug_timeline()[..., 0] > 0).sum()) > 0


@pytest.mark.parametrize("fmt", [None, (8, 64), (4, 32)], ids=["bf16", "int8", "int4"])
def test_pass_gives_the_stack_bits_on_qwen05b(fmt):
    """Every weight format of the 0.5B shape (the tiny test model is too narrow for the layer
    stack, so it runs per-layer launches and says nothing about the pass): a 40-token prompt,
    single tokens, a block of 9 and verify steps."""
    rng = np.random.default_rng(40)
    prompt = rng.integers(0, LS.QWEN2_05B["vocab"], 40).tolist()
    a, b = pass_and_stack(qwen05b(fmt), 256)
    la, lb = a.forward(prompt), b.forward(prompt)  # prompt: several tiles, not the pass
    assert np.array_equal(bits(la), bits(lb))
    for step in range(3):  # single tokens: one tile, the pass
        la, lb = a.forward([int(np.argmax(la))]), b.forward([int(np.argmax(lb))])
        assert np.array_equal(bits(la), bits(lb)), step
    p = a.pos()
    va, vb = a.forward_multi(BLOCK, len(BLOCK)), b.forward_multi(BLOCK, len(BLOCK))
    assert np.array_equal(bits(va), bits(vb))
    a.truncate(p)
    b.truncate(p)
    for i in range(3):
        assert a.verify_greedy(BLOCK) == b.verify_greedy(BLOCK)
        assert a.pos() == b.pos()
        a.truncate(p)
        b.truncate(p)
    assert pass_ran(b)


def test_pass_gives_the_stack_bits_on_qwen05b_int8_verify_steps():
    """0.5B int8 after a 512-token prompt: the workload of the verify benchmark."""
    rng = np.random.default_rng(512)
    prompt = rng.integers(0, LS.QWEN2_05B["vocab"], 512).tolist()
    a, b = pass_and_stack(qwen05b((8, 64)), 1024)
    assert np.array_equal(bits(a.forward(prompt)), bits(b.forward(prompt)))
    p = a.pos()
    block = [int(x) for x in rng.integers(0, LS.QWEN2_05B["vocab"], 9)]
    for step in range(3):
        va, vb = a.forward_multi(block, 9), b.forward_multi(block, 9)
        say("0.5B pass vs stack, step", step, "max diff", float(np.max(np.abs(va - vb))))
        assert np.array_equal(bits(va), bits(vb)), step
        block = [int(np.argmax(va[-1]))] + block[1:]
    a.truncate(p)
    b.truncate(p)
    assert a.verify_greedy(block) == b.verify_greedy(block)
    assert a.pos() == b.pos()
    assert pass_ran(b)


def test_a_failed_wait_in_the_pass_is_an_error_and_the_next_call_is_clean():
    """The host sets the error word before the pass: every wait of the pass gives up at once, the
    launch drains, the call returns LS_E_DEVICE and moves no position, and the next call gives the
    stack's bits again."""
    rng = np.random.default_rng(6)
    prompt = rng.integers(0, LS.QWEN2_05B["vocab"], 40).tolist()
    a, b = pass_and_stack(qwen05b((8, 64)), 256)
    a.forward(prompt)
    b.forward(prompt)
    p = b.pos()
    b.debug_fail_next()
    with pytest.raises(LS.LayerstreamError) as e:
        b.forward_multi(BLOCK, len(BLOCK))
    assert e.value.code == -4
    assert b.pos() == p
    va, vb = a.forward_multi(BLOCK, len(BLOCK)), b.forward_multi(BLOCK, len(BLOCK))
    assert np.array_equal(bits(va), bits(vb))


def test_pass_timeline_stamps_every_unit_of_every_layer_in_order():
    """LS_PASS_TIMELINE=1 keeps 100 MHz stamps per (workgroup, layer, stage): every stage has
    stamped units in every layer, each unit's start comes before its done, and a layer's first
    q|k|v unit starts before its last down unit is done, which is before the next layer's last
    q|k|v unit is done."""
    with env("LS_PASS", "1"), env("LS_PASS_TIMELINE", "1"):
        m = gpu_model(qwen05b((8, 64)), max_ctx=256)
    m.forward([5, 17, 301, 42, 599, 0, 3, 4, 9])
    tl = m.debug_timeline()
    assert tl is not None
    G, L, stages, words = tl.shape
    assert (L, stages, words) == (m.cfg()["layers"], 5, 32)
    start, done = tl[..., 0].astype(np.int64), tl[..., 12].astype(np.int64)
    ran = start > 0
    assert np.all(ran.sum(axis=0) > 0)
    assert np.all(done[ran] >= start[ran])
    for l in range(L):
        assert start[ran[:, l, 0], l, 0].min() <= done[ran[:, l, 4], l, 4].max()
        if l + 1 < L:
            assert done[ran[:, l, 4], l, 4].max() <= done[ran[:, l + 1, 0], l + 1, 0].max()
