"""The layer stack's per-workgroup timeline (LS_STACK_TIMELINE=1, a separate build of the stack
kernel with stamps compiled in): the same bits as the stack without stamps, and stamps that
describe the launch (every workgroup of every layer stamped, in order within a workgroup, each
layer's roles tagged, a layer's down finished before the next layer's q|k|v)."""
import numpy as np
import pytest

from test_gpu import bits, env, gpu_model, qwen05b, qwen3b, say

pytestmark = pytest.mark.gpu

BLOCK = [8, 9, 400, 33, 120, 5, 77, 301, 2]


def check_stamps(tl, layers):
    tl = tl.reshape(-1, 8).astype(np.int64)
    layer, role = tl[:, 7] >> 8, tl[:, 7] & 255
    assert np.all(tl[:, 0] > 0) and np.all(tl[:, 2] > 0), "every workgroup ran and finished"
    assert set(layer.tolist()) == set(range(layers)) and set(role.tolist()) == set(range(5))
    assert np.all(tl[:, 2] >= tl[:, 0])
    waited = tl[:, 1] > 0
    assert np.all(tl[waited, 1] >= tl[waited, 0]) and np.all(tl[waited, 2] >= tl[waited, 1])
    for l in range(1, layers):
        assert tl[(layer == l - 1) & (role == 4), 2].max() <= tl[(layer == l) & (role == 0), 2].max()


@pytest.mark.parametrize("shape", ["0.5B", "3B"])
def test_stack_timeline_keeps_the_bits_and_stamps_every_workgroup(shape):
    say("stack timeline", shape)
    m = qwen05b((8, 64)) if shape == "0.5B" else qwen3b((8, 64))
    a = gpu_model(m, max_ctx=256)
    with env("LS_STACK_TIMELINE", "1"):
        b = gpu_model(m, max_ctx=256)
    rng = np.random.default_rng(7)
    prompt = rng.integers(0, 151936, 40).tolist()
    assert np.array_equal(bits(a.forward(prompt)), bits(b.forward(prompt)))
    p = a.pos()
    va, vb = a.forward_multi(BLOCK, len(BLOCK)), b.forward_multi(BLOCK, len(BLOCK))
    assert np.array_equal(bits(va), bits(vb))
    check_stamps(b.debug_timeline(raw=True), b.cfg()["layers"])
    a.truncate(p)
    b.truncate(p)
    for _ in range(2):
        assert a.verify_greedy(BLOCK) == b.verify_greedy(BLOCK)
        assert a.pos() == b.pos()
    check_stamps(b.debug_timeline(raw=True), b.cfg()["layers"])
