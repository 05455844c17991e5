"""The draft model's proposals on the device (src/spec.rs:100-107): kk single-token passes, each fed
the argmax of the one before, run as one chain of one-token verify passes with one host wait. They
must be the tokens (and leave the positions) of kk forward + argmax calls, eager and replayed from a
graph, for the tiny model and the 0.5B shape in int4 (the draft of the int8 target in the benchmark),
and speculative decoding with such a draft must still give the oracle's greedy tokens."""
import numpy as np
import pytest

import layerstream_amd as LS
import oracle_py as O
from test_gpu import PROMPT, cpu_model, gpu_model, qwen05b, say, tiny

pytestmark = pytest.mark.gpu


def forward_loop(m, first, k):
    out, cur = [], first
    for _ in range(k):
        cur = int(np.argmax(m.forward([cur])))
        out.append(cur)
    return out


@pytest.mark.parametrize("name", ["int8", "int4", "bf16"])
def test_draft_chain_gives_the_tokens_of_single_passes(name):
    m = tiny(name)
    for graphs in (True, False):
        a, b = gpu_model(m), gpu_model(m)
        b.use_graphs(graphs)
        first = int(np.argmax(a.forward(PROMPT)))
        b.forward(PROMPT)
        for k in (1, 3, 8, 8, 5):  # 8 twice: a graph replay
            say("draft chain", name, "graphs", graphs, "k", k)
            want = forward_loop(a, first, k)
            got = b.draft_chain(first, k)
            assert got == want, (name, graphs, k)
            assert a.pos() == b.pos()
            first = got[-1]


def test_draft_chain_of_the_int4_05b_model_after_a_prompt():
    m = qwen05b((4, 32))
    rng = np.random.default_rng(7)
    prompt = rng.integers(0, LS.QWEN2_05B["vocab"], 64).tolist()
    a, b = gpu_model(m, max_ctx=256), gpu_model(m, max_ctx=256)
    first = int(np.argmax(a.forward(prompt)))
    b.forward(prompt)
    for step in range(3):
        want = forward_loop(a, first, 8)
        got = b.draft_chain(first, 8)
        say("0.5B int4 chain", step, got)
        assert got == want
        assert a.pos() == b.pos()
        first = got[-1]


def test_bad_chains_are_rejected():
    g = gpu_model(tiny("int8"), max_ctx=16)
    g.forward(PROMPT)
    for k in (0, 33):
        with pytest.raises(LS.LayerstreamError):
            g.draft_chain(1, k)
    with pytest.raises(LS.LayerstreamError):
        g.draft_chain(1, 16 - len(PROMPT) + 1)  # past the context limit
    assert g.pos() == len(PROMPT)
    s = gpu_model(tiny("int8"), LS.MODE_STREAM, 2)
    s.forward(PROMPT)
    with pytest.raises(LS.LayerstreamError) as e:
        s.draft_chain(1, 4)
    assert e.value.code == -5


@pytest.mark.parametrize("k", [1, 4, 8])
def test_speculation_with_a_device_draft_chain_matches_the_oracle(k):
    """int8 target, int4 draft of the same weights (resident, so its proposals run as chains):
    the tokens are the oracle's greedy continuation of the target."""
    target, draft = tiny("int8"), tiny("int4")
    want = O.plain_greedy(cpu_model(target, max_ctx=128), PROMPT, 30)
    t, d = gpu_model(target), gpu_model(draft)
    got, st = LS.speculative_greedy(t, LS.ModelDrafter(d), PROMPT, 30, k)
    say("spec with a draft chain, k", k, "accepted", st["accepted"], "of", st["drafted"])
    assert got == want
