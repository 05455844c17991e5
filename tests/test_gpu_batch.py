"""Batched verify (several sequences, one weight pass) on an MI355X, through the C ABI.

The reference keeps one KV cache per Model (src/model.rs:16-26), so a batch has no reference
output of its own: each sequence of a batch must give exactly what it gives alone (the same
accepted counts, next tokens and positions, and afterwards bit-identical logits, which also
checks every cached K/V row). A single sequence is pinned to the oracle by test_gpu.py.
"""
import sys

import numpy as np
import pytest

import layerstream_amd as LS
import oracle_py as O
import tinymodels as T
from test_gpu import bits, cpu_model, gpu_model, qwen05b, qwen3b, tiny

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def batch_model(m, n_seq, max_ctx=128, graphs=True):
    src = LS.Source.from_memory(m["config_text"], m["layers"], m["embed"], m["norm"])
    b = LS.Model(src, LS.MODE_RESIDENT, 2, max_ctx, 0, n_seq=n_seq)
    b.use_graphs(graphs)
    return b


def run_against_alone(m, prompts, plan, greedy, max_ctx, graphs=True, vocab=T.VOCAB):
    """plan: per step, per sequence (k, good): a block of the last token, `good` drafts from the
    greedy continuation and k - good wrong ones."""
    n = len(prompts)
    batch = batch_model(m, n, max_ctx, graphs)
    alone = [gpu_model(m, max_ctx=max_ctx) for _ in range(n)]
    last, done = [], []
    for s, p in enumerate(prompts):
        batch.select(s)
        a_b = batch.forward_argmax(p)
        a_1 = alone[s].forward_argmax(p)
        assert a_b == a_1, s
        if greedy is not None:
            assert a_b == greedy[s][0], s
        last.append(a_b)
        done.append(1)
    for step, ks in enumerate(plan):
        blocks = []
        for s, (k, good) in enumerate(ks):
            g = greedy[s]
            d = list(g[done[s] : done[s] + good]) + [(g[done[s] + good] + 5) % vocab] * (k - good)
            blocks.append([last[s]] + d[:k])
        say("batch step", step, [len(b) for b in blocks])
        got = batch.verify_greedy_batch(blocks)
        for s in range(n):
            want = alone[s].verify_greedy(blocks[s])
            assert got[s] == want, (step, s, got[s], want)
            batch.select(s)
            assert batch.pos() == alone[s].pos(), (step, s)
            acc, nxt = want
            assert nxt == greedy[s][done[s] + acc], (step, s, acc, nxt)
            done[s] += acc + 1
            last[s] = nxt
    for s in range(n):
        batch.select(s)
        lb, la = batch.forward([last[s]]), alone[s].forward([last[s]])
        assert np.array_equal(bits(lb), bits(la)), s
    return batch


def test_batched_verify_gives_each_sequence_what_it_gets_alone():
    m = tiny("int8")
    # prompt lengths put sequence boundaries at and across 16-row tiles
    prompts = [[(37 * s + 11 * i + 1) % T.VOCAB for i in range(n)] for s, n in enumerate([6, 19, 3, 40, 11])]
    cpu = cpu_model(m, max_ctx=200)
    greedy = []
    for p in prompts:
        cpu.reset()
        greedy.append(O.plain_greedy(cpu, p, 120))
    plan = [
        [(8, 2), (8, 0), (8, 8), (3, 1), (0, 0)],
        [(1, 1), (8, 3), (5, 5), (8, 0), (32, 4)],
        [(8, 2), (8, 0), (8, 8), (3, 1), (0, 0)],  # same block lengths: a graph replay
        [(32, 32), (2, 0), (0, 0), (8, 7), (8, 1)],
        [(8, 2), (8, 0), (8, 8), (3, 1), (0, 0)],
    ]
    for graphs in (True, False):
        say("graphs", graphs)
        run_against_alone(m, prompts, plan, greedy, max_ctx=160, graphs=graphs)


def test_batched_verify_bf16_tiny_and_single_sequence_batches():
    m = tiny("bf16")
    prompts = [[5, 17, 301, 42, 599, 0], [250, 3, 77]]
    cpu = cpu_model(m)
    greedy = []
    for p in prompts:
        cpu.reset()
        greedy.append(O.plain_greedy(cpu, p, 40))
    run_against_alone(m, prompts, [[(4, 2), (4, 4)], [(4, 0), (2, 1)], [(4, 4), (4, 0)]], greedy, max_ctx=96)
    run_against_alone(m, prompts[:1], [[(4, 2)], [(8, 8)], [(4, 1)]], greedy[:1], max_ctx=96)


def test_batched_verify_rejects_bad_requests():
    m = tiny("int8")
    b = batch_model(m, 3, max_ctx=30)
    for s in range(3):
        b.select(s)
        b.forward_argmax([1, 2, 3])
    with pytest.raises(ValueError):
        b.verify_greedy_batch([[1], [2]])  # two blocks for three sequences
    for bad in ([[1], [], [2]], [[1], [1] * 34, [2]], [[1], [T.VOCAB], [2]], [[1], [1] * 28, [2]]):
        with pytest.raises(LS.LayerstreamError):
            b.verify_greedy_batch(bad)  # empty, too long, outside the vocabulary, context full
    with pytest.raises(LS.LayerstreamError):
        b.select(3)
    for s in range(3):  # nothing above moved a position
        b.select(s)
        assert b.pos() == 3, s
    got = b.verify_greedy_batch([[1], [1] * 27, [2, 3]])
    for s, (acc, _) in enumerate(got):
        b.select(s)
        assert b.pos() == 3 + acc + 1, s


def batch_vs_alone(q, vocab, lens, max_ctx, plan, tag, seed=7):
    """Prompts of the given lengths through one batch model and one model per sequence, then the
    plan's verify steps (per step, per sequence: drafts from the greedy continuation accepted);
    every sequence of the batch must give what it gives alone, bit for bit."""
    src = LS.Source.from_lsq_image(q["lsq"])
    rng = np.random.default_rng(seed)
    prompts = [rng.integers(0, vocab, n).tolist() for n in lens]
    batch = LS.Model(src, LS.MODE_RESIDENT, 2, max_ctx, 0, n_seq=len(prompts))
    alone = [LS.Model(src, LS.MODE_RESIDENT, 2, max_ctx, 0) for _ in prompts]
    last = []
    for s, p in enumerate(prompts):
        batch.select(s)
        a = batch.forward_argmax(p)
        assert a == alone[s].forward_argmax(p), s
        last.append(a)
    # greedy continuations from the alone models, to script drafts that are partly accepted
    greedy = []
    for s in range(len(prompts)):
        p0 = alone[s].pos()
        g = [last[s]]
        for _ in range(24):
            g.append(alone[s].forward_argmax([g[-1]]))
        alone[s].truncate(p0)
        greedy.append(g)
    done = [1] * len(prompts)
    for step, goods in enumerate(plan):
        blocks = []
        for s, good in enumerate(goods):
            g = greedy[s]
            d = list(g[done[s] : done[s] + good]) + [(g[done[s] + good] + 1) % vocab] * (8 - good)
            blocks.append([last[s]] + d[:8])
        say(tag, "batch step", step)
        got = batch.verify_greedy_batch(blocks)
        for s in range(len(prompts)):
            want = alone[s].verify_greedy(blocks[s])
            assert got[s] == want, (step, s, got[s], want)
            acc, nxt = want
            assert nxt == greedy[s][done[s] + acc], (step, s)
            done[s] += acc + 1
            last[s] = nxt
    for s in range(len(prompts)):
        batch.select(s)
        assert batch.pos() == alone[s].pos()
        lb, la = batch.forward([last[s]]), alone[s].forward([last[s]])
        assert np.array_equal(bits(lb), bits(la)), s


def test_qwen05b_int8_batched_verify_matches_each_sequence_alone():
    """The 0.5B shape: a batch of 4 x 9 rows runs the multi-tile kernels (split gate|up and down
    launches, head over 3 tiles, attention per KV group: 7 heads x 9 rows in 4 query tiles);
    each sequence alone runs the single-tile fused ones."""
    q = qwen05b((8, 64))
    batch_vs_alone(q, LS.QWEN2_05B["vocab"], [130, 37, 300, 64], 400, [[8, 0, 3, 5], [2, 8, 0, 1], [0, 0, 8, 8]], "0.5B")


def test_qwen3b_int8_batched_verify_matches_each_sequence_alone():
    """The 3B shape (head_dim 128, 8 heads per KV group: 72 (head, row) pairs in 5 query tiles,
    256-column K shares): a batch of 3 x 9 rows against each sequence alone in the layer stack."""
    say("3B batch: synth + quantize")
    q = qwen3b((8, 64))
    batch_vs_alone(q, LS.QWEN2_3B["vocab"], [70, 260, 17], 320, [[8, 0, 3], [2, 8, 0]], "3B")
