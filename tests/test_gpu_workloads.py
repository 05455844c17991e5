"""Parity with the oracle at the benchmark workloads' own sizes, the argmax tie rule on the device,
and the error path of the in-launch waits, on an MI355X through the C ABI.

Tolerances as in test_gpu.py: logits within 1e-3 relative of the oracle's at the full model
shapes, per-row argmax and accepted counts exactly, GPU-internal comparisons bit for bit.
"""
import sys

import numpy as np
import pytest

import layerstream_amd as LS
import oracle_py as O
import tinymodels as T
from test_gpu import bits, cpu_model, env, gpu_model, qwen05b, qwen3b, tiny, PROMPT

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def oracle_block(cpu, prompt, k, rng, vocab):
    """One oracle prefill: the greedy a, g1, g2 after the prompt, then the logits of the verify
    block [a, g1, g2, random ...] of k drafts (src/spec.rs:116). Returns (block, logits)."""
    a = int(np.argmax(cpu.forward(prompt)))
    g1 = int(np.argmax(cpu.forward([a])))
    g2 = int(np.argmax(cpu.forward([g1])))
    cpu.truncate(len(prompt))
    block = [a, g1, g2] + rng.integers(0, vocab, k - 2).tolist()
    return block, cpu.forward_multi(block, k + 1)


def want_acceptance(ref, block):
    m = 0
    while m < len(block) - 1 and int(ref[m].argmax()) == block[m + 1]:
        m += 1
    return m, int(ref[m].argmax())


def check_rows(got, ref, tag):
    rel = np.max(np.abs(got - ref)) / np.max(np.abs(ref))
    srt = np.sort(ref, axis=1)
    say(tag, "max rel logit diff", rel, "top1-top2 margins", (srt[:, -1] - srt[:, -2]).round(4).tolist())
    assert rel <= 1e-3, tag
    assert np.array_equal(got.argmax(1), ref.argmax(1)), tag


def test_c3_int4_at_2048_context_resident_and_streamed_from_pinned_memory():
    """C3: 0.5B int4-g32 after a 2048-token prompt (16 prefill chunks; the verify rows attend over
    129 key blocks), one k=8 verify step against the oracle, resident; then the same run with the
    weights streamed from a pinned host copy through 2 device slots (direct DMA from the pinned
    views, reads counted when a slot is taken, the next pass's first layers copied as soon as a
    pass ends): bit-identical logits and acceptance, and every pass reads each layer block and the
    table once (tests/quant.rs:232-248)."""
    say("C3: build")
    m = qwen05b((4, 32))
    V = LS.QWEN2_05B["vocab"]
    rng = np.random.default_rng(2048)
    prompt = rng.integers(0, V, 2048).tolist()
    say("C3: oracle")
    block, ref = oracle_block(cpu_model(m, max_ctx=2100), prompt, 8, rng, V)
    want = want_acceptance(ref, block)
    say("C3: gpu resident")
    gm = gpu_model(m, max_ctx=2100)
    assert gm.forward_argmax(prompt) == block[0]
    p = gm.pos()
    got = gm.forward_multi(block, 9)
    check_rows(got, ref, "C3 resident")
    gm.truncate(p)
    assert gm.verify_greedy(block) == want and want[0] >= 2
    say("C3: gpu streamed from pinned memory")
    src = LS.Source.from_lsq_image(np.frombuffer(m["lsq"], np.uint8).copy()).pinned_copy()
    sm = LS.Model(src, LS.MODE_STREAM, 2, 2100)
    c = src.config()
    _, layer_total = LS.layer_layout(m["config_text"])
    rb = LS.row_bytes(c["embed_format"], c["hidden"])
    per_pass = c["layers"] * layer_total + c["vocab"] * rb
    r0 = src.bytes_read()
    assert sm.forward_argmax(prompt) == block[0]
    chunks = (2048 + 127) // 128
    # every prefill chunk streams the layers; only the last one also streams the table
    assert src.bytes_read() - r0 == chunks * c["layers"] * layer_total + c["vocab"] * rb + 2048 * rb
    r1 = src.bytes_read()
    got_s = sm.forward_multi(block, 9)
    assert np.array_equal(bits(got_s), bits(got)), "streamed != resident"
    assert src.bytes_read() - r1 == per_pass + 9 * rb
    sm.truncate(p)
    assert sm.verify_greedy(block) == want
    assert sm.pos() == gm.pos()


def test_c5_3b_int8_at_1024_context_two_steps():
    """C5: 3B int8-g64 after a 1024-token prompt, a k=8 verify step against the oracle (the head
    runs with only the live tokens' fragment slots in LDS and its own final reduction), then two
    more verify steps with other block lengths (13 and 1 tokens), each against the oracle's
    acceptance, so the head's finished-workgroup count is reset across graph replays."""
    say("C5: build")
    m = qwen3b((8, 64))
    V = LS.QWEN2_3B["vocab"]
    rng = np.random.default_rng(1024)
    prompt = rng.integers(0, V, 1024).tolist()
    cpu = cpu_model(m, max_ctx=1100)
    say("C5: oracle")
    block, ref = oracle_block(cpu, prompt, 8, rng, V)
    want = want_acceptance(ref, block)
    say("C5: gpu")
    gm = gpu_model(m, max_ctx=1100)
    assert gm.forward_argmax(prompt) == block[0]
    p = gm.pos()
    got = gm.forward_multi(block, 9)
    check_rows(got, ref, "C5")
    gm.truncate(p)
    assert gm.verify_greedy(block) == want and want[0] >= 2
    # the oracle follows the accepted prefix, then two more steps
    cpu.truncate(p)
    cpu.forward(block[: want[0] + 1])
    last = want[1]
    for n in (13, 1):
        nb = [last] + rng.integers(0, V, n - 1).tolist()
        p1 = cpu.pos()
        r = cpu.forward_multi(nb, n)
        w = want_acceptance(r, nb)
        got_w = gm.verify_greedy(nb)
        say("C5 step", n, got_w, w)
        assert got_w == w, n
        cpu.truncate(p1)
        cpu.forward(nb[: w[0] + 1])
        assert gm.pos() == cpu.pos()
        last = w[1]


def test_c4_sixteen_sequences_of_nine_rows():
    """C4: 16 sequences x (k=8 drafts + 1) = 144 rows in one pass (9 token tiles), prompts of
    U[128, 1024] ids. Sequences 0, 7 and 15 are checked against the oracle (acceptance of three
    steps, whose drafts follow the oracle's greedy tokens in part); every sequence against itself
    run alone on the GPU (same acceptance and positions, then bit-identical logits)."""
    say("C4: build")
    q = qwen05b((8, 64))
    V = LS.QWEN2_05B["vocab"]
    src = LS.Source.from_lsq_image(q["lsq"])
    rng = np.random.default_rng(144)
    n_seq = 16
    lens = rng.integers(128, 1025, n_seq).tolist()
    prompts = [rng.integers(0, V, n).tolist() for n in lens]
    max_ctx = 1100
    batch = LS.Model(src, LS.MODE_RESIDENT, 2, max_ctx, 0, n_seq=n_seq)
    alone = LS.Model(src, LS.MODE_RESIDENT, 2, max_ctx, 0)  # one sequence at a time
    steps = 3
    # greedy continuations from the GPU alone (verified against the oracle below for 3 sequences)
    greedy, last = [], []
    for s, p in enumerate(prompts):
        batch.select(s)
        a = batch.forward_argmax(p)
        last.append(a)
        alone.reset()
        assert alone.forward_argmax(p) == a, s
        g = [a]
        for _ in range(steps * 9 + 2):
            g.append(alone.forward_argmax([g[-1]]))
        greedy.append(g)
    checked = [0, 7, 15]
    for s in checked:
        say("C4: oracle for sequence", s, "prompt", lens[s])
        cpu = cpu_model(q, max_ctx=max_ctx)
        assert O.plain_greedy(cpu, prompts[s], 12) == greedy[s][:12], s
    goods = [[(3 * s + st) % 9 for s in range(n_seq)] for st in range(steps)]
    done = [1] * n_seq
    blocks_log = []
    for st in range(steps):
        blocks = []
        for s in range(n_seq):
            g, good = greedy[s], goods[st][s]
            d = list(g[done[s] : done[s] + good]) + [(g[done[s] + good] + 1) % V] * (8 - good)
            blocks.append([last[s]] + d[:8])
        say("C4 step", st, "rows", sum(len(b) for b in blocks))
        got = batch.verify_greedy_batch(blocks)
        blocks_log.append(blocks)
        for s in range(n_seq):
            acc, nxt = got[s]
            assert acc == min(goods[st][s], 8), (st, s, got[s])
            assert nxt == greedy[s][done[s] + acc], (st, s)
            done[s] += acc + 1
            last[s] = nxt
    # each sequence alone on the GPU replays the same blocks: same answers, same logits after
    for s in range(n_seq):
        alone.reset()
        alone.forward_argmax(prompts[s])
        for st in range(steps):
            alone.verify_greedy(blocks_log[st][s])
        batch.select(s)
        assert batch.pos() == alone.pos() == lens[s] + done[s] - 1, s
        lb, la = batch.forward([last[s]]), alone.forward([last[s]])
        assert np.array_equal(bits(lb), bits(la)), s


def tied_model():
    """The tiny int8 model with its embedding table's rows duplicated in pairs (row 2k + 1 = row
    2k): every logit has a bit-identical twin, so the argmax must take the lower, even index
    (src/spec.rs:41-49, src/model.rs:373-376)."""
    base = T.write_tiny_model(13)
    emb = np.frombuffer(base["embed"], np.uint8).reshape(T.VOCAB, -1).copy()
    emb[1::2] = emb[0::2]
    m = dict(base)
    m["embed"] = emb.reshape(-1)
    return m


def test_argmax_takes_the_lowest_index_among_tied_logits():
    m = tied_model()
    cpu = cpu_model(m)
    g = O.plain_greedy(cpu, PROMPT, 30)
    assert all(t % 2 == 0 for t in g)
    gm = gpu_model(m)
    got = LS.greedy_generate(gm, PROMPT, 30)
    assert got == g
    # a verify block over twins: the acceptance compares against even tokens only
    gm.reset()
    assert gm.forward_argmax(PROMPT) == g[0]
    block = [g[0], g[1], g[2] + 1, g[3]]  # an odd twin of g[2] is rejected
    assert gm.verify_greedy(block) == (1, g[2])
    logits = gpu_model(m).forward(PROMPT)
    assert np.array_equal(bits(logits[0::2]), bits(logits[1::2]))


def test_a_failed_in_launch_wait_is_an_error_and_the_next_call_is_clean():
    """The error word that a bounded wait sets when it gives up, set from the host before the
    pass: every wait of the pass stops at once, the call returns LS_E_DEVICE and moves no
    position, and the next call matches the oracle. Both staging paths (pinned words read by the
    kernels, and copies each way), eager and graph replay, and the layer stack of the 0.5B shape."""
    m = tiny("int8")
    g = O.plain_greedy(cpu_model(m, max_ctx=128), PROMPT, 40)
    for direct in ("1", "0"):
        for graphs in (True, False):
            say("failure path, direct", direct, "graphs", graphs)
            with env("LS_DIRECT", direct):
                gm = gpu_model(m)
            gm.use_graphs(graphs)
            assert gm.forward_argmax(PROMPT) == g[0]
            block = [g[0], g[1], g[2], 5]
            p = gm.pos()
            gm.verify_greedy(block)  # a normal step first (graph captured)
            gm.truncate(p)
            gm.debug_fail_next()
            with pytest.raises(LS.LayerstreamError) as e:
                gm.verify_greedy(block)
            assert e.value.code == -4
            assert gm.pos() == p
            assert gm.verify_greedy(block) == (2, g[3])
            gm.debug_fail_next()
            with pytest.raises(LS.LayerstreamError):
                gm.forward([g[3]])
            assert gm.pos() == p + 3
            assert gm.forward_argmax([g[3]]) == g[4]
    say("failure path, 0.5B layer stack")
    q = qwen05b((8, 64))
    gm = gpu_model(q, max_ctx=256)
    rng = np.random.default_rng(5)
    prompt = rng.integers(0, LS.QWEN2_05B["vocab"], 40).tolist()
    a = gm.forward_argmax(prompt)
    p = gm.pos()
    ref = gm.forward_multi([a, 1, 2], 3)
    gm.truncate(p)
    gm.debug_fail_next()
    with pytest.raises(LS.LayerstreamError):
        gm.forward_multi([a, 1, 2], 3)
    assert gm.pos() == p
    assert np.array_equal(bits(gm.forward_multi([a, 1, 2], 3)), bits(ref))


def test_c2_full_generation_matches_the_oracle_token_for_token():
    """The headline workload end to end: 0.5B int8-g64 (clip search), a 512-token prompt of the
    benchmark's seeded ids, then 256 generated tokens by speculative decoding with k=8 scripted
    drafts (60% of them the greedy token). Every emitted token equals the oracle's own greedy
    continuation (src/spec.rs: speculation never changes the output), and so does the GPU's plain
    greedy decoding; the accepted counts per step come from the device's verify steps."""
    say("C2: build")
    m = qwen05b((8, 64))
    prompt = np.random.default_rng(512).integers(0, 151936, 512).tolist()
    n = 256
    say("C2: oracle greedy", n)
    cpu = cpu_model(m, max_ctx=1024)
    want = O.plain_greedy(cpu, prompt, n)
    assert len(want) == n
    say("C2: gpu greedy")
    gm = gpu_model(m, max_ctx=1024)
    got_plain = LS.greedy_generate(gm, prompt, n)
    assert got_plain == want
    say("C2: gpu speculative k=8")
    d = LS.ScriptedDrafter(want, 0.6, 2024, 151936)
    got, st = LS.speculative_greedy(gpu_model(m, max_ctx=1024), d, prompt, n, 8)
    d.close()
    say("C2: stats", st)
    assert got == want
    assert st["target_passes"] < n


def test_c1_and_c3_full_generation_match_the_oracle_token_for_token():
    """The other single-sequence workloads end to end: 0.5B bf16 after a 64-token prompt with k=4
    drafts, and 0.5B int4-g32 after a 2048-token prompt with k=8 drafts, resident and streamed from
    pinned memory through two device slots; 128 generated tokens each, equal to the oracle's greedy
    continuation token for token."""
    for name, fmt, n_prompt, k, modes in (("C1", None, 64, 4, ("resident",)), ("C3", (4, 32), 2048, 8, ("resident", "stream"))):
        say(name, ": build")
        m = qwen05b(fmt)
        prompt = np.random.default_rng(512).integers(0, 151936, n_prompt).tolist()
        n = 128
        say(name, ": oracle greedy", n)
        want = O.plain_greedy(cpu_model(m, max_ctx=n_prompt + n + 16), prompt, n)
        for mode in modes:
            say(name, ": gpu speculative", mode)
            if mode == "resident":
                tm = gpu_model(m, max_ctx=n_prompt + n + 16)
            else:
                src = LS.Source.from_lsq_image(np.frombuffer(m["lsq"], np.uint8).copy()).pinned_copy()
                tm = LS.Model(src, LS.MODE_STREAM, 2, n_prompt + n + 16)
            d = LS.ScriptedDrafter(want, 0.6, 2024, 151936)
            got, st = LS.speculative_greedy(tm, d, prompt, n, k)
            d.close()
            say(name, mode, "target passes", st["target_passes"])
            assert got == want, (name, mode)


def test_c5_generation_matches_the_oracle_token_for_token():
    """The 3B workload end to end on a shorter run: int8-g64 after a 1024-token prompt, 32 tokens by
    speculation with k=8 scripted drafts through the layer stack; every token equals the oracle's
    greedy continuation."""
    say("C5 gen: build")
    m = qwen3b((8, 64))
    prompt = np.random.default_rng(512).integers(0, 151936, 1024).tolist()
    n = 32
    say("C5 gen: oracle greedy", n)
    want = O.plain_greedy(cpu_model(m, max_ctx=1100), prompt, n)
    say("C5 gen: gpu speculative")
    d = LS.ScriptedDrafter(want, 0.6, 2024, 151936)
    got, st = LS.speculative_greedy(gpu_model(m, max_ctx=1100), d, prompt, n, 8)
    d.close()
    say("C5 gen: target passes", st["target_passes"])
    assert got == want
