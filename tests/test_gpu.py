"""Parity of the HIP engine (through the C ABI) with the oracle, on an MI355X.

Tolerances: logits within 1e-4 * (1 + max|ref|) on the tiny models and 1e-3 relative on the
0.5B shape (the north star's bound); token sequences, accepted counts and argmax exactly.
Within the GPU engine, batched and single-token passes, and resident and streamed weights, are
compared bit for bit.
"""
import contextlib
import os
import sys

import numpy as np
import pytest

import layerstream_amd as LS
import oracle_py as O
import tinymodels as T

pytestmark = pytest.mark.gpu

PROMPT = [5, 17, 301, 42, 599, 0]
OTHER_PROMPT = [250, 3, 77]
FOLLOW = [7, 33, 120]


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def oracle_cfg(text):
    c = LS.config_from_json(text)
    return {k: c[k] for k in ("format", "embed_format", "hidden", "inter", "layers", "heads", "kv_heads", "head_dim", "vocab", "eps", "rope_theta")}


def gpu_model(m, mode=LS.MODE_RESIDENT, slots=2, max_ctx=128):
    src = LS.Source.from_memory(m["config_text"], m["layers"], m["embed"], m["norm"])
    return LS.Model(src, mode, slots, max_ctx)


# The oracle's threads: the cores this process may run on, at most 16 (a GPU's share of its host).
ORACLE_THREADS = max(1, min(16, len(os.sched_getaffinity(0))))


def cpu_model(m, max_ctx=128):
    return O.OracleModel(oracle_cfg(m["config_text"]), m["layers"], m["embed"], m["norm"], threads=ORACLE_THREADS, max_ctx=max_ctx)


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def close(got, ref, rel=1e-4):
    got, ref = np.asarray(got), np.asarray(ref)
    return np.max(np.abs(got - ref)) <= rel * (1 + np.max(np.abs(ref)))


# ------------------------------------------------------------------------------ operator
@pytest.mark.parametrize("f", [(16, 0), (8, 32), (8, 64), (4, 16), (4, 32), (4, 64)])
def test_matmul_matches_the_oracle_and_is_batch_invariant(f):
    from hipmem import DeviceArray

    say("matmul", f)
    rng = np.random.default_rng(1)
    pool = O.lib().or_pool_new(4)
    try:
        # the two wide shapes split K over 5 and 16 workgroups (last-arriver fixup)
        for rows, cols in [(37, 128), (64, 256), (150, 192), (96, 4864), (40, 16384)]:
            if f[0] != 16 and cols % f[1]:
                continue
            w = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float32)
            if f[0] == 16:
                wb = T.bf16_trunc_bytes(w.reshape(-1))
            else:
                wb = np.concatenate([LS.quantize_row(f, r)[0] for r in w])
            dw = DeviceArray(wb)
            for t in [1, 2, 5, 9, 16, 17, 33]:
                x = rng.standard_normal((t, cols)).astype(np.float32)
                ref = np.zeros(t * rows, np.float32)
                O.lib().or_matmul(pool, O.fmt(*f), O.u8(wb), rows, cols, O.f32(x), t, O.f32(ref))
                dx, dy = DeviceArray(x), DeviceArray(np.zeros(t * rows, np.float32))
                LS._check(LS.lib().ls_matmul(LS.fmt(*f), dw.p, rows, cols, dx.p, t, dy.p, None))
                y = dy.to_host(ref)
                assert np.all(np.abs(y - ref) <= 1e-4 * (1 + np.abs(ref))), (f, rows, cols, t)
                # each row of the batch equals the single-input product bit for bit
                for tt in (0, t - 1):
                    d1, o1 = DeviceArray(np.ascontiguousarray(x[tt])), DeviceArray(np.zeros(rows, np.float32))
                    LS._check(LS.lib().ls_matmul(LS.fmt(*f), dw.p, rows, cols, d1.p, 1, o1.p, None))
                    y1 = o1.to_host(np.zeros(rows, np.float32))
                    assert np.array_equal(bits(y1), bits(y[tt * rows : (tt + 1) * rows])), (f, t, tt)
    finally:
        O.lib().or_pool_free(pool)


# ------------------------------------------------------------------------------ tiny models
MODELS = {}


def tiny(name):
    if name not in MODELS:
        base = T.write_tiny_model(13)
        if name == "bf16":
            MODELS[name] = base
        elif name == "int8":
            MODELS[name] = T.quantized(base, (8, 32), (8, 32))
        elif name == "int4":
            MODELS[name] = T.quantized(base, (4, 32), (4, 32))
        elif name == "mixed":
            MODELS[name] = T.quantized(base, (4, 16), (8, 64))
        elif name == "unrelated":
            MODELS[name] = T.write_tiny_model(99)
    return MODELS[name]


def run_fixed(m):
    out = [m.forward(PROMPT)]
    for t in FOLLOW:
        out.append(m.forward([t]))
    return np.stack(out)


def run_greedy(m):
    out = [m.forward(PROMPT)]
    for _ in range(3):
        out.append(m.forward([int(np.argmax(out[-1]))]))
    return np.stack(out)


@pytest.mark.parametrize("name", ["bf16", "int8", "int4", "mixed"])
def test_tiny_model_logits_match_the_oracle(name):
    say("tiny logits", name)
    m = tiny(name)
    ref = run_fixed(cpu_model(m))
    for mode in (LS.MODE_RESIDENT, LS.MODE_STREAM):
        got = run_fixed(gpu_model(m, mode))
        assert close(got, ref), (name, mode, np.max(np.abs(got - ref)))
        assert np.array_equal(got.argmax(1), ref.argmax(1))


def test_checking_several_positions_at_once_gives_bit_identical_logits():
    """tests/spec.rs:63-84 on the device, for every format and both modes."""
    block = [8, 9, 400, 33, 120]
    for name in ("bf16", "int8", "int4"):
        for mode in (LS.MODE_RESIDENT, LS.MODE_STREAM):
            say("batch invariance", name, mode)
            m = tiny(name)
            for n in (1, 2, len(block)):
                a = gpu_model(m, mode)
                a.forward(PROMPT)
                together = a.forward_multi(block, n)
                b = gpu_model(m, mode)
                b.forward(PROMPT)
                one = np.stack([b.forward([t]) for t in block])
                assert np.array_equal(bits(together), bits(one[len(block) - n :])), (name, mode, n)
                assert a.pos() == b.pos()


def test_every_mode_gives_bit_identical_logits():
    """tests/pipeline.rs:79-101 and tests/quant.rs:142-158: resident vs 1, 2, 3 slots."""
    for name in ("bf16", "mixed"):
        m = tiny(name)
        ref = run_greedy(gpu_model(m, LS.MODE_RESIDENT))
        for slots in (1, 2, 3):
            say("modes", name, slots)
            got = run_greedy(gpu_model(m, LS.MODE_STREAM, slots))
            assert np.array_equal(bits(ref), bits(got)), (name, slots)


def test_streaming_reads_every_layer_and_the_table_once_per_pass():
    """tests/quant.rs:232-248: 4 passes x (layers + table) + one row per input token."""
    m = tiny("int4")
    src = LS.Source.from_lsq_image(np.frombuffer(m["lsq"], np.uint8).copy())
    g = LS.Model(src, LS.MODE_STREAM, 2, 64)
    run_greedy(g)
    c = src.config()
    _, total = LS.layer_layout(m["config_text"])
    rb = LS.row_bytes(c["embed_format"], c["hidden"])
    per_pass = c["layers"] * total + c["vocab"] * rb
    assert src.bytes_read() == 4 * per_pass + 9 * rb
    rep = g.report()
    assert rep["resident_weight_bytes"] > 0


def test_truncate_incremental_and_bad_requests():
    m = tiny("bf16")
    a = gpu_model(m)
    a.forward(PROMPT)
    a.forward([7, 8, 9])
    a.truncate(len(PROMPT))
    after = a.forward([20])
    b = gpu_model(m)
    b.forward(PROMPT)
    assert np.array_equal(bits(after), bits(b.forward([20])))
    with pytest.raises(LS.LayerstreamError):
        a.truncate(a.pos() + 1)
    # incremental == whole prompt (tests/pipeline.rs:200-217)
    toks = [(i * 31 + 7) % T.VOCAB for i in range(20)]
    whole = gpu_model(m, max_ctx=64).forward(toks)
    inc = gpu_model(m, max_ctx=64)
    inc.forward(toks[:9])
    for t in toks[9:19]:
        inc.forward([t])
    got = inc.forward(toks[19:])
    assert np.max(np.abs(whole - got)) < 1e-4 and inc.pos() == 20
    # bad requests are errors (tests/pipeline.rs:219-232)
    o = gpu_model(m, max_ctx=64)
    for bad in ([], [T.VOCAB], [1] * 65):
        with pytest.raises(LS.LayerstreamError):
            o.forward(bad)
    o.forward([1] * 60)
    with pytest.raises(LS.LayerstreamError):
        o.forward([1] * 5)
    o.reset()
    o.forward([1] * 64)
    t = gpu_model(m)
    for toks, n in ([1, 2], 3), ([1, 2], 0):
        with pytest.raises(LS.LayerstreamError):
            t.forward_multi(toks, n)


def test_prompts_longer_than_one_prefill_chunk():
    """Prompts span several 128-token chunks (src/model.rs:111-119); each chunk must see its own
    tokens and the cache of the chunks before it."""
    rng = np.random.default_rng(7)
    for name in ("bf16", "int4"):
        m = tiny(name)
        prompt = rng.integers(0, T.VOCAB, 300).tolist()
        ref = cpu_model(m, max_ctx=512).forward(prompt)
        for mode in (LS.MODE_RESIDENT, LS.MODE_STREAM):
            say("long prompt", name, mode)
            g = gpu_model(m, mode, max_ctx=512)
            got = g.forward(prompt)
            assert close(got, ref), (name, mode, np.max(np.abs(got - ref)))
            inc = gpu_model(m, mode, max_ctx=512)
            inc.forward(prompt[:150])
            got2 = inc.forward(prompt[150:])
            assert np.max(np.abs(got2 - got)) < 1e-4
            assert g.pos() == inc.pos() == 300


def test_speculation_never_changes_the_output_and_matches_the_oracle():
    """tests/spec.rs:103-132 with draft models on the device, plus token parity with the oracle."""
    base = tiny("bf16")
    for dname in ("int8", "int4", "unrelated"):
        for prompt in (PROMPT, OTHER_PROMPT):
            for max_new in (1, 2, 9, 30):
                want = O.plain_greedy(cpu_model(base), prompt, max_new)
                assert LS.greedy_generate(gpu_model(base), prompt, max_new) == want
                for k in (1, 2, 3, 5, 8):
                    for mode in (LS.MODE_RESIDENT, LS.MODE_STREAM):
                        got, st = LS.speculative_greedy(gpu_model(base, mode), gpu_model(tiny(dname)), prompt, max_new, k)
                        assert got == want, (dname, len(prompt), max_new, k, mode)
                        assert st["accepted"] <= st["drafted"]
                        assert st["target_passes"] <= max(len(got) - 1, 0)
        say("spec", dname, "ok")


def test_eos_and_perfect_draft():
    m = tiny("bf16")
    full = O.plain_greedy(cpu_model(m), PROMPT, 24)
    for cut in (0, 1, 5, 11):
        eos = [full[cut]]
        want = O.plain_greedy(cpu_model(m), PROMPT, 24, eos)
        for k in (1, 4, 8):
            got, _ = LS.speculative_greedy(gpu_model(m), gpu_model(m), PROMPT, 24, k, eos)
            assert got == want, (cut, k)
    max_new, k = 21, 3
    want = O.plain_greedy(cpu_model(m), PROMPT, max_new)
    got, st = LS.speculative_greedy(gpu_model(m), gpu_model(m), PROMPT, max_new, k)
    assert got == want and st["accepted"] == st["drafted"]
    assert st["target_passes"] == -(-(max_new - 1) // (k + 1))
    # bad requests (tests/spec.rs:175-193)
    for kk, prompt, mn in [(0, PROMPT, 5), (33, PROMPT, 5), (2, [], 5), (2, PROMPT, 0), (2, PROMPT, 500)]:
        with pytest.raises(LS.LayerstreamError):
            LS.speculative_greedy(gpu_model(m), gpu_model(m), prompt, mn, kk)
    t = gpu_model(m)
    t.forward(PROMPT)
    with pytest.raises(LS.LayerstreamError):
        LS.speculative_greedy(t, gpu_model(m), PROMPT, 5, 2)


def test_verify_step_accepts_the_longest_matching_prefix():
    m = tiny("bf16")
    g = O.plain_greedy(cpu_model(m), PROMPT, 12)
    for m_want in range(0, 6):
        tgt = gpu_model(m)
        a = tgt.forward_argmax(PROMPT)
        assert a == g[0]
        drafts = list(g[1 : 1 + m_want]) + [(g[1 + m_want] + 1) % T.VOCAB] + [3] * (5 - m_want)
        drafts = drafts[:5]
        acc, nxt = tgt.verify_greedy([a] + drafts)
        want_m = min(m_want, 5)
        assert acc == want_m and nxt == g[1 + want_m], (m_want, acc, nxt)
        assert tgt.pos() == len(PROMPT) + acc + 1


def test_graph_replays_match_eager_steps_bit_for_bit():
    """Verify steps replayed from captured HIP graphs (several block lengths, each replayed more
    than once, with eager forward passes and synchronisations in between) against a model that
    runs every step launch by launch."""
    m = tiny("int8")
    g = O.plain_greedy(cpu_model(m), PROMPT, 40)
    eager, graph = gpu_model(m), gpu_model(m)
    eager.use_graphs(False)
    a_e, a_g = eager.forward_argmax(PROMPT), graph.forward_argmax(PROMPT)
    assert a_e == a_g == g[0]
    last, done = a_e, 1
    for step, (k, good) in enumerate([(3, 1), (8, 2), (3, 0), (8, 5), (1, 0), (8, 8), (3, 3), (8, 1)]):
        say("graph step", step, k, good)
        drafts = list(g[done : done + good]) + [(g[done + good] + 7) % T.VOCAB] * (k - good)
        drafts = drafts[:k]
        r_e = eager.verify_greedy([last] + drafts)
        r_g = graph.verify_greedy([last] + drafts)
        assert r_e == r_g, (step, r_e, r_g)
        assert eager.pos() == graph.pos()
        acc, nxt = r_e
        assert nxt == g[done + acc], (step, acc, nxt)
        done += acc + 1
        last = nxt
        if step % 3 == 1:
            # eager work on the graph model between replays: one token forward, then roll back
            p = graph.pos()
            le, lg = eager.forward([last]), graph.forward([last])
            assert np.array_equal(bits(le), bits(lg)), step
            eager.truncate(p)
            graph.truncate(p)


# ------------------------------------------------------------------------------ 0.5B shape
def qwen05b(fmt=None, seed=1):
    text = LS.qwen2_config_text(**LS.QWEN2_05B)
    m = LS.synth_bf16_model(text, seed)
    if fmt is None:
        return m
    img = LS.quantize_model(text, m["layers"], m["embed"], m["norm"], fmt)
    parts = T.split_lsq(img.tobytes(), oracle_cfg(LS.inject_quant(text, *fmt)))
    return {"config_text": LS.inject_quant(text, *fmt), "lsq": img, **{k: parts[k] for k in ("layers", "embed", "norm")}}


def test_qwen05b_bf16_verify_step_matches_the_oracle():
    """The CPU-runnable configuration: 0.5B shape, bf16 weights, f32 compute, prompt of 64 random
    ids, one verify step of k=4 drafts whose first two are the greedy continuation."""
    say("0.5B bf16: synth")
    m = qwen05b()
    rng = np.random.default_rng(64)
    prompt = rng.integers(0, 151936, 64).tolist()
    cpu = cpu_model(m, max_ctx=256)
    g = O.plain_greedy(cpu, prompt, 3)  # a, g1, g2
    cpu.reset()
    drafts = [g[1], g[2]] + rng.integers(0, 151936, 2).tolist()
    block = [g[0]] + drafts
    say("0.5B bf16: oracle")
    cpu.forward(prompt)
    ref = cpu.forward_multi(block, 5)
    say("0.5B bf16: gpu")
    gm = gpu_model(m, max_ctx=256)
    a = gm.forward_argmax(prompt)
    assert a == g[0]
    got = gm.forward_multi(block, 5)
    rel = np.max(np.abs(got - ref)) / np.max(np.abs(ref))
    say("max rel logit diff", rel)
    assert rel <= 1e-3
    assert np.array_equal(got.argmax(1), ref.argmax(1))
    top2 = np.sort(ref, axis=1)[:, -2:]
    say("top1-top2 margins", (top2[:, 1] - top2[:, 0]).tolist())
    # the fused verify step gives the same acceptance
    gm2 = gpu_model(m, max_ctx=256)
    gm2.forward(prompt)
    acc, nxt = gm2.verify_greedy(block)
    want_m = 0
    while want_m < 4 and ref[want_m].argmax() == drafts[want_m]:
        want_m += 1
    assert acc == want_m >= 2 and nxt == ref[want_m].argmax()


def test_qwen05b_int8_greedy_after_a_512_token_prompt_matches_the_oracle():
    """The benchmark configuration's shape: 0.5B int8-g64 (clip search), a 512-token prompt
    (four prefill chunks), then greedy decoding and speculative decoding with scripted drafts."""
    say("0.5B int8: build")
    m = qwen05b((8, 64))
    rng = np.random.default_rng(512)
    prompt = rng.integers(0, 151936, 512).tolist()
    n = 12
    gm = gpu_model(m, max_ctx=1024)
    gl = [gm.forward(prompt)]
    for _ in range(n - 1):
        gl.append(gm.forward([int(np.argmax(gl[-1]))]))
    g = [int(np.argmax(x)) for x in gl]
    say("0.5B int8: oracle")
    cpu = cpu_model(m, max_ctx=1024)
    cl = [cpu.forward(prompt)]
    for i in range(n - 1):
        cl.append(cpu.forward([g[i]]))
    for i in range(n):
        srt = np.sort(cl[i])
        rel = np.max(np.abs(gl[i] - cl[i])) / np.max(np.abs(cl[i]))
        say(f"pos {i}: rel {rel:.2e}, margin {srt[-1] - srt[-2]:.3e}")
        assert rel <= 1e-3
        assert int(np.argmax(cl[i])) == g[i], i
    # speculation with scripted drafts reproduces greedy decoding exactly
    d = LS.ScriptedDrafter(g, 0.6, 7, 151936)
    got, st = LS.speculative_greedy(gpu_model(m, max_ctx=1024), d, prompt, n, 8)
    assert got == g and st["target_passes"] < n


def qwen3b(fmt, seed=1):
    text = LS.qwen2_config_text(**LS.QWEN2_3B)
    m = LS.synth_bf16_model(text, seed)
    if fmt is None:
        return m
    img = LS.quantize_model(text, m["layers"], m["embed"], m["norm"], fmt)
    del m
    parts = T.split_lsq(img.tobytes(), oracle_cfg(LS.inject_quant(text, *fmt)))
    return {"config_text": LS.inject_quant(text, *fmt), "lsq": img, **{k: parts[k] for k in ("layers", "embed", "norm")}}


def verify_step_vs_oracle(m, prompt, k, rng, max_ctx, tag):
    """One verify block [a, g1, g2, random...] after the prompt: logits of every row within 1e-3
    relative of the oracle's, the same per-row argmax, and the fused step's acceptance."""
    cpu = cpu_model(m, max_ctx=max_ctx)
    g = O.plain_greedy(cpu, prompt, 3)
    cpu.reset()
    vocab = LS.config_from_json(m["config_text"])["vocab"]
    drafts = [g[1], g[2]] + rng.integers(0, vocab, k - 2).tolist()
    block = [g[0]] + drafts
    say(tag, "oracle")
    cpu.forward(prompt)
    ref = cpu.forward_multi(block, k + 1)
    say(tag, "gpu")
    gm = gpu_model(m, max_ctx=max_ctx)
    assert gm.forward_argmax(prompt) == g[0]
    p = gm.pos()
    got = gm.forward_multi(block, k + 1)
    rel = np.max(np.abs(got - ref)) / np.max(np.abs(ref))
    say(tag, "max rel logit diff", rel)
    assert rel <= 1e-3
    assert np.array_equal(got.argmax(1), ref.argmax(1))
    gm.truncate(p)
    acc, nxt = gm.verify_greedy(block)
    want_m = 0
    while want_m < k and ref[want_m].argmax() == drafts[want_m]:
        want_m += 1
    assert acc == want_m >= 2 and nxt == ref[want_m].argmax()


@contextlib.contextmanager
def env(name, value):
    """An engine switch read when a model is created."""
    old = os.environ.get(name)
    os.environ[name] = value
    try:
        yield
    finally:
        if old is None:
            del os.environ[name]
        else:
            os.environ[name] = old


def test_layer_stack_and_per_layer_launches_give_identical_bits():
    """One-tile passes run every layer in one launch (k_layers) by default; LS_STACK=0 runs the
    per-layer launches. Same plans, so the same logits bit for bit, and the same acceptance. The
    0.5B shape in every weight format (the tiny model is too narrow for the stack and runs the
    per-layer launches either way)."""
    block = [8, 9, 400, 33, 120, 5, 77, 301, 2]
    rng = np.random.default_rng(3)
    cases = [("0.5B " + name, qwen05b(fmt), rng.integers(0, 151936, 40).tolist(), 256)
             for name, fmt in (("bf16", None), ("int8", (8, 64)), ("int4", (4, 32)))]
    for name, m, prompt, max_ctx in cases:
        say("stack vs per-layer", name)
        with env("LS_STACK", "0"):
            a = gpu_model(m, max_ctx=max_ctx)
        b = gpu_model(m, max_ctx=max_ctx)
        la, lb = a.forward(prompt), b.forward(prompt)
        assert np.array_equal(bits(la), bits(lb)), name
        p = a.pos()
        va, vb = a.forward_multi(block, len(block)), b.forward_multi(block, len(block))
        assert np.array_equal(bits(va), bits(vb)), name
        a.truncate(p)
        b.truncate(p)
        assert a.verify_greedy(block) == b.verify_greedy(block), name
        assert a.pos() == b.pos()


def test_verify_steps_without_copies_match_the_copying_path_and_the_oracle():
    """Resident verify steps read their staged position and tokens from pinned host memory, and the
    head's last workgroup reduces the argmax partials, applies greedy acceptance and writes
    (error, m, next) back there (the default); LS_DIRECT=0 copies each way and runs k_head_final.
    Same acceptance and positions either way, for blocks of one token tile and of several (the
    last workgroup then reduces every tile's partials), two steps in a row (graph replays), each
    checked against the oracle's greedy tokens (src/spec.rs:119-127)."""
    m = tiny("int8")
    g = O.plain_greedy(cpu_model(m, max_ctx=256), PROMPT, 100)
    for n_block, m_want in [(9, 4), (9, 8), (1, 0), (17, 16), (40, 25), (40, 39)]:
        say("verify without copies", n_block, m_want)
        with env("LS_DIRECT", "0"):
            a = gpu_model(m, max_ctx=256)
        b = gpu_model(m, max_ctx=256)
        for t in (a, b):
            assert t.forward_argmax(PROMPT) == g[0]
        at = 0  # g[at] is the token each step's block starts with
        for step in range(2):
            drafts = list(g[at + 1 : at + 1 + m_want]) + [(g[at + 1 + m_want] + 1) % T.VOCAB] * (n_block - 1 - m_want)
            block = [g[at]] + drafts[: n_block - 1]
            want_m = min(m_want, n_block - 1)
            got_a, got_b = a.verify_greedy(block), b.verify_greedy(block)
            assert got_a == got_b == (want_m, g[at + want_m + 1]), (n_block, m_want, step, got_a, got_b)
            assert a.pos() == b.pos() == len(PROMPT) + at + want_m + 1
            at += want_m + 1


def test_qwen3b_int8_verify_step_matches_the_oracle():
    """The 3B shape (hidden 2048, head_dim 128, FFN 11008; the fragments of all 16 token columns
    exceed one workgroup's LDS, so the head keeps only the live tokens' slots there and does its
    own final reduction), int8-g64, prompt of 64 ids, one verify step of k=8. The same path over
    a 1024-token prompt and three steps of different lengths: test_gpu_workloads.py."""
    say("3B int8: build")
    m = qwen3b((8, 64))
    rng = np.random.default_rng(3)
    prompt = rng.integers(0, 151936, 64).tolist()
    verify_step_vs_oracle(m, prompt, 8, rng, 256, "3B int8:")


def _same_bits_two_ways(m, env_a, env_b, what):
    """Two models of m, each created under its own engine switches, give the same logits bit for
    bit and the same acceptance over a 40-token prompt (three tiles) and blocks of 9, 1 and 9
    tokens in a row."""
    rng = np.random.default_rng(5)
    prompt = rng.integers(0, 151936, 40).tolist()
    made = []
    for sw in (env_a, env_b):
        with contextlib.ExitStack() as st:
            for k, v in sw.items():
                st.enter_context(env(k, v))
            made.append(gpu_model(m, max_ctx=256))
    a, b = made
    assert np.array_equal(bits(a.forward(prompt)), bits(b.forward(prompt)))
    for block in ([8, 9, 400, 33, 120, 5, 77, 301, 2], [17], [3, 4, 5, 6, 7, 8, 9, 10, 11]):
        say(what, "block of", len(block))
        p = a.pos()
        va, vb = a.forward_multi(block, len(block)), b.forward_multi(block, len(block))
        assert np.array_equal(bits(va), bits(vb)), len(block)
        a.truncate(p)
        b.truncate(p)
        assert a.verify_greedy(block) == b.verify_greedy(block), len(block)
        assert a.pos() == b.pos()


def test_qwen3b_pipelined_matrices_give_the_bits_of_k_mm():
    """With 128-column K shares (LS_WIDE=0: 16 wavefronts along a 2048 row) the 3B gate|up over
    one token tile (688 gate and up strip pairs, more than the device has CUs) runs as the
    pipelined launch; LS_PIPE=0 runs it as k_mm. Same plan, so the same bits."""
    say("3B pipelined vs k_mm: build")
    _same_bits_two_ways(qwen3b((8, 64)), {"LS_WIDE": "0", "LS_PIPE": "0"}, {"LS_WIDE": "0"}, "3B pipelined vs k_mm:")


def test_qwen3b_layer_stack_and_per_layer_launches_give_identical_bits():
    """The 3B shape's default plans use 256-column K shares (8 wavefronts cover a 2048 row), so its
    one-tile passes run as the layer stack (k_layers, head_dim 128, 256-column shares); LS_STACK=0
    runs the per-layer k_mm launches with the same plans. Same bits, int8-g64, int4-g32 and bf16."""
    for fmt in ((8, 64), (4, 32), None):
        say("3B stack vs per-layer: build", fmt)
        _same_bits_two_ways(qwen3b(fmt), {"LS_STACK": "0"}, {}, f"3B stack vs per-layer {fmt}:")


def test_qwen05b_int4_verify_step_after_a_long_prompt_matches_the_oracle():
    """The int4-g32 configuration's shape with a 1100-token prompt (nine prefill chunks; the
    verify rows attend over 69 blocks of 16 keys), one verify step of k=8."""
    say("0.5B int4: build")
    m = qwen05b((4, 32))
    rng = np.random.default_rng(2048)
    prompt = rng.integers(0, 151936, 1100).tolist()
    verify_step_vs_oracle(m, prompt, 8, rng, 1200, "0.5B int4:")
