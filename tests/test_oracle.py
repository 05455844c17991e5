"""Pins of the oracle (the C restatement of the reference CPU path) on the CPU.

Every check comes from the reference's own tests (known answers, invariants, f64 references)
or from an independent implementation (Hugging Face Qwen2, tests/golden/hf_tiny_logits.npz).
"""
import math
import os

import numpy as np
import pytest

import oracle_py as O
import tinymodels as T

L = O.lib


def lcg_vals(seed, n):
    """The LCG of src/kernels.rs:280-283 / src/quant.rs:258-261."""
    r = T.Lcg(seed)
    return r.take(n), r


def to_bf16(vals):
    return T.bf16_trunc_bytes(np.asarray(vals, np.float32))


# ---------------------------------------------------------------- formats (src/weights.rs:431-446)
def test_row_bytes_known_answers():
    assert O.row_bytes((16, 0), 896) == 1792
    assert O.row_bytes((8, 64), 896) == 896 + 14 * 2 == 924
    assert O.row_bytes((4, 32), 896) == 448 + 28 * 2 == 504
    assert O.row_bytes((8, 64), 4864) == 5016
    assert O.row_bytes((4, 32), 4864) == 2736


def test_format_validation():
    import ctypes as C

    cols = (C.c_size_t * 2)(896, 4864)
    assert L().or_validate(O.fmt(8, 64), cols, 2) == 0
    assert L().or_validate(O.fmt(4, 32), cols, 2) == 0
    for bad in [(6, 32), (8, 24), (8, 512), (8, 256)]:
        assert L().or_validate(O.fmt(*bad), cols, 2) != 0, bad


def test_layer_block_sizes():
    """Layer block sizes of the 0.5B shape, recomputed from the layout (src/weights.rs row sizes)."""
    import ctypes as C

    base = dict(hidden=896, inter=4864, layers=24, heads=14, kv_heads=2, head_dim=64, vocab=151936, eps=1e-6, rope_theta=1e6)
    r = (C.c_size_t * 24)()
    for f, want in [((8, 64), 15_381_248), ((4, 32), 8_392_448)]:
        c = O.cfg_struct(dict(base, format=f, embed_format=f))
        assert L().or_layer_layout(C.byref(c), r) == want
    c3 = O.cfg_struct(dict(base, hidden=2048, inter=11008, heads=16, head_dim=128, format=(8, 64), embed_format=(8, 64)))
    assert L().or_layer_layout(C.byref(c3), r) == 79_492_096


# ---------------------------------------------------------------- quant.rs:272-282
def test_bf16_round_is_round_to_nearest_even():
    r = L().or_bf16_round
    assert r(1.0) == 1.0
    assert r(1.0 + 2.0**-8) == 1.0
    assert r(1.0 + 3.0 * 2.0**-8) == 1.0 + 2.0**-6
    assert r(1.0 + 2.0**-9) == 1.0
    assert math.isnan(r(float("nan")))
    assert r(float("inf")) == float("inf")
    v = np.float32(0.12345679)
    assert r(r(v)) == r(v)


# ---------------------------------------------------------------- argmax (src/model.rs:373-376)
def test_argmax_first_maximum_and_nan_rule():
    f = lambda v: L().or_argmax(O.f32(np.asarray(v, np.float32)), len(v))  # noqa: E731
    assert f([0.1, 3.0, 3.0, -1.0]) == 1
    nan = float("nan")
    assert f([nan, 5.0, 6.0]) == 0  # `x > NaN` is never true
    assert f([1.0, nan, 0.5, 2.0, 2.0]) == 3
    assert f([-np.inf, -np.inf]) == 0


# ---------------------------------------------------------------- kernels.rs:286-316
def test_dot_bf16_matches_double_precision():
    seed = 7
    r = T.Lcg(seed)
    for n in [1, 7, 8, 9, 16, 17, 64, 896, 4864]:
        w = r.take(n)
        x = r.take(n)
        wb = to_bf16(w)
        wf = T.bf16_bytes_to_f32(wb).astype(np.float64)
        want = float(np.sum(wf * x.astype(np.float64)))
        got = L().or_dot_bf16(O.u8(wb), O.f32(x), n)
        assert abs(got - want) < 1e-4 * (1 + abs(want)), n


def test_matmul_single_and_batched_agree_and_match_naive():
    pool = L().or_pool_new(4)
    try:
        rows, cols = 50, 40
        r = T.Lcg(99)
        w = r.take(rows * cols)
        wb = to_bf16(w)
        wf = T.bf16_bytes_to_f32(wb).reshape(rows, cols).astype(np.float64)
        for t in [1, 2, 5]:
            x = r.take(t * cols)
            y = np.zeros(t * rows, np.float32)
            L().or_matmul(pool, O.fmt(16, 0), O.u8(wb), rows, cols, O.f32(x), t, O.f32(y))
            want = (x.reshape(t, cols).astype(np.float64) @ wf.T).reshape(-1)
            assert np.all(np.abs(y - want) < 1e-4), t
            # each batched row equals the single-input product bit for bit
            for tt in range(t):
                y1 = np.zeros(rows, np.float32)
                xs = np.ascontiguousarray(x[tt * cols : (tt + 1) * cols])
                L().or_matmul(pool, O.fmt(16, 0), O.u8(wb), rows, cols, O.f32(xs), 1, O.f32(y1))
                assert np.array_equal(y1.view(np.uint32), y[tt * rows : (tt + 1) * rows].view(np.uint32))
    finally:
        L().or_pool_free(pool)


# ---------------------------------------------------------------- kernels.rs:318-347
def test_rms_norm_has_unit_rms_for_unit_weights():
    x = np.array([3.0, -4.0, 12.0, 0.5], np.float32)
    ones = to_bf16([1.0] * 4)
    out = np.zeros(4, np.float32)
    L().or_rms_norm_bf16(O.f32(x), 4, O.u8(ones), 4, 0.0, O.f32(out))
    assert abs(math.sqrt(float(np.mean(out.astype(np.float64) ** 2))) - 1.0) < 1e-5
    # closed form: x / sqrt(mean(x^2) + eps) * w
    w = to_bf16([0.5, 2.0, 1.0, -1.0])
    L().or_rms_norm_bf16(O.f32(x), 4, O.u8(w), 4, 1e-6, O.f32(out))
    want = x / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6) * T.bf16_bytes_to_f32(w)
    assert np.allclose(out, want, rtol=1e-6)


def test_rope_identity_at_zero_and_norm_preserving():
    inv = np.array([10000.0 ** (-i / 4) for i in range(4)], np.float32)
    v = np.arange(1, 9, dtype=np.float32)
    orig = v.copy()
    L().or_rope_inplace(O.f32(v), O.f32(inv), 8, 0)
    assert np.array_equal(v, orig)
    L().or_rope_inplace(O.f32(v), O.f32(inv), 8, 37)
    assert abs(float(np.sum(orig**2)) - float(np.sum(v**2))) < 1e-3
    # rotate-half convention: element i pairs with i + d/2 (closed form in f64)
    ang = 37 * inv.astype(np.float64)
    a, b = orig[:4].astype(np.float64), orig[4:].astype(np.float64)
    want = np.concatenate([a * np.cos(ang) - b * np.sin(ang), b * np.cos(ang) + a * np.sin(ang)])
    assert np.allclose(v, want, atol=1e-5)


def test_softmax_sums_to_one_and_is_stable():
    v = np.array([1000.0, 1001.0, 999.0], np.float32)
    L().or_softmax_inplace(O.f32(v), 3)
    assert abs(float(v.sum()) - 1.0) < 1e-6
    assert v[1] > v[0] > v[2]
    assert abs(L().or_silu(0.0)) == 0.0 and abs(L().or_silu(10.0) - 10.0 / (1 + math.exp(-10))) < 1e-6


# ---------------------------------------------------------------- quant.rs:284-373
def qrow(n, r):
    """quant.rs:263-266: a few large outliers among small weights."""
    return np.array([r.next() * np.float32(0.5 if i % 37 == 0 else 0.05) for i in range(n)], np.float32)


def quantize_row(f, w, clip):
    out = np.zeros(O.row_bytes(f, len(w)), np.uint8)
    import ctypes as C

    e, nn = C.c_double(), C.c_double()
    L().or_quantize_row(O.fmt(*f), O.f32(w), len(w), int(clip), O.u8(out), C.byref(e), C.byref(nn))
    return out, e.value


def dequant(f, raw, cols):
    out = np.zeros(cols, np.float32)
    L().or_dequant_row(O.fmt(*f), O.u8(raw), O.f32(out), cols)
    return out


def test_quant_round_trip_error_is_bounded_by_half_a_step():
    r = T.Lcg(5)
    for bits, group in [(8, 16), (8, 32), (8, 64), (4, 16), (4, 32), (4, 64)]:
        w = qrow(256, r)
        packed, _ = quantize_row((bits, group), w, False)
        back = dequant((bits, group), packed, 256)
        for g in range(256 // group):
            wg, bg = w[g * group : (g + 1) * group], back[g * group : (g + 1) * group]
            amax = float(np.max(np.abs(wg)))
            step = amax / (127.0 if bits == 8 else 7.0)
            assert np.all(np.abs(wg - bg) <= step * 0.52)
            i = int(np.argmax(np.abs(wg)))
            assert abs(wg[i] - bg[i]) <= amax * 0.01


def test_clip_search_never_does_worse_and_helps_four_bit():
    r = T.Lcg(11)
    plain = clipped = 0.0
    for _ in range(40):
        w = qrow(128, r)
        _, ea = quantize_row((4, 32), w, False)
        _, eb = quantize_row((4, 32), w, True)
        assert eb <= ea * (1 + 1e-9)
        plain += ea
        clipped += eb
    assert clipped < plain * 0.97


def test_zero_and_tiny_rows_do_not_produce_nan():
    for f in [(8, 32), (4, 32)]:
        for w in [np.zeros(64, np.float32), np.full(64, 1e-45, np.float32), np.full(64, -3.0, np.float32)]:
            packed, _ = quantize_row(f, w, True)
            assert np.all(np.isfinite(dequant(f, packed, 64)))
    packed, _ = quantize_row((8, 32), np.zeros(32, np.float32), True)
    assert np.all(dequant((8, 32), packed, 32) == 0.0)


def test_int4_nibble_order_and_offset():
    """src/quant.rs:7-9: byte j holds weight j (low nibble) and j + group/2 (high), each +8."""
    w = np.array([(j % 15) - 7 for j in range(32)], np.float32)  # on the grid with scale 1
    packed, _ = quantize_row((4, 32), w, False)
    for j in range(16):
        assert packed[j] & 15 == int(w[j]) + 8 and packed[j] >> 4 == int(w[j + 16]) + 8
    assert np.array_equal(dequant((4, 32), packed, 32), w)


def test_quantized_matmul_equals_matmul_over_dequantized_weights():
    pool = L().or_pool_new(4)
    try:
        r = T.Lcg(21)
        for bits, group in [(8, 32), (8, 64), (4, 32), (4, 64)]:
            f = (bits, group)
            rows, cols = 37, 128
            rb = O.row_bytes(f, cols)
            packed = np.zeros(rows * rb, np.uint8)
            deq = np.zeros((rows, cols), np.float32)
            for i in range(rows):
                w = qrow(cols, r)
                p, _ = quantize_row(f, w, True)
                packed[i * rb : (i + 1) * rb] = p
                deq[i] = dequant(f, p, cols)
            for t in [1, 3]:
                x = r.take(t * cols)
                y = np.zeros(t * rows, np.float32)
                L().or_matmul(pool, O.fmt(*f), O.u8(packed), rows, cols, O.f32(x), t, O.f32(y))
                want = (x.reshape(t, cols).astype(np.float64) @ deq.astype(np.float64).T).reshape(-1)
                assert np.all(np.abs(y - want) < 1e-4 * (1 + np.abs(want))), (f, t)
    finally:
        L().or_pool_free(pool)


# ---------------------------------------------------------------- independent implementation
def test_logits_match_an_independent_qwen2_implementation():
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "hf_tiny_logits.npz"))
    toks = g["tokens"]
    for s in g["seeds"]:
        m = T.write_tiny_model(int(s))
        om = O.OracleModel(m["cfg"], m["layers"], m["embed"], m["norm"], threads=3, max_ctx=64)
        got = om.forward_multi(toks, len(toks))
        ref = g[f"logits_seed{s}"]
        assert np.max(np.abs(got - ref)) < 1e-4 * (1 + np.max(np.abs(ref)))
        assert np.array_equal(got.argmax(1), ref.argmax(1))
        # incremental decoding reaches the same logits
        om.reset()
        om.forward(toks[:5])
        last = None
        for t in toks[5:]:
            last = om.forward([t])
        assert np.max(np.abs(last - ref[-1])) < 1e-4 * (1 + np.max(np.abs(ref)))


# ---------------------------------------------------------------- tests/spec.rs, tests/pipeline.rs
PROMPT = [5, 17, 301, 42, 599, 0]
OTHER_PROMPT = [250, 3, 77]


def mk(model, max_ctx=128, threads=3):
    return O.OracleModel(model["cfg"], model["layers"], model["embed"], model["norm"], threads=threads, max_ctx=max_ctx)


def bit_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def test_checking_several_positions_at_once_gives_bit_identical_logits():
    m = T.write_tiny_model(11)
    block = [8, 9, 400, 33, 120]
    for n in [1, 2, len(block)]:
        a = mk(m)
        a.forward(PROMPT)
        together = a.forward_multi(block, n)
        b = mk(m)
        b.forward(PROMPT)
        one = [b.forward([t]) for t in block]
        assert bit_equal(together, np.stack(one[len(block) - n :]))
        assert a.pos() == b.pos()


def test_truncating_the_cache_forgets_the_tail_exactly():
    m = T.write_tiny_model(12)
    a = mk(m)
    a.forward(PROMPT)
    a.forward([7, 8, 9])
    a.truncate(len(PROMPT))
    after = a.forward([20])
    b = mk(m)
    b.forward(PROMPT)
    assert bit_equal(after, b.forward([20]))
    with pytest.raises(O.OracleError):
        a.truncate(a.pos() + 1)


def test_incremental_decoding_matches_processing_the_whole_prompt():
    m = T.write_tiny_model(6)
    toks = [(i * 31 + 7) % T.VOCAB for i in range(20)]
    whole = mk(m, 64).forward(toks)
    inc = mk(m, 64)
    inc.forward(toks[:9])
    for t in toks[9:19]:
        inc.forward([t])
    got = inc.forward(toks[19:])
    assert np.max(np.abs(whole - got)) < 1e-4
    assert inc.pos() == 20


def test_bad_requests_are_errors_not_panics():
    m = T.write_tiny_model(7)
    o = mk(m, 64)
    for bad in ([], [T.VOCAB], [1] * 65):
        with pytest.raises(O.OracleError):
            o.forward(bad)
    o.forward([1] * 60)
    with pytest.raises(O.OracleError):
        o.forward([1] * 5)
    o.reset()
    o.forward([1] * 64)
    t = mk(m)
    for toks, n in [([1, 2], 3), ([1, 2], 0)]:
        with pytest.raises(O.OracleError):
            t.forward_multi(toks, n)


@pytest.fixture(scope="module")
def spec_models():
    base = T.write_tiny_model(13)
    other = T.write_tiny_model(99)
    q8 = T.quantized(base, (8, 32), (8, 32))
    q4 = T.quantized(base, (4, 32), (4, 32))
    return base, {"int8 copy": q8, "int4 copy": q4, "unrelated model": other}


def test_speculation_never_changes_the_output_whatever_the_draft_guesses(spec_models):
    base, drafts = spec_models
    for name, d in drafts.items():
        for prompt in (PROMPT, OTHER_PROMPT):
            for max_new in (1, 2, 9, 30):
                want = O.plain_greedy(mk(base), prompt, max_new)
                for k in (1, 2, 3, 5, 8):
                    got, st = O.speculative_greedy(mk(base), O.model_drafter(mk(d)), prompt, max_new, k)
                    assert got == want, (name, len(prompt), max_new, k)
                    assert st["accepted"] <= st["drafted"]
                    assert st["target_passes"] <= max(len(got) - 1, 0)


def test_it_stops_at_an_end_of_sequence_token_exactly_where_plain_greedy_does():
    m = T.write_tiny_model(14)
    full = O.plain_greedy(mk(m), PROMPT, 24)
    for cut in (0, 1, 5, 11):
        eos = [full[cut]]
        want = O.plain_greedy(mk(m), PROMPT, 24, eos)
        assert len(want) <= cut + 1 and want[-1] == eos[0]
        for k in (1, 4, 8):
            got, _ = O.speculative_greedy(mk(m), O.model_drafter(mk(m)), PROMPT, 24, k, eos)
            assert got == want, (cut, k)


def test_a_perfect_draft_needs_far_fewer_passes():
    m = T.write_tiny_model(15)
    max_new, k = 21, 3
    want = O.plain_greedy(mk(m), PROMPT, max_new)
    got, st = O.speculative_greedy(mk(m), O.model_drafter(mk(m)), PROMPT, max_new, k)
    assert got == want
    assert st["accepted"] == st["drafted"]
    assert st["target_passes"] == -(-(max_new - 1) // (k + 1))


def test_bad_speculation_requests_are_errors():
    m = T.write_tiny_model(16)
    t, d = mk(m), mk(m)
    for k, prompt, max_new in [(0, PROMPT, 5), (33, PROMPT, 5), (2, [], 5), (2, PROMPT, 0), (2, PROMPT, 500)]:
        with pytest.raises(O.OracleError):
            O.speculative_greedy(t, O.model_drafter(d), prompt, max_new, k)
    t.forward(PROMPT)
    with pytest.raises(O.OracleError):
        O.speculative_greedy(t, O.model_drafter(d), PROMPT, 5, 2)


def test_scripted_drafter_equals_greedy_and_hits_its_acceptance_rate():
    m = T.write_tiny_model(17)
    want = O.plain_greedy(mk(m), PROMPT, 40)
    for p in (0.0, 0.6, 1.0):
        got, st = O.speculative_greedy(mk(m), O.scripted_drafter(want, p, 1234, T.VOCAB), PROMPT, 40, 8)
        assert got == want
        if p == 1.0:
            assert st["accepted"] == st["drafted"]
        if p == 0.0:
            assert st["accepted"] == 0
    d = O.scripted_drafter(list(range(5000)), 0.6, 7, 151936)
    hits = sum(L().or_scripted_draft(d, i) == i for i in range(5000))
    assert 0.57 < hits / 5000 < 0.63


# ---------------------------------------------------------------- tests/quant.rs:75-122
GRIDS = [
    ((8, 32), (8, 32)),
    ((8, 16), (8, 64)),
    ((4, 32), (4, 32)),
    ((4, 16), (4, 64)),
    ((4, 32), (8, 16)),
    ((8, 64), (4, 16)),
]

FOLLOW = [7, 33, 120]


def run_fixed(o):
    out = [o.forward(PROMPT)]
    for t in FOLLOW:
        out.append(o.forward([t]))
    return np.stack(out)


@pytest.mark.parametrize("i", range(len(GRIDS)))
def test_quantized_model_equals_bf16_when_weights_fit_the_grid(i):
    body, embed = GRIDS[i]
    m = T.write_tiny_model(100 + i, grid=(body, embed))
    ref = run_fixed(mk(m, 64))
    assert np.max(np.abs(ref)) > 0.01
    for clip in (False, True):
        q = T.quantized(m, body, embed, clip)
        got = run_fixed(mk(q, 64))
        tol = 1e-3 * (1 + np.max(np.abs(ref)))
        assert np.max(np.abs(ref - got)) < tol, (body, embed, clip)


def test_rounding_real_weights_stays_close_and_eight_bits_is_closer_than_four():
    m = T.write_tiny_model(7)
    ref = run_fixed(mk(m, 64))
    scale = np.max(np.abs(ref))

    def err(body):
        q = T.quantized(m, body, body, True)
        got = run_fixed(mk(q, 64))
        assert np.all(np.isfinite(got))
        return np.max(np.abs(ref - got)) / scale

    e8, e4 = err((8, 32)), err((4, 32))
    assert e8 < 0.05 and e8 < e4 < 1.0
