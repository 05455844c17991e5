"""Host-side (CPU) tests of the product library: the C ABI exports, the formats, the quantizer's
bytes against the oracle, `.lsq` validation and the scripted drafter. No GPU calls."""
import os
import re

import numpy as np
import pytest

import layerstream_amd as LS
import oracle_py as O
import tinymodels as T

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_library_exports_every_declared_symbol():
    hdr = open(os.path.join(ROOT, "include", "layerstream.h")).read()
    names = set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]*?\b(ls_\w+)\s*\(", hdr, re.M))
    assert len(names) >= 35
    lib = LS.lib()
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing
    assert set(LS.SIGNATURES) <= names


def test_row_bytes_and_validation():
    assert LS.row_bytes((16, 0), 896) == 1792
    assert LS.row_bytes((8, 64), 896) == 924
    assert LS.row_bytes((4, 32), 896) == 504
    import ctypes as C

    cols = (C.c_size_t * 2)(896, 4864)
    assert LS.lib().ls_format_validate(LS.fmt(8, 64), cols, 2) == 0
    for bad in [(6, 32), (8, 24), (8, 512), (8, 256)]:
        assert LS.lib().ls_format_validate(LS.fmt(*bad), cols, 2) != 0


BASE = (
    '{"model_type":"qwen2","hidden_act":"silu","tie_word_embeddings":true,"hidden_size":896,\n'
    '"num_attention_heads":14,"num_key_value_heads":2,"intermediate_size":4864,"num_hidden_layers":24,\n'
    '"vocab_size":151936,"rms_norm_eps":1e-6,"rope_theta":1000000.0,"max_position_embeddings":32768}'
)


def test_config_rejects_unsupported_architectures():
    """src/weights.rs:448-464"""
    c = LS.config_from_json(BASE)
    assert (c["head_dim"], c["heads"] // c["heads"] * 128, LS.row_bytes(c["embed_format"], 896)) == (64, 128, 1792)
    for a, b in [('"qwen2"', '"llama"'), ('"silu"', '"gelu"'), ('"tie_word_embeddings":true', '"tie_word_embeddings":false'), ('"num_key_value_heads":2', '"num_key_value_heads":5')]:
        with pytest.raises(LS.LayerstreamError):
            LS.config_from_json(BASE.replace(a, b))


def test_inject_quant_produces_a_config_that_parses_back():
    """src/quant.rs:376-397"""
    text = LS.inject_quant(BASE + "\n", 4, 32)
    assert text == T.inject_quant(BASE + "\n", 4, 32)
    c = LS.config_from_json(text)
    assert c["format"] == (4, 32) and c["embed_format"] == (4, 32)
    text = LS.inject_quant(BASE, 4, 32, (8, 64))
    c = LS.config_from_json(text)
    assert c["format"] == (4, 32) and c["embed_format"] == (8, 64)
    assert LS.row_bytes(c["embed_format"], 896) == 896 + 28
    plain = LS.config_from_json(BASE)
    assert plain["format"] == (16, 0)
    with pytest.raises(LS.LayerstreamError):
        LS.config_from_json(LS.inject_quant(BASE, 8, 256))
    with pytest.raises(LS.LayerstreamError):
        LS.config_from_json(text.replace(',"embed_group":64', ""))


def test_layer_layout_matches_the_oracle():
    import ctypes as C

    for f in [(16, 0), (8, 64), (4, 32), (8, 32)]:
        text = BASE if f[0] == 16 else LS.inject_quant(BASE, *f)
        ranges, total = LS.layer_layout(text)
        r = (C.c_size_t * 24)()
        c = O.cfg_struct(dict(hidden=896, inter=4864, layers=24, heads=14, kv_heads=2, head_dim=64, vocab=151936, eps=1e-6, rope_theta=1e6, format=f, embed_format=f))
        assert O.lib().or_layer_layout(C.byref(c), r) == total
        assert [(r[2 * i], r[2 * i + 1]) for i in range(12)] == ranges


def test_quantize_row_is_bit_identical_to_the_oracle():
    r = T.Lcg(3)
    for f in [(8, 16), (8, 32), (8, 64), (4, 16), (4, 32), (4, 64), (8, 256)]:
        for clip in (False, True):
            for _ in range(5):
                w = np.array([r.next() * np.float32(0.5 if i % 37 == 0 else 0.05) for i in range(256)], np.float32)
                got, e, n = LS.quantize_row(f, w, clip)
                want = np.zeros_like(got)
                import ctypes as C

                ee, nn = C.c_double(), C.c_double()
                O.lib().or_quantize_row(O.fmt(*f), O.f32(w), 256, int(clip), O.u8(want), C.byref(ee), C.byref(nn))
                assert np.array_equal(got, want), (f, clip)
                assert e == ee.value
    # special rows (quant.rs:328-343)
    for w in [np.zeros(64, np.float32), np.full(64, 1e-45, np.float32), np.full(64, -3.0, np.float32), np.array([np.inf] + [1.0] * 63, np.float32)]:
        got, _, _ = LS.quantize_row((4, 32), w, True)
        want = np.zeros_like(got)
        O.lib().or_quantize_row(O.fmt(4, 32), O.f32(w), 64, 1, O.u8(want), None, None)
        assert np.array_equal(got, want)


@pytest.mark.parametrize("body,embed", [((8, 32), (8, 32)), ((4, 32), (8, 64)), ((4, 16), (4, 16)), ((8, 64), (4, 16))])
def test_quantize_model_image_is_bit_identical_to_the_oracle(body, embed):
    m = T.write_tiny_model(3)
    got = LS.quantize_model(m["config_text"], m["layers"], m["embed"], m["norm"], body, embed)
    want = T.quantized(m, body, embed)["lsq"]
    assert got.tobytes() == want


def test_quantizer_rejects_bad_requests():
    """tests/quant.rs:194-213"""
    m = T.write_tiny_model(5)
    for bad in [(8, 48), (6, 32), (8, 512)]:
        with pytest.raises(LS.LayerstreamError):
            LS.quantize_model(m["config_text"], m["layers"], m["embed"], m["norm"], bad)
    q = T.quantized(m, (8, 32), (8, 32))
    with pytest.raises(LS.LayerstreamError, match="already quantized"):
        LS.quantize_model(q["config_text"], m["layers"], m["embed"], m["norm"], (8, 32))


def test_damaged_lsq_images_are_errors():
    """tests/quant.rs:215-229"""
    m = T.write_tiny_model(5)
    good = np.frombuffer(T.quantized(m, (8, 32), (8, 32))["lsq"], np.uint8)
    s = LS.Source.from_lsq_image(good.copy())
    assert s.config()["format"] == (8, 32)
    bads = [good[:-3], np.concatenate([good, [0]]).astype(np.uint8), good[:5]]
    magic = good.copy()
    magic[0] ^= 1
    bads.append(magic)
    for b in bads:
        with pytest.raises(LS.LayerstreamError):
            LS.Source.from_lsq_image(np.ascontiguousarray(b, np.uint8))


def test_lsq_file_source(tmp_path):
    m = T.write_tiny_model(6)
    img = T.quantized(m, (4, 32), (4, 32))["lsq"]
    p = tmp_path / "m.lsq"
    p.write_bytes(img)
    s = LS.Source.open_lsq(str(p))
    assert s.config()["format"] == (4, 32) and s.bytes_read() == 0
    (tmp_path / "bad.lsq").write_bytes(img[:-1])
    with pytest.raises(LS.LayerstreamError):
        LS.Source.open_lsq(str(tmp_path / "bad.lsq"))
    with pytest.raises(LS.LayerstreamError):
        LS.Source.open_lsq(str(tmp_path / "missing.lsq"))


def test_memory_source_checks_sizes():
    m = T.write_tiny_model(7)
    LS.Source.from_memory(m["config_text"], m["layers"], m["embed"], m["norm"])
    with pytest.raises(LS.LayerstreamError):
        LS.Source.from_memory(m["config_text"], m["layers"][:-2], m["embed"], m["norm"])


def test_synthetic_weights_are_seeded_and_shaped():
    text = LS.qwen2_config_text(hidden=64, inter=128, layers=2, heads=4, kv_heads=2, vocab=300)
    a = LS.synth_bf16_model(text, 5, threads=2)
    b = LS.synth_bf16_model(text, 5, threads=3)
    c = LS.synth_bf16_model(text, 6)
    assert all(np.array_equal(a[k], b[k]) for k in ("layers", "embed", "norm"))
    assert not np.array_equal(a["embed"], c["embed"])
    e = T.bf16_bytes_to_f32(a["embed"]).astype(np.float64)
    assert abs(e.mean()) < 2e-3 and abs(e.std() - 0.02) < 1e-3
    n = T.bf16_bytes_to_f32(a["norm"])
    assert abs(float(n.mean()) - 1.0) < 0.01
    # values are bf16 round-to-nearest results: re-rounding changes nothing
    assert all(O.lib().or_bf16_round(float(v)) == float(v) for v in e[:200])


def test_scripted_drafter_matches_the_oracle_proposer():
    g = list(range(100, 400))
    d = LS.ScriptedDrafter(g, 0.6, 99, 151936)
    od = O.scripted_drafter(g, 0.6, 99, 151936)
    for i in range(0, 350):
        assert d.token(i) == O.lib().or_scripted_draft(od, i)
