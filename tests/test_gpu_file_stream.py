"""Streaming weights from a `.lsq` file (FileSource, src/source.rs:90-182) through the stream
provider's I/O thread, which reads ahead of the copies in schedule order (src/provider.rs:187-206,
288-305): logits against the oracle on the tiny model for 1, 2 and 3 device slots, bit-identical to
the resident model on the 0.5B shape, every pass reading each layer block and the table once, and a
file that shrinks under the model turning into an error instead of a hang."""
import os

import numpy as np
import pytest

import layerstream_amd as LS
import tinymodels as T
from test_gpu import FOLLOW, PROMPT, bits, close, cpu_model, gpu_model, qwen05b, run_fixed, say, tiny

pytestmark = pytest.mark.gpu


def write_lsq(tmp_path, m, name):
    path = os.path.join(str(tmp_path), name + ".lsq")
    with open(path, "wb") as f:
        f.write(bytes(m["lsq"]))
    return path


@pytest.mark.parametrize("name", ["int4", "mixed", "int8"])
def test_streaming_from_a_file_matches_the_oracle(tmp_path, name):
    m = tiny(name)
    ref = run_fixed(cpu_model(m))
    path = write_lsq(tmp_path, m, name)
    for slots in (1, 2, 3):
        say("file stream", name, "slots", slots)
        src = LS.Source.open_lsq(path)
        g = LS.Model(src, LS.MODE_STREAM, slots, 128)
        got = run_fixed(g)
        assert close(got, ref), (name, slots, float(np.max(np.abs(got - ref))))
        assert np.array_equal(got.argmax(1), ref.argmax(1))
        # one pass per call: every layer block and the table once, plus one row per token
        c = src.config()
        _, total = LS.layer_layout(m["config_text"])
        rb = LS.row_bytes(c["embed_format"], c["hidden"])
        passes = 1 + len(FOLLOW)
        assert src.bytes_read() == passes * (c["layers"] * total + c["vocab"] * rb) + (len(PROMPT) + len(FOLLOW)) * rb
        rep = g.report()
        assert rep["h2d_bytes"] >= passes * c["layers"] * total


def test_qwen05b_streamed_from_a_file_gives_the_resident_bits(tmp_path):
    """0.5B int8-g64: a 40-token prompt and a k=8 verify step, streamed from a file through 2
    slots, give the resident model's logits bit for bit and its acceptance."""
    m = qwen05b((8, 64))
    path = write_lsq(tmp_path, m, "q05b_int8")
    rng = np.random.default_rng(9)
    V = LS.QWEN2_05B["vocab"]
    prompt = rng.integers(0, V, 40).tolist()
    res = gpu_model(m, max_ctx=128)
    st = LS.Model(LS.Source.open_lsq(path), LS.MODE_STREAM, 2, 128)
    la, lb = res.forward(prompt), st.forward(prompt)
    assert np.array_equal(bits(la), bits(lb))
    a = int(np.argmax(la))
    block = [a] + rng.integers(0, V, 8).tolist()
    p = res.pos()
    va, vb = res.forward_multi(block, 9), st.forward_multi(block, 9)
    assert np.array_equal(bits(va), bits(vb))
    res.truncate(p)
    st.truncate(p)
    assert res.verify_greedy(block) == st.verify_greedy(block)
    rep = st.report()
    say("0.5B file stream: host wait for reads per pass (ms)", rep["wait_ns"] / 1e6 / 4)


def test_a_file_that_shrinks_under_the_model_is_an_error(tmp_path):
    """The I/O thread's read failure reaches the caller as LS_E_IO (the reference returns the
    read error from forward), and the model is not left waiting on it."""
    m = tiny("int4")
    path = write_lsq(tmp_path, m, "shrink")
    src = LS.Source.open_lsq(path)
    g = LS.Model(src, LS.MODE_STREAM, 2, 64)
    g.forward(PROMPT)
    size = os.path.getsize(path)
    with open(path, "r+b") as f:
        f.truncate(size // 2)
    with pytest.raises(LS.LayerstreamError) as e:
        g.forward([1])
    assert e.value.code == -3


@pytest.mark.parametrize("name", ["int4", "mixed"])
def test_pinned_streaming_from_the_tiled_mirror_gives_the_resident_bits(name):
    """A pinned source is streamed from a pinned copy already in the tile layout (built once by the
    provider, no rearrangement per pass); LS_STREAM_TILED=0 copies the source's own bytes and
    rearranges them on the device every pass. Both give the resident logits bit for bit, for 1, 2
    and 3 slots, and the reads are counted the same way."""
    from test_gpu import env

    m = tiny(name)
    ref = run_fixed(gpu_model(m))
    img = np.frombuffer(bytes(m["lsq"]), np.uint8).copy()
    for tiled in ("1", "0"):
        for slots in (1, 2, 3):
            say("pinned stream", name, "tiled", tiled, "slots", slots)
            src = LS.Source.from_lsq_image(img).pinned_copy()
            with env("LS_STREAM_TILED", tiled):
                g = LS.Model(src, LS.MODE_STREAM, slots, 128)
            got = run_fixed(g)
            assert np.array_equal(bits(ref), bits(got)), (name, tiled, slots)
            c = src.config()
            _, total = LS.layer_layout(m["config_text"])
            rb = LS.row_bytes(c["embed_format"], c["hidden"])
            passes = 1 + len(FOLLOW)
            assert src.bytes_read() == passes * (c["layers"] * total + c["vocab"] * rb) + (len(PROMPT) + len(FOLLOW)) * rb
