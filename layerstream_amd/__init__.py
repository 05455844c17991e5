"""layerstream_amd: MI355X speculative-decoding verify engine (Python binding of the C ABI).

The classes mirror the reference crate's API (themaker00001/layerstream): `Model` with
forward / forward_multi / truncate / pos / reset / max_ctx (src/model.rs:58-140),
`speculative_greedy` (src/spec.rs:57-152), sources (src/source.rs) and the quantizer
(src/quant.rs). All compute runs in liblayerstream_amd.so (HIP, gfx950); there is no CPU
fallback: if the library is missing this module raises on import of the binding.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liblayerstream_amd.so")

MODE_RESIDENT = 0
MODE_STREAM = 1
MAX_DRAFT = 32


class LayerstreamError(RuntimeError):
    """A bad request or failure reported by the engine (the reference's Err(String))."""

    def __init__(self, code: int, msg: str):
        super().__init__(msg)
        self.code = code


class Format(C.Structure):
    _fields_ = [("bits", C.c_int32), ("group", C.c_int32)]


class Config(C.Structure):
    _fields_ = [
        ("format", Format),
        ("embed_format", Format),
        ("hidden", C.c_int64),
        ("inter", C.c_int64),
        ("layers", C.c_int64),
        ("heads", C.c_int64),
        ("kv_heads", C.c_int64),
        ("head_dim", C.c_int64),
        ("vocab", C.c_int64),
        ("max_pos", C.c_int64),
        ("eps", C.c_float),
        ("rope_theta", C.c_float),
    ]

    def as_dict(self) -> dict:
        return {
            "format": (self.format.bits, self.format.group),
            "embed_format": (self.embed_format.bits, self.embed_format.group),
            "hidden": self.hidden,
            "inter": self.inter,
            "layers": self.layers,
            "heads": self.heads,
            "kv_heads": self.kv_heads,
            "head_dim": self.head_dim,
            "vocab": self.vocab,
            "max_pos": self.max_pos,
            "eps": self.eps,
            "rope_theta": self.rope_theta,
        }


class Report(C.Structure):
    _fields_ = [("resident_weight_bytes", C.c_uint64), ("bytes_read", C.c_uint64), ("wait_ns", C.c_uint64), ("h2d_bytes", C.c_uint64)]


class SpecStats(C.Structure):
    _fields_ = [
        ("target_passes", C.c_uint64),
        ("drafted", C.c_uint64),
        ("accepted", C.c_uint64),
        ("draft_forwards", C.c_uint64),
        ("target_secs", C.c_double),
        ("draft_secs", C.c_double),
        ("first_secs", C.c_double),
        ("decode_secs", C.c_double),
    ]

    def as_dict(self) -> dict:
        return {f: getattr(self, f) for f, _ in self._fields_}


class KernelStat(C.Structure):
    _fields_ = [("launches", C.c_uint64), ("ms", C.c_double), ("bytes", C.c_double), ("flops", C.c_double)]


PREFILL = C.CFUNCTYPE(C.c_int, C.c_void_p, C.POINTER(C.c_uint32), C.c_size_t)
PROPOSE = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_uint32, C.c_size_t, C.POINTER(C.c_uint32))
COMMIT = C.CFUNCTYPE(C.c_int, C.c_void_p, C.POINTER(C.c_uint32), C.c_size_t, C.c_size_t)


class Drafter(C.Structure):
    _fields_ = [("ctx", C.c_void_p), ("prefill", C.c_void_p), ("propose", C.c_void_p), ("commit", C.c_void_p)]


# Symbols of include/layerstream.h and their signatures.
P, SZ, U8, U32, F32 = C.c_void_p, C.c_size_t, C.POINTER(C.c_uint8), C.POINTER(C.c_uint32), C.POINTER(C.c_float)
SIGNATURES = {
    "ls_last_error": (C.c_char_p, []),
    "ls_version": (C.c_char_p, []),
    "ls_row_bytes": (SZ, [Format, SZ]),
    "ls_format_validate": (C.c_int, [Format, C.POINTER(SZ), SZ]),
    "ls_config_from_json": (C.c_int, [C.c_char_p, C.POINTER(Config)]),
    "ls_layer_layout": (SZ, [C.POINTER(Config), C.POINTER(SZ)]),
    "ls_inject_quant": (C.c_int, [C.c_char_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_char_p, SZ, C.POINTER(SZ)]),
    "ls_quantize_row": (C.c_int, [Format, F32, SZ, C.c_int, U8, C.POINTER(C.c_double), C.POINTER(C.c_double)]),
    "ls_quantize_model": (C.c_int, [C.c_char_p, U8, U8, U8, Format, Format, C.c_int, C.c_int, U8, SZ, C.POINTER(SZ), C.POINTER(C.c_double)]),
    "ls_synth_bf16_model": (C.c_int, [C.POINTER(Config), C.c_uint64, C.c_float, U8, U8, U8, C.c_int]),
    "ls_source_from_memory": (C.c_int, [C.c_char_p, U8, SZ, U8, SZ, U8, SZ, C.POINTER(P)]),
    "ls_source_open_lsq": (C.c_int, [C.c_char_p, C.POINTER(P)]),
    "ls_source_from_lsq_image": (C.c_int, [U8, SZ, C.POINTER(P)]),
    "ls_source_pinned_copy": (C.c_int, [P, C.POINTER(P)]),
    "ls_source_free": (None, [P]),
    "ls_source_config": (C.c_int, [P, C.POINTER(Config)]),
    "ls_source_bytes_read": (C.c_uint64, [P]),
    "ls_model_create": (C.c_int, [P, C.c_int, C.c_int, SZ, C.c_int, C.POINTER(P)]),
    "ls_model_create_batch": (C.c_int, [P, C.c_int, C.c_int, SZ, C.c_int, C.c_int, C.POINTER(P)]),
    "ls_model_n_seq": (C.c_int, [P]),
    "ls_model_select": (C.c_int, [P, C.c_int]),
    "ls_model_verify_greedy_batch": (C.c_int, [P, U32, C.POINTER(SZ), C.c_int, U32, U32]),
    "ls_model_free": (None, [P]),
    "ls_model_pos": (SZ, [P]),
    "ls_model_max_ctx": (SZ, [P]),
    "ls_model_reset": (None, [P]),
    "ls_model_truncate": (C.c_int, [P, SZ]),
    "ls_model_forward": (C.c_int, [P, U32, SZ, F32, U32]),
    "ls_model_forward_multi": (C.c_int, [P, U32, SZ, SZ, F32, U32]),
    "ls_model_verify_greedy": (C.c_int, [P, U32, SZ, U32, U32]),
    "ls_model_report": (C.c_int, [P, C.POINTER(Report)]),
    "ls_model_last_step_ms": (C.c_double, [P]),
    "ls_model_draft_chain": (C.c_int, [P, C.c_uint32, SZ, U32]),
    "ls_tokenizer_load": (C.c_int, [C.c_char_p, C.POINTER(P)]),
    "ls_tokenizer_free": (None, [P]),
    "ls_tokenizer_vocab_size": (SZ, [P]),
    "ls_tokenizer_encode": (C.c_int, [P, C.c_char_p, SZ, U32, SZ, C.POINTER(SZ)]),
    "ls_tokenizer_decode": (C.c_int, [P, U32, SZ, C.c_char_p, SZ, C.POINTER(SZ)]),
    "ls_tokenizer_token_bytes": (C.c_int, [P, C.c_uint32, C.c_int, C.c_char_p, SZ, C.POINTER(SZ)]),
    "ls_tokenizer_token_id": (C.c_int, [P, C.c_char_p, U32]),
    "ls_tokenizer_is_special": (C.c_int, [P, C.c_uint32]),
    "ls_tokenizer_pretokens": (C.c_int, [C.c_char_p, SZ, U32, SZ, C.POINTER(SZ)]),
    "ls_stream_decoder_new": (C.c_int, [C.POINTER(P)]),
    "ls_stream_decoder_free": (None, [P]),
    "ls_stream_decoder_push": (C.c_int, [P, C.c_char_p, SZ, C.c_char_p, SZ, C.POINTER(SZ)]),
    "ls_stream_decoder_finish": (C.c_int, [P, C.c_char_p, SZ, C.POINTER(SZ)]),
    "ls_sampler_new": (C.c_int, [C.c_float, SZ, C.c_float, C.c_uint64, C.POINTER(P)]),
    "ls_sampler_free": (None, [P]),
    "ls_sampler_sample": (C.c_int, [P, F32, SZ, U32]),
    "ls_drafter_from_model": (C.c_int, [P, C.POINTER(Drafter)]),
    "ls_drafter_scripted": (C.c_int, [U32, SZ, C.c_double, C.c_uint64, C.c_uint64, C.POINTER(Drafter)]),
    "ls_drafter_scripted_token": (C.c_uint32, [C.POINTER(Drafter), SZ]),
    "ls_drafter_free": (None, [C.POINTER(Drafter)]),
    "ls_speculative_greedy": (C.c_int, [P, C.POINTER(Drafter), U32, SZ, SZ, SZ, U32, SZ, U32, C.POINTER(SZ), C.POINTER(SpecStats)]),
    "ls_greedy_generate": (C.c_int, [P, U32, SZ, SZ, U32, SZ, U32, C.POINTER(SZ)]),
    "ls_spec_begin": (C.c_int, [P, C.POINTER(Drafter), U32, SZ, SZ, SZ, U32, SZ, C.POINTER(P)]),
    "ls_spec_step": (C.c_int, [P, SZ, C.POINTER(C.c_int)]),
    "ls_spec_result": (C.c_int, [P, U32, SZ, C.POINTER(SZ), C.POINTER(SpecStats)]),
    "ls_spec_step_log": (SZ, [P, C.POINTER(C.c_double), U32, SZ]),
    "ls_spec_free": (None, [P]),
    "ls_model_profile": (C.c_int, [P, C.c_int]),
    "ls_model_profile_read": (C.c_int, [P, C.POINTER(KernelStat)]),
    "ls_model_use_graphs": (C.c_int, [P, C.c_int]),
    "ls_model_debug_fail_next": (C.c_int, [P]),
    "ls_model_debug_timeline": (SZ, [P, C.POINTER(C.c_uint64), SZ]),
    "ls_model_debug_read": (SZ, [P, C.c_char_p, P, SZ]),
    "ls_matmul": (C.c_int, [Format, P, SZ, SZ, P, SZ, P, P]),
    "ls_matmul_noalloc": (C.c_int, [Format, P, SZ, SZ, P, SZ, P, P]),
}

_lib = None


def lib():
    """The loaded C library; raises if it has not been built (no fallback exists)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with `python -m layerstream_amd.build`")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _check(rc: int):
    if rc != 0:
        raise LayerstreamError(rc, lib().ls_last_error().decode())


def _u8(a: np.ndarray):
    return a.ctypes.data_as(U8)


def _u32(a: np.ndarray):
    return a.ctypes.data_as(U32)


def _f32(a: np.ndarray):
    return a.ctypes.data_as(F32)


def _toks(tokens) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32).reshape(-1))


# ---------------------------------------------------------------------------------- formats
def fmt(bits: int, group: int = 0) -> Format:
    return Format(bits, group)


def row_bytes(f, cols: int) -> int:
    return lib().ls_row_bytes(Format(*f), cols)


def config_from_json(text: str) -> dict:
    c = Config()
    _check(lib().ls_config_from_json(text.encode(), C.byref(c)))
    return c.as_dict()


def inject_quant(text: str, bits: int, group: int, embed=None) -> str:
    n = C.c_size_t(0)
    eb, eg = embed if embed else (0, 0)
    _check(lib().ls_inject_quant(text.encode(), bits, group, eb, eg, None, 0, C.byref(n)))
    buf = C.create_string_buffer(n.value + 1)
    _check(lib().ls_inject_quant(text.encode(), bits, group, eb, eg, buf, n.value + 1, C.byref(n)))
    return buf.value.decode()


def layer_layout(cfg_text: str):
    c = Config()
    _check(lib().ls_config_from_json(cfg_text.encode(), C.byref(c)))
    r = (C.c_size_t * 24)()
    total = lib().ls_layer_layout(C.byref(c), r)
    return [(r[2 * i], r[2 * i + 1]) for i in range(12)], total


def quantize_row(f, row, clip: bool = True):
    row = np.ascontiguousarray(row, np.float32)
    out = np.zeros(row_bytes(f, len(row)), np.uint8)
    e, n = C.c_double(), C.c_double()
    _check(lib().ls_quantize_row(Format(*f), _f32(row), len(row), int(clip), _u8(out), C.byref(e), C.byref(n)))
    return out, e.value, n.value


def quantize_model(config_text: str, layers, embed, norm, body, embed_fmt=None, clip: bool = True, threads: int = 0) -> bytes:
    """quantize_model (src/quant.rs:158-251) of in-memory bf16 parts into a `.lsq` image."""
    embed_fmt = embed_fmt or body
    layers = np.ascontiguousarray(layers, np.uint8)
    embed = np.ascontiguousarray(embed, np.uint8)
    norm = np.ascontiguousarray(norm, np.uint8)
    n = C.c_size_t(0)
    args = (config_text.encode(), _u8(layers), _u8(embed), _u8(norm), Format(*body), Format(*embed_fmt), int(clip), threads)
    _check(lib().ls_quantize_model(*args, None, 0, C.byref(n), None))
    out = np.zeros(n.value, np.uint8)
    rel = C.c_double()
    _check(lib().ls_quantize_model(*args, _u8(out), n.value, C.byref(n), C.byref(rel)))
    return out


# ---------------------------------------------------------------------------------- models
QWEN2_05B = dict(hidden=896, inter=4864, layers=24, heads=14, kv_heads=2, vocab=151936, eps=1e-6, rope_theta=1e6, max_pos=32768)
QWEN2_3B = dict(hidden=2048, inter=11008, layers=36, heads=16, kv_heads=2, vocab=151936, eps=1e-6, rope_theta=1e6, max_pos=32768)


def qwen2_config_text(hidden, inter, layers, heads, kv_heads, vocab, eps=1e-6, rope_theta=1e6, max_pos=32768) -> str:
    """A Hugging Face style config.json for a Qwen2 model with tied embeddings."""
    return (
        '{"model_type":"qwen2","hidden_act":"silu","tie_word_embeddings":true,'
        f'"hidden_size":{hidden},"num_attention_heads":{heads},"num_key_value_heads":{kv_heads},'
        f'"intermediate_size":{inter},"num_hidden_layers":{layers},"vocab_size":{vocab},'
        f'"rms_norm_eps":{eps!r},"rope_theta":{float(rope_theta)!r},"max_position_embeddings":{max_pos}}}'
    )


def synth_bf16_model(config_text: str, seed: int, std: float = 0.02, threads: int = 0) -> dict:
    """Seeded random-init bf16 weights of the config's shape (layers, embedding, final norm)."""
    c = Config()
    _check(lib().ls_config_from_json(config_text.encode(), C.byref(c)))
    r = (C.c_size_t * 24)()
    total = lib().ls_layer_layout(C.byref(c), r)
    layers = np.empty(total * c.layers, np.uint8)
    embed = np.empty(c.vocab * c.hidden * 2, np.uint8)
    norm = np.empty(c.hidden * 2, np.uint8)
    _check(lib().ls_synth_bf16_model(C.byref(c), seed, std, _u8(layers), _u8(embed), _u8(norm), threads))
    return {"config_text": config_text, "layers": layers, "embed": embed, "norm": norm}


class Source:
    """A byte source (trait Source, src/source.rs:23-33)."""

    def __init__(self, handle, keep=()):
        self.h = handle
        self._keep = keep

    @classmethod
    def from_memory(cls, config_text: str, layers, embed, norm) -> "Source":
        layers = np.ascontiguousarray(layers, np.uint8)
        embed = np.ascontiguousarray(embed, np.uint8)
        norm = np.ascontiguousarray(norm, np.uint8)
        h = C.c_void_p()
        _check(lib().ls_source_from_memory(config_text.encode(), _u8(layers), layers.size, _u8(embed), embed.size, _u8(norm), norm.size, C.byref(h)))
        return cls(h, (layers, embed, norm))

    @classmethod
    def from_lsq_image(cls, image) -> "Source":
        img = np.ascontiguousarray(np.frombuffer(image, np.uint8) if isinstance(image, (bytes, bytearray)) else image, np.uint8)
        h = C.c_void_p()
        _check(lib().ls_source_from_lsq_image(_u8(img), img.size, C.byref(h)))
        return cls(h, (img,))

    @classmethod
    def open_lsq(cls, path: str) -> "Source":
        h = C.c_void_p()
        _check(lib().ls_source_open_lsq(os.fsencode(path), C.byref(h)))
        return cls(h)

    def pinned_copy(self) -> "Source":
        h = C.c_void_p()
        _check(lib().ls_source_pinned_copy(self.h, C.byref(h)))
        return Source(h)

    def config(self) -> dict:
        c = Config()
        _check(lib().ls_source_config(self.h, C.byref(c)))
        return c.as_dict()

    def bytes_read(self) -> int:
        return lib().ls_source_bytes_read(self.h)

    def close(self):
        if self.h:
            lib().ls_source_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Model:
    """Model (src/model.rs:16-140) on an MI355X. mode: MODE_RESIDENT or MODE_STREAM.

    With n_seq > 1 it holds that many independent sequences (K/V caches and positions) over one
    copy of the weights: the single-sequence calls act on the selected one (select()), and
    verify_greedy_batch() verifies a block of every sequence in one pass."""

    def __init__(self, source: Source, mode: int = MODE_RESIDENT, slots: int = 2, max_ctx: int = 1024, device: int = 0,
                 n_seq: int = 1):
        self.source = source
        h = C.c_void_p()
        if n_seq == 1:
            _check(lib().ls_model_create(source.h, mode, slots, max_ctx, device, C.byref(h)))
        else:
            _check(lib().ls_model_create_batch(source.h, mode, slots, max_ctx, device, n_seq, C.byref(h)))
        self.h = h
        self._cfg = source.config()

    def close(self):
        if getattr(self, "h", None):
            lib().ls_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def cfg(self) -> dict:
        return self._cfg

    @property
    def vocab(self) -> int:
        return self._cfg["vocab"]

    def pos(self) -> int:
        return lib().ls_model_pos(self.h)

    def max_ctx(self) -> int:
        return lib().ls_model_max_ctx(self.h)

    def reset(self):
        lib().ls_model_reset(self.h)

    def truncate(self, pos: int):
        _check(lib().ls_model_truncate(self.h, pos))

    def forward(self, tokens) -> np.ndarray:
        t = _toks(tokens)
        out = np.zeros(self.vocab, np.float32)
        _check(lib().ls_model_forward(self.h, _u32(t), t.size, _f32(out), None))
        return out

    def forward_argmax(self, tokens) -> int:
        t = _toks(tokens)
        a = np.zeros(1, np.uint32)
        _check(lib().ls_model_forward(self.h, _u32(t), t.size, None, _u32(a)))
        return int(a[0])

    def forward_multi(self, tokens, n: int) -> np.ndarray:
        t = _toks(tokens)
        out = np.zeros((max(n, 1), self.vocab), np.float32)
        _check(lib().ls_model_forward_multi(self.h, _u32(t), t.size, n, _f32(out), None))
        return out

    def forward_multi_argmax(self, tokens, n: int) -> np.ndarray:
        t = _toks(tokens)
        a = np.zeros(max(n, 1), np.uint32)
        _check(lib().ls_model_forward_multi(self.h, _u32(t), t.size, n, None, _u32(a)))
        return a

    def verify_greedy(self, block):
        """One fused verify step: returns (accepted m, next token); the cache keeps p + m + 1."""
        t = _toks(block)
        m, nx = C.c_uint32(), C.c_uint32()
        _check(lib().ls_model_verify_greedy(self.h, _u32(t), t.size, C.byref(m), C.byref(nx)))
        return m.value, nx.value

    def report(self) -> dict:
        r = Report()
        _check(lib().ls_model_report(self.h, C.byref(r)))
        return {f: getattr(r, f) for f, _ in Report._fields_}

    def last_step_ms(self) -> float:
        return lib().ls_model_last_step_ms(self.h)

    def profile(self, enable: bool, dominant: bool = False):
        """Bracket every weight-streaming matvec launch with HIP events (for roofline figures);
        with dominant, only each pass's dominant launch (the layer stack when a pass runs as one)."""
        _check(lib().ls_model_profile(self.h, (2 if dominant else 1) if enable else 0))

    def profile_read(self) -> dict:
        st = KernelStat()
        _check(lib().ls_model_profile_read(self.h, C.byref(st)))
        return {f: getattr(st, f) for f, _ in KernelStat._fields_}

    def use_graphs(self, enable: bool):
        """Replay verify steps from captured HIP graphs (default on; resident weights only)."""
        _check(lib().ls_model_use_graphs(self.h, int(enable)))

    def debug_timeline(self, raw: bool = False) -> np.ndarray:
        """Per-unit stamps of the last persistent pass (LS_PASS_TIMELINE=1 at creation), or None:
        [workgroup][layer][stage (qkv, attention, o, gate|up, down)][32] in 100 MHz ticks:
        0 start, 1 + w wavefront w's input ready, 9 1/rms known, 10 products summed, 11 stores
        issued, 12 done, 13 flags seen, 14/15 stale re-fetches (counts), 16 + w wavefront w's
        products done, 24 flag store acknowledged; 0 where a unit did not run or reach a stamp.
        With raw, the words as they are: also the layer stack's [workgroup][4] stamps
        (LS_STACK_TIMELINE=1 at creation: [workgroup][8]: entry, input there, done, inputs loaded,
        products issued, row-group sums done, epilogue stores issued, layer << 8 | role)."""
        n = lib().ls_model_debug_timeline(self.h, None, 0)
        if n == 0:
            return None
        out = np.zeros(n, np.uint64)
        lib().ls_model_debug_timeline(self.h, out.ctypes.data_as(C.POINTER(C.c_uint64)), n)
        if raw:
            return out
        L = self.cfg()["layers"]
        return out.reshape(-1, L, 5, 32)

    def debug_read(self, name: str) -> np.ndarray:
        """A copy of an internal device buffer (debugging) as bytes."""
        n = lib().ls_model_debug_read(self.h, name.encode(), None, 0)
        if n == 0:
            raise LayerstreamError(-1, lib().ls_last_error().decode())
        out = np.zeros(n, np.uint8)
        lib().ls_model_debug_read(self.h, name.encode(), out.ctypes.data, n)
        return out

    def draft_chain(self, first: int, k: int) -> list:
        """k greedy single-token passes chained on the device: the draft model's proposals after
        `first` (the same tokens as k forward + argmax calls); the model advances by k."""
        out = np.zeros(k, np.uint32)
        _check(lib().ls_model_draft_chain(self.h, first, k, _u32(out)))
        return out.tolist()

    def debug_fail_next(self):
        """Test hook: the next device pass starts with its error word set and fails with
        LS_E_DEVICE (every in-launch wait gives up at once); positions stay unchanged."""
        _check(lib().ls_model_debug_fail_next(self.h))

    @property
    def n_seq(self) -> int:
        return lib().ls_model_n_seq(self.h)

    def select(self, seq: int):
        """Make sequence `seq` the one the single-sequence calls act on."""
        _check(lib().ls_model_select(self.h, seq))

    def verify_greedy_batch(self, blocks):
        """One verify pass over blocks[s] for every sequence s: [(accepted m_s, next_s)], as
        verify_greedy would return for each sequence alone; sequence s keeps p_s + m_s + 1."""
        if len(blocks) != self.n_seq:
            raise ValueError(f"{len(blocks)} blocks for {self.n_seq} sequences")
        lens = np.array([len(b) for b in blocks], np.uint64)
        flat = _toks(np.concatenate([np.asarray(b, np.uint32) for b in blocks]) if len(blocks) else [])
        m = np.zeros(len(blocks), np.uint32)
        nx = np.zeros(len(blocks), np.uint32)
        _check(lib().ls_model_verify_greedy_batch(self.h, _u32(flat), lens.ctypes.data_as(C.POINTER(SZ)), len(blocks), _u32(m),
                                                  _u32(nx)))
        return [(int(a), int(b)) for a, b in zip(m, nx)]


class ModelDrafter:
    """A draft Model, as the reference's `draft: &mut Model` (src/spec.rs:59)."""

    def __init__(self, model: Model):
        self.model = model
        self.d = Drafter()
        _check(lib().ls_drafter_from_model(model.h, C.byref(self.d)))

    def close(self):
        pass


class ScriptedDrafter:
    """Proposes greedy[i] with probability p_accept, else another token (seeded)."""

    def __init__(self, greedy, p_accept: float, seed: int, vocab: int):
        g = _toks(greedy)
        self.d = Drafter()
        _check(lib().ls_drafter_scripted(_u32(g), g.size, p_accept, seed, vocab, C.byref(self.d)))

    def token(self, i: int) -> int:
        return lib().ls_drafter_scripted_token(C.byref(self.d), i)

    def close(self):
        if self.d.ctx:
            lib().ls_drafter_free(C.byref(self.d))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def speculative_greedy(target: Model, draft, prompt, max_new: int, k: int, eos=()):
    """speculative_greedy (src/spec.rs:57-152): returns (tokens, stats dict)."""
    if isinstance(draft, Model):
        draft = ModelDrafter(draft)
    p = _toks(prompt) if len(prompt) else np.zeros(0, np.uint32)
    e = _toks(list(eos) or [0])
    out = np.zeros(max(max_new, 1), np.uint32)
    n = C.c_size_t(0)
    st = SpecStats()
    pp = _u32(p) if p.size else None
    rc = lib().ls_speculative_greedy(target.h, C.byref(draft.d), pp, p.size, max_new, k, _u32(e), len(eos), _u32(out), C.byref(n), C.byref(st))
    _check(rc)
    return out[: n.value].tolist(), st.as_dict()


class SpecRun:
    """speculative_greedy in resumable form: the prompt pass at construction, then step(n) runs n
    verify passes; tokens(), stats() and step_log() report progress."""

    def __init__(self, target: Model, draft, prompt, max_new: int, k: int, eos=()):
        if isinstance(draft, Model):
            draft = ModelDrafter(draft)
        self._draft = draft
        p = _toks(prompt)
        e = _toks(list(eos) or [0])
        h = C.c_void_p()
        _check(lib().ls_spec_begin(target.h, C.byref(draft.d), _u32(p), p.size, max_new, k, _u32(e), len(eos), C.byref(h)))
        self.h = h
        self.max_new = max_new

    def step(self, n: int = 1) -> bool:
        done = C.c_int(0)
        _check(lib().ls_spec_step(self.h, n, C.byref(done)))
        return bool(done.value)

    def tokens(self):
        out = np.zeros(max(self.max_new, 1), np.uint32)
        n = C.c_size_t(0)
        _check(lib().ls_spec_result(self.h, _u32(out), out.size, C.byref(n), None))
        return out[: n.value].tolist()

    def stats(self) -> dict:
        st = SpecStats()
        _check(lib().ls_spec_result(self.h, None, 0, None, C.byref(st)))
        return st.as_dict()

    def step_log(self):
        n = lib().ls_spec_step_log(self.h, None, None, 0)
        ms = np.zeros(max(n, 1), np.float64)
        m = np.zeros(max(n, 1), np.uint32)
        lib().ls_spec_step_log(self.h, ms.ctypes.data_as(C.POINTER(C.c_double)), _u32(m), n)
        return ms[:n], m[:n]

    def close(self):
        if getattr(self, "h", None):
            lib().ls_spec_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def greedy_generate(m: Model, prompt, max_new: int, eos=()):
    """Plain greedy decoding (Sampler::greedy, src/model.rs:328-336)."""
    p = _toks(prompt)
    e = _toks(list(eos) or [0])
    out = np.zeros(max(max_new, 1), np.uint32)
    n = C.c_size_t(0)
    _check(lib().ls_greedy_generate(m.h, _u32(p), p.size, max_new, _u32(e), len(eos), _u32(out), C.byref(n)))
    return out[: n.value].tolist()


def _sized_bytes(call):
    """Runs call(buf, cap, n_ptr) twice when the first buffer is too small; returns the bytes."""
    n = C.c_size_t(0)
    buf = C.create_string_buffer(256)
    _check(call(buf, 256, C.byref(n)))
    if n.value > 256:
        buf = C.create_string_buffer(n.value)
        _check(call(buf, n.value, C.byref(n)))
    return buf.raw[: n.value]


class Tokenizer:
    """The Qwen2 byte-level BPE tokenizer (src/tokenizer.rs), in the library (host code)."""

    def __init__(self, model_dir: str):
        h = C.c_void_p()
        _check(lib().ls_tokenizer_load(os.fsencode(model_dir), C.byref(h)))
        self.h = h

    def vocab_size(self) -> int:
        return lib().ls_tokenizer_vocab_size(self.h)

    def encode(self, text: str) -> list:
        b = text.encode("utf-8")
        n = C.c_size_t(0)
        _check(lib().ls_tokenizer_encode(self.h, b, len(b), None, 0, C.byref(n)))
        out = np.zeros(max(n.value, 1), np.uint32)
        _check(lib().ls_tokenizer_encode(self.h, b, len(b), _u32(out), out.size, C.byref(n)))
        return out[: n.value].tolist()

    def decode(self, ids) -> str:
        a = _toks(list(ids) or [0])
        k = len(list(ids))
        return _sized_bytes(lambda buf, cap, n: lib().ls_tokenizer_decode(self.h, _u32(a), k, buf, cap, n)).decode("utf-8")

    def token_bytes(self, tid: int, show_special: bool = False) -> bytes:
        return _sized_bytes(lambda buf, cap, n: lib().ls_tokenizer_token_bytes(self.h, tid, int(show_special), buf, cap, n))

    def token_id(self, token: str):
        i = np.zeros(1, np.uint32)
        return int(i[0]) if lib().ls_tokenizer_token_id(self.h, token.encode("utf-8"), _u32(i)) else None

    def is_special(self, tid: int) -> bool:
        return bool(lib().ls_tokenizer_is_special(self.h, tid))

    def close(self):
        if getattr(self, "h", None):
            lib().ls_tokenizer_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def pretokens(text: str) -> list:
    """The pre-token split of text (the Qwen2 pattern), as strings."""
    b = text.encode("utf-8")
    n = C.c_size_t(0)
    _check(lib().ls_tokenizer_pretokens(b, len(b), None, 0, C.byref(n)))
    ends = np.zeros(max(n.value, 1), np.uint32)
    _check(lib().ls_tokenizer_pretokens(b, len(b), _u32(ends), ends.size, C.byref(n)))
    out, start = [], 0
    for e in ends[: n.value].tolist():
        out.append(text[start:e])
        start = e
    return out


class StreamDecoder:
    """Incremental UTF-8 decoder (src/tokenizer.rs:311-346)."""

    def __init__(self):
        h = C.c_void_p()
        _check(lib().ls_stream_decoder_new(C.byref(h)))
        self.h = h

    def push(self, data: bytes) -> str:
        cap = 3 * (len(data) + 4)
        buf = C.create_string_buffer(cap)
        n = C.c_size_t(0)
        _check(lib().ls_stream_decoder_push(self.h, data, len(data), buf, cap, C.byref(n)))
        return buf.raw[: n.value].decode("utf-8")

    def finish(self) -> str:
        buf = C.create_string_buffer(16)
        n = C.c_size_t(0)
        _check(lib().ls_stream_decoder_finish(self.h, buf, 16, C.byref(n)))
        return buf.raw[: n.value].decode("utf-8")

    def __del__(self):
        try:
            lib().ls_stream_decoder_free(self.h)
        except Exception:
            pass


class Sampler:
    """Sampler (src/model.rs:300-366): greedy at temperature <= 0, else top-k / top-p sampling."""

    def __init__(self, temperature: float, top_k: int, top_p: float, seed: int):
        h = C.c_void_p()
        _check(lib().ls_sampler_new(temperature, top_k, top_p, seed, C.byref(h)))
        self.h = h

    @classmethod
    def greedy(cls) -> "Sampler":
        return cls(0.0, 1, 1.0, 0)

    def sample(self, logits) -> int:
        a = np.ascontiguousarray(np.asarray(logits, np.float32))
        t = np.zeros(1, np.uint32)
        _check(lib().ls_sampler_sample(self.h, a.ctypes.data_as(C.POINTER(C.c_float)), a.size, _u32(t)))
        return int(t[0])

    def __del__(self):
        try:
            lib().ls_sampler_free(self.h)
        except Exception:
            pass
