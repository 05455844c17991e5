"""ctypes binding of the oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the CPU-baseline
leg of bench.py, always as the checker. The product package never imports this module.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")


class Fmt(C.Structure):
    _fields_ = [("bits", C.c_int32), ("group", C.c_int32)]


class Cfg(C.Structure):
    _fields_ = [
        ("format", Fmt),
        ("embed_format", Fmt),
        ("hidden", C.c_int64),
        ("inter", C.c_int64),
        ("layers", C.c_int64),
        ("heads", C.c_int64),
        ("kv_heads", C.c_int64),
        ("head_dim", C.c_int64),
        ("vocab", C.c_int64),
        ("eps", C.c_float),
        ("rope_theta", C.c_float),
    ]


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


class OrSampler(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_size_t), ("top_p", C.c_float), ("state", C.c_uint64)]


class Sampler:
    """The oracle's Sampler (src/model.rs:300-366)."""

    def __init__(self, temperature: float, top_k: int, top_p: float, seed: int):
        self.s = OrSampler()
        lib().or_sampler_init(C.byref(self.s), temperature, top_k, top_p, seed)

    def uniform(self) -> float:
        return lib().or_sampler_uniform(C.byref(self.s))

    def sample(self, logits) -> int:
        a = np.ascontiguousarray(np.asarray(logits, np.float32))
        return int(lib().or_sampler_sample(C.byref(self.s), f32(a), a.size))


class Drafter(C.Structure):
    _fields_ = [
        ("model", C.c_void_p),
        ("greedy", C.POINTER(C.c_uint32)),
        ("n_greedy", C.c_size_t),
        ("p_accept", C.c_double),
        ("seed", C.c_uint64),
        ("vocab", C.c_uint64),
    ]


def build() -> None:
    """Compile liboracle.so with its Makefile (gcc)."""
    subprocess.run(["make", "-s", "-C", HERE, "-B"], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        P, F32, U8, U32, SZ = C.c_void_p, C.POINTER(C.c_float), C.POINTER(C.c_uint8), C.POINTER(C.c_uint32), C.c_size_t
        sig = {
            "or_row_bytes": (SZ, [Fmt, SZ]),
            "or_validate": (C.c_int, [Fmt, C.POINTER(SZ), SZ]),
            "or_layer_layout": (SZ, [C.POINTER(Cfg), C.POINTER(SZ)]),
            "or_bf16_round": (C.c_float, [C.c_float]),
            "or_quantize_row": (None, [Fmt, F32, SZ, C.c_int, U8, C.POINTER(C.c_double), C.POINTER(C.c_double)]),
            "or_quantize_model": (C.c_int, [C.POINTER(Cfg), C.c_char_p, U8, U8, U8, C.c_int, C.c_int, U8, SZ, C.POINTER(SZ)]),
            "or_dot_bf16": (C.c_float, [U8, F32, SZ]),
            "or_dot_q8": (C.c_float, [U8, F32, SZ, SZ]),
            "or_dot_q4": (C.c_float, [U8, F32, SZ, SZ]),
            "or_dequant_row": (None, [Fmt, U8, F32, SZ]),
            "or_rms_norm_bf16": (None, [F32, SZ, U8, SZ, C.c_float, F32]),
            "or_rms_norm_f32": (None, [F32, F32, SZ, C.c_float, F32]),
            "or_rope_inplace": (None, [F32, F32, SZ, SZ]),
            "or_softmax_inplace": (None, [F32, SZ]),
            "or_silu": (C.c_float, [C.c_float]),
            "or_argmax": (C.c_uint32, [F32, SZ]),
            "or_sampler_init": (None, [C.POINTER(OrSampler), C.c_float, SZ, C.c_float, C.c_uint64]),
            "or_sampler_uniform": (C.c_float, [C.POINTER(OrSampler)]),
            "or_sampler_sample": (C.c_uint32, [C.POINTER(OrSampler), F32, SZ]),
            "or_pool_new": (P, [C.c_int]),
            "or_pool_free": (None, [P]),
            "or_matmul": (None, [P, Fmt, U8, SZ, SZ, F32, SZ, F32]),
            "or_model_new": (P, [C.POINTER(Cfg), U8, U8, U8, C.c_int, SZ]),
            "or_model_free": (None, [P]),
            "or_model_pos": (SZ, [P]),
            "or_model_max_ctx": (SZ, [P]),
            "or_model_reset": (None, [P]),
            "or_model_truncate": (C.c_int, [P, SZ]),
            "or_model_forward": (C.c_int, [P, U32, SZ, F32]),
            "or_model_forward_multi": (C.c_int, [P, U32, SZ, SZ, F32]),
            "or_last_error": (C.c_char_p, []),
            "or_scripted_draft": (C.c_uint32, [C.POINTER(Drafter), SZ]),
            "or_speculative_greedy": (C.c_int, [P, C.POINTER(Drafter), U32, SZ, SZ, SZ, U32, SZ, U32, C.POINTER(SZ), C.POINTER(SpecStats)]),
            "or_plain_greedy": (C.c_int, [P, U32, SZ, SZ, U32, SZ, U32, C.POINTER(SZ)]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def fmt(bits: int, group: int = 0) -> Fmt:
    return Fmt(bits, group)


def ptr(a: np.ndarray, ctype):
    return a.ctypes.data_as(C.POINTER(ctype))


def u8(a):
    return ptr(a, C.c_uint8)


def f32(a):
    return ptr(a, C.c_float)


def u32(a):
    return ptr(a, C.c_uint32)


class OracleError(RuntimeError):
    pass


def _check(rc: int):
    if rc != 0:
        raise OracleError(lib().or_last_error().decode())


def cfg_struct(cfg: dict) -> Cfg:
    f = cfg["format"]
    e = cfg["embed_format"]
    return Cfg(
        Fmt(*f),
        Fmt(*e),
        cfg["hidden"],
        cfg["inter"],
        cfg["layers"],
        cfg["heads"],
        cfg["kv_heads"],
        cfg["head_dim"],
        cfg["vocab"],
        cfg["eps"],
        cfg["rope_theta"],
    )


def row_bytes(f, cols: int) -> int:
    return lib().or_row_bytes(Fmt(*f), cols)


class OracleModel:
    """The reference's `Model` (src/model.rs:58-140) over resident weights."""

    def __init__(self, cfg: dict, layers: np.ndarray, embed: np.ndarray, norm_raw: np.ndarray, threads: int = 0, max_ctx: int = 1024):
        self.cfg = cfg
        self._keep = (np.ascontiguousarray(layers, np.uint8), np.ascontiguousarray(embed, np.uint8), np.ascontiguousarray(norm_raw, np.uint8))
        self._c = cfg_struct(cfg)
        threads = threads or os.cpu_count() or 1
        self.threads = threads
        self.h = lib().or_model_new(C.byref(self._c), u8(self._keep[0]), u8(self._keep[1]), u8(self._keep[2]), threads, max_ctx)

    def close(self):
        if self.h:
            lib().or_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def vocab(self) -> int:
        return self.cfg["vocab"]

    def pos(self) -> int:
        return lib().or_model_pos(self.h)

    def max_ctx(self) -> int:
        return lib().or_model_max_ctx(self.h)

    def reset(self):
        lib().or_model_reset(self.h)

    def truncate(self, pos: int):
        _check(lib().or_model_truncate(self.h, pos))

    def forward(self, tokens) -> np.ndarray:
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32))
        out = np.zeros(self.vocab, np.float32)
        _check(lib().or_model_forward(self.h, u32(t), len(t), f32(out)))
        return out

    def forward_multi(self, tokens, n: int) -> np.ndarray:
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32))
        out = np.zeros((max(n, 1), self.vocab), np.float32)
        _check(lib().or_model_forward_multi(self.h, u32(t), len(t), n, f32(out)))
        return out


def scripted_drafter(greedy, p_accept: float, seed: int, vocab: int):
    g = np.ascontiguousarray(np.asarray(greedy, dtype=np.uint32))
    d = Drafter(None, u32(g), len(g), p_accept, seed, vocab)
    d._keep = g
    return d


def model_drafter(model: OracleModel):
    d = Drafter(model.h, None, 0, 0.0, 0, model.vocab)
    d._keep = model
    return d


def speculative_greedy(target: OracleModel, drafter: Drafter, prompt, max_new: int, k: int, eos=()):
    p = np.ascontiguousarray(np.asarray(prompt, dtype=np.uint32))
    e = np.ascontiguousarray(np.asarray(list(eos) or [0], dtype=np.uint32))
    out = np.zeros(max(max_new, 1), np.uint32)
    n = C.c_size_t(0)
    st = SpecStats()
    rc = lib().or_speculative_greedy(target.h, C.byref(drafter), u32(p), len(p), max_new, k, u32(e), len(eos), u32(out), C.byref(n), C.byref(st))
    _check(rc)
    stats = {f: getattr(st, f) for f, _ in SpecStats._fields_}
    return out[: n.value].tolist(), stats


def plain_greedy(m: OracleModel, prompt, max_new: int, eos=()):
    p = np.ascontiguousarray(np.asarray(prompt, dtype=np.uint32))
    e = np.ascontiguousarray(np.asarray(list(eos) or [0], dtype=np.uint32))
    out = np.zeros(max(max_new, 1), np.uint32)
    n = C.c_size_t(0)
    _check(lib().or_plain_greedy(m.h, u32(p), len(p), max_new, u32(e), len(eos), u32(out), C.byref(n)))
    return out[: n.value].tolist()


def quantize_model(qcfg: dict, qconfig_text: str, layers, embed, norm_raw, clip: bool = True, threads: int = 0) -> bytes:
    c = cfg_struct(qcfg)
    n = C.c_size_t(0)
    layers = np.ascontiguousarray(layers, np.uint8)
    embed = np.ascontiguousarray(embed, np.uint8)
    norm_raw = np.ascontiguousarray(norm_raw, np.uint8)
    txt = qconfig_text.encode()
    _check(lib().or_quantize_model(C.byref(c), txt, u8(layers), u8(embed), u8(norm_raw), int(clip), threads or os.cpu_count(), None, 0, C.byref(n)))
    out = np.zeros(n.value, np.uint8)
    _check(lib().or_quantize_model(C.byref(c), txt, u8(layers), u8(embed), u8(norm_raw), int(clip), threads or os.cpu_count(), u8(out), n.value, C.byref(n)))
    return out.tobytes()
