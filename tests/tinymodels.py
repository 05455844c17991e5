"""Synthetic test models, restating the reference's test fixtures (tests/common/mod.rs:9-135).

The reference writes a tiny Qwen2 model (hidden 64, 4 heads / 2 KV heads, inter 128, 3 layers,
vocab 600) to a `.safetensors` file with an LCG; the "grid" variant puts every matrix exactly
on a quantization grid. Here the same values are produced in memory: the layer blocks in the
slot order of src/weights.rs:158-171 (alphabetical, as in the file), the embedding table and
the final norm, as raw bf16 bytes.
"""
from __future__ import annotations

import numpy as np

HIDDEN, HEADS, KV_HEADS, INTER, LAYERS, VOCAB = 64, 4, 2, 128, 3, 600

TINY_CONFIG_TEXT = (
    '{"model_type":"qwen2","hidden_act":"silu","tie_word_embeddings":true,"hidden_size":64,\n'
    '"num_attention_heads":4,"num_key_value_heads":2,"intermediate_size":128,\n'
    '"num_hidden_layers":3,"vocab_size":600,"rms_norm_eps":1e-6,"rope_theta":10000.0,\n'
    '"max_position_embeddings":512}'
)

# Slot order inside a layer block (src/weights.rs:158-186).
SLOTS = [
    "input_layernorm.weight",
    "mlp.down_proj.weight",
    "mlp.gate_proj.weight",
    "mlp.up_proj.weight",
    "post_attention_layernorm.weight",
    "self_attn.k_proj.bias",
    "self_attn.k_proj.weight",
    "self_attn.o_proj.weight",
    "self_attn.q_proj.bias",
    "self_attn.q_proj.weight",
    "self_attn.v_proj.bias",
    "self_attn.v_proj.weight",
]

M64 = (1 << 64) - 1


class Lcg:
    """tests/common/mod.rs:17-24: state*6364136223846793005 + 1442695040888963407, top 31 bits
    to f32 (round to nearest), / 2^31 * 2 - 1, all in f32."""

    def __init__(self, seed: int):
        self.s = seed & M64

    def next(self) -> np.float32:
        self.s = (self.s * 6364136223846793005 + 1442695040888963407) & M64
        v = np.float32(self.s >> 33) / np.float32(2147483648.0)
        return np.float32(v * np.float32(2.0) - np.float32(1.0))

    def take(self, n: int) -> np.ndarray:
        out = np.empty(n, np.float32)
        for i in range(n):
            out[i] = self.next()
        return out


def bf16_trunc_bytes(vals: np.ndarray) -> np.ndarray:
    """tests/common/mod.rs:26-28: the top 16 bits of each f32 (truncation), little endian."""
    u = np.ascontiguousarray(vals, np.float32).view(np.uint32) >> 16
    return u.astype("<u2").view(np.uint8)


def bf16_bytes_to_f32(b: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(b, np.uint8).view("<u2").astype(np.uint32) << 16
    return u.view(np.float32)


def _grid(rng: Lcg, rows: int, cols: int, bits: int, group: int) -> np.ndarray:
    """tests/common/mod.rs:44-62"""
    qmax, scale = (127, np.float32(2.0**-10)) if bits == 8 else (7, np.float32(2.0**-6))
    vals = np.empty(rows * cols, np.float32)
    n = 0
    for _ in range(rows):
        for g in range(cols // group):
            for j in range(group):
                v = np.float32(rng.next() * np.float32(qmax + 0.5))
                code = int(_round_half_away(v))
                code = max(-qmax, min(qmax, code))
                if j == (g * 7) % group:
                    code = -qmax if rng.next() < 0 else qmax
                vals[n] = np.float32(code) * scale
                n += 1
    return bf16_trunc_bytes(vals)


def _round_half_away(v: np.float32) -> float:
    """Rust f32::round: half away from zero."""
    f = float(v)
    return np.floor(f + 0.5) if f >= 0 else -np.floor(-f + 0.5)


def _shapes(hidden, heads, kv_heads, inter):
    hd = hidden // heads
    kv = kv_heads * hd
    return {
        "input_layernorm.weight": [hidden],
        "mlp.down_proj.weight": [hidden, inter],
        "mlp.gate_proj.weight": [inter, hidden],
        "mlp.up_proj.weight": [inter, hidden],
        "post_attention_layernorm.weight": [hidden],
        "self_attn.k_proj.bias": [kv],
        "self_attn.k_proj.weight": [kv, hidden],
        "self_attn.o_proj.weight": [hidden, hidden],
        "self_attn.q_proj.bias": [hidden],
        "self_attn.q_proj.weight": [hidden, hidden],
        "self_attn.v_proj.bias": [kv],
        "self_attn.v_proj.weight": [kv, hidden],
    }


def tiny_cfg(fmt=(16, 0), embed_fmt=None) -> dict:
    return {
        "format": tuple(fmt),
        "embed_format": tuple(embed_fmt or fmt),
        "hidden": HIDDEN,
        "inter": INTER,
        "layers": LAYERS,
        "heads": HEADS,
        "kv_heads": KV_HEADS,
        "head_dim": HIDDEN // HEADS,
        "vocab": VOCAB,
        "eps": 1e-6,
        "rope_theta": 10000.0,
    }


def write_tiny_model(seed: int, grid=None) -> dict:
    """tests/common/mod.rs:64-135. `grid` = ((bits, group), (embed_bits, embed_group)) or None.

    Returns {cfg, config_text, layers, embed, norm} with bf16 bytes; the draw order follows the
    alphabetical tensor order of the file (embedding, then each layer's 12 tensors, then the
    final norm)."""
    rng = Lcg(seed)
    shapes = _shapes(HIDDEN, HEADS, KV_HEADS, INTER)

    def make(name, shape):
        n = int(np.prod(shape))
        is_norm = name.endswith("layernorm.weight") or name == "model.norm.weight"
        if is_norm:
            v = rng.take(n)
            return bf16_trunc_bytes(np.float32(1.0) + np.float32(0.1) * v)
        if grid is not None and len(shape) == 2:
            bits, group = grid[1] if name == "model.embed_tokens.weight" else grid[0]
            return _grid(rng, shape[0], shape[1], bits, group)
        v = rng.take(n)
        return bf16_trunc_bytes(np.float32(0.15) * v)

    embed = make("model.embed_tokens.weight", [VOCAB, HIDDEN])
    blocks = []
    for _ in range(LAYERS):
        parts = [make(s, shapes[s]) for s in SLOTS]
        blocks.append(np.concatenate(parts))
    norm = make("model.norm.weight", [HIDDEN])
    return {
        "cfg": tiny_cfg(),
        "config_text": TINY_CONFIG_TEXT,
        "layers": np.concatenate(blocks),
        "embed": embed,
        "norm": norm,
    }


def inject_quant(config_text: str, bits: int, group: int, embed=None) -> str:
    """src/quant.rs:137-145"""
    end = config_text.rfind("}")
    head = config_text[:end].rstrip()
    extra = f',"embed_bits":{embed[0]},"embed_group":{embed[1]}' if embed else ""
    return f'{head},"layerstream_quant":{{"bits":{bits},"group":{group}{extra}}}}}'


def split_lsq(img: bytes, cfg: dict) -> dict:
    """Split a `.lsq` image (src/weights.rs:340-358, 389-424) into its parts."""
    import json
    import struct

    assert img[:4] == b"LSQ1"
    (jl,) = struct.unpack("<I", img[4:8])
    hdr = json.loads(img[8 : 8 + jl].decode())
    lb, eb, nb = hdr["layer_bytes"], hdr["embed_bytes"], hdr["norm_bytes"]
    a = 8 + jl
    arr = np.frombuffer(img, np.uint8)
    layers = arr[a : a + cfg["layers"] * lb]
    embed = arr[a + cfg["layers"] * lb : a + cfg["layers"] * lb + eb]
    norm = arr[a + cfg["layers"] * lb + eb : a + cfg["layers"] * lb + eb + nb]
    assert a + cfg["layers"] * lb + eb + nb == len(img)
    return {"header": hdr, "layers": layers, "embed": embed, "norm": norm}


def quantized(model: dict, body, embed, clip=True) -> dict:
    """Quantize a tiny bf16 model with the oracle's quantizer (src/quant.rs:158-251)."""
    import oracle_py as O  # noqa: WPS433  (tests put oracle/ on sys.path)

    text = inject_quant(model["config_text"], body[0], body[1], None if tuple(embed) == tuple(body) else embed)
    qcfg = dict(model["cfg"], format=tuple(body), embed_format=tuple(embed))
    img = O.quantize_model(qcfg, text, model["layers"], model["embed"], model["norm"], clip=clip)
    parts = split_lsq(img, qcfg)
    return {"cfg": qcfg, "config_text": text, "lsq": img, **{k: parts[k] for k in ("layers", "embed", "norm")}}
