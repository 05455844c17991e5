"""Write tests/golden/hf_tiny_logits.npz: logits of an independent Qwen2 implementation
(Hugging Face transformers' Qwen2ForCausalLM, float32, eager attention) on the reference's
tiny synthetic model (tests/common/mod.rs:64-135, seeds below).

This pins the model semantics of the oracle (GQA head mapping, rotate-half RoPE, q/k/v bias,
RMSNorm placement, SwiGLU, tied head) against a second implementation, independently of the
restatement. It builds the model from a config object and our own weights: nothing is
downloaded. Run: python tests/golden/make_hf_golden.py
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import tinymodels as T  # noqa: E402

SEEDS = [11, 12]
TOKENS = [5, 17, 301, 42, 599, 0, 7, 33, 120, 250, 3, 77]


def hf_logits(model: dict, tokens) -> np.ndarray:
    from transformers import Qwen2Config, Qwen2ForCausalLM

    cfg = Qwen2Config(
        vocab_size=T.VOCAB,
        hidden_size=T.HIDDEN,
        intermediate_size=T.INTER,
        num_hidden_layers=T.LAYERS,
        num_attention_heads=T.HEADS,
        num_key_value_heads=T.KV_HEADS,
        hidden_act="silu",
        max_position_embeddings=512,
        rms_norm_eps=1e-6,
        rope_theta=10000.0,
        tie_word_embeddings=True,
        use_sliding_window=False,
        attn_implementation="eager",
    )
    torch.manual_seed(0)
    m = Qwen2ForCausalLM(cfg).float().eval()
    f = T.bf16_bytes_to_f32
    shapes = T._shapes(T.HIDDEN, T.HEADS, T.KV_HEADS, T.INTER)
    sd = {"model.embed_tokens.weight": f(model["embed"]).reshape(T.VOCAB, T.HIDDEN), "model.norm.weight": f(model["norm"])}
    total = len(model["layers"]) // T.LAYERS
    for l in range(T.LAYERS):
        blk = model["layers"][l * total : (l + 1) * total]
        off = 0
        for s in T.SLOTS:
            n = int(np.prod(shapes[s]))
            sd[f"model.layers.{l}.{s}"] = f(blk[off : off + 2 * n]).reshape(shapes[s])
            off += 2 * n
    sd = {k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in sd.items()}
    sd["lm_head.weight"] = sd["model.embed_tokens.weight"]
    missing, unexpected = m.load_state_dict(sd, strict=False)
    assert not unexpected, unexpected
    assert all("rotary" in k for k in missing), missing
    with torch.no_grad():
        out = m(torch.tensor([tokens]), use_cache=False).logits[0].float().numpy()
    return out


def main():
    out = {"tokens": np.array(TOKENS, np.uint32), "seeds": np.array(SEEDS)}
    for s in SEEDS:
        out[f"logits_seed{s}"] = hf_logits(T.write_tiny_model(s), TOKENS).astype(np.float32)
    np.savez_compressed(os.path.join(HERE, "hf_tiny_logits.npz"), **out)
    print("wrote", {k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main()
