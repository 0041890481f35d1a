"""Writes tests/golden/hf_goldens.npz: input/output vectors of Hugging Face's Llama modules on
small synthetic fp16 inputs, computed on the CPU.

The reference anchors its kernel tests to Hugging Face outputs (ref: tests/test_rmsnorm.cu,
tests/test_rope.cu, tests/test_swiglu.cu, tests/test_embedding.cu read prompt_XX_*.f16 files
written by scripts/make_*_reference.py from the real model). Those fixtures are not in the
reference checkout and the model weights are not available offline, so this script applies the
same Hugging Face modules (transformers' LlamaRMSNorm, LlamaRotaryEmbedding +
apply_rotary_pos_emb, the llama3 rope-init routine, SiLU, nn.Embedding) to seeded synthetic
inputs of the reference's shapes. The vectors pin the oracle's rounding conventions
independently of the oracle's own code. It also runs LlamaForCausalLM in float32 over a prompt
of a small Llama-3 shape with seeded random weights (tests/_helpers.py: TINY, tiny_weights), the
whole-model anchor the reference takes from Hugging Face logits of the real model (ref:
tests/test_generate_batched.cu:44-53); the fixture holds the token ids, the logits and a hash of
the weights. Run with the versions recorded in the file (transformers 5.15.0, torch 2.10.0).

    python tests/golden/make_hf_goldens.py
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np
import torch
import transformers
from transformers import LlamaConfig
from transformers.modeling_rope_utils import ROPE_INIT_FUNCTIONS
from transformers.models.llama.modeling_llama import (LlamaRMSNorm, LlamaRotaryEmbedding,
                                                      apply_rotary_pos_emb)

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "hf_goldens.npz")
SEED = 0x5EED0001
# The whole-model case: tiny_weights(LLAMA_WEIGHT_SEED, embed_std=0.5), LLAMA_T token ids drawn
# with default_rng(LLAMA_IDS_SEED).integers(0, vocab, LLAMA_T).
LLAMA_WEIGHT_SEED, LLAMA_IDS_SEED, LLAMA_T = 0x5EED0110, 0x5EED0111, 40


def weights_digest(w: dict) -> str:
    """sha256 over the weights' names and fp16 bits in sorted-name order."""
    h = hashlib.sha256()
    for k in sorted(w):
        h.update(k.encode())
        h.update(np.ascontiguousarray(w[k]).view(np.uint16).tobytes())
    return h.hexdigest()


def tiny_llama_logits(c: dict, w: dict, ids) -> np.ndarray:
    """Logits [T, vocab] of transformers' LlamaForCausalLM in float32 (eager attention, tied
    embeddings, llama3 rope scaling) with the weights `w` (Hugging Face names), over one prompt."""
    cfg = LlamaConfig(
        vocab_size=c["vocab"], hidden_size=c["hidden"], intermediate_size=c["inter"],
        num_hidden_layers=c["n_layers"], num_attention_heads=c["n_heads"],
        num_key_value_heads=c["n_kv_heads"], head_dim=c["head_dim"],
        max_position_embeddings=131072, rms_norm_eps=c["eps"], tie_word_embeddings=True,
        rope_parameters={"rope_type": "llama3", "rope_theta": c["rope_theta"],
                         "factor": c["rope_factor"], "low_freq_factor": c["rope_low_freq_factor"],
                         "high_freq_factor": c["rope_high_freq_factor"],
                         "original_max_position_embeddings": int(c["rope_original_max_pos"])},
        attn_implementation="eager")
    model = transformers.LlamaForCausalLM(cfg).float().eval()
    state = {k: torch.from_numpy(v.astype(np.float32)) for k, v in w.items()}
    state["lm_head.weight"] = state["model.embed_tokens.weight"]
    missing, unexpected = model.load_state_dict(state, strict=False)
    assert not unexpected and all("rotary" in m for m in missing), (missing, unexpected)
    with torch.no_grad():
        return model(torch.tensor(ids, dtype=torch.long)[None]).logits[0].numpy()


def llama32_1b_config() -> LlamaConfig:
    # Llama-3.2-1B shape constants (ref: engine/layer.h:6-9, engine/model.cu:20).
    return LlamaConfig(
        vocab_size=128256, hidden_size=2048, intermediate_size=8192, num_hidden_layers=16,
        num_attention_heads=32, num_key_value_heads=8, head_dim=64,
        max_position_embeddings=131072, rms_norm_eps=1e-5,
        rope_parameters={"rope_type": "llama3", "rope_theta": 500000.0, "factor": 32.0,
                         "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                         "original_max_position_embeddings": 8192})


def main() -> None:
    torch.manual_seed(0)
    rng = np.random.default_rng(SEED)
    cfg = llama32_1b_config()
    out = {}

    # llama3 rotation speeds
    inv_freq, attn_scale = ROPE_INIT_FUNCTIONS["llama3"](cfg, torch.device("cpu"))
    assert attn_scale == 1.0
    out["inv_freq"] = inv_freq.to(torch.float32).numpy()

    # RMSNorm, fp16 in / weight / out
    rows, hidden = 8, 2048
    x = rng.standard_normal((rows, hidden), dtype=np.float32).astype(np.float16)
    x[1] *= np.float16(8.0)             # a row with large values
    x[2] *= np.float16(1e-3)            # a row of small values
    x[3] = np.float16(0.5)              # a constant row
    w = (1.0 + 0.1 * rng.standard_normal(hidden, dtype=np.float32)).astype(np.float16)
    norm = LlamaRMSNorm(hidden, eps=cfg.rms_norm_eps).half()
    with torch.no_grad():
        norm.weight.copy_(torch.from_numpy(w))
        y = norm(torch.from_numpy(x))
    out.update(rms_x=x.view(np.uint16), rms_w=w.view(np.uint16),
               rms_out=y.numpy().view(np.uint16))

    # RoPE on Q [T, 32, 64] and K [T, 8, 64]
    T, nh, nkv, hd = 16, 32, 8, 64
    pos = np.array([0, 1, 2, 7, 100, 401, 2047, 8191, 8192, 12345, 65535, 65536, 100000, 131071,
                    rng.integers(0, 131072), rng.integers(0, 131072)], dtype=np.int32)
    q = rng.standard_normal((T, nh, hd), dtype=np.float32).astype(np.float16)
    k = rng.standard_normal((T, nkv, hd), dtype=np.float32).astype(np.float16)
    rot = LlamaRotaryEmbedding(cfg)
    qt = torch.from_numpy(q).transpose(0, 1).unsqueeze(0)   # [1, heads, T, hd]
    kt = torch.from_numpy(k).transpose(0, 1).unsqueeze(0)
    with torch.no_grad():
        cos, sin = rot(qt, torch.from_numpy(pos).long().unsqueeze(0))
        qo, ko = apply_rotary_pos_emb(qt, kt, cos, sin)
    out.update(rope_pos=pos, rope_q_in=q.view(np.uint16), rope_k_in=k.view(np.uint16),
               rope_q_out=qo.squeeze(0).transpose(0, 1).contiguous().numpy().view(np.uint16),
               rope_k_out=ko.squeeze(0).transpose(0, 1).contiguous().numpy().view(np.uint16))

    # SwiGLU: silu(gate) * up, with special gate values in the first row
    g = rng.standard_normal((4, 2048), dtype=np.float32).astype(np.float16)
    u = rng.standard_normal((4, 2048), dtype=np.float32).astype(np.float16)
    specials = np.array([0.0, -0.0, 6e-8, -6e-8, 1e-4, -1e-4, 8.0, -8.0, 16.0, -16.0, 20.0,
                         -20.0, 88.0, -88.0, 1000.0, -1000.0, 65504.0, -65504.0],
                        dtype=np.float32).astype(np.float16)
    g[0, :specials.size] = specials
    u[0, :specials.size] = np.float16(1.5)
    g[1] *= np.float16(6.0)
    with torch.no_grad():
        s = torch.nn.functional.silu(torch.from_numpy(g)) * torch.from_numpy(u)
    out.update(swiglu_gate=g.view(np.uint16), swiglu_up=u.view(np.uint16),
               swiglu_out=s.numpy().view(np.uint16))

    # Embedding gather
    vocab, eh, n = 64, 256, 32
    table = (0.02 * rng.standard_normal((vocab, eh), dtype=np.float32)).astype(np.float16)
    ids = rng.integers(0, vocab, n).astype(np.int32)
    ids[:3] = [0, vocab - 1, ids[5]]
    emb = torch.nn.Embedding(vocab, eh).half()
    with torch.no_grad():
        emb.weight.copy_(torch.from_numpy(table))
        e = emb(torch.from_numpy(ids).long())
    out.update(emb_table=table.view(np.uint16), emb_ids=ids, emb_out=e.numpy().view(np.uint16))

    # Whole model: LlamaForCausalLM over a prompt, small Llama-3 shape, seeded random weights
    sys.path.insert(0, os.path.dirname(HERE))
    from _helpers import TINY, tiny_weights
    w_tiny = tiny_weights(LLAMA_WEIGHT_SEED, embed_std=0.5)
    llama_ids = np.random.default_rng(LLAMA_IDS_SEED).integers(0, TINY["vocab"], LLAMA_T)
    out.update(llama_ids=llama_ids.astype(np.int32),
               llama_logits=tiny_llama_logits(TINY, w_tiny, llama_ids).astype(np.float32))

    meta = {"seed": SEED, "transformers": transformers.__version__, "torch": torch.__version__,
            "eps": cfg.rms_norm_eps, "rope": cfg.rope_parameters,
            "llama": {"config": TINY, "weight_seed": LLAMA_WEIGHT_SEED, "embed_std": 0.5,
                      "ids_seed": LLAMA_IDS_SEED, "T": LLAMA_T,
                      "weights_sha256": weights_digest(w_tiny)}}
    out["meta_json"] = np.frombuffer(json.dumps(meta).encode(), dtype=np.uint8)
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: " + ", ".join(f"{k}{list(v.shape)}" for k, v in out.items()))


if __name__ == "__main__":
    main()
