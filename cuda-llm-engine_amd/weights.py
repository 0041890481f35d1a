"""Weight files and synthetic weights for the decode-step engine.

The file format is the reference's: ``weights.bin`` holds the fp16 tensors back to back in
sorted-name order, ``index.tsv`` one line per tensor, ``name<TAB>offset<TAB>nbytes<TAB>d0,d1``,
and ``index.json`` the same as a list of records (ref: scripts/export_for_cpp.py:14-24,
scripts/make_index_tsv.py:4-7; read by engine/util.h:29-50). Tensor names are Hugging Face's
(ref: engine/layer.cu:13-27, engine/model.cu:12-15); the lm head is the embedding matrix.

There is no network here, so no real checkpoint: the tests and the bench use seeded random
weights of the model's shapes.
"""
from __future__ import annotations

import json
import os

import numpy as np
import torch

LAYER_TENSORS = (
    ("attn_norm", "input_layernorm.weight"),
    ("wq", "self_attn.q_proj.weight"),
    ("wk", "self_attn.k_proj.weight"),
    ("wv", "self_attn.v_proj.weight"),
    ("wo", "self_attn.o_proj.weight"),
    ("mlp_norm", "post_attention_layernorm.weight"),
    ("w_gate", "mlp.gate_proj.weight"),
    ("w_up", "mlp.up_proj.weight"),
    ("w_down", "mlp.down_proj.weight"),
)


def tensor_shapes(cfg) -> dict:
    """Hugging Face name -> shape of every tensor the engine reads."""
    c = cfg if isinstance(cfg, dict) else cfg.as_dict()
    H, I, V = c["hidden"], c["inter"], c["vocab"]
    qdim, kvdim = c["n_heads"] * c["head_dim"], c["n_kv_heads"] * c["head_dim"]
    per = {"attn_norm": (H,), "wq": (qdim, H), "wk": (kvdim, H), "wv": (kvdim, H),
           "wo": (H, qdim), "mlp_norm": (H,), "w_gate": (I, H), "w_up": (I, H),
           "w_down": (H, I)}
    out = {"model.embed_tokens.weight": (V, H), "model.norm.weight": (H,)}
    for l in range(c["n_layers"]):
        for key, suffix in LAYER_TENSORS:
            out[f"model.layers.{l}.{suffix}"] = per[key]
    return out


def random_weights(cfg, seed: int, device="cpu", std: float = 0.02,
                   embed_std: float = 0.02) -> dict:
    """Seeded synthetic weights: projections ~N(0, std), the embedding ~N(0, embed_std), norm
    weights ~N(1, 0.1). Returns Hugging Face name -> fp16 torch tensor on `device`."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    out = {}
    for name, shape in tensor_shapes(cfg).items():
        if name.endswith("norm.weight") or name.endswith("layernorm.weight"):
            t = 1.0 + 0.1 * torch.randn(shape, generator=g, device=device)
        else:
            s = embed_std if name == "model.embed_tokens.weight" else std
            t = s * torch.randn(shape, generator=g, device=device)
        out[name] = t.to(torch.float16).contiguous()
    return out


def engine_layers(tensors: dict, cfg) -> tuple:
    """(embed, final_norm, [per-layer dict keyed by llmk.LayerWeights.NAMES]) for
    Engine.set_weights."""
    c = cfg if isinstance(cfg, dict) else cfg.as_dict()
    layers = []
    for l in range(c["n_layers"]):
        layers.append({key: tensors[f"model.layers.{l}.{suffix}"] for key, suffix in LAYER_TENSORS})
    return tensors["model.embed_tokens.weight"], tensors["model.norm.weight"], layers


def write_weights_dir(path: str, tensors: dict) -> None:
    """Writes weights.bin, index.tsv and index.json in the reference's format."""
    os.makedirs(path, exist_ok=True)
    index, offset = [], 0
    with open(os.path.join(path, "weights.bin"), "wb") as f:
        for name in sorted(tensors):
            t = tensors[name]
            a = t.detach().cpu().numpy() if isinstance(t, torch.Tensor) else np.asarray(t)
            b = np.ascontiguousarray(a.astype(np.float16)).tobytes()
            f.write(b)
            index.append({"name": name, "shape": list(a.shape), "dtype": "f16",
                          "offset": offset, "nbytes": len(b)})
            offset += len(b)
    with open(os.path.join(path, "index.json"), "w") as f:
        json.dump(index, f, indent=1)
    with open(os.path.join(path, "index.tsv"), "w") as f:
        for t in index:
            f.write(f"{t['name']}\t{t['offset']}\t{t['nbytes']}\t"
                    f"{','.join(map(str, t['shape']))}\n")


def read_weights_dir(path: str) -> dict:
    """name -> numpy float16 array, from index.tsv + weights.bin (memory-mapped)."""
    data = np.memmap(os.path.join(path, "weights.bin"), dtype=np.uint8, mode="r")
    out = {}
    with open(os.path.join(path, "index.tsv")) as f:
        for line in f:
            parts = line.rstrip("\n").split("\t")
            if len(parts) != 4:
                continue
            name, off, nb, shape = parts[0], int(parts[1]), int(parts[2]), parts[3]
            dims = tuple(int(d) for d in shape.split(",") if d)
            out[name] = np.frombuffer(data[off:off + nb], dtype=np.float16).reshape(dims)
    return out
