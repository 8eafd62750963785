"""Writes small synthetic safetensors checkpoints with MoE blocks in the thinker's key layout
(`{prefix}.experts.{e}.{gate,up,down}_proj.weight`, `{prefix}.shared_experts.*`), sharded like a real
checkpoint with a model.safetensors.index.json, plus unrelated tensors. Test helper only."""
import json
import os

import torch
from safetensors.torch import save_file


def expert_tensors(prefix, n_experts, hidden, inter, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    out = {}
    for e in list(range(n_experts)) + ["shared"]:
        p = f"{prefix}.shared_experts." if e == "shared" else f"{prefix}.experts.{e}."
        out[p + "gate_proj.weight"] = (torch.randn(inter, hidden, generator=g) * 0.05).to(dtype)
        out[p + "up_proj.weight"] = (torch.randn(inter, hidden, generator=g) * 0.05).to(dtype)
        out[p + "down_proj.weight"] = (torch.randn(hidden, inter, generator=g) * 0.05).to(dtype)
    return out


def write_checkpoint(root, tensors, shards=2, extra=True):
    """Spreads `tensors` over `shards` files (round robin, interleaved with unrelated tensors) and writes the
    index. Returns the directory."""
    os.makedirs(root, exist_ok=True)
    keys = sorted(tensors)
    files = [{} for _ in range(shards)]
    for i, k in enumerate(keys):
        files[i % shards][k] = tensors[k].contiguous()
    if extra:
        for s in range(shards):
            files[s][f"model.layers.{s}.input_layernorm.weight"] = torch.ones(64, dtype=torch.bfloat16)
            files[s][f"model.layers.{s}.self_attn.q_proj.weight"] = torch.zeros(8, 64, dtype=torch.float32)
    weight_map = {}
    for s, f in enumerate(files):
        name = f"model-{s + 1:05d}-of-{shards:05d}.safetensors"
        save_file(f, os.path.join(root, name), metadata={"format": "pt"})
        weight_map.update({k: name for k in f})
    with open(os.path.join(root, "model.safetensors.index.json"), "w") as fh:
        json.dump({"metadata": {}, "weight_map": weight_map}, fh)
    return root


def stacked(tensors, prefix, n_experts):
    """The reference restacking (engine.py:343-361) on the CPU: w_gu [E1, 2I, H], w_d [E1, H, I]."""
    gu, d = [], []
    for e in list(range(n_experts)) + ["shared"]:
        p = f"{prefix}.shared_experts." if e == "shared" else f"{prefix}.experts.{e}."
        gu.append(torch.cat([tensors[p + "gate_proj.weight"], tensors[p + "up_proj.weight"]]))
        d.append(tensors[p + "down_proj.weight"])
    return torch.stack(gu), torch.stack(d)
