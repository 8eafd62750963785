"""CPU checks of the checkpoint reader: safetensors headers against the safetensors library's own reader,
the index, and the expert key map (no GPU work)."""
import os

import pytest
import torch
from safetensors import safe_open

import expert_load as EL
from workloads import expert_tensors, write_checkpoint


def test_read_header_matches_safetensors_library(tmp_path):
    t = expert_tensors("model.layers.1.mlp", 3, 64, 32, seed=1)
    t["odd.f32"] = torch.randn(5, 7)
    root = write_checkpoint(str(tmp_path / "ck"), t, shards=2)
    idx = EL.checkpoint_index(root)
    assert set(t) <= set(idx)
    for path in set(idx.values()):
        hdr = EL.read_header(path)
        data = open(path, "rb").read()
        with safe_open(path, framework="pt") as f:
            assert sorted(hdr) == sorted(f.keys())
            for k in f.keys():
                ref = f.get_tensor(k)
                dt, shape, a, b = hdr[k]
                assert shape == tuple(ref.shape)
                assert dt == {torch.bfloat16: "BF16", torch.float32: "F32"}[ref.dtype]
                got = torch.frombuffer(bytearray(data[a:b]), dtype=ref.dtype).reshape(shape)
                assert torch.equal(got, ref)


def test_single_file_index(tmp_path):
    from safetensors.torch import save_file
    save_file({"a": torch.zeros(2, 2)}, str(tmp_path / "model.safetensors"))
    assert EL.checkpoint_index(str(tmp_path)) == {"a": str(tmp_path / "model.safetensors")}
    with pytest.raises(FileNotFoundError):
        EL.checkpoint_index(str(tmp_path / "nothing"))


def test_expert_items_order_slots_and_missing_keys():
    idx = {f"p.experts.{e}.{n}_proj.weight": "f" for e in range(4) for n in ("gate", "up", "down")}
    idx.update({f"p.shared_experts.{n}_proj.weight": "f" for n in ("gate", "up", "down")})
    items = EL.expert_items(idx, "p", 4)
    assert len(items) == 15
    assert items[-3:] == [("p.shared_experts.gate_proj.weight", 0, 4), ("p.shared_experts.up_proj.weight", 1, 4),
                          ("p.shared_experts.down_proj.weight", 2, 4)]
    assert items[3] == ("p.experts.1.gate_proj.weight", 0, 1)
    assert len(EL.expert_items(idx, "p", 4, shared=False)) == 12
    del idx["p.experts.2.up_proj.weight"]
    with pytest.raises(ValueError, match="experts.2.up_proj"):
        EL.expert_items(idx, "p", 4)
