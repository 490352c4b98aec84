"""Checkpoint packer (q4rdna.pack_model) and the streaming sidecar writer.

The packer reads a local Hugging Face checkpoint the way the reference's
packer does (source/pack_q4rdna_sidecar.py:100-161) and quantizes on the GPU;
its file must equal the sidecar the oracle builds from the same bf16 weights
with the native packer's search (oracle pinned byte-exact to
source/q4rdna_sidecar_pack.cpp in test_oracle.py)."""
import json
import os

import numpy as np
import pytest

import oracle as O
from q4rdna import sidecar
from q4rdna.pack_model import HF_TO_GGML, scoped_tensors

# A miniature Qwen3 shape set: hidden 256, 2 KV heads of 32, FFN 512.
MINI = {"self_attn.q_proj.weight": (256, 256), "self_attn.k_proj.weight": (64, 256),
        "self_attn.v_proj.weight": (64, 256), "self_attn.o_proj.weight": (256, 256),
        "mlp.gate_proj.weight": (512, 256), "mlp.up_proj.weight": (512, 256),
        "mlp.down_proj.weight": (256, 512)}


def mini_checkpoint(path, layers=2):
    """Two bf16 shards plus the index; returns {hf name: bf16 bits}."""
    import torch
    from safetensors.torch import save_file
    bits = {}
    shards = {"model-00001-of-00002.safetensors": {}, "model-00002-of-00002.safetensors": {}}
    weight_map = {}
    for layer in range(layers):
        for i, (suffix, (rows, cols)) in enumerate(MINI.items()):
            name = f"model.layers.{layer}.{suffix}"
            w = O.gaussian_weights(rows, cols, 1000 * layer + i)
            b, _ = O.bf16_round(w)
            bits[name] = b
            shard = list(shards)[(layer + i) % 2]
            shards[shard][name] = torch.from_numpy(b.view(np.int16).copy()).view(torch.bfloat16)
            weight_map[name] = shard
    shards[list(shards)[0]]["model.embed_tokens.weight"] = torch.zeros(8, 256, dtype=torch.bfloat16)
    weight_map["model.embed_tokens.weight"] = list(shards)[0]
    for shard, tensors in shards.items():
        save_file(tensors, os.path.join(path, shard))
    with open(os.path.join(path, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": weight_map}, f)
    return bits


def expected_image(bits, layers, max_tensors=0):
    tensors = []
    for layer in range(layers):
        for suffix, ggml in HF_TO_GGML:
            b = bits[f"model.layers.{layer}.{suffix}"]
            rows, cols = b.shape
            w = (b.astype(np.uint32) << 16).view(np.float32)
            tensors.append((f"blk.{layer}.{ggml}", rows, cols, O.pack(w, O.ALGO_SIDECAR)))
    if max_tensors:
        tensors = tensors[:max_tensors]
    return O.build_sidecar(tensors)


def test_streaming_writer_matches_oracle_image(tmp_path):
    rng = np.random.default_rng(3)
    tensors = [("blk.0.attn_q.weight", 64, 128), ("blk.0.attn_k.weight", 32, 64), ("blk.0.ffn_down.weight", 96, 192)]
    data = [rng.integers(0, 256, r * c * 34 // 64, dtype=np.uint8) for _, r, c in tensors]
    path = tmp_path / "s.q4rdna"
    with sidecar.SidecarWriter(path, tensors) as w:
        for (name, _, _), d in zip(tensors, data):
            w.add(name, d)
    want = O.build_sidecar([(n, r, c, d) for (n, r, c), d in zip(tensors, data)])
    assert path.read_bytes() == want
    assert O.validate_sidecar(want) == len(tensors)


def test_streaming_writer_rejects_misuse(tmp_path):
    tensors = [("a.weight", 32, 64), ("b.weight", 32, 64)]
    size = 32 * 64 * 34 // 64
    w = sidecar.SidecarWriter(tmp_path / "x", tensors)
    with pytest.raises(ValueError):
        w.add("b.weight", bytes(size))  # out of order
    with pytest.raises(ValueError):
        w.add("a.weight", bytes(size - 1))  # wrong size
    w.add("a.weight", bytes(size))
    with pytest.raises(ValueError):
        w.close()  # b.weight missing


def test_scoped_tensors_order_and_missing_names():
    weight_map = {f"model.layers.{l}.{s}": f"shard{l}" for l in range(3) for s, _ in HF_TO_GGML}
    got = scoped_tensors(weight_map, 3)
    assert [g for _, g, _ in got[:7]] == [f"blk.0.{g}" for _, g in HF_TO_GGML]
    assert got[7][1] == "blk.1.attn_q.weight" and got[-1][2] == "shard2"
    assert len(scoped_tensors(weight_map, 3, max_tensors=5)) == 5
    del weight_map["model.layers.1.mlp.up_proj.weight"]
    with pytest.raises(KeyError):
        scoped_tensors(weight_map, 3)


@pytest.mark.gpu
@pytest.mark.parametrize("max_tensors", [0, 9])
def test_pack_model_matches_oracle_sidecar(cuda, tmp_path, max_tensors):
    from q4rdna.pack_model import pack_model
    bits = mini_checkpoint(str(tmp_path))
    out = tmp_path / "out" / "mini.q4rdna"
    size = pack_model(str(tmp_path), str(out), layers=2, max_tensors=max_tensors)
    got = out.read_bytes()
    assert len(got) == size
    assert got == expected_image(bits, 2, max_tensors)
