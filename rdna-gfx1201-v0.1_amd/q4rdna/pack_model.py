"""Pack a local Hugging Face Qwen3 checkpoint into a Q4_RDNA sidecar.

The command line, tensor selection and file follow the reference packer
(source/pack_q4rdna_sidecar.py:25-33,100-161): the seven linear weights of
each decoder layer, in layer-major order, named by their ggml names, read
from the shards that model.safetensors.index.json lists.  Quantization runs
on the GPU through q4rdna_pack with the sidecar scale search, which is
bit-identical to the reference's native packer
(source/q4rdna_sidecar_pack.cpp:126-179).  The reference's Python packer
runs the same search with torch float32 reductions and an exact fp16 decode,
so the two write different bytes for a few groups: where a scale and its
negation tie exactly (a group with symmetric extremes), where two adjacent
fp16 scales tie to float32 rounding (the summation orders rank them
differently), where a scale is an fp16 subnormal (the native search decodes
it at half its value), where the Python search overflows to an infinite
scale, and in the sign of a zero scale.  On N(0, 0.02) bf16 weights the
first two kinds are 24 of 262,144 groups.

    python -m q4rdna.pack_model --model DIR --output FILE [--layers N] [--max-tensors K]
"""
from __future__ import annotations

import argparse
import json
import sys
import time
from contextlib import ExitStack
from pathlib import Path

from .sidecar import SidecarWriter

# Hugging Face suffix -> ggml suffix, one decoder layer, in file order.
HF_TO_GGML = (
    ("self_attn.q_proj.weight", "attn_q.weight"),
    ("self_attn.k_proj.weight", "attn_k.weight"),
    ("self_attn.v_proj.weight", "attn_v.weight"),
    ("self_attn.o_proj.weight", "attn_output.weight"),
    ("mlp.gate_proj.weight", "ffn_gate.weight"),
    ("mlp.up_proj.weight", "ffn_up.weight"),
    ("mlp.down_proj.weight", "ffn_down.weight"),
)


def scoped_tensors(weight_map: dict, layers: int, max_tensors: int = 0):
    """[(hf name, ggml name, shard file)] in the sidecar's order."""
    out = []
    for layer in range(layers):
        for hf_suffix, ggml_suffix in HF_TO_GGML:
            hf = f"model.layers.{layer}.{hf_suffix}"
            if hf not in weight_map:
                raise KeyError(f"{hf} is not in the checkpoint index")
            out.append((hf, f"blk.{layer}.{ggml_suffix}", weight_map[hf]))
    return out[:max_tensors] if max_tensors else out


def pack_model(model_dir, output, layers: int = 36, max_tensors: int = 0, device: int = 0, log=None) -> int:
    """Write the sidecar of `model_dir` to `output`; returns the file size."""
    import torch
    from safetensors import safe_open

    from . import api

    model_dir = Path(model_dir)
    index = json.loads((model_dir / "model.safetensors.index.json").read_text())
    tensors = scoped_tensors(index["weight_map"], layers, max_tensors)
    dev = torch.device("cuda", device)
    started = time.monotonic()
    with ExitStack() as stack:
        shards = {name: stack.enter_context(safe_open(str(model_dir / name), framework="pt", device="cpu"))
                  for name in sorted({shard for _, _, shard in tensors})}
        shapes = []
        for hf, ggml, shard in tensors:
            rows, cols = shards[shard].get_slice(hf).get_shape()
            shapes.append((ggml, int(rows), int(cols)))
        Path(output).parent.mkdir(parents=True, exist_ok=True)
        with SidecarWriter(output, shapes) as writer:
            for number, ((hf, ggml, shard), (_, rows, cols)) in enumerate(zip(tensors, shapes), 1):
                t0 = time.monotonic()
                w = shards[shard].get_tensor(hf).to(dev).to(torch.float32).contiguous()
                tiles = api.pack(w)
                writer.add(ggml, tiles.cpu().numpy())
                del w, tiles
                if log is not None:
                    log(f"[{number:3d}/{len(tensors)}] {ggml:31s} {rows:5d}x{cols:5d} "
                        f"{time.monotonic() - t0:6.2f}s total {time.monotonic() - started:7.1f}s")
            size = writer.end
    return size


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--model", required=True, help="local Hugging Face checkpoint directory")
    ap.add_argument("--output", required=True)
    ap.add_argument("--layers", type=int, default=36)
    ap.add_argument("--max-tensors", type=int, default=0)
    ap.add_argument("--device", type=int, default=0)
    args = ap.parse_args(argv)
    size = pack_model(args.model, args.output, args.layers, args.max_tensors, args.device,
                      log=lambda m: print(m, flush=True))
    print(f"wrote {args.output} ({size} bytes)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
