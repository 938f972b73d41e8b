"""Offline packer: HF safetensors checkpoint -> per-layer packed MLP weight caches.

The reference converts each layer's HF tensors into device block-float tiles when the model loads
and caches the converted tensors next to the checkpoint (``cache_file_name``,
``docker/qwen-c2-graft/graft/mlp.py:64-66,155-162``; ``layer.py:178-182``).  This tool does that
conversion ahead of time for every layer:

* ``<out>/layer_<i>/mlp.<name>.weight.<fmt>.qmlp`` -- the packed device layout with its header
  (``weight_cache``); ``load_mlp_weights(..., tensor_cache_path=<out>/layer_<i>)`` and
  ``Qwen36MLP(..., tensor_cache_path=...)`` memory-map it instead of quantising again;
  (``--format bf4`` writes gate/up as bf4 and down as bfp8, the reference's mixed layout);
* with ``--planar`` (block-float formats) also the canonical planar form, ``<name>.q.npy`` (int8
  ``[rows, cols]`` signed mantissas) and ``<name>.e8.npy`` (uint8 ``[rows, cols/16]`` group
  exponents, scale ``2^(e8 - 127)``), plain ``.npy`` files that ``numpy.load(mmap_mode="r")`` maps.

Quantisation and packing run on the GPU with the library's own kernels, so the caches are
bit-identical to what a load-time conversion produces.

Usage (from the repository root)::

    python tenstorrent.blackhole-qwen3.8-27b_amd/pack_checkpoint.py --checkpoint DIR --out DIR
        [--format bfp8|bf4|bf16] [--layers 0-63] [--planar]
"""
import argparse
import glob
import json
import os
import re
import sys

import numpy as np
import torch

_KEY = re.compile(r"(?:^|\.)layers\.(\d+)\.mlp\.(gate_proj|up_proj|down_proj)\.weight$")


def checkpoint_files(directory):
    """The safetensors files of a checkpoint directory (sharded via the index, or all of them)."""
    index = os.path.join(directory, "model.safetensors.index.json")
    if os.path.exists(index):
        with open(index) as f:
            files = sorted(set(json.load(f)["weight_map"].values()))
        return [os.path.join(directory, name) for name in files]
    files = sorted(glob.glob(os.path.join(directory, "*.safetensors")))
    if not files:
        raise FileNotFoundError(f"no .safetensors files in {directory}")
    return files


def mlp_keys(files):
    """{layer: {name: (file, key)}} for every MLP weight in the checkpoint."""
    from safetensors import safe_open

    found = {}
    for path in files:
        with safe_open(path, framework="pt") as f:
            for key in f.keys():
                m = _KEY.search(key)
                if m:
                    found.setdefault(int(m.group(1)), {})[m.group(2)] = (path, key)
    return found


def parse_layers(spec, available):
    if spec is None:
        return sorted(available)
    out = set()
    for part in spec.split(","):
        if "-" in part:
            lo, hi = part.split("-")
            out.update(range(int(lo), int(hi) + 1))
        else:
            out.add(int(part))
    missing = sorted(out - set(available))
    if missing:
        raise ValueError(f"layers {missing} have no MLP weights in the checkpoint")
    return sorted(out)


def pack_layer(entries, out_dir, fmt, device, planar=False):
    """Packs one layer's three matrices into ``out_dir``; returns the cache file paths."""
    from safetensors import safe_open

    from . import mlp, weight_cache

    gu_fmt, down_fmt = mlp.matrix_formats(fmt)
    if planar and fmt == "bf16":
        raise ValueError("--planar writes block-float mantissa/exponent planes (bfp8 or bf4)")
    written = []
    for name in ("gate_proj", "up_proj", "down_proj"):
        mfmt = down_fmt if name == "down_proj" else gu_fmt
        if name not in entries:
            raise ValueError(f"missing {name}.weight")
        path, key = entries[name]
        with safe_open(path, framework="pt") as f:
            w = f.get_tensor(key)
        w = w.to(device=device, dtype=torch.bfloat16).contiguous()
        pw = mlp.pack_weight(w, mfmt)
        cache = weight_cache.cache_file(out_dir, name, mfmt)
        weight_cache.save(cache, pw)
        written.append(cache)
        if planar:
            q, e8 = mlp.quantize_bf4(w) if mfmt == "bf4" else mlp.quantize_bfp8(w)
            np.save(os.path.join(out_dir, f"{name}.q.npy"), q.cpu().numpy())
            np.save(os.path.join(out_dir, f"{name}.e8.npy"), e8.cpu().numpy())
        del w, pw
    return written


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--checkpoint", required=True, help="directory holding the HF *.safetensors files")
    ap.add_argument("--out", required=True, help="output directory (one layer_<i> subdirectory per layer)")
    ap.add_argument("--format", default="bfp8", choices=("bfp8", "bf4", "bf16"))
    ap.add_argument("--layers", default=None, help="e.g. 0-63 or 0,5,7 (default: every layer found)")
    ap.add_argument("--planar", action="store_true", help="also write the canonical block-float planes as .npy")
    ap.add_argument("--device", default="cuda:0")
    args = ap.parse_args(argv)
    device = torch.device(args.device)
    if device.type != "cuda" or not torch.cuda.is_available():
        print("pack_checkpoint: the packer runs the library's GPU kernels; no GPU is available", file=sys.stderr)
        return 2
    found = mlp_keys(checkpoint_files(args.checkpoint))
    layers = parse_layers(args.layers, found)
    for i in layers:
        out_dir = os.path.join(args.out, f"layer_{i}")
        os.makedirs(out_dir, exist_ok=True)
        pack_layer(found[i], out_dir, args.format, device, planar=args.planar)
        print(f"layer {i}: packed into {out_dir}", flush=True)
    return 0


if __name__ == "__main__":
    # Run as a script: load the package (it registers as qwen_mlp_amd) and call its copy of main.
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    import __graft_entry__

    __graft_entry__.load_package()
    from qwen_mlp_amd import pack_checkpoint

    sys.exit(pack_checkpoint.main())
