"""On-disk cache of packed MLP weights (load time only).

The reference caches converted device tensors next to the checkpoint (``cache_file_name`` in
``docker/qwen-c2-graft/graft/mlp.py:64-66,155-162``).  Here a cache file holds one packed matrix:
a 256-byte JSON header (magic, shape, format, byte count, max row norm, flushed groups) followed by
the packed bytes exactly as ``qmlp_pack`` wrote them.  Loading memory-maps the file and copies it to
the GPU; nothing in the file is executed.
"""
import json
import os

import numpy as np
import torch

HEADER_BYTES = 256
MAGIC = "qwen-mlp-packed-v1"


def cache_file(directory, name, fmt):
    return os.path.join(str(directory), f"mlp.{name}.weight.{fmt}.qmlp")


def save(path, pw):
    from . import _lib

    expected = _lib.lib().qmlp_packed_bytes(pw.rows, pw.cols, pw.fmt_code)
    if pw.buf.numel() != expected:
        raise ValueError("packed buffer has the wrong size")
    header = json.dumps({"magic": MAGIC, "rows": pw.rows, "cols": pw.cols, "fmt": pw.fmt, "bytes": expected,
                         "max_row_norm": pw.max_row_norm, "flushed_groups": pw.flushed_groups}).encode()
    if len(header) >= HEADER_BYTES:
        raise ValueError("header too long")
    os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
    tmp = path + ".tmp"
    with open(tmp, "wb") as f:
        f.write(header.ljust(HEADER_BYTES, b" "))
        f.write(pw.buf.cpu().numpy().tobytes())
    os.replace(tmp, path)


def load(path, device):
    """Returns a PackedWeight, or None when the file is not a valid cache entry."""
    from . import _lib
    from .mlp import PackedWeight

    with open(path, "rb") as f:
        raw = f.read(HEADER_BYTES)
    try:
        meta = json.loads(raw.decode().strip())
    except (UnicodeDecodeError, json.JSONDecodeError):
        return None
    if meta.get("magic") != MAGIC or meta.get("fmt") not in _lib.FORMATS:
        return None
    rows, cols, fmt = int(meta["rows"]), int(meta["cols"]), meta["fmt"]
    nbytes = _lib.lib().qmlp_packed_bytes(rows, cols, _lib.FORMATS[fmt])
    if nbytes != int(meta["bytes"]) or os.path.getsize(path) != HEADER_BYTES + nbytes:
        return None
    data = np.memmap(path, dtype=np.uint8, mode="r", offset=HEADER_BYTES, shape=(nbytes,))
    buf = torch.from_numpy(np.array(data)).to(device)
    return PackedWeight(buf, rows, cols, fmt, float(meta["max_row_norm"]), int(meta["flushed_groups"]))
