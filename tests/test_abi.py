"""The C ABI library without a GPU: it loads, exports every declared symbol, sizes buffers like the
oracle's layout, rejects bad arguments before touching a device, and its work split covers every
unit exactly once (cf. the reference's worker-to-pair coverage tests,
scripts/ci/test_fused_1d.py:71-79)."""
import ctypes
import os
import re

import pytest

from oracle import bfp8 as obfp8

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "qwen_mlp.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(qmlp_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported(pkg):
    lib = pkg.lib()
    names = _declared()
    assert len(names) >= 12
    for name in names:
        assert hasattr(lib, name), name
    from qwen_mlp_amd import _lib

    assert sorted(_lib.SIGNATURES) == names


def test_version_and_error_strings(pkg):
    lib = pkg.lib()
    assert b"gfx950" in lib.qmlp_version()
    assert lib.qmlp_forward(None, None, None, None, None, None, None, 0, 1, 256, 256, 1, None) == -6
    assert b"null" in lib.qmlp_last_error()


@pytest.mark.parametrize("rows,cols", [(16, 256), (3072, 1024), (1024, 3072), (17408, 5120), (5120, 17408)])
@pytest.mark.parametrize("fmt", ["bf16", "bfp8"])
def test_packed_bytes_matches_layout(pkg, rows, cols, fmt):
    code = pkg.FMT_BFP8 if fmt == "bfp8" else pkg.FMT_BF16
    assert pkg.lib().qmlp_packed_bytes(rows, cols, code) == obfp8.packed_bytes(rows, cols, fmt)


def test_packed_bytes_rejects_bad_shapes(pkg):
    lib = pkg.lib()
    for rows, cols, fmt in ((15, 256, 1), (16, 255, 1), (0, 256, 0), (16, 256, 2), (-16, 256, 0)):
        assert lib.qmlp_packed_bytes(rows, cols, fmt) == 0


def test_workspace_bytes(pkg):
    lib = pkg.lib()
    a = lib.qmlp_workspace_bytes(16, 5120, 17408, 1)
    b = lib.qmlp_workspace_bytes(16, 5120, 17408, 0)
    assert a > b > 16 * 17408 * 2  # bfp8 also holds the scaled fp16 activations
    assert a % 256 == 0
    assert lib.qmlp_workspace_bytes(0, 5120, 17408, 1) == 0
    assert lib.qmlp_workspace_bytes(16, 5000, 17408, 1) == 0
    assert lib.qmlp_workspace_bytes(2048, 5120, 17408, 1) > lib.qmlp_workspace_bytes(32, 5120, 17408, 1)


def test_forward_argument_errors_need_no_gpu(pkg):
    lib = pkg.lib()
    p = ctypes.c_void_p(1 << 20)          # never dereferenced: validation fails first
    q = ctypes.c_void_p((1 << 20) + 8)    # misaligned
    ws = lib.qmlp_workspace_bytes(4, 256, 512, 1)
    big = ctypes.c_void_p(1 << 30)
    assert lib.qmlp_forward(p, p, p, p, None, big, p, ws, 4, 256, 512, 7, None) == -3
    assert lib.qmlp_forward(p, p, p, p, None, big, p, ws, 0, 256, 512, 1, None) == -1
    assert lib.qmlp_forward(p, p, p, p, None, big, p, ws, 4, 250, 512, 1, None) == -1
    assert lib.qmlp_forward(q, p, p, p, None, big, p, ws, 4, 256, 512, 1, None) == -2
    assert lib.qmlp_forward(p, p, p, p, None, p, p, ws, 4, 256, 512, 1, None) == -1   # out aliases x
    assert lib.qmlp_forward(p, p, p, p, None, big, p, ws - 256, 4, 256, 512, 1, None) == -5
    assert b"workspace" in lib.qmlp_last_error()
    assert lib.qmlp_pack(p, None, 16, 256, 1, p, 1 << 20, None) == -6
    assert lib.qmlp_pack(p, p, 17, 256, 1, p, 1 << 20, None) == -1
    assert lib.qmlp_pack(p, p, 16, 256, 1, p, 10, None) == -5


def test_python_wrapper_raises_value_error(pkg):
    from qwen_mlp_amd import _lib

    with pytest.raises(ValueError):
        _lib.check(-1, "x")
    with pytest.raises(_lib.QmlpError):
        _lib.check(-4, "x")


def _plan(pkg, rows, K, cus):
    out = (ctypes.c_int * 4)()
    assert pkg.lib().qmlp_plan_skinny(rows, K, 16, cus, out) == 0
    return list(out)


def _simulate(P, NW, T, C, aligned, SPU):
    """Python restatement of the kernel's range arithmetic."""
    U = T * C
    covered = [0] * U
    tiles_of_wg = []
    for w in range(P):
        if aligned:
            a, b = (w * T // P) * C, ((w + 1) * T // P) * C
        else:
            a, b = w * U // P, (w + 1) * U // P
        tiles_of_wg.append(set(range(a // C, (b - 1) // C + 1)) if a < b else set())
        for v in range(NW):
            sa = a * SPU + v * (b - a) * SPU // NW
            sb = a * SPU + (v + 1) * (b - a) * SPU // NW
            if sa < sb:
                spt = SPU * C
                assert (sb - 1) // spt - sa // spt + 1 <= 2, "a wave may touch at most two tiles"
            for st in range(sa, sb):
                if st % SPU == 0:
                    covered[st // SPU] += 1
        # the kernel's closed form for the owner of a unit agrees with the ranges
        for u in range(a, b):
            owner = ((u // C + 1) * P - 1) // T if aligned else ((u + 1) * P - 1) // U
            assert owner == w
    return covered, tiles_of_wg


@pytest.mark.parametrize("rows,K,cus", [(17408, 5120, 256), (5120, 17408, 256), (3072, 1024, 256),
                                        (1024, 3072, 256), (17408, 5120, 304), (8704, 5120, 256),
                                        (5120, 8704, 256), (256, 256, 256), (16, 256, 256), (5120, 17408, 7)])
def test_skinny_split_covers_every_unit_once(pkg, rows, K, cus):
    P, NW, U, aligned = _plan(pkg, rows, K, cus)
    T, C = rows // 16, K // 256
    assert U == T * C and 1 <= P <= min(T, 512)
    for SPU in (1, 2):
        for al in (0, 1):
            covered, tiles = _simulate(P, NW, T, C, al, SPU)
            assert covered == [1] * U
            owners = [sum(t in s for s in tiles) for t in range(T)]
            assert max(owners) <= 2 and min(owners) >= 1
            if al:
                assert max(owners) == 1


def test_pack_checkpoint_finds_mlp_weights(tmp_path, pkg):
    """The offline packer's checkpoint scan (CPU only): sharded index, key pattern, layer ranges."""
    import json

    import torch
    from safetensors.torch import save_file

    from qwen_mlp_amd import pack_checkpoint as pc

    def t():
        return torch.zeros((32, 256), dtype=torch.bfloat16)

    save_file({"model.layers.0.mlp.gate_proj.weight": t(), "model.layers.0.mlp.up_proj.weight": t(),
               "model.layers.0.self_attn.q_proj.weight": t()}, str(tmp_path / "a.safetensors"))
    save_file({"model.layers.0.mlp.down_proj.weight": t(), "model.layers.3.mlp.gate_proj.weight": t()},
              str(tmp_path / "b.safetensors"))
    with open(tmp_path / "model.safetensors.index.json", "w") as f:
        json.dump({"weight_map": {"x": "a.safetensors", "y": "b.safetensors"}}, f)
    files = pc.checkpoint_files(str(tmp_path))
    assert [p.split("/")[-1] for p in files] == ["a.safetensors", "b.safetensors"]
    found = pc.mlp_keys(files)
    assert sorted(found) == [0, 3] and sorted(found[0]) == ["down_proj", "gate_proj", "up_proj"]
    assert pc.parse_layers("0", found) == [0] and pc.parse_layers(None, found) == [0, 3]
    with pytest.raises(ValueError):
        pc.parse_layers("0-2", found)
