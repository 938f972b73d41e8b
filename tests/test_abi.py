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
    from qwen_mlp_amd import _lib

    # the loaded binary was built from exactly these sources (lib() refuses any other)
    assert _lib.library_source_hash() == _lib.tree_source_hash()
    assert re.fullmatch(r"[0-9a-f]{16}", _lib.tree_source_hash())
    assert lib.qmlp_forward(None, None, None, None, None, None, None, 0, 1, 256, 256, 1, None) == -6
    assert b"null" in lib.qmlp_last_error()


@pytest.mark.parametrize("rows,cols", [(16, 256), (3072, 1024), (1024, 3072), (17408, 5120), (5120, 17408)])
@pytest.mark.parametrize("fmt", ["bf16", "bfp8", "bf4"])
def test_packed_bytes_matches_layout(pkg, rows, cols, fmt):
    code = {"bfp8": pkg.FMT_BFP8, "bf4": pkg.FMT_BF4, "bf16": pkg.FMT_BF16}[fmt]
    assert pkg.lib().qmlp_packed_bytes(rows, cols, code) == obfp8.packed_bytes(rows, cols, fmt)


def test_stale_library_is_refused(pkg, tmp_path, monkeypatch):
    """A library whose stamp is not the digest of the sources beside it does not load."""
    from qwen_mlp_amd import _lib

    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "tree_source_hash", lambda: "0" * 16)
    with pytest.raises(RuntimeError, match="built from other sources"):
        _lib.lib()


def test_packed_bytes_rejects_bad_shapes(pkg):
    lib = pkg.lib()
    for rows, cols, fmt in ((15, 256, 1), (16, 255, 1), (0, 256, 0), (16, 256, 3), (16, 256, -1), (-16, 256, 0),
                            (16, 128, 2)):
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
    assert lib.qmlp_workspace_bytes(16, 5120, 17408, 2) == a  # bf4 stages the activations like bfp8
    assert lib.qmlp_workspace_bytes(16, 5120, 17408, 3) == 0


@pytest.mark.parametrize("H,I", [(5120, 17408), (1024, 3072), (5120, 8704), (256, 76800)])
@pytest.mark.parametrize("fmt", [0, 1, 2])
def test_workspace_bytes_never_shrink_as_m_grows(pkg, H, I, fmt):
    """A workspace sized for M tokens serves every call with fewer tokens: the size is
    non-decreasing in M (the split kernels' partial slots at M <= 32 can exceed what 33..~400
    tokens need otherwise, and the many-token kernels' K-split pieces need room at 2048 tokens
    but none at 2049)."""
    lib = pkg.lib()
    Ms = list(range(1, 4353)) + [6144, 8191, 8192, 8193, 16384, 65536]
    sizes = [lib.qmlp_workspace_bytes(M, H, I, fmt) for M in Ms]
    assert all(s > 0 for s in sizes)
    for (m0, s0), (m1, s1) in zip(zip(Ms, sizes), zip(Ms[1:], sizes[1:])):
        assert s1 >= s0, f"workspace shrinks from M={m0} ({s0} B) to M={m1} ({s1} B)"


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
    # activations addressed with 32-bit offsets: M * max(H, I) must stay below 2^30
    assert lib.qmlp_forward(p, p, p, p, None, big, p, 1 << 62, 65536, 256, 16384, 1, None) == -1
    assert b"2^30" in lib.qmlp_last_error()
    assert lib.qmlp_pack(p, None, 16, 256, 1, p, 1 << 20, None) == -6
    assert lib.qmlp_pack(p, p, 17, 256, 1, p, 1 << 20, None) == -1
    assert lib.qmlp_pack(p, p, 16, 256, 1, p, 10, None) == -5


def test_python_wrapper_raises_value_error(pkg):
    from qwen_mlp_amd import _lib

    with pytest.raises(ValueError):
        _lib.check(-1, "x")
    with pytest.raises(_lib.QmlpError):
        _lib.check(-4, "x")


SHAPES = [(17408, 5120), (5120, 17408), (3072, 1024), (1024, 3072), (8704, 5120), (5120, 8704), (256, 256),
          (16, 256), (65536, 256), (512, 65536), (48, 768)]
CUS = [256, 304, 80, 7, 1]


def _wg_of_step(s, S, P):
    """The stream-K kernel's closed form for the workgroup that owns step s."""
    return ((s + 1) * P - 1) // S


@pytest.mark.parametrize("rows,K", SHAPES)
def test_stream_split_covers_every_step_once(pkg, rows, K):
    """Stream-K fallback kernel: the workgroup and wave step ranges tile [0, S) exactly, no wave touches
    more tiles than the plan's LDS slots, the owner formula matches the ranges, and every tile
    shared by workgroups is the first or last tile of each (its partial slot) -- the reference's
    worker-to-pair coverage test (scripts/ci/test_fused_1d.py:71-79) for this split."""
    for cus in CUS:
        out = (ctypes.c_int * 2)()
        assert pkg.lib().qmlp_plan_stream(rows, K, cus, out) == 0
        P, maxseg = list(out)
        T, SPT = rows // 16, (K // 256) * 4
        S = T * SPT
        assert 1 <= P <= min(S, 512) and maxseg <= 4
        covered = [0] * S
        share = {}
        for w in range(P):
            s0, s1 = w * S // P, (w + 1) * S // P
            assert s1 > s0 and _wg_of_step(s0, S, P) == w and _wg_of_step(s1 - 1, S, P) == w
            for v in range(8):
                sa, sb = s0 + v * (s1 - s0) // 8, s0 + (v + 1) * (s1 - s0) // 8
                for st in range(sa, sb):
                    covered[st] += 1
                if sb > sa:
                    assert (sb - 1) // SPT - sa // SPT + 1 <= maxseg
            for t in range(s0 // SPT, (s1 - 1) // SPT + 1):
                share.setdefault(t, []).append(w)
        assert covered == [1] * S
        for t, ws in share.items():
            assert ws == list(range(_wg_of_step(t * SPT, S, P), _wg_of_step((t + 1) * SPT - 1, S, P) + 1))
            if len(ws) > 1:
                for w in ws:
                    assert t in ((w * S // P) // SPT, (((w + 1) * S // P) - 1) // SPT)


@pytest.mark.parametrize("rows,K", SHAPES)
@pytest.mark.parametrize("nmat", [1, 2])
@pytest.mark.parametrize("M", [16, 32])
def test_gemv_split_covers_every_unit_once(pkg, rows, K, nmat, M):
    """M <= 32 kernel: tile groups x K splits (split q = superblocks [q*C/S, (q+1)*C/S)) cover every
    (tile, superblock) unit once, each workgroup's waves split its rectangle exactly, no wave
    touches more than maxseg tiles, and the staged activations fit the register chunks."""
    mg = 1 if M <= 16 else 2
    for cus in CUS:
        out = (ctypes.c_int * 6)()
        rc = pkg.lib().qmlp_plan_split(rows, K, nmat, M, cus, out)
        if rc != 0:
            continue  # no split fits (K too long for the staged activations): the caller falls back
        P, G, S, KQ, Ng, maxseg = list(out)
        T, C = rows // 16, K // 256
        assert KQ == -(-C // S) and KQ * mg <= 18 and maxseg <= 12 // (nmat * mg)
        assert Ng == -(-T // G) and P == Ng * S and P <= max(cus, 1)
        covered = [[0] * C for _ in range(T)]
        for w in range(P):
            g, q = w // S, w % S
            c0, c1 = q * C // S, (q + 1) * C // S
            kq = c1 - c0
            assert kq in (KQ, KQ - 1) and kq >= 1
            Gw = min(G, T - g * G)
            U = Gw * kq
            done = 0
            for v in range(8):
                ua, ub = v * U // 8, (v + 1) * U // 8
                if ua < ub:
                    assert (ub - 1) // kq - ua // kq + 1 <= maxseg
                for u in range(ua, ub):
                    covered[g * G + u // kq][c0 + u % kq] += 1
                done += ub - ua
            assert done == U
        assert all(c == 1 for row in covered for c in row)


def test_plan_split_rejects_bad_widths(pkg):
    out = (ctypes.c_int * 6)()
    assert pkg.lib().qmlp_plan_split(17408, 5120, 2, 0, 256, out) != 0
    assert pkg.lib().qmlp_plan_split(17408, 5120, 2, 33, 256, out) != 0


def test_gemv_split_at_the_27b_shape(pkg):
    """The splits quoted for the Qwen3-27B shape on 256 CUs."""
    out = (ctypes.c_int * 6)()
    want = {(17408, 5120, 2, 16): (242, 9, 2, 10), (5120, 17408, 1, 16): (256, 5, 4, 17),
            (17408, 5120, 2, 32): (256, 17, 4, 5), (5120, 17408, 1, 32): (256, 10, 8, 9)}
    for (rows, K, nmat, M), (P, G, S, KQ) in want.items():
        assert pkg.lib().qmlp_plan_split(rows, K, nmat, M, 256, out) == 0
        assert tuple(out)[:4] == (P, G, S, KQ), (rows, K, nmat, M, tuple(out))


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


def test_bench_refuses_several_gpus():
    """bench.py measures one GPU; asking for more exits with a message and status 2 before any
    GPU work."""
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_no_kernel_waits_for_another_block():
    """Cross-block hand-offs are last-arrival only: no loop under csrc/ waits on a value in memory
    (no loop condition reads memory, no sleep, no do-while), so every kernel finishes whatever else
    holds the CUs."""
    csrc = os.path.join(os.path.dirname(HEADER), "..", "tenstorrent.blackhole-qwen3.8-27b_amd", "csrc")
    names = [n for n in os.listdir(csrc) if n.endswith((".hip", ".h"))]
    assert len(names) >= 8
    loops = 0
    for name in names:
        text = open(os.path.join(csrc, name)).read()
        for m in re.finditer(r"\b(while|for)\s*\(", text):
            depth, i = 1, m.end()
            while depth:  # the condition up to its matching parenthesis
                depth += {"(": 1, ")": -1}.get(text[i], 0)
                i += 1
            cond = text[m.end():i - 1]
            if m.group(1) == "for":  # for (init; cond; step): the condition part
                parts = cond.split(";")
                if len(parts) != 3:
                    continue
                cond = parts[1]
            loops += 1
            assert not re.search(r"load|atomic|volatile|\[|->", cond), f"{name}: loop on memory ({cond})"
        assert not re.search(r"\bdo\s*\{", text), f"{name}: do-while loop"
        assert "s_sleep" not in text, name
    assert loops > 100


def test_traffic_summary_matches_the_kernel_sources():
    """bench.py puts the committed HBM counter figures in its roofline only when they were measured
    on the current M <= 32 kernel sources; a kernel change must come with a new counter run."""
    import importlib.util

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    spec = importlib.util.spec_from_file_location("bench_for_test", os.path.join(root, "bench.py"))
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    traffic, source = bench.read_traffic("qwen3-27b-mlp-m16-bfp8")
    assert traffic is not None, source
    assert traffic["gate_up"] > 189_562_880 and traffic["down"] > 94_863_360  # at least the algorithmic bytes
