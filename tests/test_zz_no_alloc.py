"""qmlp_forward_noalloc (the forward without a workspace argument, for callers that cannot allocate)
against qmlp_forward_ex with a caller-owned workspace, through the C ABI.

The two entry points run the same kernels on the same plan, so the outputs must be bit-identical.
Each case makes two no-allocation calls in a row, the second with fewer tokens, so the second runs
on the scratch contents the first left behind.  A call whose workspace does not fit the scratch
array must fail with QMLP_E_WORKSPACE and leave its output untouched.
"""
import pytest

pytestmark = pytest.mark.gpu

H27, I27 = 5120, 17408


def _noalloc(lib, _lib, x, w, residual, out, flags, stream):
    M, H = x.shape
    return lib.qmlp_forward_noalloc(_lib.ptr(x), _lib.ptr(w.w1.buf), _lib.ptr(w.w3.buf), _lib.ptr(w.w2.buf),
                                    _lib.ptr(residual), _lib.ptr(out), M, H, w.intermediate, w.w1.fmt_code, flags,
                                    stream)


def _with_workspace(lib, _lib, x, w, residual, out, flags, stream, pkg):
    M, H = x.shape
    ws = pkg.new_workspace(M, H, w.intermediate, w.fmt, x.device)
    rc = lib.qmlp_forward_ex(_lib.ptr(x), _lib.ptr(w.w1.buf), _lib.ptr(w.w3.buf), _lib.ptr(w.w2.buf),
                             _lib.ptr(residual), _lib.ptr(out), _lib.ptr(ws), ws.numel(), M, H, w.intermediate,
                             w.w1.fmt_code, flags, stream)
    return rc


@pytest.mark.parametrize("H,I,fmt,widths", [
    (H27, I27, "bfp8", (32, 16)),
    (H27, I27, "bf4", (16, 1)),
    (1024, 3072, "bf16", (32, 7)),
])
def test_noalloc_matches_workspace_entry(pkg, cuda, H, I, fmt, widths):
    import torch
    from qwen_mlp_amd import _lib, workloads

    lib = pkg.lib()
    stream = _lib.stream_handle()
    sd = workloads.state_dict(H, I, layer=3, device=cuda)
    w = pkg.load_mlp_weights(cuda, sd, weight_format=fmt)
    for M in widths:
        for f32 in (False, True):
            print(f"case noalloc {fmt} H={H} I={I} M={M} out={'fp32' if f32 else 'bf16'}", flush=True)
            x = workloads.activations(M, H, seed=5100 + M, device=cuda)
            res = workloads.activations(M, H, seed=5200 + M, device=cuda)
            dt = torch.float32 if f32 else torch.bfloat16
            flags = _lib.OUT_F32 if f32 else 0
            out_a = torch.full((M, H), float("nan"), dtype=dt, device=cuda)
            out_b = torch.full((M, H), float("nan"), dtype=dt, device=cuda)
            rc = _noalloc(lib, _lib, x, w, res, out_a, flags, stream)
            assert rc == 0, _lib.last_error()
            rc = _with_workspace(lib, _lib, x, w, res, out_b, flags, stream, pkg)
            assert rc == 0, _lib.last_error()
            torch.cuda.synchronize()
            assert bool(torch.isfinite(out_a).all())
            assert torch.equal(out_a, out_b), f"{fmt} M={M}: no-allocation output differs"


def test_noalloc_rejects_calls_beyond_the_scratch(pkg, cuda):
    import torch
    from qwen_mlp_amd import _lib, workloads

    lib = pkg.lib()
    M = 2048
    assert lib.qmlp_workspace_bytes(M, H27, I27, _lib.FMT_BFP8) > _lib.SCRATCH_BYTES
    assert lib.qmlp_workspace_bytes(32, H27, I27, _lib.FMT_BFP8) <= _lib.SCRATCH_BYTES
    sd = workloads.state_dict(1024, 3072, layer=0, device=cuda)
    w = pkg.load_mlp_weights(cuda, sd, weight_format="bfp8")
    # the packed weights are only read after the size check, so the small layer's buffers serve
    x = torch.zeros((M, H27), dtype=torch.bfloat16, device=cuda)
    out = torch.full((M, H27), 7.0, dtype=torch.bfloat16, device=cuda)
    rc = lib.qmlp_forward_noalloc(_lib.ptr(x), _lib.ptr(w.w1.buf), _lib.ptr(w.w3.buf), _lib.ptr(w.w2.buf), None,
                                  _lib.ptr(out), M, H27, I27, _lib.FMT_BFP8, 0, _lib.stream_handle())
    assert rc == _lib.E_WORKSPACE
    assert "scratch" in _lib.last_error()
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
    rc = lib.qmlp_forward_noalloc(None, None, None, None, None, None, 16, 5000, I27, 1, 0, None)
    assert rc == _lib.E_NULL
    x16 = torch.zeros((16, 1024), dtype=torch.bfloat16, device=cuda)
    o16 = torch.zeros((16, 1024), dtype=torch.bfloat16, device=cuda)
    rc = lib.qmlp_forward_noalloc(_lib.ptr(x16), _lib.ptr(w.w1.buf), _lib.ptr(w.w3.buf), _lib.ptr(w.w2.buf), None,
                                  _lib.ptr(o16), 16, 1000, 3072, 1, 0, _lib.stream_handle())
    assert rc == _lib.E_SHAPE
    rc = lib.qmlp_forward_noalloc(_lib.ptr(x16), _lib.ptr(w.w1.buf), _lib.ptr(w.w3.buf), _lib.ptr(w.w2.buf), None,
                                  _lib.ptr(o16), 16, 1024, 3072, 9, 0, _lib.stream_handle())
    assert rc == _lib.E_FORMAT


def test_noalloc_captured_in_a_graph(pkg, cuda):
    """After an eager first call on the device, no-allocation calls captured in a HIP graph replay
    correctly: every replay (new inputs, eager work in between) equals the workspace entry point."""
    import torch
    from qwen_mlp_amd import _lib, workloads

    lib = pkg.lib()
    H, I, M = 1024, 3072, 16
    w = pkg.load_mlp_weights(cuda, workloads.state_dict(H, I, layer=6, device=cuda), weight_format="bfp8")
    x = workloads.activations(M, H, seed=1, device=cuda)
    out = torch.empty_like(x)
    assert _noalloc(lib, _lib, x, w, x, out, 0, _lib.stream_handle()) == 0, _lib.last_error()  # eager first call
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        rc = _noalloc(lib, _lib, x, w, x, out, 0, _lib.stream_handle(s))
    assert rc == 0, _lib.last_error()
    for seed in range(4):
        new_x = workloads.activations(M, H, seed=400 + seed, device=cuda)
        x.copy_(new_x)
        g.replay()
        torch.cuda.synchronize()
        ref = torch.empty_like(x)
        assert _with_workspace(lib, _lib, new_x, w, new_x, ref, 0, _lib.stream_handle(), pkg) == 0
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {seed} differs from the workspace entry point"


def test_noalloc_first_call_under_capture_is_refused(pkg, cuda):
    """In a fresh process, a first no-allocation call made while a graph captures is refused with
    QMLP_E_LAUNCH (the address lookup must run eagerly); an eager call then succeeds."""
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    code = f"""
import sys
sys.path.insert(0, {root!r})
import torch
import __graft_entry__
pkg = __graft_entry__.load_package()
from qwen_mlp_amd import _lib, workloads
lib = pkg.lib()
dev = torch.device("cuda:0")
w = pkg.load_mlp_weights(dev, workloads.state_dict(1024, 3072, layer=6, device=dev), weight_format="bfp8")
x = workloads.activations(16, 1024, seed=1, device=dev)
out = torch.empty_like(x)
args = lambda st: (_lib.ptr(x), _lib.ptr(w.w1.buf), _lib.ptr(w.w3.buf), _lib.ptr(w.w2.buf), _lib.ptr(x),
                   _lib.ptr(out), 16, 1024, 3072, w.w1.fmt_code, 0, st)
torch.cuda.synchronize()
s = torch.cuda.Stream()
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g, stream=s):
    rc = lib.qmlp_forward_noalloc(*args(_lib.stream_handle(s)))
    msg = _lib.last_error()
rc2 = lib.qmlp_forward_noalloc(*args(_lib.stream_handle()))
torch.cuda.synchronize()
print("RESULT", rc, rc2, msg, flush=True)
"""
    res = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    line = [l for l in res.stdout.splitlines() if l.startswith("RESULT")]
    assert res.returncode == 0 and line, res.stdout + res.stderr
    _, rc, rc2, msg = line[0].split(" ", 3)
    from qwen_mlp_amd import _lib

    assert int(rc) == _lib.E_LAUNCH and "outside graph capture" in msg
    assert int(rc2) == 0
