"""GPU parity: the HIP path through the C ABI against the CPU oracle on the same seeded inputs.

Integer work (quantisation, packing, unpacking, dequantisation) must be bit-exact.  The MLP output
must satisfy max|out - oracle| <= 1e-2 * RMS(oracle), the oracle being the fp32 SwiGLU on the
identically dequantised weights (scripts/ci/mlp-sweep.py:121-126, layer.py:357)."""
import numpy as np
import pytest

from oracle import bf16 as obf16
from oracle import bfp8 as obfp8
from oracle import mlp as omlp

pytestmark = pytest.mark.gpu

from parity_helpers import TOL, bits as _bits, check as _check, check_bf16 as _check_bf16  # noqa: E402
from parity_helpers import host_weights as _host_weights, oracle as _oracle  # noqa: E402


# ---------------------------------------------------------------- load-time kernels (bit-exact)


def test_quantize_bit_exact(pkg, cuda):
    import torch
    from qwen_mlp_amd import workloads

    w = workloads.weight(512, 5120, seed=77, device=cuda)
    edge = np.array([[0] * 16, [0x7F7F] + [1] * 15, [1, 0x8002] + [0] * 14, [0x3F80] * 15 + [0xBF81]], np.uint16)
    edge_words = np.tile(edge.reshape(1, 64), (16, 4))  # 16 rows x 256 cols
    scales = torch.tensor([1e-30, 1e-3, 1.0, 3e4], device=cuda).repeat_interleave(128).view(512, 1)
    wide = (torch.randn((512, 5120), device=cuda, generator=torch.Generator(cuda).manual_seed(3)) * scales)
    for mat in (w, wide.to(torch.bfloat16)):
        q, e8 = pkg.quantize_bfp8(mat)
        qo, eo = obfp8.quantize(_bits(mat))
        assert np.array_equal(q.cpu().numpy(), qo)
        assert np.array_equal(e8.cpu().numpy(), eo)
    ew = torch.from_numpy(edge_words.view(np.int16)).to(cuda).view(torch.bfloat16).contiguous()
    q, e8 = pkg.quantize_bfp8(ew)
    qo, eo = obfp8.quantize(edge_words)
    assert np.array_equal(q.cpu().numpy(), qo) and np.array_equal(e8.cpu().numpy(), eo)


def test_quantize_rejects_non_finite(pkg, cuda):
    import torch

    w = torch.zeros((16, 256), dtype=torch.bfloat16, device=cuda)
    w[3, 17] = float("inf")
    with pytest.raises(ValueError):
        pkg.quantize_bfp8(w)


@pytest.mark.parametrize("rows,cols", [(48, 768), (3072, 1024), (1024, 3072)])
def test_pack_matches_oracle_layout(pkg, cuda, rows, cols):
    from qwen_mlp_amd import workloads

    w = workloads.weight(rows, cols, seed=rows + cols, device=cuda)
    wb = _bits(w)
    # bfp8
    q, e8 = pkg.quantize_bfp8(w)
    pw = pkg.pack_canonical_bfp8(q, e8)
    qo, eo = obfp8.quantize(wb)
    tiles, rowexp, flushed = obfp8.pack_tiles(qo, eo)
    buf = pw.buf.cpu().numpy()
    assert np.array_equal(buf[: tiles.size], tiles)
    assert np.array_equal(buf[tiles.size: tiles.size + rows * 4].view(np.int32), rowexp)
    assert pw.flushed_groups == flushed == 0
    norms = obfp8.row_norms(obfp8.dequantize(qo, eo))
    assert abs(pw.max_row_norm - norms.max()) <= 1e-9 * norms.max()
    qu, eu = pkg.unpack_bfp8(pw)
    assert np.array_equal(qu.cpu().numpy(), qo) and np.array_equal(eu.cpu().numpy(), eo)
    assert np.array_equal(pkg.dequantize(pw).cpu().numpy(), obfp8.dequantize(qo, eo))
    # bf16
    pb = pkg.pack_weight(w, "bf16")
    tb = obfp8.pack_tiles_bf16(wb)
    assert np.array_equal(pb.buf.cpu().numpy()[: tb.size], tb)
    assert np.array_equal(pkg.dequantize(pb).cpu().numpy(), obf16.bits_to_f32(wb))


@pytest.mark.parametrize("rows,cols", [(48, 768), (3072, 1024), (1024, 3072)])
def test_bf4_pack_matches_oracle_layout(pkg, cuda, rows, cols):
    """bf4: quantiser, packed bytes, row exponents, trailer, unpack and the kernels' dequant
    routine all bit-exact against the oracle."""
    import torch
    from qwen_mlp_amd import workloads

    w = workloads.weight(rows, cols, seed=3 * rows + cols, device=cuda)
    # a few groups at the quantiser's edges: ties, a group maximum that rounds to 8 (clamped to
    # 7), zero groups and groups far below the row maximum
    w[0, :16] = torch.tensor([0.5625, -0.4375, 0.0625, 0.03125] * 4, dtype=torch.bfloat16, device=cuda)
    w[1, :16] = 0.0
    w[2, 16:32] = torch.full((16,), 0.96875, dtype=torch.bfloat16, device=cuda)  # 7.75 -> 8 -> 7
    w[3, 32:48] *= 2.0 ** -12
    wb = _bits(w)
    q, e8 = pkg.quantize_bf4(w)
    qo, eo = obfp8.quantize(wb, mantissa_bits=3)
    assert np.array_equal(q.cpu().numpy(), qo) and np.array_equal(e8.cpu().numpy(), eo)
    pw = pkg.pack_canonical(q, e8, "bf4")
    tiles, rowexp, flushed = obfp8.pack_tiles_bf4(qo, eo)
    buf = pw.buf.cpu().numpy()
    assert buf.size == obfp8.packed_bytes(rows, cols, "bf4")
    assert np.array_equal(buf[: tiles.size], tiles)
    assert np.array_equal(buf[tiles.size: tiles.size + rows * 4].view(np.int32), rowexp)
    assert pw.flushed_groups == flushed == 0
    ref = obfp8.dequantize(qo, eo)
    norms = obfp8.row_norms(ref)
    assert abs(pw.max_row_norm - norms.max()) <= 1e-9 * norms.max()
    qu, eu = pkg.unpack_canonical(pw)
    assert np.array_equal(qu.cpu().numpy(), qo) and np.array_equal(eu.cpu().numpy(), eo)
    d = pkg.dequantize(pw).cpu().numpy()
    assert np.array_equal(d, ref) and np.array_equal(d, obfp8.dequant_tiles_bf4(tiles, rowexp, rows, cols))
    # pack_weight takes the same route
    assert torch.equal(pkg.pack_weight(w, "bf4").buf, pw.buf)


def test_pack_reports_flushed_groups(pkg, cuda):
    import torch

    w = torch.zeros((16, 256), dtype=torch.float32, device=cuda)
    w[:, :16] = 1.0
    w[:, 16:32] = 2.0 ** -19
    w[:, 32:48] = 2.0 ** -20
    q, e8 = pkg.quantize_bfp8(w.to(torch.bfloat16))
    with pytest.raises(ValueError):
        pkg.pack_canonical_bfp8(q, e8)
    pw = pkg.pack_canonical_bfp8(q, e8, strict=False)
    assert pw.flushed_groups == 16
    d = pkg.dequantize(pw).cpu().numpy()
    assert (d[:, 16:32] == 2.0 ** -19).all() and (d[:, 32:48] == 0).all()


# ---------------------------------------------------------------- forward parity


@pytest.mark.parametrize("name", ["plumbing-h1024-i3072-m1-bf16", "qwen3-27b-mlp-m16-bf16", "qwen3-27b-mlp-m16-bfp8",
                                  "qwen3-27b-mlp-m1-bfp8", "qwen3-27b-mlp-m32-bfp8", "qwen3-27b-mlp-m16-bf4",
                                  "qwen3-27b-mlp-m1-bf4", "qwen3-27b-mlp-m32-bf4", "qwen3-27b-tp2-share-m16-bfp8",
                                  "qwen3-27b-tp2-share-m16-bf4", "qwen3-27b-mlp-m64-bfp8"])
def test_forward_workloads(pkg, cuda, name):
    import torch
    from qwen_mlp_amd import workloads

    wl = workloads.WORKLOADS[name]
    print(f"case {name}", flush=True)
    sd = workloads.state_dict(wl.hidden, wl.intermediate, layer=0, device=cuda)
    mlp = pkg.Qwen36MLP(cuda, sd, weight_format=wl.fmt, max_tokens=wl.tokens)
    x = workloads.activations(wl.tokens, wl.hidden, gain=wl.gain, device=cuda)
    x4 = x.view(1, 1, wl.tokens, wl.hidden)
    y32 = mlp.forward(x4, residual=x4, out_dtype=torch.float32)
    y16 = mlp.forward(x4, residual=x4)
    n32 = mlp.forward(x4, out_dtype=torch.float32)  # bare MLP output (the reference's forward(x))
    n16 = mlp.forward(x4)
    torch.cuda.synchronize()
    assert tuple(y16.shape) == (1, 1, wl.tokens, wl.hidden) and y16.dtype == torch.bfloat16
    # the bf16 output is exactly the fp32 output rounded once
    assert torch.equal(y32.to(torch.bfloat16), y16) and torch.equal(n32.to(torch.bfloat16), n16)
    hw = _host_weights(pkg, sd, wl.fmt)
    xf = x.float().cpu().numpy()
    ref, nref = _oracle(xf, hw), _oracle(xf, hw, residual=False)
    _check(y32.reshape(wl.tokens, wl.hidden).cpu().numpy(), ref, name)
    _check(n32.reshape(wl.tokens, wl.hidden).cpu().numpy(), nref, name + " (no residual)")
    _check_bf16(y16.reshape(wl.tokens, wl.hidden).float().cpu().numpy(), ref, name)


@pytest.mark.parametrize("fmt", ["bf16", "bfp8", "bf4"])
def test_forward_every_small_width(pkg, cuda, fmt):
    import torch
    from qwen_mlp_amd import workloads

    H, I = 1024, 3072
    sd = workloads.state_dict(H, I, layer=1, device=cuda)
    mlp = pkg.Qwen36MLP(cuda, sd, weight_format=fmt, max_tokens=128)
    hw = _host_weights(pkg, sd, fmt)
    for M in list(range(1, 34)) + [47, 64, 100]:
        x = workloads.activations(M, H, seed=3891 + M, device=cuda)
        y = mlp.forward(x, residual=x, out_dtype=torch.float32)
        torch.cuda.synchronize()
        xf = x.float().cpu().numpy()
        _check(y.cpu().numpy(), _oracle(xf, hw), f"{fmt} H={H} I={I} M={M}")


def test_forward_random_shapes(pkg, cuda):
    """Seeded irregular shapes (odd superblock and tile counts, every dispatch width, every format)
    against the oracle, fp32 and bf16 outputs."""
    import numpy as np
    import torch
    from qwen_mlp_amd import workloads

    rng = np.random.default_rng(20261201)
    Hs, Is = [256, 768, 1280, 2304, 4352], [256, 1280, 2816, 4864, 6400]
    Ms = [1, 3, 8, 15, 16, 17, 24, 31, 32, 33, 40, 64, 96, 130]
    for case in range(18):
        H, I = int(rng.choice(Hs)), int(rng.choice(Is))
        M, fmt = int(rng.choice(Ms)), str(rng.choice(["bf16", "bfp8", "bf4"]))
        print(f"case random {case}: {fmt} H={H} I={I} M={M}", flush=True)
        sd = workloads.state_dict(H, I, layer=30 + case, device=cuda)
        mlp = pkg.Qwen36MLP(cuda, sd, weight_format=fmt, max_tokens=M)
        x = workloads.activations(M, H, seed=7391 + case, device=cuda)
        y32 = mlp.forward(x, residual=x, out_dtype=torch.float32)
        y16 = mlp.forward(x, residual=x)
        torch.cuda.synchronize()
        ref = _oracle(x.float().cpu().numpy(), _host_weights(pkg, sd, fmt))
        _check(y32.cpu().numpy(), ref, f"random {case} {fmt} H={H} I={I} M={M}")
        _check_bf16(y16.float().cpu().numpy(), ref, f"random {case} {fmt} H={H} I={I} M={M}")
        del mlp, sd
        torch.cuda.empty_cache()


@pytest.mark.parametrize("fmt", ["bf16", "bfp8"])
def test_forward_stream_fallback(pkg, cuda, fmt):
    """A down projection too long for the split kernel's staged activations (K = 76800 > 16 splits
    x 18 superblocks) takes the stream-K weight-streaming kernels instead, at every width."""
    import ctypes

    import torch
    from qwen_mlp_amd import workloads

    H, I = 256, 76800
    out = (ctypes.c_int * 6)()
    assert pkg.lib().qmlp_plan_split(H, I, 1, 16, 256, out) != 0
    sd = workloads.state_dict(H, I, layer=4, device=cuda)
    mlp = pkg.Qwen36MLP(cuda, sd, weight_format=fmt, max_tokens=32)
    hw = _host_weights(pkg, sd, fmt)
    for M in (1, 16, 17, 32):
        print(f"case stream fallback {fmt} M={M}", flush=True)
        x = workloads.activations(M, H, seed=4100 + M, device=cuda)
        y = mlp.forward(x, residual=x, out_dtype=torch.float32)
        torch.cuda.synchronize()
        _check(y.cpu().numpy(), _oracle(x.float().cpu().numpy(), hw), f"stream fallback {fmt} M={M}")


@pytest.mark.parametrize("H,I,M,want_extra", [(2560, 36864, 32, 4), (4864, 53248, 16, 10), (4864, 24576, 32, 16)])
def test_forward_wide_gate_up_groups(pkg, cuda, H, I, M, want_extra):
    """Wide intermediates give gate/up tile groups of more than two tiles per wave (G = 18..26
    tiles for 8 waves).  The last arrival spreads the (tile, token group) pieces beyond two tiles
    per wave over the waves, one per wave with its first batch of loads and the rest in later
    rounds; both paths are checked here (want_extra = pieces beyond 16 tiles)."""
    import ctypes

    import torch
    from qwen_mlp_amd import workloads

    out = (ctypes.c_int * 6)()
    assert pkg.lib().qmlp_plan_split(I, H, 2, M, 256, out) == 0
    G, mg = out[1], 2 if M > 16 else 1
    assert (G - 16) * mg == want_extra, list(out)
    assert pkg.lib().qmlp_plan_split(H, I, 1, M, 256, out) == 0  # the whole forward stays on this kernel
    print(f"case wide gate/up H={H} I={I} M={M} G={G}", flush=True)
    sd = workloads.state_dict(H, I, layer=5, device=cuda)
    mlp = pkg.Qwen36MLP(cuda, sd, weight_format="bfp8", max_tokens=M)
    hw = _host_weights(pkg, sd, "bfp8")
    x = workloads.activations(M, H, seed=4300 + M, device=cuda)
    y = mlp.forward(x, residual=x, out_dtype=torch.float32)
    torch.cuda.synchronize()
    _check(y.cpu().numpy(), _oracle(x.float().cpu().numpy(), hw), f"wide gate/up H={H} I={I} M={M}")


@pytest.mark.parametrize("fmt", ["bf16", "bfp8", "bf4"])
def test_zero_input_and_aliasing(pkg, cuda, fmt):
    import torch
    from qwen_mlp_amd import workloads

    H, I = 1024, 3072
    sd = workloads.state_dict(H, I, layer=2, device=cuda)
    mlp = pkg.Qwen36MLP(cuda, sd, weight_format=fmt, max_tokens=16)
    x = torch.zeros((5, H), dtype=torch.bfloat16, device=cuda)
    r = workloads.activations(5, H, seed=5, device=cuda)
    assert torch.equal(mlp.forward(x, residual=r), r)
    assert not mlp.forward(x).float().abs().max().item()
    # out may alias the residual (in-place residual stream update)
    x = workloads.activations(5, H, seed=6, device=cuda)
    expect = mlp.forward(x, residual=r)
    rr = r.clone()
    mlp.forward(x, residual=rr, out=rr)
    assert torch.equal(rr, expect)


@pytest.mark.parametrize("fmt", ["bf16", "bfp8", "bf4"])
def test_bitwise_deterministic(pkg, cuda, fmt):
    import torch
    from qwen_mlp_amd import workloads

    H, I = 5120, 17408
    sd = workloads.state_dict(H, I, layer=3, device=cuda)
    mlp = pkg.Qwen36MLP(cuda, sd, weight_format=fmt, max_tokens=32)
    for M in (1, 16, 32):
        x = workloads.activations(M, H, seed=7391 + M, device=cuda)
        a = mlp.forward(x, residual=x)
        b = mlp.forward(x, residual=x)
        torch.cuda.synchronize()
        assert torch.equal(a, b)


@pytest.mark.parametrize("fmt", ["bf16", "bfp8", "bf4"])
@pytest.mark.parametrize("H,I,M", [(1024, 4352, 2048), (5376, 2048, 2048), (1024, 3072, 64)])
def test_prefill_bitwise_deterministic(pkg, cuda, fmt, H, I, M):
    """Many-token forwards repeated give identical bits, also where tiles split their K range into
    pieces whose partial tiles meet in the workspace and are added in a fixed order: at 2048
    tokens the tiles beyond the last whole round (gate/up at I = 4352: 16 tiles in 4 pieces; down
    at H = 5376: 80 tiles in 3 pieces), at 64 tokens every tile."""
    import torch
    from qwen_mlp_amd import workloads

    print(f"case prefill determinism {fmt} H={H} I={I} M={M}", flush=True)
    sd = workloads.state_dict(H, I, layer=5, device=cuda)
    mlp = pkg.Qwen36MLP(cuda, sd, weight_format=fmt, max_tokens=M)
    x = workloads.activations(M, H, seed=7391 + M, device=cuda)
    a = mlp.forward(x, residual=x)
    b = mlp.forward(x, residual=x)
    c = mlp.forward(x, residual=x, out_dtype=torch.float32)
    d = mlp.forward(x, residual=x, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    assert torch.equal(c, d)


@pytest.mark.parametrize("fmt", ["bf16", "bfp8", "bf4"])
@pytest.mark.parametrize("H,I,M", [(1024, 3072, 16), (1024, 3072, 64), (1024, 4352, 2048)])
def test_graph_capture_replays(pkg, cuda, fmt, H, I, M):
    """A forward captured in a HIP graph and replayed five times on new inputs, each replay
    equal to the eager forward: the weight-streaming kernels at 16 tokens, the tiled kernels at 64
    tokens (every tile split, padding blocks) and at 2048 tokens with split pieces (their arrival
    counters must be back at zero after every replay)."""
    import torch
    from qwen_mlp_amd import workloads

    print(f"case graph {fmt} H={H} I={I} M={M}", flush=True)
    sd = workloads.state_dict(H, I, layer=4, device=cuda)
    mlp = pkg.Qwen36MLP(cuda, sd, weight_format=fmt, max_tokens=M)
    static_x = workloads.activations(M, H, seed=1, device=cuda)
    static_out = torch.empty_like(static_x)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        mlp.forward(static_x, residual=static_x, out=static_out)  # warm-up outside the graph
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):  # the warm-up gave this stream its workspace
        mlp.forward(static_x, residual=static_x, out=static_out)
    for seed in range(5):
        new_x = workloads.activations(M, H, seed=100 + seed, device=cuda)
        static_x.copy_(new_x)
        g.replay()
        torch.cuda.synchronize()
        eager = mlp.forward(new_x, residual=new_x)
        torch.cuda.synchronize()
        assert torch.equal(static_out, eager), f"replay {seed} differs from eager"


def test_layer_chain(pkg, cuda):
    """Four chained layers (residual stream) checked layer by layer against the oracle."""
    import torch
    from qwen_mlp_amd import workloads

    H, I, M = 1024, 3072, 16
    x = workloads.activations(M, H, seed=9, device=cuda)
    for layer in range(4):
        fmt = "bfp8" if layer % 2 else "bf16"
        sd = workloads.state_dict(H, I, layer=10 + layer, device=cuda)
        mlp = pkg.Qwen36MLP(cuda, sd, weight_format=fmt, max_tokens=M)
        y = mlp.forward(x, residual=x)
        torch.cuda.synchronize()
        xf = x.float().cpu().numpy()
        _check_bf16(y.float().cpu().numpy(), _oracle(xf, _host_weights(pkg, sd, fmt)), f"chain layer {layer} {fmt}")
        x = y


def test_shape_errors(pkg, cuda):
    import torch
    from qwen_mlp_amd import workloads

    sd = workloads.state_dict(1024, 3072, layer=5, device=cuda)
    mlp = pkg.Qwen36MLP(cuda, sd, weight_format="bfp8", max_tokens=4)
    with pytest.raises(ValueError):
        mlp.forward(torch.zeros((2, 1000), dtype=torch.bfloat16, device=cuda))
    with pytest.raises(ValueError):
        mlp.forward(torch.zeros((2, 1024), dtype=torch.float32, device=cuda))
    with pytest.raises(ValueError):
        mlp.forward(torch.zeros((2, 1024), dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        pkg.pack_weight(torch.zeros((17, 256), dtype=torch.bfloat16, device=cuda))
    # an output that a reshape could only copy is refused (the result would land in the copy)
    x = torch.zeros((2, 1024), dtype=torch.bfloat16, device=cuda)
    strided = torch.zeros((1024, 2), dtype=torch.bfloat16, device=cuda).t()
    with pytest.raises(ValueError):
        mlp.forward(x, out=strided)
    with pytest.raises(ValueError):
        mlp.forward_rmsnorm(x, torch.zeros(1024, dtype=torch.bfloat16, device=cuda), out=strided)


@pytest.mark.parametrize("fmt", ["bf16", "bfp8", "bf4"])
@pytest.mark.parametrize("H,I,M", [(1024, 3072, 2048), (5120, 17408, 256), (1024, 3072, 200), (1024, 3072, 33),
                                   (1024, 4352, 2048), (5120, 512, 2048), (6144, 2048, 2048), (5376, 2048, 2048),
                                   (1024, 41728, 160), (1024, 3072, 2049), (2048, 2048, 4100)])
def test_prefill_tiled(pkg, cuda, fmt, H, I, M):
    """Many-token forwards (the LDS-tiled matrix-core kernels): a full 2048-token chunk, the 27B
    shape at 256 tokens, a token count that leaves a partial token block, the narrowest width that
    takes this path (one partial block in each projection), chunks longer than 2048 tokens with a
    ragged last block (2049: 204 gate/up tiles, fewer than one round; 4100: 264 tiles in each
    projection, one whole round and 8 tiles in 4 pieces that meet in the workspace's fixed-size
    split region), and, for the block-float formats,
    shapes whose tiles do not fill whole rounds of a 256-CU GPU, so that the tiles beyond the last
    whole round split their K range into pieces that meet in the workspace: gate/up at I = 4352
    (16 tiles in 4 pieces) and I = 41728 (70 tiles in 3 pieces, block order left as is), down at
    H = 5120, K = 512 and H = 6144 (2 pieces) and at H = 5376 (80 tiles in 3 pieces)."""
    import torch
    from qwen_mlp_amd import workloads

    print(f"case prefill {fmt} H={H} I={I} M={M}", flush=True)
    sd = workloads.state_dict(H, I, layer=8, device=cuda)
    mlp = pkg.Qwen36MLP(cuda, sd, weight_format=fmt, max_tokens=M)
    x = workloads.activations(M, H, seed=4242 + M, gain=False, device=cuda)
    y32 = mlp.forward(x, residual=x, out_dtype=torch.float32)
    y16 = mlp.forward(x, residual=x)
    torch.cuda.synchronize()
    assert torch.equal(y32.to(torch.bfloat16), y16)
    hw = _host_weights(pkg, sd, fmt)
    xf = x.float().cpu().numpy()
    _check(y32.cpu().numpy(), _oracle(xf, hw), f"prefill {fmt} H={H} I={I} M={M}")


@pytest.mark.parametrize("fmt", ["bf16", "bfp8", "bf4"])
def test_fp32_residual_stream(pkg, cuda, fmt):
    """An fp32 residual stream (out = residual + MLP(x), the residual read as fp32) at every kind of
    dispatch: the weight-streaming kernel (16 tokens), the 16x16 tiled kernels (200 tokens), and at
    2048 tokens the 32x32 kernel's down projection whose last tiles split K into pieces (block-float
    formats; bf16 weights take the 16x16 kernel there too); then in place (out = residual)."""
    import torch
    from qwen_mlp_amd import workloads

    H, I = 6144, 2048
    sd = workloads.state_dict(H, I, layer=21, device=cuda)
    mlp = pkg.Qwen36MLP(cuda, sd, weight_format=fmt, max_tokens=2048)
    hw = _host_weights(pkg, sd, fmt)
    for M in (16, 200, 2048):
        print(f"case fp32 residual {fmt} M={M}", flush=True)
        x = workloads.activations(M, H, seed=7100 + M, gain=False, device=cuda)
        res = workloads.activations(M, H, seed=7200 + M, gain=False, device=cuda).float() * 3.0 + 0.125
        ref = omlp.swiglu(x.float().cpu().numpy(), hw["gate_proj"], hw["up_proj"], hw["down_proj"],
                          residual=res.cpu().numpy())
        y = mlp.forward(x, residual=res, out_dtype=torch.float32)
        torch.cuda.synchronize()
        _check(y.cpu().numpy(), ref, f"fp32 residual {fmt} M={M}")
        r2 = res.clone()
        mlp.forward(x, residual=r2, out=r2, out_dtype=torch.float32)
        torch.cuda.synchronize()
        assert torch.equal(r2, y), f"{fmt} M={M}: in-place fp32 residual differs"


@pytest.mark.parametrize("fmt", ["bf16", "bfp8", "bf4"])
def test_rmsnorm_prologue(pkg, cuda, fmt):
    """h + MLP(rmsnorm(h) * (1 + w)) against the oracle's composition (the norm output rounded to
    bf16 as the reference's separate norm produces it), across every dispatch width: fused into
    the M <= 32 weight-streaming kernel, a separate pass for the others; then in place (out = h)."""
    import torch
    from qwen_mlp_amd import workloads

    H, I = 1024, 3072
    sd = workloads.state_dict(H, I, layer=9, device=cuda)
    mlp = pkg.Qwen36MLP(cuda, sd, weight_format=fmt, max_tokens=200)
    hw = _host_weights(pkg, sd, fmt)
    g = torch.Generator(cuda).manual_seed(31)
    nw = (torch.randn(H, generator=g, device=cuda) * 0.3).to(torch.bfloat16)
    nwf = nw.float().cpu().numpy()
    for M in (1, 5, 16, 24, 32, 64, 200):
        h = (workloads.activations(M, H, seed=600 + M, device=cuda).float() * 7.0).to(torch.bfloat16)
        y = mlp.forward_rmsnorm(h, nw, eps=1e-6, out_dtype=torch.float32)
        y16 = mlp.forward_rmsnorm(h, nw, eps=1e-6)
        torch.cuda.synchronize()
        assert torch.equal(y.to(torch.bfloat16), y16)
        hf = h.float().cpu().numpy()
        ref = omlp.norm_swiglu(hf, nwf, hw["gate_proj"], hw["up_proj"], hw["down_proj"], 1e-6)
        _check(y.cpu().numpy(), ref, f"rmsnorm {fmt} M={M}")
        hh = h.clone()
        mlp.forward_rmsnorm(hh, nw, eps=1e-6, out=hh)
        torch.cuda.synchronize()
        assert torch.equal(hh, y16)


def test_rmsnorm_prologue_27b(pkg, cuda):
    import torch
    from qwen_mlp_amd import workloads

    H, I, M = 5120, 17408, 16
    sd = workloads.state_dict(H, I, layer=10, device=cuda)
    mlp = pkg.Qwen36MLP(cuda, sd, weight_format="bfp8", max_tokens=M)
    nw = (torch.randn(H, generator=torch.Generator(cuda).manual_seed(5), device=cuda) * 0.3).to(torch.bfloat16)
    h = (workloads.activations(M, H, seed=77, device=cuda).float() * 30.0).to(torch.bfloat16)
    y = mlp.forward_rmsnorm(h, nw, eps=1e-6, out_dtype=torch.float32)
    torch.cuda.synchronize()
    hw = _host_weights(pkg, sd, "bfp8")
    ref = omlp.norm_swiglu(h.float().cpu().numpy(), nw.float().cpu().numpy(), hw["gate_proj"], hw["up_proj"],
                           hw["down_proj"], 1e-6)
    _check(y.cpu().numpy(), ref, "rmsnorm 27B M=16 bfp8")


@pytest.mark.parametrize("fmt", ["bfp8", "bf4"])
def test_offline_packer_round_trip(pkg, cuda, tmp_path, fmt):
    """HF safetensors -> pack_checkpoint -> cache files: the cached layer loads bit-identical to a
    load-time conversion and the planar files hold the canonical mantissas/exponents."""
    import numpy as np
    import torch
    from safetensors.torch import save_file
    from qwen_mlp_amd import pack_checkpoint, workloads

    H, I = 1024, 3072
    sds = [workloads.state_dict(H, I, layer=20 + i, device=cuda) for i in range(2)]
    save_file({f"model.layers.{i}.mlp.{k}": v.cpu().contiguous() for i, sd in enumerate(sds) for k, v in sd.items()},
              str(tmp_path / "model.safetensors"))
    assert pack_checkpoint.main(["--checkpoint", str(tmp_path), "--out", str(tmp_path / "packed"), "--planar",
                                 "--format", fmt]) == 0
    quant = pkg.quantize_bf4 if fmt == "bf4" else pkg.quantize_bfp8
    for i, sd in enumerate(sds):
        d = tmp_path / "packed" / f"layer_{i}"
        cached = pkg.load_mlp_weights(cuda, {}, tensor_cache_path=str(d), weight_format=fmt)  # nothing to convert
        direct = pkg.load_mlp_weights(cuda, sd, weight_format=fmt)
        assert (cached.w1.fmt, cached.w2.fmt, cached.w3.fmt) == (fmt, "bfp8", fmt)
        for f in ("w1", "w2", "w3"):
            assert torch.equal(getattr(cached, f).buf, getattr(direct, f).buf)
        q, e8 = quant(sd["gate_proj.weight"])
        assert np.array_equal(np.load(d / "gate_proj.q.npy", mmap_mode="r"), q.cpu().numpy())
        assert np.array_equal(np.load(d / "gate_proj.e8.npy", mmap_mode="r"), e8.cpu().numpy())
        q, e8 = pkg.quantize_bfp8(sd["down_proj.weight"])
        assert np.array_equal(np.load(d / "down_proj.q.npy", mmap_mode="r"), q.cpu().numpy())


@pytest.mark.parametrize("rows", [16, 32])
def test_verify_arm_routes_decoder_mlps(pkg, cuda, rows):
    """A toy 2-layer decoder (norm -> MLP -> residual, layer.py:352-357, attention left out) whose
    feed-forward modules are plain torch MLPs: inside the arm's scope the verify-width calls (16 or
    32 token rows, the reference's T16 and T32 arms) run the library and match the torch path,
    other widths fall back, and the bindings come back.  Before the first scope the arm checks
    each layer's packed weights byte for byte against that layer's own (2 x 3 matrices)."""
    import types

    import torch
    from qwen_mlp_amd import verify_arm, workloads

    H, I = 1024, 3072

    class TorchMLP:
        def __init__(self, sd):
            for k in ("gate_proj", "up_proj", "down_proj"):
                setattr(self, k, types.SimpleNamespace(weight=sd[f"{k}.weight"]))

        def forward(self, x):
            xf = x.float()
            g, u, d = (getattr(self, k).weight.float() for k in ("gate_proj", "up_proj", "down_proj"))
            return ((torch.nn.functional.silu(xf @ g.T) * (xf @ u.T)) @ d.T).to(torch.bfloat16)

    class ToyLayer:
        def __init__(self, mlp):
            self.feed_forward = mlp

        def forward(self, h):
            hf = h.float()
            n = (hf * torch.rsqrt(hf.pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16)
            return (hf + self.feed_forward.forward(n).float()).to(torch.bfloat16)

    sds = [workloads.state_dict(H, I, layer=30 + i, device=cuda) for i in range(2)]
    layers = [ToyLayer(TorchMLP(sd)) for sd in sds]
    amd = [pkg.Qwen36MLP(cuda, sd, weight_format="bf16", max_tokens=rows) for sd in sds]
    arm = verify_arm.VerifyArm([l.feed_forward for l in layers], amd, token_rows=rows)

    def run(h):
        for layer in layers:
            h = layer.forward(h)
        return h

    hv = workloads.activations(rows, H, seed=4, device=cuda).view(1, 1, rows, H)
    h8 = workloads.activations(8, H, seed=5, device=cuda).view(1, 1, 8, H)
    refv, ref8 = run(hv), run(h8)
    with arm.install():
        outv, out8 = run(hv), run(h8)
    torch.cuda.synchronize()
    assert arm.audit == dict(rows=rows, layers=2, hits=[1, 1], fallbacks=[1, 1], restored=True,
                             weights_unchanged=True, weights_checked=6)
    assert len(arm.weight_checks) == 6 and all(c["exact"] for c in arm.weight_checks)
    assert torch.equal(out8, ref8)  # fell back to the torch path
    # The torch decoder rounds the MLP output to bf16 before the residual add, the library rounds
    # the sum once: besides the 1e-2 * RMS bar allow two bf16 ulps of the reference per element.
    y = outv.double().reshape(rows, H).cpu().numpy()
    r = refv.double().reshape(rows, H).cpu().numpy()
    _, e = np.frexp(np.abs(r))
    excess = float(np.max(np.abs(y - r) - 2 * np.ldexp(1.0, e - 8)))
    bar = TOL * float(np.sqrt(np.mean(r * r)))
    print(f"verify arm T{rows} vs torch decoder: max(|err| - 2 ulp)={excess:.4e} bar={bar:.4e}", flush=True)
    assert excess <= bar
    assert all("forward" not in l.feed_forward.__dict__ for l in layers)
    with pytest.raises(ZeroDivisionError):
        with arm.install():
            1 / 0
    assert arm.audit["restored"] and not arm.active
    # a swapped pairing (layer 0's library weights serving layer 1 and back) is refused, unbound
    swapped = verify_arm.VerifyArm([l.feed_forward for l in layers], amd[::-1], token_rows=rows)
    with pytest.raises(ValueError, match="layer 0: the library's packed gate_proj is not this decoder layer"):
        with swapped.install():
            pytest.fail("a swapped pairing must not install")
    assert all("forward" not in l.feed_forward.__dict__ for l in layers) and not swapped.active
    # one stale matrix (layer 1's down projection re-packed from other weights) is refused too
    stale = pkg.Qwen36MLP(cuda, dict(sds[1], **{"down_proj.weight": sds[0]["down_proj.weight"]}),
                          weight_format="bf16", max_tokens=rows)
    bad = verify_arm.VerifyArm([l.feed_forward for l in layers], [amd[0], stale], token_rows=rows)
    with pytest.raises(ValueError, match="layer 1: the library's packed down_proj"):
        bad.__enter__()
    assert not bad.active
