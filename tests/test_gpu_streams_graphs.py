"""Concurrent forwards on two streams and HIP-graph capture of whole layer stacks.

* Two streams running many-token forwards at once: the split tiles of the matrix-core kernels
  meet by last arrival, so no block waits for another and the two kernels' blocks may interleave
  on the CUs in any way; every output must equal the eager, one-at-a-time result bit for bit.
* ``torch.cuda.graph(g)`` with no stream argument (torch's own capture stream), and a graph
  replayed after the shared workspace grew: the replaced workspace stays alive.
* The 64-layer bfp8 stack (27B, 16 tokens, the decoder's RMSNorm -> MLP -> residual chain)
  captured in one graph and replayed A-B-A against eager runs, with the input left unmodified and
  the missing-input-update negative control of the reference's replay check
  (scripts/ci/fusion_trace.py:42-62; the captured verify step, scripts/ci/verifier_engine.py:565-572).
"""
import pytest

pytestmark = pytest.mark.gpu

H27, I27 = 5120, 17408


@pytest.mark.parametrize("fmt,H,I,M", [("bfp8", H27, I27, 16), ("bf4", H27, I27, 16), ("bfp8", H27, I27, 2048),
                                       ("bfp8", H27, I27, 64), ("bf4", 1024, 4352, 2048), ("bf16", 1024, 4352, 2048),
                                       ("bfp8", 5376, 2048, 2048)])
def test_two_streams_concurrent_forwards(pkg, cuda, fmt, H, I, M):
    """Forwards of two layers issued alternately on two streams with no synchronisation between
    them.  27B at 16 tokens: the split-K weight-streaming kernels, whose partial sums meet by last
    arrival in per-stream counters; 27B at 2048 tokens: 64 gate/up and 64 down tiles in 4 pieces;
    27B at 64 tokens: every tile split; I = 4352: 16 gate/up tiles in 4 pieces; H = 5376: 80 down
    tiles in 3 pieces."""
    import torch
    from qwen_mlp_amd import workloads

    print(f"case two streams {fmt} H={H} I={I} M={M}", flush=True)
    pool = pkg.WorkspacePool()
    mlps = [pkg.Qwen36MLP(cuda, workloads.state_dict(H, I, layer=70 + i, device=cuda), weight_format=fmt,
                          max_tokens=M, pool=pool) for i in range(2)]
    xs = [workloads.activations(M, H, seed=300 + i, device=cuda) for i in range(4)]
    ref = [[m.forward(x, residual=x) for x in xs] for m in mlps]  # eager, one at a time
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    outs = [[torch.empty_like(x) for x in xs] for _ in mlps]
    for rnd in range(3):
        for j, x in enumerate(xs):
            for k, (m, s) in enumerate(zip(mlps, streams)):
                with torch.cuda.stream(s):
                    m.forward(x, residual=x, out=outs[k][j])
        for s in streams:
            torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        for k in range(2):
            for j in range(len(xs)):
                assert torch.equal(outs[k][j], ref[k][j]), f"round {rnd}: layer {k} input {j} differs from eager"
    assert len(pool._ws) >= 3  # the current stream, torch's capture stream and the two side streams


def test_graph_on_torch_default_capture_stream(pkg, cuda):
    """The usual PyTorch pattern: warm up on a side stream, then ``torch.cuda.graph(g)`` with no
    stream argument (it captures on its own side stream, for which the MLP reserved a workspace)."""
    import torch
    from qwen_mlp_amd import workloads

    H, I, M = 1024, 3072, 16
    mlp = pkg.Qwen36MLP(cuda, workloads.state_dict(H, I, layer=80, device=cuda), weight_format="bfp8", max_tokens=M)
    static_x = workloads.activations(M, H, seed=1, device=cuda)
    static_out = torch.empty_like(static_x)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        mlp.forward(static_x, residual=static_x, out=static_out)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        mlp.forward(static_x, residual=static_x, out=static_out)
    for seed in range(3):
        new_x = workloads.activations(M, H, seed=200 + seed, device=cuda)
        static_x.copy_(new_x)
        g.replay()
        torch.cuda.synchronize()
        eager = mlp.forward(new_x, residual=new_x)
        torch.cuda.synchronize()
        assert torch.equal(static_out, eager), f"replay {seed} differs from eager"


def test_graph_replays_after_workspace_growth(pkg, cuda):
    """A graph captured at 16 tokens, then an eager call with more tokens than max_tokens grows the
    shared workspace: the graph keeps the workspace it captured (kept alive by the pool), so its
    replays stay correct and write nowhere else."""
    import torch
    from qwen_mlp_amd import workloads

    H, I = 1024, 3072
    pool = pkg.WorkspacePool()
    mlp = pkg.Qwen36MLP(cuda, workloads.state_dict(H, I, layer=81, device=cuda), weight_format="bfp8", max_tokens=16,
                        pool=pool)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    static_x = workloads.activations(16, H, seed=2, device=cuda)
    static_out = torch.empty_like(static_x)
    with torch.cuda.stream(s):
        mlp.forward(static_x, residual=static_x, out=static_out)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        mlp.forward(static_x, residual=static_x, out=static_out)
    torch.cuda.synchronize()
    before = pool.total_bytes()
    with torch.cuda.stream(s):  # 300 tokens on the graph's stream: its workspace must grow
        big = workloads.activations(300, H, seed=3, device=cuda)
        ybig = mlp.forward(big, residual=big)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    assert pool.total_bytes() > before and pool.retired_bytes() > 0
    # fill fresh allocations with a pattern: were the old workspace freed, they could take its place
    junk = [torch.full((1 << 20,), 7, dtype=torch.int32, device=cuda) for _ in range(8)]
    for seed in range(3):
        new_x = workloads.activations(16, H, seed=210 + seed, device=cuda)
        static_x.copy_(new_x)
        g.replay()
        torch.cuda.synchronize()
        eager = mlp.forward(new_x, residual=new_x)
        torch.cuda.synchronize()
        assert torch.equal(static_out, eager), f"replay {seed} after the growth differs from eager"
    assert all(bool((j == 7).all()) for j in junk)
    assert torch.equal(mlp.forward(big, residual=big), ybig)


def test_stack_64_layers_graph_aba(pkg, cuda):
    """64 independently seeded bfp8 layers at the 27B shape, 16 tokens, chained as the decoder's
    feed-forward sublayers h <- h + MLP(rmsnorm(h) * (1 + w)), captured in one HIP graph.  Replays
    with inputs A, B, A each equal the eager chain bit for bit and leave the input buffer as it was
    given; a replay without copying the next input (the missing-input-update negative control)
    reproduces the previous output and differs from the other input's."""
    import torch
    from qwen_mlp_amd import workloads

    M, L = 16, 64
    layers = []
    for i in range(L):
        sd = workloads.state_dict(H27, I27, layer=100 + i, device=cuda)
        layers.append(pkg.load_mlp_weights(cuda, sd, weight_format="bfp8"))
        del sd
    g0 = torch.Generator(cuda).manual_seed(11)
    norms = [(torch.randn(H27, generator=g0, device=cuda) * 0.2).to(torch.bfloat16) for _ in range(L)]
    print(f"case graph stack: {L} layers packed", flush=True)
    ws = pkg.new_workspace(M, H27, I27, "bfp8", cuda)
    static_in = torch.empty((M, H27), dtype=torch.bfloat16, device=cuda)
    bufs = [torch.empty_like(static_in), torch.empty_like(static_in)]

    def chain(src):
        h = src
        for i in range(L):
            out = bufs[i % 2]
            pkg.mlp_forward_rmsnorm(h, norms[i], layers[i], eps=1e-6, out=out, workspace=ws)
            h = out
        return h

    a = workloads.activations(M, H27, seed=500, device=cuda)
    b = workloads.activations(M, H27, seed=501, device=cuda)
    ref = {}
    for name, v in (("A", a), ("B", b)):
        static_in.copy_(v)
        ref[name] = chain(static_in).clone()
    torch.cuda.synchronize()
    assert not torch.equal(ref["A"], ref["B"])
    assert bool(torch.isfinite(ref["A"].float()).all()) and bool(torch.isfinite(ref["B"].float()).all())

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        chain(static_in)  # warm-up on the capturing stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=s):
        result = chain(static_in)
    addrs = (static_in.data_ptr(), result.data_ptr(), ws.data_ptr())
    for step, name in enumerate(("A", "B", "A")):
        given = a if name == "A" else b
        static_in.copy_(given)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(result, ref[name]), f"replay {step} ({name}) differs from the eager chain"
        assert torch.equal(static_in, given), f"replay {step} ({name}) modified its input"
        x_eager = given.clone()
        eager = chain(x_eager)  # eager work between replays, on the same buffers
        torch.cuda.synchronize()
        assert torch.equal(eager, ref[name])
    assert (static_in.data_ptr(), result.data_ptr(), ws.data_ptr()) == addrs  # nothing captured moved
    # negative control: the next input (B) is not copied in, so the replay reads the stale input
    # A; the output buffer is poisoned first, so only a replay that ran can pass
    assert torch.equal(static_in, a)
    result.fill_(float("nan"))
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(result, ref["A"]) and not torch.equal(result, ref["B"])
