"""Qwen3 SwiGLU MLP for MI355X: the host-side mirror of the reference module.

Reference interface being replaced (``docker/qwen-c2-graft/graft/mlp.py``):

* ``MLPWeights`` (``mlp.py:15-20``): w1 = gate_proj, w2 = down_proj, w3 = up_proj.
* ``load_mlp_weights(mesh_device, state_dict, tensor_cache_path=None, args=None)``
  (``mlp.py:45-169``): converts the HF tensors ``{gate,up,down}_proj.weight`` into device tiles.
* ``Qwen36MLP(mesh_device, state_dict, tensor_cache_path=None, args=None, tt_ccl=None)`` with
  ``forward(x)`` (``mlp.py:359-423``): ``down(silu(gate(x)) * up(x))`` on a ``[1, 1, M, H]`` bf16
  activation; the decoder layer then adds the residual (``layer.py:354-357``), which
  ``forward(x, residual=h)`` fuses.

Shapes: x ``[1, 1, M, H]`` or ``[M, H]`` (any leading dims multiply into M), bf16, on the GPU.
Errors: ``ValueError`` for wrong shape/dtype/device (as ``FusedProjection.__call__``,
``scripts/ci/fused_1d.py:124-128``), ``QmlpError`` for launch failures.  There is no CPU fallback.
"""
import ctypes
import os
from dataclasses import dataclass

import torch

from . import _lib

# MLP weight formats.  "bf4" is the reference's mixed layout (``mlp.py:17-19,164-169``): gate/up in
# bf4 (3 magnitude bits), down in bfp8.
WEIGHT_FORMATS = ("bf16", "bfp8", "bf4")
MATRIX_FORMATS = ("bf16", "bfp8", "bf4")
_MANTISSA_BITS = {"bfp8": 7, "bf4": 3}


def matrix_formats(fmt):
    """(gate/up, down) matrix formats of an MLP weight format."""
    if fmt not in WEIGHT_FORMATS:
        raise ValueError(f"weight format must be one of {WEIGHT_FORMATS}, got {fmt!r}")
    return (fmt, "bfp8") if fmt == "bf4" else (fmt, fmt)


@dataclass
class PackedWeight:
    """One weight matrix in the library's packed layout (device bytes + shape + format)."""

    buf: torch.Tensor  # uint8 device tensor, qmlp_packed_bytes(rows, cols, fmt) bytes
    rows: int
    cols: int
    fmt: str
    max_row_norm: float = 0.0
    flushed_groups: int = 0

    @property
    def fmt_code(self):
        return _lib.FORMATS[self.fmt]

    @property
    def nbytes(self):
        return self.buf.numel()

    @property
    def stream_bytes(self):
        """Bytes of the weight values the forward pass streams (excludes row exponents/trailer)."""
        per_value = {"bfp8": 17 / 16, "bf4": 9 / 16, "bf16": 2}[self.fmt]
        return int(self.rows * self.cols * per_value)

    def data_ptr(self):
        return self.buf.data_ptr()


def _check_device_tensor(t, name, dtype=None):
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be on the GPU, got {t.device}")
    if dtype is not None and t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def quantize_bfp8(w, stream=None):
    """Canonical bfp8 of a bf16 ``[rows, cols]`` GPU tensor -> ``(q int8 [rows, cols], e8 uint8 [rows, cols/16])``."""
    return _quantize(w, "bfp8", stream)


def quantize_bf4(w, stream=None):
    """Canonical bf4 (q in [-7, 7]) of a bf16 ``[rows, cols]`` GPU tensor -> ``(q, e8)``."""
    return _quantize(w, "bf4", stream)


def _quantize(w, fmt, stream):
    _check_device_tensor(w, "w", torch.bfloat16)
    if w.dim() != 2:
        raise ValueError("w must be 2-D")
    rows, cols = w.shape
    q = torch.empty((rows, cols), dtype=torch.int8, device=w.device)
    e8 = torch.empty((rows, cols // 16), dtype=torch.uint8, device=w.device)
    bad = torch.zeros(1, dtype=torch.int32, device=w.device)
    fn = "qmlp_quantize_" + fmt
    _lib.check(getattr(_lib.lib(), fn)(_lib.ptr(w), rows, cols, _lib.ptr(q), _lib.ptr(e8), _lib.ptr(bad),
                                       _lib.stream_handle(stream)), fn)
    if int(bad.item()):
        raise ValueError(f"weight holds non-finite values in {int(bad.item())} groups")
    return q, e8


def _read_info(pw, stream=None):
    norm = ctypes.c_double(0.0)
    flushed = ctypes.c_uint32(0)
    _lib.check(_lib.lib().qmlp_packed_info(_lib.ptr(pw.buf), pw.rows, pw.cols, pw.fmt_code, ctypes.byref(norm),
                                           ctypes.byref(flushed), _lib.stream_handle(stream)), "qmlp_packed_info")
    pw.max_row_norm = float(norm.value)
    pw.flushed_groups = int(flushed.value)
    return pw


def pack_canonical_bfp8(q, e8, strict=True, stream=None):
    """Pack canonical bfp8 (q int8 [rows, cols], e8 uint8 [rows, cols/16]) into the device layout."""
    return pack_canonical(q, e8, "bfp8", strict, stream)


def pack_canonical(q, e8, fmt="bfp8", strict=True, stream=None):
    """Pack canonical block float (``fmt`` "bfp8" or "bf4") into the device layout."""
    if fmt not in _MANTISSA_BITS:
        raise ValueError(f"canonical format must be bfp8 or bf4, got {fmt!r}")
    _check_device_tensor(q, "q", torch.int8)
    _check_device_tensor(e8, "e8", torch.uint8)
    rows, cols = q.shape
    if tuple(e8.shape) != (rows, cols // 16):
        raise ValueError("e8 must be [rows, cols/16]")
    code = _lib.FORMATS[fmt]
    nbytes = _lib.lib().qmlp_packed_bytes(rows, cols, code)
    if nbytes == 0:
        raise ValueError(f"unsupported shape {rows}x{cols}: rows must be a multiple of 16 and cols of 256")
    buf = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
    _lib.check(_lib.lib().qmlp_pack(_lib.ptr(q), _lib.ptr(e8), rows, cols, code, _lib.ptr(buf), nbytes,
                                    _lib.stream_handle(stream)), "qmlp_pack")
    pw = _read_info(PackedWeight(buf, rows, cols, fmt), stream)
    if strict and pw.flushed_groups:
        raise ValueError(f"{pw.flushed_groups} {fmt} groups lie more than 19 binades below their row maximum")
    return pw


def pack_weight(w, fmt="bfp8", strict=True, stream=None):
    """bf16 ``[rows, cols]`` GPU tensor (HF layout: [out, in]) -> PackedWeight in the matrix format
    ``fmt`` ("bf16", "bfp8" or "bf4")."""
    if fmt not in MATRIX_FORMATS:
        raise ValueError(f"matrix format must be one of {MATRIX_FORMATS}, got {fmt!r}")
    _check_device_tensor(w, "w", torch.bfloat16)
    if w.dim() != 2:
        raise ValueError("w must be 2-D")
    if fmt in _MANTISSA_BITS:
        q, e8 = _quantize(w, fmt, stream)
        return pack_canonical(q, e8, fmt, strict=strict, stream=stream)
    rows, cols = w.shape
    nbytes = _lib.lib().qmlp_packed_bytes(rows, cols, _lib.FMT_BF16)
    if nbytes == 0:
        raise ValueError(f"unsupported shape {rows}x{cols}: rows must be a multiple of 16 and cols of 256")
    buf = torch.empty(nbytes, dtype=torch.uint8, device=w.device)
    _lib.check(_lib.lib().qmlp_pack(_lib.ptr(w), None, rows, cols, _lib.FMT_BF16, _lib.ptr(buf), nbytes,
                                    _lib.stream_handle(stream)), "qmlp_pack")
    return _read_info(PackedWeight(buf, rows, cols, "bf16"), stream)


def unpack_bfp8(pw, stream=None):
    """Packed bfp8 -> canonical (q, e8) (lossless for unflushed groups)."""
    if pw.fmt != "bfp8":
        raise ValueError("unpack_bfp8 needs a bfp8 weight")
    return unpack_canonical(pw, stream)


def unpack_canonical(pw, stream=None):
    """Packed bfp8 or bf4 -> canonical (q, e8) (lossless for unflushed groups)."""
    if pw.fmt not in _MANTISSA_BITS:
        raise ValueError("unpacking needs a bfp8 or bf4 weight")
    q = torch.empty((pw.rows, pw.cols), dtype=torch.int8, device=pw.buf.device)
    e8 = torch.empty((pw.rows, pw.cols // 16), dtype=torch.uint8, device=pw.buf.device)
    fn = "qmlp_unpack_" + pw.fmt
    _lib.check(getattr(_lib.lib(), fn)(_lib.ptr(pw.buf), pw.rows, pw.cols, _lib.ptr(q), _lib.ptr(e8),
                                       _lib.stream_handle(stream)), fn)
    return q, e8


def dequantize(pw, stream=None):
    """Packed weight -> float32 ``[rows, cols]`` via the kernels' own dequant routine."""
    out = torch.empty((pw.rows, pw.cols), dtype=torch.float32, device=pw.buf.device)
    _lib.check(_lib.lib().qmlp_dequant_packed(_lib.ptr(pw.buf), pw.rows, pw.cols, pw.fmt_code, _lib.ptr(out),
                                              _lib.stream_handle(stream)), "qmlp_dequant_packed")
    return out


def workspace_bytes(M, H, I, fmt):
    n = _lib.lib().qmlp_workspace_bytes(M, H, I, _lib.FORMATS[fmt])
    if n == 0:
        raise ValueError(f"unsupported sizes M={M} H={H} I={I} fmt={fmt}")
    return n


def _new_workspace_bytes(n, device, stream=None):
    ws = torch.empty(n, dtype=torch.uint8, device=device)
    _lib.check(_lib.lib().qmlp_workspace_init(_lib.ptr(ws), n, _lib.stream_handle(stream)), "qmlp_workspace_init")
    return ws


def new_workspace(M, H, I, fmt, device, stream=None):
    """Allocate and initialise a forward workspace (outside any graph capture).  A workspace sized
    for M tokens serves every call with M or fewer tokens, of any shape whose size fits."""
    return _new_workspace_bytes(workspace_bytes(M, H, I, fmt), device, stream)


def graph_capture_stream(device=None):
    """The stream ``torch.cuda.graph(g)`` captures on when it is given no ``stream``: torch's
    ``torch.cuda.graph.default_capture_stream``, created here the way torch creates it (lazily, one
    per process) if no graph has been built yet."""
    cls = torch.cuda.graphs.graph
    if cls.default_capture_stream is None:
        with torch.cuda.device(device):
            cls.default_capture_stream = torch.cuda.Stream()
    return cls.default_capture_stream


class WorkspacePool:
    """One forward workspace per (device, stream), shared by every MLP that runs there.

    Forwards on one stream run one after another, so they can share a workspace.  Forwards on
    different streams may overlap, so each stream gets its own.  A workspace only grows, and only
    outside graph capture: during a capture the stream must already hold a large enough one.  Run
    one forward on that stream first, or call ``reserve`` (``Qwen36MLP`` reserves for the current
    stream and for the stream ``torch.cuda.graph`` captures on by default).  The reference keeps one
    scratch buffer per device for all layers in the same way
    (``docker/qwen-c2-graft/graft/mlp.py:274-356``).

    A workspace replaced by a larger one is kept alive, not freed: a HIP graph captured before the
    growth still addresses it, and its replays must not write into memory the caching allocator has
    handed to other tensors.  ``clear()`` drops every workspace, the replaced ones included; call it
    only once no captured graph that used them will be replayed.
    """

    def __init__(self):
        self._ws = {}
        self._retired = []

    @staticmethod
    def _key(device, stream):
        s = stream if stream is not None else torch.cuda.current_stream(device)
        return (torch.device(device).index if torch.device(device).index is not None else torch.cuda.current_device(),
                s.cuda_stream)

    def reserve(self, nbytes, device, stream=None):
        """The workspace of (device, stream), grown to at least ``nbytes`` (outside capture only)."""
        key = self._key(device, stream)
        ws = self._ws.get(key)
        if ws is None or ws.numel() < nbytes:
            if torch.cuda.is_current_stream_capturing():
                raise ValueError(f"no workspace of {nbytes} bytes for stream {key[1]:#x} during graph capture: run one "
                                 "forward on the capturing stream before capturing, or call WorkspacePool.reserve")
            if ws is not None:
                nbytes = max(nbytes, ws.numel())
                self._retired.append(ws)  # a graph captured earlier may still address it
            # allocated with the stream current, so that the caching allocator keeps the new memory
            # stream-ordered with this stream's work
            s = stream if stream is not None else torch.cuda.current_stream(device)
            with torch.cuda.stream(s):
                ws = _new_workspace_bytes(nbytes, device, s)
            self._ws[key] = ws
        return ws

    def total_bytes(self):
        """Bytes of the live workspaces (the replaced ones kept for captured graphs not counted)."""
        return sum(ws.numel() for ws in self._ws.values())

    def retired_bytes(self):
        """Bytes of replaced workspaces kept alive for graphs captured before a growth."""
        return sum(ws.numel() for ws in self._retired)

    def clear(self):
        """Drop every workspace, the replaced ones included (no captured graph may use them again)."""
        self._ws.clear()
        self._retired.clear()


# Shared by every Qwen36MLP unless one is given its own pool.
workspace_pool = WorkspacePool()


@dataclass(frozen=True)
class MLPWeights:
    """Packed MLP weights; field names follow ``docker/qwen-c2-graft/graft/mlp.py:15-20``."""

    w1: PackedWeight  # gate_proj [I, H]
    w2: PackedWeight  # down_proj [H, I]
    w3: PackedWeight  # up_proj   [I, H]

    @property
    def hidden(self):
        return self.w1.cols

    @property
    def intermediate(self):
        return self.w1.rows

    @property
    def fmt(self):
        """MLP weight format ("bf4" = bf4 gate/up with bfp8 down)."""
        return self.w1.fmt

    @property
    def stream_bytes(self):
        return self.w1.stream_bytes + self.w2.stream_bytes + self.w3.stream_bytes


def load_mlp_weights(device, state_dict, tensor_cache_path=None, args=None, weight_format="bfp8", strict=True):
    """Per-layer MLP state -> MLPWeights (``mlp.py:45-169``).

    ``state_dict`` holds ``gate_proj.weight`` / ``up_proj.weight`` ``[I, H]`` and
    ``down_proj.weight`` ``[H, I]`` (HF layout).  ``tensor_cache_path`` (a directory) enables the
    on-disk cache of packed weights, like the reference's ``cache_file_name``.  ``weight_format``
    may also come from ``args.mlp_weight_format``.  A cache entry passes the same checks as a fresh
    conversion: with ``strict`` it must hold no flushed groups, and its shape must match the
    state-dict tensor when the state dict has one.
    """
    fmt = getattr(args, "mlp_weight_format", weight_format) if args is not None else weight_format
    gu_fmt, down_fmt = matrix_formats(fmt)
    device = torch.device(device) if not isinstance(device, torch.device) else device
    if device.type != "cuda":
        raise ValueError(f"device must be a GPU, got {device}")
    names = {"w1": "gate_proj", "w2": "down_proj", "w3": "up_proj"}
    packed = {}
    for field, name in names.items():
        mfmt = down_fmt if field == "w2" else gu_fmt
        cache = None
        if tensor_cache_path is not None:
            from . import weight_cache

            cache = weight_cache.cache_file(tensor_cache_path, name, mfmt)
            pw = weight_cache.load(cache, device) if os.path.exists(cache) else None
            if pw is not None:
                if pw.fmt != mfmt:
                    raise ValueError(f"cache entry {cache} holds {pw.fmt}, expected {mfmt}")
                src = state_dict.get(f"{name}.weight") if hasattr(state_dict, "get") else None
                if src is not None and tuple(src.shape) != (pw.rows, pw.cols):
                    raise ValueError(f"cache entry {cache} is [{pw.rows}, {pw.cols}] but {name}.weight is "
                                     f"{list(src.shape)}: stale cache")
                header = (pw.max_row_norm, pw.flushed_groups)
                _read_info(pw)  # the trailer the kernels read, not the file header's copy of it
                if header != (pw.max_row_norm, pw.flushed_groups):
                    raise ValueError(f"cache entry {cache}: header and packed trailer disagree")
                if strict and pw.flushed_groups:
                    raise ValueError(f"cache entry {cache}: {pw.flushed_groups} {mfmt} groups lie more than 19 "
                                     "binades below their row maximum")
                packed[field] = pw
                continue
        w = state_dict[f"{name}.weight"]
        if not isinstance(w, torch.Tensor):
            w = torch.as_tensor(w)
        w = w.to(device=device, dtype=torch.bfloat16).contiguous()
        packed[field] = pack_weight(w, mfmt, strict=strict)
        del w
        if cache is not None:
            from . import weight_cache

            weight_cache.save(cache, packed[field])
    weights = MLPWeights(**packed)
    I, H = weights.w1.rows, weights.w1.cols
    if (weights.w3.rows, weights.w3.cols) != (I, H) or (weights.w2.rows, weights.w2.cols) != (H, I):
        raise ValueError("gate/up must be [I, H] and down [H, I]")
    check_formats(weights)
    return weights


def check_formats(weights):
    """The three matrices must form one MLP weight format (all alike, or bf4 gate/up + bfp8 down)."""
    gu, down = matrix_formats(weights.w1.fmt) if weights.w1.fmt in WEIGHT_FORMATS else (None, None)
    if weights.w3.fmt != gu or weights.w2.fmt != down:
        raise ValueError(f"weight formats gate={weights.w1.fmt} up={weights.w3.fmt} down={weights.w2.fmt} do not form "
                         f"one of {WEIGHT_FORMATS} (bf4 takes a bfp8 down_proj)")


def mlp_forward(x2d, weights, residual=None, out=None, workspace=None, stream=None, out_dtype=None):
    """``out = residual + down(silu(gate(x)) * up(x))`` for a 2-D bf16 ``[M, H]`` GPU tensor.

    ``residual`` may be bf16 or fp32; ``out`` (or ``out_dtype`` when ``out`` is None) may be bf16
    (rounded once to nearest-even) or fp32 (the unrounded fp32 sum).  ``out`` may be the residual
    tensor itself (in-place residual update).
    """
    _check_device_tensor(x2d, "x", torch.bfloat16)
    M, H = x2d.shape
    I = weights.intermediate
    if H != weights.hidden:
        raise ValueError(f"x has hidden size {H}, weights expect {weights.hidden}")
    flags = 0
    if residual is not None:
        _check_device_tensor(residual, "residual")
        if residual.dtype not in (torch.bfloat16, torch.float32):
            raise ValueError("residual must be bf16 or fp32")
        if tuple(residual.shape) != (M, H):
            raise ValueError("residual must match x")
        if residual.dtype == torch.float32:
            flags |= _lib.RESIDUAL_F32
    if out is None:
        dt = torch.bfloat16 if out_dtype is None else out_dtype
        if dt not in (torch.bfloat16, torch.float32):
            raise ValueError("out_dtype must be bf16 or fp32")
        out = torch.empty((M, H), dtype=dt, device=x2d.device)
    else:
        _check_device_tensor(out, "out")
        if out.dtype not in (torch.bfloat16, torch.float32):
            raise ValueError("out must be bf16 or fp32")
        if tuple(out.shape) != (M, H):
            raise ValueError("out must match x")
    if out.dtype == torch.float32:
        flags |= _lib.OUT_F32
    if workspace is None:
        workspace = new_workspace(M, H, I, weights.fmt, x2d.device, stream)
    rc = _lib.lib().qmlp_forward_ex(_lib.ptr(x2d), _lib.ptr(weights.w1.buf), _lib.ptr(weights.w3.buf),
                                    _lib.ptr(weights.w2.buf), _lib.ptr(residual), _lib.ptr(out),
                                    _lib.ptr(workspace), workspace.numel(), M, H, I, weights.w1.fmt_code, flags,
                                    _lib.stream_handle(stream))
    _lib.check(rc, "qmlp_forward")
    return out


def mlp_forward_rmsnorm(h2d, norm_weight, weights, eps=1e-6, out=None, workspace=None, stream=None,
                        out_dtype=None):
    """``out = h + down(silu(gate(n)) * up(n))`` with ``n = rmsnorm(h) * (1 + norm_weight)``: the
    decoder's ``ffn_norm`` + MLP + residual add (``docker/qwen-c2-graft/graft/layer.py:352-357``)
    in one call.  ``h2d`` bf16 ``[M, H]``; ``norm_weight`` bf16 ``[H]``; ``out`` may be ``h2d``."""
    _check_device_tensor(h2d, "h", torch.bfloat16)
    _check_device_tensor(norm_weight, "norm_weight", torch.bfloat16)
    M, H = h2d.shape
    I = weights.intermediate
    if H != weights.hidden:
        raise ValueError(f"h has hidden size {H}, weights expect {weights.hidden}")
    if tuple(norm_weight.shape) != (H,):
        raise ValueError(f"norm_weight must have shape ({H},)")
    if out is None:
        dt = torch.bfloat16 if out_dtype is None else out_dtype
        if dt not in (torch.bfloat16, torch.float32):
            raise ValueError("out_dtype must be bf16 or fp32")
        out = torch.empty((M, H), dtype=dt, device=h2d.device)
    else:
        _check_device_tensor(out, "out")
        if out.dtype not in (torch.bfloat16, torch.float32) or tuple(out.shape) != (M, H):
            raise ValueError("out must be a bf16 or fp32 [M, H] tensor")
    flags = _lib.OUT_F32 if out.dtype == torch.float32 else 0
    if workspace is None:
        workspace = new_workspace(M, H, I, weights.fmt, h2d.device, stream)
    rc = _lib.lib().qmlp_forward_rmsnorm(_lib.ptr(h2d), _lib.ptr(norm_weight), float(eps), _lib.ptr(weights.w1.buf),
                                         _lib.ptr(weights.w3.buf), _lib.ptr(weights.w2.buf), _lib.ptr(out),
                                         _lib.ptr(workspace), workspace.numel(), M, H, I, weights.w1.fmt_code, flags,
                                         _lib.stream_handle(stream))
    _lib.check(rc, "qmlp_forward_rmsnorm")
    return out


class Qwen36MLP:
    """SwiGLU feed-forward network (``docker/qwen-c2-graft/graft/mlp.py:359-423``) on MI355X.

    ``Qwen36MLP(device, state_dict, tensor_cache_path=None, args=None, tt_ccl=None,
    weight_format="bfp8", max_tokens=2048, pool=None)``; ``forward(x, residual=None, out=None)``.
    Every instance takes its workspace from ``pool`` (the module's shared ``workspace_pool`` by
    default): one workspace per (device, stream) for all layers, reserved here for up to
    ``max_tokens`` rows on the current stream and on the stream ``torch.cuda.graph`` captures on by
    default.  ``forward`` allocates nothing but its output (and nothing at all when ``out`` is
    given), so it may run inside a HIP graph capture on a stream that already holds a large enough
    workspace.
    """

    def __init__(self, mesh_device, state_dict, tensor_cache_path=None, args=None, tt_ccl=None,
                 weight_format="bfp8", max_tokens=2048, pool=None):
        self.device = torch.device(mesh_device) if not isinstance(mesh_device, torch.device) else mesh_device
        self.args = args
        self.tt_ccl = tt_ccl
        self.weights = load_mlp_weights(self.device, state_dict, tensor_cache_path, args, weight_format)
        self.max_tokens = int(max_tokens)
        self.pool = workspace_pool if pool is None else pool
        nbytes = self._workspace_bytes(self.max_tokens)
        self.pool.reserve(nbytes, self.device)
        # torch.cuda.graph(g) without a stream captures on its own side stream: give it a workspace
        # too, so that the usual warm-up-then-capture pattern needs no stream argument
        cap = graph_capture_stream(self.device)
        if cap.device == self.device or (cap.device.index is None and self.device.index in (None, 0)):
            self.pool.reserve(nbytes, self.device, cap)

    @property
    def weight_format(self):
        return self.weights.fmt

    def _workspace_bytes(self, M):
        return workspace_bytes(M, self.weights.hidden, self.weights.intermediate, self.weights.fmt)

    def _workspace_for(self, M):
        # sizes never shrink as M grows, so the reservation for max_tokens covers every smaller call
        if M > self.max_tokens and not torch.cuda.is_current_stream_capturing():
            self.max_tokens = M
        return self.pool.reserve(self._workspace_bytes(max(M, self.max_tokens)), self.device)

    def forward(self, x, residual=None, out=None, out_dtype=None):
        if not isinstance(x, torch.Tensor) or x.dtype != torch.bfloat16:
            raise ValueError("BF16 activation tensor required")
        if x.dim() < 1 or x.shape[-1] != self.weights.hidden:
            raise ValueError(f"activation must end in hidden size {self.weights.hidden}, got {tuple(x.shape)}")
        if x.device.type != "cuda":
            raise ValueError("activation must be on the GPU")
        shape = x.shape
        x2d = x.reshape(-1, shape[-1])
        if not x2d.is_contiguous():
            x2d = x2d.contiguous()
        M = x2d.shape[0]
        if M == 0:
            raise ValueError("empty activation")
        r2d = None
        if residual is not None:
            if tuple(residual.shape) != tuple(shape):
                raise ValueError("residual must have the activation's shape")
            r2d = residual.reshape(M, shape[-1])
        o2d = None
        if out is not None:
            if tuple(out.shape) != tuple(shape):
                raise ValueError("out must have the activation's shape")
            if not out.is_contiguous():  # a reshape would write into a copy
                raise ValueError("out must be contiguous")
            o2d = out.reshape(M, shape[-1])
        y = mlp_forward(x2d, self.weights, residual=r2d, out=o2d, workspace=self._workspace_for(M),
                        out_dtype=out_dtype)
        return y.reshape(shape) if out is None else out

    __call__ = forward

    def forward_rmsnorm(self, h, norm_weight, eps=1e-6, out=None, out_dtype=None):
        """``h + self.forward(rmsnorm(h) * (1 + norm_weight))`` in one call: the decoder's
        ``ffn_norm`` -> MLP -> residual add (``layer.py:352-357``).  ``h`` ``[..., H]`` bf16;
        ``out`` may be ``h`` itself."""
        if not isinstance(h, torch.Tensor) or h.dtype != torch.bfloat16 or h.device.type != "cuda":
            raise ValueError("h must be a bf16 GPU tensor")
        if h.dim() < 1 or h.shape[-1] != self.weights.hidden:
            raise ValueError(f"h must end in hidden size {self.weights.hidden}, got {tuple(h.shape)}")
        shape = h.shape
        h2d = h.reshape(-1, shape[-1])
        if not h2d.is_contiguous():
            h2d = h2d.contiguous()
        M = h2d.shape[0]
        o2d = None
        if out is not None:
            if tuple(out.shape) != tuple(shape):
                raise ValueError("out must have h's shape")
            if not out.is_contiguous():  # a reshape would write into a copy
                raise ValueError("out must be contiguous")
            o2d = out.reshape(M, shape[-1])
        y = mlp_forward_rmsnorm(h2d, norm_weight, self.weights, eps=eps, out=o2d, workspace=self._workspace_for(M),
                                out_dtype=out_dtype)
        return y.reshape(shape) if out is None else out
