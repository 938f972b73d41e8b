"""Verify-loop integration: route a decoder's MLP calls at the verify width to this library.

Counterpart of the reference's opt-in M = 16 arm ``FusedT16Arm``
(``scripts/ci/fused_t16_scope.py:11-94``).  The contract is the same:
* while a scope is open, each decoder MLP instance answers calls of the verify shape
  ``[1, 1, token_rows, H]`` with this library and every other call with its own ``forward``;
* the scope counts hits and fallbacks per layer;
* on exit it checks that every binding is back and that no weight moved
  (``fused_t16_scope.py:40-43,84-94``);
* before the first scope opens, it checks that each layer's library weights are that layer's own
  weights, byte for byte, and refuses to install otherwise (the reference's admission check
  ``qualify_target_weights``, ``scripts/ci/fused_t16_admission.py:36-69``, which compares the
  fused op's packed gate/up with each layer's own w1/w3 for all 64 layers).

The design here is a context-manager object.  It stores a small callable ``_Route`` per layer in
that instance's own ``__dict__``, keeps a snapshot of what the ``__dict__`` held before, and puts
the snapshot back on exit.  The weights it audits are the packed buffers this library streams:
their device addresses and sizes must be the same on exit as on entry.  Platform differences:
* activations are torch GPU tensors;
* each layer's weights are this library's packed copies (one ``Qwen36MLP`` per layer);
* there is no collective, because one GPU runs the unsharded layer.
"""
import torch

_ABSENT = object()  # marks an instance that had no ``forward`` attribute of its own
_PROJECTIONS = (("w1", "gate_proj"), ("w3", "up_proj"), ("w2", "down_proj"))


def decoder_mlp_weights(mlp):
    """The HF-layout weights ``{gate,up,down}_proj.weight`` of a decoder MLP module: from its
    ``state_dict()`` (a torch ``nn.Module`` MLP such as HF's), else from ``gate_proj.weight``-style
    attributes.  Returns None if the module exposes neither."""
    keys = [f"{name}.weight" for _, name in _PROJECTIONS]
    if callable(getattr(mlp, "state_dict", None)):
        sd = mlp.state_dict()
        if all(k in sd for k in keys):
            return {k: sd[k] for k in keys}
    out = {}
    for _, name in _PROJECTIONS:
        w = getattr(getattr(mlp, name, None), "weight", None)
        if not isinstance(w, torch.Tensor):
            return None
        out[f"{name}.weight"] = w
    return out


class _Route:
    """Installed as one decoder MLP's ``forward`` while a scope is open: sends the call to the arm
    together with the layer's index."""

    __slots__ = ("arm", "index")

    def __init__(self, arm, index):
        self.arm = arm
        self.index = index

    def __call__(self, value):
        return self.arm._dispatch(self.index, value)


class VerifyArm:
    """``VerifyArm(mlps, amd_mlps, token_rows=16, source_weights=None, check_weights=True)``.

    ``mlps`` are the decoder's feed-forward modules (objects with a ``forward(x)`` method).
    ``amd_mlps`` are the matching ``Qwen36MLP`` instances.  ``with arm.install(): ...`` opens a
    scope.  After it closes, ``arm.audit`` holds the per-layer hit and fallback counts, whether
    every binding was restored, and whether every packed weight stayed at its address.  A failed
    audit raises ``AssertionError``, unless the scope is already ending with an exception: that
    exception then propagates unchanged, and the audit records what went wrong.

    Layer correspondence: before the first scope opens (outside any graph capture), each layer's
    three packed matrices must be byte-equal to what the library packs from that decoder layer's
    own ``{gate,up,down}_proj.weight`` in the same format -- ``source_weights(i, mlp)`` returns
    them, by default ``decoder_mlp_weights(mlp)``.  A mismatch (a swapped, stale or foreign
    pairing) raises ``ValueError`` and nothing is installed.  ``check_weights=False`` skips the
    check, for decoder modules that do not expose their weights.
    """

    def __init__(self, mlps, amd_mlps, token_rows=16, source_weights=None, check_weights=True):
        mlps, amd_mlps = list(mlps), list(amd_mlps)
        if token_rows not in (16, 32):
            raise ValueError("verify width must be 16 or 32 token rows")
        if len(mlps) != len(amd_mlps):
            raise ValueError("one library MLP per decoder MLP required")
        if len({id(m) for m in mlps}) != len(mlps):
            raise ValueError("distinct MLP instances required")
        self.token_rows = token_rows
        self._modules = mlps
        self._amd = amd_mlps
        self._source = source_weights if source_weights is not None else (lambda i, m: decoder_mlp_weights(m))
        self._check = bool(check_weights)
        self._checked = None  # the weight bindings that passed the correspondence check
        self.weight_checks = []
        self._native = [None] * len(mlps)  # each layer's own forward, resolved when a scope opens
        self._saved = []
        self._weights_at_entry = None
        self.hits = [0] * len(mlps)
        self.fallbacks = [0] * len(mlps)
        self._open = False
        self.audit = {}

    @property
    def active(self):
        return self._open

    # ------------------------------------------------------------------ routing

    def _dispatch(self, index, value):
        if not self._open:
            raise RuntimeError("the arm requires an active scope")
        amd = self._amd[index]
        verify_shape = (1, 1, self.token_rows, amd.weights.hidden)
        if not (isinstance(value, torch.Tensor) and value.device.type == "cuda" and tuple(value.shape) == verify_shape):
            self.fallbacks[index] += 1
            return self._native[index](value)
        if value.dtype != torch.bfloat16:
            raise ValueError("bf16 activation required")
        self.hits[index] += 1
        return amd.forward(value)

    # ------------------------------------------------------------------ audit helpers

    def _weight_bindings(self):
        """(weights object, then address and size of each packed buffer) per layer."""
        out = []
        for amd in self._amd:
            w = amd.weights
            out.append((id(w),) + tuple((pw.buf.data_ptr(), pw.buf.numel()) for pw in (w.w1, w.w2, w.w3)))
        return out

    def check_layer_weights(self):
        """Byte-compares every layer's packed matrices with the library's packing of that layer's
        own weights; raises ``ValueError`` naming the first layer and matrix that differ."""
        from .mlp import pack_weight

        if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
            raise RuntimeError("the layer weight check cannot run during graph capture")
        checks = []
        for i, (mlp, amd) in enumerate(zip(self._modules, self._amd)):
            sd = self._source(i, mlp)
            if sd is None:
                raise ValueError(f"layer {i}: the decoder MLP exposes no gate_proj/up_proj/down_proj weights to check "
                                 "the library's packed copy against (pass source_weights=, or check_weights=False)")
            for field, name in _PROJECTIONS:
                pw = getattr(amd.weights, field)
                w = sd[f"{name}.weight"]
                if tuple(w.shape) != (pw.rows, pw.cols):
                    raise ValueError(f"layer {i}: {name} is {list(w.shape)} in the decoder but [{pw.rows}, {pw.cols}] "
                                     "in the library")
                w = w.to(device=pw.buf.device, dtype=torch.bfloat16).contiguous()
                ref = pack_weight(w, pw.fmt, strict=False)
                exact = ref.buf.numel() == pw.buf.numel() and bool(torch.equal(ref.buf, pw.buf))
                del ref, w
                if not exact:
                    raise ValueError(f"layer {i}: the library's packed {name} is not this decoder layer's weight "
                                     f"(swapped, stale or foreign pairing)")
                checks.append(dict(layer=i, matrix=name, fmt=pw.fmt, bytes=pw.buf.numel(), exact=True))
        self.weight_checks = checks
        self._checked = self._weight_bindings()
        return checks

    # ------------------------------------------------------------------ scope

    def install(self):
        """The scope object itself: ``with arm.install(): ...``."""
        return self

    def __enter__(self):
        if self._open:
            raise RuntimeError("scope already active")
        if self._check and self._checked != self._weight_bindings():
            self.check_layer_weights()  # raises before anything is installed
        self._saved = [m.__dict__.get("forward", _ABSENT) for m in self._modules]
        self._native = [m.forward for m in self._modules]
        self._weights_at_entry = self._weight_bindings()
        try:
            for i, m in enumerate(self._modules):
                m.forward = _Route(self, i)
        except BaseException:
            self._restore()
            raise
        self._open = True
        return self

    def _restore(self):
        for m, saved in zip(self._modules, self._saved):
            if saved is _ABSENT:
                m.__dict__.pop("forward", None)
            else:
                m.__dict__["forward"] = saved

    def __exit__(self, exc_type, exc, tb):
        self._open = False
        self._restore()
        restored = all(m.forward == native for m, native in zip(self._modules, self._native))
        weights_unchanged = self._weight_bindings() == self._weights_at_entry
        self.audit = dict(rows=self.token_rows, layers=len(self._modules), hits=list(self.hits),
                          fallbacks=list(self.fallbacks), restored=restored, weights_unchanged=weights_unchanged,
                          weights_checked=len(self.weight_checks) if self._check else 0)
        if exc_type is None:
            if not restored:
                raise AssertionError("MLP bindings changed during the scope")
            if not weights_unchanged:
                raise AssertionError("packed MLP weights moved during the scope")
        return False  # never swallow the scope's own exception
