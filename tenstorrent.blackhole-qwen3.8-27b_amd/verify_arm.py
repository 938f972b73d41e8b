"""Verify-loop integration: route a decoder's MLP calls at the verify width to this library.

Counterpart of the reference's opt-in M = 16 arm ``FusedT16Arm``
(``scripts/ci/fused_t16_scope.py:11-94``).  The contract is the same:
* while a scope is open, each decoder MLP instance answers calls of the verify shape
  ``[1, 1, token_rows, H]`` with this library and every other call with its own ``forward``;
* the scope counts hits and fallbacks per layer;
* on exit it checks that every binding is back and that no weight moved
  (``fused_t16_scope.py:40-43,84-94``).

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
    """``VerifyArm(mlps, amd_mlps, token_rows=16)``.

    ``mlps`` are the decoder's feed-forward modules (objects with a ``forward(x)`` method).
    ``amd_mlps`` are the matching ``Qwen36MLP`` instances.  ``with arm.install(): ...`` opens a
    scope.  After it closes, ``arm.audit`` holds the per-layer hit and fallback counts, whether
    every binding was restored, and whether every packed weight stayed at its address.  A failed
    audit raises ``AssertionError``, unless the scope is already ending with an exception: that
    exception then propagates unchanged, and the audit records what went wrong.
    """

    def __init__(self, mlps, amd_mlps, token_rows=16):
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

    # ------------------------------------------------------------------ scope

    def install(self):
        """The scope object itself: ``with arm.install(): ...``."""
        return self

    def __enter__(self):
        if self._open:
            raise RuntimeError("scope already active")
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
                          fallbacks=list(self.fallbacks), restored=restored, weights_unchanged=weights_unchanged)
        if exc_type is None:
            if not restored:
                raise AssertionError("MLP bindings changed during the scope")
            if not weights_unchanged:
                raise AssertionError("packed MLP weights moved during the scope")
        return False  # never swallow the scope's own exception
