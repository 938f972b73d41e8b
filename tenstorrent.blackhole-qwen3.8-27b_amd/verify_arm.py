"""Verify-loop integration: route a decoder's MLP calls at the verify width to this library.

Counterpart of the reference's opt-in M = 16 arm ``FusedT16Arm`` (``scripts/ci/fused_t16_scope.py:11-94``):
for the duration of a scope every layer's ``feed_forward.forward`` is replaced, per instance, by a
function that runs this library when the activation has the verify shape ``[1, 1, token_rows, H]``
and calls the layer's original ``forward`` otherwise; the scope counts hits and fallbacks per layer
and checks on exit that every original binding is back (``fused_t16_scope.py:84-94``).

Differences that follow from the platform: the activations are torch GPU tensors, the weights are
this library's packed copies (``Qwen36MLP`` per layer, built from each layer's HF state dict), and
there is no collective (one GPU runs the unsharded layer).
"""
from contextlib import contextmanager

import torch


@contextmanager
def instance_overrides(bindings):
    """Set ``instance.name = value`` for each ``(instance, name, value)`` and restore the previous
    instance attribute (or its absence) on exit, even after an exception."""
    previous = []
    try:
        for instance, name, value in bindings:
            previous.append((instance, name, name in instance.__dict__, instance.__dict__.get(name)))
            setattr(instance, name, value)
        yield
    finally:
        for instance, name, existed, value in reversed(previous):
            if existed:
                setattr(instance, name, value)
            else:
                delattr(instance, name)


class VerifyArm:
    """``VerifyArm(mlps, amd_mlps, token_rows=16)``: ``mlps`` are the decoder's feed-forward modules
    (objects with a ``forward(x)`` method), ``amd_mlps`` the matching ``Qwen36MLP`` instances."""

    def __init__(self, mlps, amd_mlps, token_rows=16):
        if token_rows not in (16, 32):
            raise ValueError("verify width must be 16 or 32 token rows")
        if len(mlps) != len(amd_mlps):
            raise ValueError("one library MLP per decoder MLP required")
        if len({id(m) for m in mlps}) != len(mlps):
            raise ValueError("distinct MLP instances required")
        self.token_rows = token_rows
        self.originals = [(m, m.forward) for m in mlps]
        self.amd = list(amd_mlps)
        self.hits = [0] * len(mlps)
        self.fallbacks = [0] * len(mlps)
        self.active = False
        self.audit = {}

    def forward(self, index, value):
        if not self.active:
            raise RuntimeError("the arm requires an active scope")
        mlp, original = self.originals[index]
        amd = self.amd[index]
        if (not isinstance(value, torch.Tensor) or tuple(value.shape) != (1, 1, self.token_rows, amd.weights.hidden)
                or value.device.type != "cuda"):
            self.fallbacks[index] += 1
            return original(value)
        if value.dtype != torch.bfloat16:
            raise ValueError("bf16 activation required")
        self.hits[index] += 1
        return amd.forward(value)

    @contextmanager
    def install(self):
        if self.active:
            raise RuntimeError("scope already active")
        self.active = True
        try:
            with instance_overrides([(mlp, "forward", lambda value, index=index: self.forward(index, value))
                                     for index, (mlp, original) in enumerate(self.originals)]):
                yield self
        finally:
            self.active = False
            restored = all(mlp.forward == original for mlp, original in self.originals)
            self.audit = dict(rows=self.token_rows, layers=len(self.originals), hits=list(self.hits),
                              fallbacks=list(self.fallbacks), restored=restored)
            if not restored:
                raise AssertionError("MLP bindings changed during the scope")
