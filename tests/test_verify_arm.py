"""The verify arm's scope logic on the CPU (no kernel calls): instance bindings installed and
restored, fallbacks counted, the packed-weight address audit, and exceptions inside the scope
propagating unchanged -- the contract of the reference's FusedT16Arm
(scripts/ci/fused_t16_scope.py:40-51,78-94)."""
import types

import pytest
import torch


def _arm_module(pkg):
    from qwen_mlp_amd import verify_arm

    return verify_arm


class FakeMLP:
    def __init__(self, tag):
        self.tag = tag
        self.calls = 0

    def forward(self, x):
        self.calls += 1
        return x + self.tag


def _fake_amd(hidden=8):
    def pw():
        return types.SimpleNamespace(buf=torch.zeros(64, dtype=torch.uint8))

    weights = types.SimpleNamespace(hidden=hidden, w1=pw(), w2=pw(), w3=pw())
    return types.SimpleNamespace(weights=weights, forward=lambda x: pytest.fail("no library call expected on the CPU"))


def test_scope_routes_falls_back_and_restores(pkg):
    va = _arm_module(pkg)
    mlps = [FakeMLP(1.0), FakeMLP(2.0)]
    own = lambda x: x * 10  # noqa: E731 -- an instance-level override that must survive the scope
    mlps[1].forward = own
    arm = va.VerifyArm(mlps, [_fake_amd(), _fake_amd()], token_rows=16, check_weights=False)
    x = torch.zeros(1, 1, 16, 8)  # the verify shape, but on the CPU: falls back
    with arm.install() as scope:
        assert scope is arm and arm.active
        assert "forward" in mlps[0].__dict__ and mlps[1].forward is not own
        assert torch.equal(mlps[0].forward(x), x + 1.0)
        assert torch.equal(mlps[1].forward(x), x * 10)
        assert torch.equal(mlps[0].forward(torch.ones(3)), torch.ones(3) + 1.0)
    assert not arm.active
    assert "forward" not in mlps[0].__dict__ and mlps[1].forward is own
    assert arm.audit == dict(rows=16, layers=2, hits=[0, 0], fallbacks=[2, 1], restored=True, weights_unchanged=True,
                          weights_checked=0)
    assert mlps[0].calls == 2


def test_route_outside_scope_raises(pkg):
    va = _arm_module(pkg)
    mlp = FakeMLP(0.0)
    arm = va.VerifyArm([mlp], [_fake_amd()], check_weights=False)
    with arm.install():
        route = mlp.forward
    with pytest.raises(RuntimeError):
        route(torch.zeros(2))


def test_nested_scope_refused(pkg):
    va = _arm_module(pkg)
    arm = va.VerifyArm([FakeMLP(0.0)], [_fake_amd()], check_weights=False)
    with arm.install():
        with pytest.raises(RuntimeError):
            arm.__enter__()
    assert not arm.active


def test_moved_weights_fail_the_audit(pkg):
    va = _arm_module(pkg)
    amd = _fake_amd()
    mlp = FakeMLP(0.0)
    arm = va.VerifyArm([mlp], [amd], check_weights=False)
    with pytest.raises(AssertionError, match="moved"):
        with arm.install():
            amd.weights.w2.buf = torch.zeros(64, dtype=torch.uint8)  # a new allocation
    assert arm.audit["weights_unchanged"] is False and arm.audit["restored"] is True
    assert "forward" not in mlp.__dict__


def test_rebinding_inside_scope_is_undone(pkg):
    va = _arm_module(pkg)
    mlp = FakeMLP(0.0)
    arm = va.VerifyArm([mlp], [_fake_amd()], check_weights=False)
    with arm.install():
        mlp.forward = lambda x: x  # someone else rebinds during the scope
    assert "forward" not in mlp.__dict__ and arm.audit["restored"]


def test_exception_in_scope_propagates_unchanged(pkg):
    va = _arm_module(pkg)
    amd = _fake_amd()
    mlp = FakeMLP(0.0)
    arm = va.VerifyArm([mlp], [amd], check_weights=False)
    with pytest.raises(ZeroDivisionError):
        with arm.install():
            amd.weights.w1.buf = torch.zeros(64, dtype=torch.uint8)  # would fail the audit ...
            1 / 0  # ... but the scope's own error is what the caller sees
    assert arm.audit["weights_unchanged"] is False
    assert "forward" not in mlp.__dict__ and not arm.active


def test_constructor_checks(pkg):
    va = _arm_module(pkg)
    m = FakeMLP(0.0)
    with pytest.raises(ValueError):
        va.VerifyArm([m], [_fake_amd()], token_rows=8)
    with pytest.raises(ValueError):
        va.VerifyArm([m, m], [_fake_amd(), _fake_amd()])
    with pytest.raises(ValueError):
        va.VerifyArm([m], [])


def test_weight_check_needs_the_decoder_weights(pkg):
    """With the correspondence check on, a decoder MLP that exposes no weights is refused at
    install, before anything is bound."""
    va = _arm_module(pkg)
    mlp = FakeMLP(0.0)
    arm = va.VerifyArm([mlp], [_fake_amd()])
    with pytest.raises(ValueError, match="exposes no gate_proj"):
        with arm.install():
            pytest.fail("the scope must not open")
    assert "forward" not in mlp.__dict__ and not arm.active


def test_decoder_mlp_weights_sources(pkg):
    """The decoder's weights come from an nn.Module's state_dict (HF's gate_proj / up_proj /
    down_proj Linear layers) or from gate_proj.weight-style attributes."""
    va = _arm_module(pkg)
    H, I = 8, 16

    class HFMLP(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.gate_proj = torch.nn.Linear(H, I, bias=False)
            self.up_proj = torch.nn.Linear(H, I, bias=False)
            self.down_proj = torch.nn.Linear(I, H, bias=False)

    m = HFMLP()
    sd = va.decoder_mlp_weights(m)
    assert sorted(sd) == ["down_proj.weight", "gate_proj.weight", "up_proj.weight"]
    assert sd["gate_proj.weight"].data_ptr() == m.gate_proj.weight.data_ptr()
    plain = types.SimpleNamespace(**{k: types.SimpleNamespace(weight=torch.zeros(2)) for k in
                                     ("gate_proj", "up_proj", "down_proj")})
    assert va.decoder_mlp_weights(plain)["up_proj.weight"] is plain.up_proj.weight
    assert va.decoder_mlp_weights(FakeMLP(0.0)) is None


def test_weight_check_refuses_a_shape_mismatch(pkg):
    """Matrices of another shape than the library's packed copy are refused (before any packing)."""
    va = _arm_module(pkg)

    def pw(rows, cols):
        return types.SimpleNamespace(buf=torch.zeros(64, dtype=torch.uint8), rows=rows, cols=cols, fmt="bfp8")

    weights = types.SimpleNamespace(hidden=256, w1=pw(512, 256), w2=pw(256, 512), w3=pw(512, 256))
    amd = types.SimpleNamespace(weights=weights)
    src = {"gate_proj.weight": torch.zeros(256, 512), "up_proj.weight": torch.zeros(512, 256),
           "down_proj.weight": torch.zeros(256, 512)}
    mlp = FakeMLP(0.0)
    arm = va.VerifyArm([mlp], [amd], source_weights=lambda i, m: src)
    with pytest.raises(ValueError, match="layer 0: gate_proj is"):
        with arm.install():
            pytest.fail("the scope must not open")
    assert "forward" not in mlp.__dict__
