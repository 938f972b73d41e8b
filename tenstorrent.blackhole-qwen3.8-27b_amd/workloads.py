"""Seeded synthetic MLP workloads (activations and random-init weights of the Qwen3 shapes).

There are no checkpoints offline, so weights are ``N(0, 0.02)`` bf16 and activations ``N(0, 1)``
bf16, optionally scaled per hidden channel by an RMSNorm-like gain ``U(0.5, 1.5)``.  The seeds follow
the reference's convention of separate activation and weight seeds (``1000 + seed`` /
``2000 + seed``, ``optimisation/ttnn-op/c1e_gateup/c1e_gateup_card_b.py:128-151``).
"""
from dataclasses import dataclass

import torch

QWEN3_27B = {"hidden": 5120, "intermediate": 17408}
PLUMBING = {"hidden": 1024, "intermediate": 3072}
X_SEED = 1000
W_SEED = 2000


@dataclass(frozen=True)
class Workload:
    name: str
    hidden: int
    intermediate: int
    tokens: int
    fmt: str
    gain: bool  # RMSNorm-like per-channel gain on the activations

    def weight_bytes(self):
        """Bytes of the three matrices' values (gate/up and down per the weight format; "bf4"
        pairs bf4 gate/up with a bfp8 down)."""
        per = {"bfp8": 17 / 16, "bf4": 9 / 16, "bf16": 2}
        gu = self.fmt
        down = "bfp8" if self.fmt == "bf4" else self.fmt
        return int(self.hidden * self.intermediate * (2 * per[gu] + per[down]))

    def algorithmic_bytes(self):
        """Weights streamed once + activation read + output write + residual read (bf16):
        W + 4*M*H bytes per layer."""
        return self.weight_bytes() + 4 * self.tokens * self.hidden

    def flops(self):
        return 6 * self.tokens * self.hidden * self.intermediate


WORKLOADS = {
    "plumbing-h1024-i3072-m1-bf16": Workload("plumbing-h1024-i3072-m1-bf16", 1024, 3072, 1, "bf16", False),
    "qwen3-27b-mlp-m16-bf16": Workload("qwen3-27b-mlp-m16-bf16", 5120, 17408, 16, "bf16", True),
    "qwen3-27b-mlp-m16-bfp8": Workload("qwen3-27b-mlp-m16-bfp8", 5120, 17408, 16, "bfp8", True),
    "qwen3-27b-mlp-m1-bfp8": Workload("qwen3-27b-mlp-m1-bfp8", 5120, 17408, 1, "bfp8", True),
    "qwen3-27b-mlp-m32-bfp8": Workload("qwen3-27b-mlp-m32-bfp8", 5120, 17408, 32, "bfp8", True),
    # a 64-token verify window: the many-token kernels with every tile split
    "qwen3-27b-mlp-m64-bfp8": Workload("qwen3-27b-mlp-m64-bfp8", 5120, 17408, 64, "bfp8", True),
    "qwen3-27b-mlp-prefill-m2048-bfp8": Workload("qwen3-27b-mlp-prefill-m2048-bfp8", 5120, 17408, 2048, "bfp8", False),
    "qwen3-27b-mlp-m16-bf4": Workload("qwen3-27b-mlp-m16-bf4", 5120, 17408, 16, "bf4", True),
    "qwen3-27b-mlp-m1-bf4": Workload("qwen3-27b-mlp-m1-bf4", 5120, 17408, 1, "bf4", True),
    "qwen3-27b-mlp-m32-bf4": Workload("qwen3-27b-mlp-m32-bf4", 5120, 17408, 32, "bf4", True),
    "qwen3-27b-mlp-prefill-m2048-bf4": Workload("qwen3-27b-mlp-prefill-m2048-bf4", 5120, 17408, 2048, "bf4", False),
    # one GPU's share of a layer split two ways along the intermediate dimension (the reference's
    # TP2 shard: gate/up rows and down columns 8704 of 17408, docker/qwen-c2-graft/graft/mlp.py:49-151)
    "qwen3-27b-tp2-share-m16-bfp8": Workload("qwen3-27b-tp2-share-m16-bfp8", 5120, 8704, 16, "bfp8", True),
    "qwen3-27b-tp2-share-m16-bf4": Workload("qwen3-27b-tp2-share-m16-bf4", 5120, 8704, 16, "bf4", True),
}


def _gen(seed, device):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def activations(tokens, hidden, seed=X_SEED, gain=True, device="cuda"):
    """bf16 ``[tokens, hidden]``: N(0,1), times a per-channel gain U(0.5, 1.5) when ``gain``."""
    g = _gen(seed, device)
    x = torch.randn((tokens, hidden), generator=g, device=device, dtype=torch.float32)
    if gain:
        x = x * (0.5 + torch.rand((hidden,), generator=g, device=device, dtype=torch.float32))
    return x.to(torch.bfloat16)


def weight(rows, cols, seed, std=0.02, device="cuda"):
    """bf16 ``[rows, cols]`` ~ N(0, std)."""
    g = _gen(seed, device)
    return (torch.randn((rows, cols), generator=g, device=device, dtype=torch.float32) * std).to(torch.bfloat16)


def state_dict(hidden, intermediate, layer=0, device="cuda"):
    """HF-layout MLP tensors of one layer, seeds 2000 + 3*layer + {0: gate, 1: up, 2: down}."""
    base = W_SEED + 3 * layer
    return {
        "gate_proj.weight": weight(intermediate, hidden, base + 0, device=device),
        "up_proj.weight": weight(intermediate, hidden, base + 1, device=device),
        "down_proj.weight": weight(hidden, intermediate, base + 2, device=device),
    }
