"""Seeded synthetic inputs for the benchmark configurations.

Seeds: 0 activations, 1 router logits, 2 router bias, 3 weights, 4 grads,
5 expert-id shuffle.  Generators run on the requested device; CPU generation
is bit-reproducible everywhere and is what the parity tests use.

Benchmark configurations 1-5:
  tiny     T=2048  H=1024 E=8   K=2 I=2048     whole layer, CPU-checkable
  permute  T=16384 H=7168 E=256 K=8            permute + quantise (headline)
  mixtral  T=8192  H=4096 E=8   K=2 I=14336    whole layer
  dsv3     R=65536 H=7168 E=32      I=2048     grouped GEMM, Zipf(1.2) loads
  qwen3    T=16384 H=2048 E=128 K=8 I=768      forward (+ backward later)
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

SEED_X, SEED_LOGITS, SEED_BIAS, SEED_W, SEED_GRAD, SEED_SHUFFLE = 0, 1, 2, 3, 4, 5


@dataclass(frozen=True)
class Config:
    name: str
    T: int
    H: int
    E: int
    K: int
    I: int = 0
    bias: bool = False
    outliers: bool = False


CONFIGS = {
    "tiny": Config("tiny", T=2048, H=1024, E=8, K=2, I=2048),
    "permute": Config("permute", T=16384, H=7168, E=256, K=8, bias=True, outliers=True),
    "mixtral": Config("mixtral", T=8192, H=4096, E=8, K=2, I=14336),
    "dsv3": Config("dsv3", T=65536, H=7168, E=32, K=1, I=2048),
    "qwen3": Config("qwen3", T=16384, H=2048, E=128, K=8, I=768),
}


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def tokens(T: int, H: int, device="cpu", outliers: bool = False, seed: int = SEED_X) -> torch.Tensor:
    """bf16 [T,H] ~ N(0,1); with ``outliers`` 0.1% of entries (seeded index
    sample, duplicates possible) are scaled by 50."""
    g = _gen(seed, device)
    x = torch.randn((T, H), generator=g, device=device, dtype=torch.float32)
    if outliers:
        n = max(1, (T * H) // 1000)
        pos = torch.randint(0, T * H, (n,), generator=g, device=device)
        x.view(-1)[pos] *= 50.0
    return x.to(torch.bfloat16)


def logits(T: int, E: int, device="cpu", seed: int = SEED_LOGITS) -> torch.Tensor:
    return torch.randn((T, E), generator=_gen(seed, device), device=device, dtype=torch.float32)


def router_bias(E: int, device="cpu", seed: int = SEED_BIAS) -> torch.Tensor:
    return torch.randn((E,), generator=_gen(seed, device), device=device, dtype=torch.float32) * 0.5


def weights(E: int, N: int, K: int, device="cpu", seed: int = SEED_W, std: float = 0.02) -> torch.Tensor:
    """bf16 [E,N,K] ~ N(0, std), generated in slabs to bound fp32 scratch."""
    g = _gen(seed, device)
    out = torch.empty((E, N, K), dtype=torch.bfloat16, device=device)
    for e in range(E):
        out[e] = (torch.randn((N, K), generator=g, device=device, dtype=torch.float32) * std).to(torch.bfloat16)
    return out


def zipf_counts(R: int = 65536, E: int = 32, alpha: float = 1.2, zeros: int = 4,
                seed: int = SEED_SHUFFLE) -> list[int]:
    """Per-expert row counts: Zipf(alpha) shares over ranks 1..E-zeros, rounded
    by largest remainder to sum exactly R; ``zeros`` experts get no rows; the
    rank -> expert-id assignment is a seeded shuffle."""
    n = E - zeros
    w = [1.0 / (k ** alpha) for k in range(1, n + 1)]
    tot = sum(w)
    raw = [R * x / tot for x in w]
    base = [int(v) for v in raw]
    rem = R - sum(base)
    order = sorted(range(n), key=lambda i: (-(raw[i] - base[i]), i))
    for i in order[:rem]:
        base[i] += 1
    perm = torch.randperm(E, generator=_gen(seed, "cpu")).tolist()
    counts = [0] * E
    for rank, c in enumerate(base):
        counts[perm[rank]] = c
    return counts


def offsets_from_counts(counts, device="cpu") -> torch.Tensor:
    off = [0]
    for c in counts:
        off.append(off[-1] + int(c))
    return torch.tensor(off, dtype=torch.int32, device=device)
