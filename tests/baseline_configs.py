"""The five BASELINE.json configurations (config 4 has variants 4a and 4b).

Shapes, paths and value distributions as BASELINE.json states them:
x ~ N(0,1); dt = softplus(N(mu, sigma)) (the ABI receives the pre-softplus
value); A = -exp(U(ln 1, ln 16)); B, C ~ N(0,1)/sqrt(N); h0 zero or N(0, 0.1)
(0.1 read as the standard deviation). Seed 1000 + config index.
"""
from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class Config:
    name: str
    L: int
    S: int
    H: int
    P: int
    N: int
    G: int
    paths: tuple          # "fp32" and/or "bf16"
    seed: int
    s0_sigma: float = 0.0
    dt_mu: float = -1.0
    dt_sigma: float = 0.5
    check_heads: tuple = ()   # heads the CPU oracle recomputes at full size

    @property
    def shape(self):
        return self.L, self.S, self.H, self.P, self.N, self.G


CONFIGS = {
    "cfg0": Config("cfg0", 256, 1, 8, 64, 64, 1, ("fp32",), 1000, check_heads=tuple(range(8))),
    "cfg1": Config("cfg1", 2048, 1, 64, 64, 128, 8, ("fp32",), 1001, check_heads=(0, 9, 36, 63)),
    "cfg2": Config("cfg2", 8192, 1, 64, 64, 128, 8, ("bf16", "fp32"), 1002, check_heads=(0, 15, 40, 63)),
    "cfg3": Config("cfg3", 1000, 4, 32, 128, 128, 1, ("fp32",), 1003, s0_sigma=0.1, dt_mu=-2.0,
                   dt_sigma=1.0, check_heads=(0, 13, 31)),
    "cfg4a": Config("cfg4a", 4096, 8, 80, 64, 128, 1, ("bf16",), 1004, s0_sigma=0.1,
                    check_heads=(0, 41, 79)),
    "cfg4b": Config("cfg4b", 4096, 8, 27, 192, 128, 1, ("bf16",), 1005, s0_sigma=0.1,
                    check_heads=(0, 26)),
}
