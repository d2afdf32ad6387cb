"""Seeded synthetic decode workloads (Qwen3-VL-2B text-decoder attention shapes).

Mirrors the input construction of the reference's decode microbenchmark
(message/run_triton_attention_microbench.py:199-215: q [B,Hq,1,D], k/v [B,Hkv,L,D] drawn N(0,1)) and
extends it to the five measured configurations:

  c1  B=1, 1 layer, cache 1024 -> append 1 -> attend over 1025                      (seed 1)
  c2  B=8, 28 layers, cache 2048 (K scaled by 0.5), 128 steps of append 1 + attend   (seed 2)
  c3  B=1, 1 layer, cache 32768, 64 steps, one planted high-logit key per kv head    (seed 3)
  c4  B=64, 28 layers, ragged cache lengths ~ U{512..4096}, one step                 (seed 4)
  c5  B=32, 1 layer, lengths ~ U{256..8192}, paged (16-token pages, permuted block
      table), fp8 e4m3 K/V with per-(token, head) fp32 scales, 1% outliers at +-8     (seed 5)

All shapes use 16 query heads, 8 kv heads, head_dim 128 and sm_scale = 1/sqrt(128). Values are drawn in
float32 from a seeded generator on the target device and rounded to bf16.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

HQ = 16
HKV = 8
HEAD_DIM = 128
SM_SCALE = 1.0 / math.sqrt(HEAD_DIM)
PAGE = 16


@dataclass(frozen=True)
class Workload:
    name: str
    batch: int
    layers: int
    steps: int
    seed: int
    prefill: int | None = None          # uniform prefilled length
    len_range: tuple[int, int] | None = None  # ragged: lengths ~ U{lo..hi}
    k_scale: float = 1.0                 # multiplier on prefilled K
    paged: bool = False
    fp8: bool = False
    planted: bool = False
    outlier_frac: float = 0.0
    outlier_value: float = 8.0
    extra: dict = field(default_factory=dict)

    @property
    def group(self) -> int:
        return HQ // HKV


WORKLOADS = {
    "c1": Workload("c1", batch=1, layers=1, steps=1, seed=1, prefill=1024),
    "c2": Workload("c2", batch=8, layers=28, steps=128, seed=2, prefill=2048, k_scale=0.5),
    "c3": Workload("c3", batch=1, layers=1, steps=64, seed=3, prefill=32768, planted=True),
    "c4": Workload("c4", batch=64, layers=28, steps=1, seed=4, len_range=(512, 4096)),
    "c5": Workload("c5", batch=32, layers=1, steps=1, seed=5, len_range=(256, 8192), paged=True, fp8=True,
                   outlier_frac=0.01),
}


def generator(device: torch.device | str, seed: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def normal(shape, gen: torch.Generator, device, dtype=torch.bfloat16, scale: float = 1.0,
           outlier_frac: float = 0.0, outlier_value: float = 8.0) -> torch.Tensor:
    x = torch.randn(shape, generator=gen, device=device, dtype=torch.float32)
    if scale != 1.0:
        x.mul_(scale)
    if outlier_frac > 0.0:
        pick = torch.rand(shape, generator=gen, device=device) < outlier_frac
        sign = torch.where(torch.rand(shape, generator=gen, device=device) < 0.5, -1.0, 1.0)
        x = torch.where(pick, sign * outlier_value, x)
    return x.to(dtype)


def seq_lengths(w: Workload, gen: torch.Generator) -> list[int]:
    """Cache lengths before the first append (host list)."""
    if w.len_range is None:
        return [w.prefill] * w.batch
    lo, hi = w.len_range
    lens = torch.randint(lo, hi + 1, (w.batch,), generator=gen, device=gen.device)
    return [int(x) for x in lens.cpu()]


def plant_keys(k: torch.Tensor, q: torch.Tensor, gen: torch.Generator, lens: list[int], margin: float = 10.0):
    """For every kv head j, overwrite the key at a random position p_j with c * q_hat (q_hat = unit vector of
    query head j*G, the first head of the group) so that this key's logit exceeds the largest other logit
    of that query head by at least ``margin`` (natural-log units). Returns [(b, j, p_j, c)]."""
    B, Hkv, _, D = k.shape
    G = q.shape[1] // Hkv
    planted = []
    for b in range(B):
        L = lens[b]
        for j in range(Hkv):
            qh = q[b, j * G, 0].float()
            logits = (k[b, j, :L].float() @ qh) * SM_SCALE
            p = int(torch.randint(0, L, (1,), generator=gen, device=gen.device))
            others = torch.cat([logits[:p], logits[p + 1 :]])
            target = float(others.max()) + margin
            qn = float(qh.norm())
            c = target / (SM_SCALE * qn)
            k[b, j, p] = (qh / qn * c).to(k.dtype)
            planted.append((b, j, p, c))
    return planted
