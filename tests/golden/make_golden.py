"""Write the golden fixtures in this directory from the oracle (run: python tests/golden/make_golden.py).

fixtures.safetensors holds:
  c1.*        the single-layer decode step of the c1 workload (batch 1, 16 q / 8 kv heads, head_dim 128, cache
              1024 -> append 1 -> attend over 1025), inputs drawn on the CPU from torch.Generator seed 1:
              a SHA-256 of the input bytes (pins the generator) and the float64 closed-form output;
  tiny.*      a brute-force-sized case stored whole (inputs and float64 output): B=2, 4 q / 2 kv heads,
              head_dim 16, 8 tokens;
  fp8.table   the value of each of the 256 OCP e4m3 codes (float32, NaN for 0x7f / 0xff);
  fp8.rows_x / fp8.rows_codes / fp8.rows_scale
              rows quantized on write (scale = amax/448), chosen to hit round-half-even ties in the normal
              and subnormal ranges, the 448 clamp, zero rows and +-8 outliers.
The reference repository ships no vectors for this path; these are produced by the oracle, whose functions
are pinned independently in tests/test_oracle.py.
"""

from __future__ import annotations

import hashlib
import math
import os
import sys

import torch
from safetensors.torch import save_file

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import reference_path as ref  # noqa: E402

C1_SEED = 1
HQ, HKV, D, L0 = 16, 8, 128, 1024


def c1_inputs():
    """The c1 step's inputs, drawn in float32 from one CPU generator and rounded to bf16."""
    g = torch.Generator().manual_seed(C1_SEED)
    mk = lambda *shape: torch.randn(shape, generator=g).to(torch.bfloat16)  # noqa: E731
    cache_k, cache_v = mk(1, HKV, L0, D), mk(1, HKV, L0, D)
    k_new, v_new = mk(1, HKV, 1, D), mk(1, HKV, 1, D)
    q = mk(1, HQ, 1, D)
    return cache_k, cache_v, k_new, v_new, q


def digest(*tensors) -> torch.Tensor:
    h = hashlib.sha256()
    for t in tensors:
        h.update(t.contiguous().view(torch.int16).numpy().tobytes())
    return torch.frombuffer(bytearray(h.digest()), dtype=torch.uint8).clone()


def fp8_rows() -> torch.Tensor:
    rows = torch.zeros(6, 16)
    # scale 1 (amax 448): ties at 1.0625 -> 1.0, 1.1875 -> 1.25, subnormal ties 2^-10 -> 0, 3*2^-10 -> 2^-8
    rows[0] = torch.tensor([448.0, 1.0625, 1.1875, 2.0 ** -10, 3 * 2.0 ** -10, -1e-3, 15 * 2.0 ** -10, 0.0,
                            -448.0, 416.0, 432.0, 2.0 ** -6, -(2.0 ** -9), 1.125, 3.0, -0.5])
    rows[1] = 0.0  # all-zero row: scale 0, zero codes
    g = torch.Generator().manual_seed(5)
    rows[2] = torch.randn(16, generator=g)
    rows[3] = torch.randn(16, generator=g)
    rows[3, 4] = 8.0  # outlier
    rows[4] = torch.randn(16, generator=g) * 1e-3
    rows[5] = -torch.logspace(-4, 2, 16)
    return rows.to(torch.bfloat16)


def build() -> dict[str, torch.Tensor]:
    cache_k, cache_v, k_new, v_new, q = c1_inputs()
    k, v = ref.dynamic_layer_update(cache_k, cache_v, k_new, v_new)
    out = {
        "c1.input_sha256": digest(cache_k, cache_v, k_new, v_new, q),
        "c1.out_fp64": ref.decode_fp64(q, k, v, 1.0 / math.sqrt(D), HQ // HKV),
    }
    g = torch.Generator().manual_seed(2)
    tq = torch.randn((2, 4, 1, 16), generator=g).to(torch.bfloat16)
    tk = torch.randn((2, 2, 8, 16), generator=g).to(torch.bfloat16)
    tv = torch.randn((2, 2, 8, 16), generator=g).to(torch.bfloat16)
    out.update({"tiny.q": tq, "tiny.k": tk, "tiny.v": tv, "tiny.out_fp64": ref.decode_fp64(tq, tk, tv, 0.25, 2)})
    out["fp8.table"] = torch.tensor([ref.e4m3_value(c) for c in range(256)], dtype=torch.float32)
    x = fp8_rows()
    codes, scale = ref.fp8_quantize_rows(x)
    out.update({"fp8.rows_x": x, "fp8.rows_codes": codes.view(torch.uint8), "fp8.rows_scale": scale})
    return out


if __name__ == "__main__":
    path = os.path.join(HERE, "fixtures.safetensors")
    save_file(build(), path)
    print(path, os.path.getsize(path), "bytes")
