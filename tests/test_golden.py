"""Golden fixtures (tests/golden/fixtures.safetensors, written by tests/golden/make_golden.py) against the
oracle on the CPU. The GPU parity tests compare the kernels with the same fixtures."""

import math
import os
import sys

import torch
from safetensors.torch import load_file

from oracle import reference_path as ref

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, GOLDEN)
import make_golden  # noqa: E402

FIX = load_file(os.path.join(GOLDEN, "fixtures.safetensors"))


def test_c1_inputs_are_reproduced():
    """The seeded generator still produces the inputs the fixture was made from."""
    assert torch.equal(make_golden.digest(*make_golden.c1_inputs()), FIX["c1.input_sha256"])


def test_c1_oracle_matches_fixture():
    cache_k, cache_v, k_new, v_new, q = make_golden.c1_inputs()
    k, v = ref.dynamic_layer_update(cache_k, cache_v, k_new, v_new)
    assert k.shape[2] == 1025
    exact = ref.decode_fp64(q, k, v, 1 / math.sqrt(128), 2)
    assert (exact - FIX["c1.out_fp64"]).abs().max() < 1e-12
    # the bf16 SDPA reference path lands within the bf16 bar of the exact result
    sdpa = ref.sdpa_decode(q, k, v, 1 / math.sqrt(128), 2).double()
    assert (sdpa - FIX["c1.out_fp64"]).abs().max() < 2e-2


def test_tiny_case_matches_fixture():
    out = ref.decode_fp64(FIX["tiny.q"], FIX["tiny.k"], FIX["tiny.v"], 0.25, 2)
    assert (out - FIX["tiny.out_fp64"]).abs().max() < 1e-12


def test_fp8_table_and_rows_match_fixture():
    table = ref.e4m3_decode_table()
    both_nan = torch.isnan(table) & torch.isnan(FIX["fp8.table"])
    assert bool((both_nan | (table == FIX["fp8.table"])).all())
    codes, scale = ref.fp8_quantize_rows(FIX["fp8.rows_x"])
    assert torch.equal(codes.view(torch.uint8), FIX["fp8.rows_codes"])
    assert torch.equal(scale, FIX["fp8.rows_scale"])
    # the tie cases in row 0 (scale 1): 1.0625 -> 0x38, 1.1875 -> 0x3a, 2^-10 -> 0, 3*2^-10 -> 0x02
    assert FIX["fp8.rows_codes"][0, :5].tolist() == [0x7E, 0x38, 0x3A, 0x00, 0x02]
