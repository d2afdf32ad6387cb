"""The fp8 encoding of the append kernels, and the launch-constant integer division of the append kernel.

The kernels quantise with gfx950's fp8 conversion instruction (e4m3x4). Exhaustively, on every float with
|x| <= 448, it must give the codes of the encoder written out from the OCP e4m3 format (round to nearest even);
the quotients a hair above 448 that the kernels also feed it (|x / s| <= 448 (1 + 2^-23) for a normal scale) are
covered by the row quantiser's check, which compares with the codes of the clamped IEEE quotient. The row scale amax / 448 comes from a corrected product, and the
quotient x / scale from one reciprocal per row (hardware reciprocal and a Newton step) and a corrected product per
value (fp8_quantize); for every row maximum of bf16 and of fp16 sources the scale and the reciprocal must be the
IEEE quotients' bits, and for every (row maximum, value) pair the codes those of the IEEE quotient. On rows of every magnitude, through the product's own append, codes and
scales must be the oracle's (torch's cast of clamp(x / scale)). The append kernel divides row indexes by the
launch's new-row count with a multiplier (fast_div); on 2^25 dividends spread over the 31-bit range it must
equal the division for every divisor tried.
"""

import ctypes

import pytest
import torch

from aicas_amd import ops
from aicas_amd.build import CALIB_OUTPUT
from oracle import reference_path as ref

pytestmark = pytest.mark.gpu


def test_hardware_encoder_matches_format_encoder_on_every_float(dev):
    lib = ctypes.CDLL(CALIB_OUTPUT, mode=ctypes.RTLD_LOCAL)
    lib.aicas_calib_fp8_encoder_check.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    mism = torch.zeros(1, dtype=torch.int64, device=dev)
    first = torch.zeros(1, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev)
    rc = lib.aicas_calib_fp8_encoder_check(mism.data_ptr(), first.data_ptr(), stream.cuda_stream)
    assert rc == 0
    assert int(mism.item()) == 0, f"first differing pattern {int(first.item()) & 0xffffffff:#010x}"


@pytest.mark.parametrize("src_dtype, name", [(0, "bf16"), (1, "fp16")])
def test_row_quantiser_gives_the_ieee_quotient_codes(dev, src_dtype, name):
    lib = ctypes.CDLL(CALIB_OUTPUT, mode=ctypes.RTLD_LOCAL)
    lib.aicas_calib_fp8_divide_check.argtypes = [ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    mism = torch.zeros(3, dtype=torch.int64, device=dev)
    first = torch.zeros(1, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev)
    assert lib.aicas_calib_fp8_divide_check(src_dtype, mism.data_ptr(), first.data_ptr(), stream.cuda_stream) == 0
    f = int(first.item()) & 0xffffffff
    codes, scales, recips = mism.cpu().tolist()
    assert (codes, scales, recips) == (0, 0, 0), \
        f"{name}: {codes} code groups, {scales} scales, {recips} reciprocals differ; first at row maximum " \
        f"{f >> 16:#06x}, values from {f & 0xffff:#06x}"


def test_launch_constant_division(dev):
    divisors = list(range(1, 4097)) + [1 << k for k in range(13, 31)]
    divisors += [(1 << k) + e for k in range(13, 31) for e in (-1, 1)] + [3 * 2048 * 8, 6000, 65535, 65537,
                                                                           1000003, 123456789, 2147483647]
    arr = (ctypes.c_int32 * len(divisors))(*divisors)
    lib = ctypes.CDLL(CALIB_OUTPUT, mode=ctypes.RTLD_LOCAL)
    lib.aicas_calib_fast_div_check.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p,
                                               ctypes.c_void_p]
    mism = torch.zeros(1, dtype=torch.int64, device=dev)
    first = torch.zeros(1, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev)
    rc = lib.aicas_calib_fast_div_check(ctypes.cast(arr, ctypes.c_void_p), len(divisors), mism.data_ptr(),
                                        first.data_ptr(), stream.cuda_stream)
    assert rc == 0
    assert int(mism.item()) == 0, f"first divisor with a difference: {int(first.item())}"


@pytest.mark.parametrize("magnitude", [1e-6, 3e-3, 1.0, 250.0, 6.0e4])
def test_append_codes_match_oracle_across_magnitudes(dev, magnitude):
    """4096 rows of 128 per magnitude (bf16 sources, half of them with a planted +-8x outlier and a run of exact
    ties), written by the append kernel: codes and scales equal the oracle's."""
    g = torch.Generator().manual_seed(int(magnitude * 1000) % 9973)
    B, H, n, D = 4, 8, 128, 128
    x = torch.randn((B, H, n, D), generator=g) * magnitude
    x[:, :, ::2, 3] *= 8.0
    # values on e4m3 rounding boundaries of the row's scale: k / 16 of the amax for small k
    x[:, :, 1::4, 10:26] = x[:, :, 1::4, :1].abs() * torch.arange(1, 17) / 16.0
    x = x.to(torch.bfloat16)
    k = torch.zeros((B, H, n, D), dtype=ops.FP8_DTYPE, device=dev)
    v = torch.zeros_like(k)
    ks = torch.zeros((B, H, n), dtype=torch.float32, device=dev)
    vs = torch.zeros_like(ks)
    ops.kv_append(ops.KVCacheView(k, v, ks, vs), x.to(dev), x.to(dev), torch.zeros(B, dtype=torch.int32, device=dev))
    codes, scale = ref.fp8_quantize_rows(x)
    assert torch.equal(k.cpu().view(torch.uint8), codes.view(torch.uint8))
    assert torch.equal(ks.cpu(), scale)
