"""bench.py's byte accounting and its single-GPU contract, on the CPU.

The algorithmic bytes per layer-step are what the roofline fraction divides by, so they are pinned here by
hand-counted cases: B=8 L=2048 with 64.5 decode steps on average (the headline's mean length after the
append, 2112.5 tokens), a small paged fp8 case counted term by term, and the prefill writer's launch.
"""

import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_headline_bytes_per_launch():
    # K and V read: 2 x 2112.5 tokens x 8 kv heads x 256 B per row, for 8 sequences
    kv = 8 * 2 * 2112.5 * 8 * 256
    new_rows = 2 * 8 * 8 * 128 * 2 * 2          # read bf16, written bf16
    q_out = 2 * 8 * 16 * 128 * 2                 # q read, output written
    assert kv == 69_222_400 and new_rows == 65_536 and q_out == 65_536
    assert bench.algorithmic_bytes(8, 16, 8, 128, [2112.5] * 8) == 69_353_472


def test_paged_fp8_bytes_term_by_term():
    lens, page = [20, 33], 16
    row = 128 * 1 + 4                            # e4m3 codes and one fp32 scale per token and kv head
    kv = sum(2 * L * 2 * row for L in lens)      # K and V, 2 kv heads
    new_rows = 2 * 2 * 2 * 128 * 2 + 2 * 2 * 2 * row
    q_out = 2 * 2 * 4 * 128 * 2
    table = (2 + 3) * 4 + 2 * 4                  # block-table entries of 2 and 3 pages, and the lengths
    got = bench.algorithmic_bytes(2, 4, 2, 128, lens, fp8=True, page=page)
    assert got == kv + new_rows + q_out + table


def test_prefill_bytes_term_by_term():
    # 2 sequences x 3 kv heads x 40 new tokens, head_dim 64, from position 0
    rows = 2 * 2 * 3 * 40                        # K and V rows
    src = rows * 64 * 2                          # bf16 rows read
    assert bench.prefill_bytes(2, 3, 40, 64) == src + rows * 64 * 2 + 2 * 4
    # paged fp8 with 16-token pages: 3 pages per sequence written, one table entry each
    assert bench.prefill_bytes(2, 3, 40, 64, fp8=True, page=16) == src + rows * (64 + 4) + 2 * 3 * 4 + 2 * 4
    # the bench's prefill line: 32 sequences, 8 kv heads, a 2048-token prompt, 16-token pages
    assert bench.prefill_bytes(32, 8, 2048, 128, fp8=True, page=16) == 268_435_456 + 138_412_032 + 16_384 + 128


def test_more_than_one_gpu_is_refused_before_any_gpu_work():
    proc = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                          text=True, timeout=120)
    assert proc.returncode == 2
    assert "one GPU" in proc.stdout + proc.stderr
