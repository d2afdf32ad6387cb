"""The oracle's block allocator (reference_path.block_alloc / block_free), pinned on the CPU.

Known answers worked by hand, and invariants over random alloc / free sequences against an independent
brute-force model (a set of free ids and a dict per sequence): every live page holds a distinct block, free +
held == num_blocks, a released sequence's blocks come back in page order, and exhaustion leaves exactly the
pages the pool could not cover at -1.
"""

import random

import torch

from oracle import reference_path as ref


def test_known_answers():
    stack, count = ref.block_pool_init(6)
    assert stack == [5, 4, 3, 2, 1, 0] and count == 6
    table = torch.full((2, 4), -1, dtype=torch.int32)
    # pages of 4 tokens: sequence 0 appends tokens 0..2 (page 0), sequence 1 tokens 5..7 (page 1)
    count, st = ref.block_alloc(stack, count, table, [0, 5], 3, 4)
    assert st == 0 and count == 4 and table.tolist() == [[0, -1, -1, -1], [-1, 1, -1, -1]]
    # tokens 3..4 -> pages 0 (held) and 1; tokens 8..9 -> page 2
    count, st = ref.block_alloc(stack, count, table, [3, 8], 2, 4)
    assert st == 0 and count == 2 and table.tolist() == [[0, 2, -1, -1], [-1, 1, 3, -1]]
    lens = [5, 10]
    count, st = ref.block_free(stack, count, table, [0, 1], lens, 6)  # sequence 1 gives back 1 then 3
    assert st == 0 and count == 4 and lens == [5, 0]
    assert table.tolist() == [[0, 2, -1, -1], [-1, -1, -1, -1]] and stack[:count] == [5, 4, 1, 3]
    count, st = ref.block_alloc(stack, count, table, [0, 0], 1, 4)  # sequence 0 page 0 held; sequence 1 page 0
    assert st == 0 and count == 3 and table.tolist() == [[0, 2, -1, -1], [3, -1, -1, -1]]
    fresh = torch.full((1, 4), -1, dtype=torch.int32)
    count, st = ref.block_alloc(stack, count, fresh, [0], 8, 4)  # pages 0, 1 take the top two: 1 then 4
    assert st == 0 and count == 1 and fresh.tolist() == [[1, 4, -1, -1]]


def test_overflow_and_exhaustion():
    stack, count = ref.block_pool_init(2)
    table = torch.full((2, 2), -1, dtype=torch.int32)
    count, st = ref.block_alloc(stack, count, table, [0, 6], 3, 4)  # sequence 1 tokens 6..8 reach page 2 > width
    assert st & 4 and table.tolist() == [[0, -1], [-1, 1]] and count == 0
    count, st = ref.block_alloc(stack, count, table, [4, 0], 1, 4)
    assert st == 8 and table.tolist() == [[0, -1], [-1, 1]] and count == 0  # nothing left for page 1 / page 0
    count, st = ref.block_free(stack, count, torch.tensor([[7, -1], [-1, -1]], dtype=torch.int32), [1, 0], None, 2)
    assert st == 2 and count == 0  # id 7 is outside the pool


def test_random_sequences_against_a_set_model():
    rng = random.Random(5)
    for trial in range(40):
        N, B, W, page = rng.randint(1, 40), rng.randint(1, 6), rng.randint(1, 8), rng.choice([1, 2, 4, 8])
        stack, count = ref.block_pool_init(N)
        table = torch.full((B, W), -1, dtype=torch.int32)
        free = set(range(N))
        held = [dict() for _ in range(B)]
        lens = [0] * B
        for step in range(30):
            if rng.random() < 0.25:
                rel = [rng.random() < 0.5 for _ in range(B)]
                order = []
                for b in range(B):
                    if rel[b]:
                        order += [held[b][pg] for pg in sorted(held[b])]
                        free |= set(held[b].values())
                        held[b].clear()
                before = count
                count, st = ref.block_free(stack, count, table, [int(r) for r in rel], lens, N)
                assert st == 0 and stack[before:count] == order
            else:
                n = rng.randint(1, 5)
                pos = [lens[b] for b in range(B)]
                count, st = ref.block_alloc(stack, count, table, pos, n, page)
                for b in range(B):
                    for pg in range(pos[b] // page, min((pos[b] + n - 1) // page, W - 1) + 1):
                        e = int(table[b, pg])
                        if pg in held[b]:
                            assert e == held[b][pg]
                        elif e >= 0:
                            assert e in free
                            free.discard(e)
                            held[b][pg] = e
                        else:
                            assert st & 8  # only exhaustion leaves a touched page empty
                    lens[b] = min(pos[b] + n, W * page)
            live = [e for h in held for e in h.values()]
            assert len(live) == len(set(live))
            assert count == len(free) and count + len(live) == N
            assert sorted(stack[:count]) == sorted(free)
