"""Host logic: the product's zigzag schedule covers the global causal triangle exactly
once, gives every rank equal work, and tags first/last touches correctly."""

import pytest
import torch

from ringmaster_amd.balancers import contiguous_indices, head_tail_indices
from ringmaster_amd.ring.schedule import (contiguous_gidx, contiguous_schedule, distflash_work,
                                          ring_pairs_per_rank, zigzag_gidx, zigzag_schedule)


def coverage(world, L, split_final):
    h = L // 2
    S = world * L
    cnt = torch.zeros(S, S, dtype=torch.int32)
    per_rank = [0] * world
    for s, blocks in enumerate(zigzag_schedule(world, L, split_final=split_final)):
        for bl in blocks:
            assert bl.kv_rank == (bl.rank - s) % world
            qg = torch.tensor(zigzag_gidx(bl.rank, h, world))[bl.q_lo:bl.q_hi]
            kg = torch.tensor(zigzag_gidx(bl.kv_rank, h, world))[bl.k_lo:bl.k_hi]
            sq, sk = len(qg), len(kg)
            allow = torch.ones(sq, sk, dtype=torch.bool)
            if bl.causal:
                allow = allow.tril(sk - sq)
            # every attended pair must be causal on global indices
            assert bool((kg.unsqueeze(0) <= qg.unsqueeze(1))[allow].all())
            cnt[qg.unsqueeze(1).expand(sq, sk)[allow], kg.unsqueeze(0).expand(sq, sk)[allow]] += 1
            per_rank[bl.rank] += int(allow.sum())
            assert bl.pairs == int(allow.sum())
    return cnt, per_rank


@pytest.mark.parametrize("world,L", [(1, 8), (2, 8), (4, 6), (8, 4), (3, 10)])
@pytest.mark.parametrize("split_final", [False, True])
def test_schedule_covers_causal_triangle_once(world, L, split_final):
    cnt, per_rank = coverage(world, L, split_final)
    S = world * L
    assert torch.equal(cnt, torch.ones(S, S, dtype=torch.int32).tril())
    assert per_rank == [ring_pairs_per_rank(world, L)] * world
    assert sum(per_rank) == S * (S + 1) // 2


@pytest.mark.parametrize("world", [1, 2, 4, 8])
def test_first_last_touch_tags(world):
    L = 8
    h = L // 2
    seen_first, seen_last = {}, {}
    for s, blocks in enumerate(zigzag_schedule(world, L, split_final=True)):
        for bl in blocks:
            for row in range(bl.q_lo, bl.q_hi):
                key = (bl.rank, row)
                if bl.first:
                    assert key not in seen_first
                    seen_first[key] = s
                if bl.last:
                    assert key not in seen_last
                    seen_last[key] = s
    for r in range(world):
        for row in range(L):
            assert seen_first[(r, row)] == 0
            assert seen_last[(r, row)] == (r if row < h else world - 1)


def test_backward_schedule_one_block_per_rank_and_kv_once():
    for world in (2, 4, 8):
        for s, blocks in enumerate(zigzag_schedule(world, 8, split_final=False)):
            assert sorted(b.rank for b in blocks) == list(range(world))
            assert sorted(b.kv_rank for b in blocks) == list(range(world))


def test_balancer_literals(golden):
    for case in golden["head_tail_indices"]["cases"]:
        assert head_tail_indices(case["seq_len"], case["world"]) == case["expected"]
    for case in golden["contiguous_indices"]["cases"]:
        assert contiguous_indices(case["seq_len"], case["world"]) == case["expected"]
    for case in golden["balancer_errors"]["cases"]:
        fn = {"contiguous_indices": contiguous_indices, "head_tail_indices": head_tail_indices}
        with pytest.raises(ValueError):
            fn[case["fn"]](case["seq_len"], case["world"])
    g = golden["head_tail_global_positions"]
    half = g["local_len"] // 2
    assert zigzag_gidx(g["cp_rank"], half, g["cp_size"]) == g["expected"]


@pytest.mark.parametrize("world,L", [(1, 5), (2, 4), (4, 3), (8, 2), (5, 3)])
@pytest.mark.parametrize("causal", [True, False])
def test_contiguous_schedule_covers_each_pair_once(world, L, causal):
    S = world * L
    cnt = torch.zeros(S, S, dtype=torch.int32)
    last = {}
    for s, blocks in enumerate(contiguous_schedule(world, L, causal=causal)):
        assert sorted(b.kv_rank for b in blocks) == sorted({b.kv_rank for b in blocks})
        for bl in blocks:
            assert bl.kv_rank == (bl.rank - s) % world and bl.first == (s == 0)
            qg = torch.tensor(contiguous_gidx(bl.rank, L))
            kg = torch.tensor(contiguous_gidx(bl.kv_rank, L))
            allow = torch.ones(L, L, dtype=torch.bool)
            if bl.causal:
                allow = allow.tril()
            if causal:
                assert bool((kg.unsqueeze(0) <= qg.unsqueeze(1))[allow].all())
            cnt[qg.unsqueeze(1).expand(L, L)[allow], kg.unsqueeze(0).expand(L, L)[allow]] += 1
            if bl.last:
                assert bl.rank not in last
                last[bl.rank] = s
    full = torch.ones(S, S, dtype=torch.int32)
    assert torch.equal(cnt, full.tril() if causal else full)
    assert last == {r: (r if causal else world - 1) for r in range(world)}


def test_distflash_balance_literals():
    # ring/distflash.py:15: "P=4 -> 3,3,2,2 vs ring's 1,2,3,4"
    assert distflash_work(4) == [3, 3, 2, 2]
    ring = [sum(1 for blocks in contiguous_schedule(4, 1, causal=True) for b in blocks
                if b.rank == r) for r in range(4)]
    assert ring == [1, 2, 3, 4]
    for world in range(1, 10):
        work = distflash_work(world)
        assert sum(work) == world * (world + 1) // 2  # every causal block exactly once
        assert max(work) - min(work) <= 1


@pytest.mark.parametrize("world,L", [(1, 8), (2, 8), (4, 6), (3, 10)])
def test_device_row_tables_match_host_lists(world, L):
    from ringmaster_amd.ring.zigzag import _global_rows

    zz = _global_rows("zigzag", world, L, "cpu")
    assert zz.dtype == torch.int32 and zz.shape == (world, L)
    assert zz.tolist() == [zigzag_gidx(r, L // 2, world) for r in range(world)]
    ct = _global_rows("contiguous", world, L, "cpu")
    assert ct.tolist() == [contiguous_gidx(r, L) for r in range(world)]
    assert _global_rows("zigzag", world, L, "cpu") is zz  # cached


@pytest.mark.parametrize("lens", [[16], [1, 15], [5, 0, 7, 4], [3, 3, 3, 3, 4], [0, 16]])
def test_sync_free_doc_ids_match_repeat_interleave(lens):
    # ring/varlen_blocks.py:45-48 builds the ids with repeat_interleave; zero-length
    # documents (repeated offsets) must be skipped the same way
    from ringmaster_amd.ring.zigzag import doc_ids_from_cu

    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32)
    ref = doc_ids_from_cu(cu, "cpu")
    fast = doc_ids_from_cu(cu, "cpu", sum(lens))
    assert fast.dtype == ref.dtype == torch.int32
    assert torch.equal(fast, ref)
