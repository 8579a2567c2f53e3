"""Host logic: the product's zigzag schedule covers the global causal triangle exactly
once, gives every rank equal work, and tags first/last touches correctly."""

import pytest
import torch

from ringmaster_amd.balancers import contiguous_indices, head_tail_indices
from ringmaster_amd.ring.schedule import (contiguous_gidx, contiguous_schedule,
                                          distflash_schedule, distflash_work,
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


def _reference_distflash_blocks(world):
    """(query owner, KV owner, worker) in the order the reference's forward merges them
    into the owner's rows, read off its loops (ring/distflash.py:113-133): the diagonal,
    the phase-2 loop over d = 1..P-1 keeping d > P//2 and r - d >= 0, then the phase-1
    loop over d = 1..P//2 where helper r computes q_{r+d} for r + d < P."""
    half = world // 2
    per_owner = {r: [(r, r, r)] for r in range(world)}
    for r in range(world):
        for d in range(1, world):
            if d > half and r - d >= 0:
                per_owner[r].append((r, r - d, r))
    for d in range(1, half + 1):
        for r in range(world):
            if r + d < world:
                per_owner[r + d].append((r + d, r, r))
    return per_owner


@pytest.mark.parametrize("world", [1, 2, 3, 4, 5, 8])
def test_distflash_schedule_is_the_reference_placement(world):
    L = 4
    steps = distflash_schedule(world, L)
    seen, per_owner, per_worker = set(), {r: [] for r in range(world)}, [0] * world
    for s, blocks in enumerate(steps):
        assert blocks, "no empty steps"
        assert len({b.rank for b in blocks}) == len(blocks)      # one block per owner per step
        assert len({b.kv_rank for b in blocks}) == len(blocks)   # one dK/dV target per step
        for b in blocks:
            i, j, w = b.rank, b.kv_rank, b.runs_on
            assert i >= j and (i, j) not in seen
            seen.add((i, j))
            assert (b.q_lo, b.q_hi, b.k_lo, b.k_hi) == (0, L, 0, L)
            assert b.causal == (s == 0) == (i == j) == b.first
            d = i - j
            assert w == (i if (d == 0 or d > world // 2) else j)  # owner / helper placement
            per_owner[i].append((i, j, w))
            per_worker[w] += 1
    assert len(seen) == world * (world + 1) // 2                 # every causal block once
    assert per_owner == _reference_distflash_blocks(world)       # the reference's merge order
    assert per_worker == distflash_work(world)
    last = {b.rank: s for s, blocks in enumerate(steps) for b in blocks}
    for s, blocks in enumerate(steps):
        for b in blocks:
            assert b.last == (last[b.rank] == s)


def test_distflash_balance_at_eight_ranks():
    assert distflash_work(8) == [5, 5, 5, 5, 4, 4, 4, 4]
    steps = distflash_schedule(8, 1)
    # in units of a full block (the diagonal is half of one): 4.5 for ranks 0-3, 3.5 for 4-7
    units = [sum(0.5 if b.causal else 1.0 for st in steps for b in st if b.runs_on == r)
             for r in range(8)]
    assert units == [4.5] * 4 + [3.5] * 4


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


def test_cu_seqlens_checks():
    from ringmaster_amd.ring.zigzag import check_cu_seqlens, doc_for

    check_cu_seqlens(torch.tensor([0, 3, 3, 8]), 8)  # empty documents are allowed
    for bad, match in (([1, 8], "from 0"), ([0, 7], "from 0"), ([0, 5, 4, 8], "decrease"),
                       ([8], "two entries")):
        with pytest.raises(ValueError, match=match):
            check_cu_seqlens(torch.tensor(bad), 8)
    q = torch.zeros(2, 1, 1, 4, 8)                      # [P, b, H, L, d]: total 8
    assert doc_for(torch.tensor([0, 5, 8], dtype=torch.int32), q).tolist() == [0] * 5 + [1] * 3
    with pytest.raises(ValueError):
        doc_for(torch.tensor([0, 5, 9], dtype=torch.int32), q)
