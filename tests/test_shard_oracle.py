"""Pin the zigzag shard oracle (oracle/shard.py) on the CPU.

The checks follow the reference's own tests of the batch-dict shard
(tests/test_zigzag_shard.py:15-83 and tests/test_core.py:115-122) and the rules of
shard.py:120-176, checked element by element rather than by rebuilding the index:

* rank r holds the global positions of chunks r and 2P-1-r of the padded sequence,
  early chunk first, and its ``position_ids`` are exactly those positions (pads
  continue the numbering);
* every real token comes back at its position (round trip), every position is owned
  by exactly one rank (disjoint cover);
* padding rows hold 0 (ids, masks, features) and -100 (labels, shift labels);
* shift labels are global: position p's target is token p+1 of the whole sequence,
  -100 at the last real token;
* the literal vectors the reference tests hold (rank 0 of cp2 over 16 tokens, the
  6 -> 8 pad case) and the unshard (inverse scatter, tests/test_zigzag_shard.py:39-43).

The reference's round-trip lengths (32, 48) divide 2P for every P it uses, so they
never pad; the lengths 45, 37, 22 and 6 below do.
"""

import pytest
import torch

from oracle import shard as osh

WORLDS = (2, 4, 8)
LENGTHS = (32, 48, 45, 37, 22, 6)


def _batch(seq_len):
    g = torch.Generator().manual_seed(seq_len)
    return {
        "input_ids": torch.arange(seq_len).view(1, seq_len) + 1000,
        "labels": torch.arange(seq_len).view(1, seq_len) + 5000,
        "attention_mask": torch.ones(1, seq_len, dtype=torch.long),
        "features": torch.randn(1, seq_len, 3, generator=g),
    }


def check_shard_batch(shard_fn, unshard_fn=None, shard_tensor_fn=None):
    """Run the reference's rules against ``shard_fn(batch, rank, world) -> (batch,
    (seq_len, pad_len))`` (and the tensor shard / unshard when given)."""
    for world in WORLDS:
        for seq_len in LENGTHS:
            pad = (-seq_len) % (2 * world)
            total = seq_len + pad
            half = total // (2 * world)
            src = _batch(seq_len)
            owner = {}
            for r in range(world):
                out, (orig, pad_len) = shard_fn({k: v.clone() for k, v in src.items()}, r, world)
                ctx = f"world {world} seq {seq_len} rank {r}"
                assert (orig, pad_len) == (seq_len, pad), ctx
                want = list(range(r * half, (r + 1) * half)) + \
                    list(range((2 * world - 1 - r) * half, (2 * world - r) * half))
                assert out["position_ids"][0].tolist() == want, f"{ctx}: positions"
                for j, p in enumerate(want):
                    assert p not in owner, f"{ctx}: position {p} also on rank {owner[p]}"
                    owner[p] = r
                    real = p < seq_len
                    assert out["input_ids"][0, j] == (src["input_ids"][0, p] if real else 0), ctx
                    assert out["labels"][0, j] == (src["labels"][0, p] if real else -100), ctx
                    target = src["labels"][0, p + 1] if p + 1 < seq_len else -100
                    assert out["shift_labels"][0, j] == target, f"{ctx}: shift label at {p}"
                    assert out["attention_mask"][0, j] == (1 if real else 0), ctx
                    feat = src["features"][0, p] if real else torch.zeros(3)
                    assert torch.equal(out["features"][0, j], feat), ctx
                if shard_tensor_fn is not None:
                    assert torch.equal(shard_tensor_fn(src["features"], world, r), out["features"])
                    assert torch.equal(shard_tensor_fn(src["labels"], world, r, pad_value=-100),
                                       out["labels"])
            assert sorted(owner) == list(range(total)), f"world {world} seq {seq_len}: cover"
            if unshard_fn is not None:
                for key in ("input_ids", "features"):
                    shards = [osh.zigzag_shard_tensor(src[key], world, r) for r in range(world)]
                    assert torch.equal(unshard_fn(shards, seq_len), src[key]), key


def test_shard_oracle_rules():
    check_shard_batch(osh.zigzag_shard_batch, osh.zigzag_unshard_tensor, osh.zigzag_shard_tensor)


def test_shard_oracle_reference_literals(golden):
    lit = golden["zigzag_shard_rank0_cp2_16"]
    n = lit["seq_len"]
    batch = {"input_ids": torch.arange(n).view(1, n), "labels": torch.arange(n).view(1, n)}
    out, _ = osh.zigzag_shard_batch(batch, lit["cp_rank"], lit["cp_size"])
    assert out["position_ids"][0].tolist() == lit["expected_position_ids"]
    assert "shift_labels" in out
    # tests/test_core.py:115-122: 6 tokens over 4 ranks pad to 8, two per rank
    base = {"input_ids": torch.arange(6).view(1, 6), "labels": torch.arange(6).view(1, 6)}
    out, (orig, pad) = osh.zigzag_shard_batch(base, 0, 4)
    assert (orig, pad) == (6, 2) and out["input_ids"].shape == (1, 2)


def test_shard_oracle_reference_roundtrip_cases(golden):
    """The reference's round-trip grid (tests/test_zigzag_shard.py:15-43): ids equal to
    positions come back in place; position ids are the rank's global indices."""
    cases = golden["zigzag_roundtrip_cases"]
    for world in cases["cp_sizes"]:
        for seq_len in cases["seq_lens"]:
            ids = torch.arange(seq_len).view(1, seq_len)
            total = seq_len + (-seq_len) % (2 * world)
            recon = torch.full((1, total), -1, dtype=torch.long)
            for r in range(world):
                out, _ = osh.zigzag_shard_batch({"input_ids": ids.clone()}, r, world)
                assert out["input_ids"].shape == (1, total // world)
                for p, tok in zip(out["position_ids"][0].tolist(), out["input_ids"][0].tolist()):
                    recon[0, p] = tok
            assert torch.equal(recon[0, :seq_len], ids[0])


def test_shard_oracle_existing_position_ids_and_prepadded_tensor():
    """Given position ids are kept (and continued over the pad); a tensor already at the
    padded length is sharded as it is (shard.py:173-175 shards every [b, total] tensor)."""
    seq_len, world = 10, 2
    pos = (torch.arange(seq_len) + 100).view(1, seq_len)
    pre = torch.arange(12).view(1, 12) + 7  # padded length 12 already
    out, (orig, pad) = osh.zigzag_shard_batch(
        {"input_ids": torch.zeros(1, seq_len, dtype=torch.long), "position_ids": pos.clone(),
         "prepadded": pre.clone()}, 1, world)
    assert (orig, pad) == (10, 2)
    idx = [3, 4, 5, 6, 7, 8]  # chunks 1 and 2 of 4 chunks of 3
    full_pos = torch.cat([pos[0], torch.tensor([110, 111])])
    assert out["position_ids"][0].tolist() == full_pos[idx].tolist()
    assert out["prepadded"][0].tolist() == pre[0, idx].tolist()


def test_balancer_literals(golden):
    from ringmaster_amd.balancers import contiguous_indices, head_tail_indices

    for fn, key in ((osh.head_tail_indices, "head_tail_indices"),
                    (osh.contiguous_indices, "contiguous_indices"),
                    (head_tail_indices, "head_tail_indices"),
                    (contiguous_indices, "contiguous_indices")):
        for case in golden[key]["cases"]:
            assert fn(case["seq_len"], case["world"]) == case["expected"], (fn, case)


@pytest.mark.parametrize("world", WORLDS)
def test_head_tail_indices_match_shard_positions(world):
    """The index generator and the batch shard agree (balancers.py:18-29 vs shard.py:165-171)."""
    seq_len = 8 * world
    idx = osh.head_tail_indices(seq_len, world)
    for r in range(world):
        out, _ = osh.zigzag_shard_batch({"input_ids": torch.zeros(1, seq_len, dtype=torch.long)},
                                        r, world)
        assert out["position_ids"][0].tolist() == idx[r]
