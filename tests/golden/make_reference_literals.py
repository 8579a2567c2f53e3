"""Write reference_literals.json: literal input/output vectors transcribed from the
reference's own tests (no reference code is imported or run). Each entry cites the
test file:line that holds the literal."""

import json
from pathlib import Path

LITERALS = {
    "contiguous_indices": {
        "source": "tests/test_core.py:61-62",
        "cases": [{"seq_len": 8, "world": 2, "expected": [[0, 1, 2, 3], [4, 5, 6, 7]]}],
    },
    "head_tail_indices": {
        "source": "tests/test_core.py:65-67",
        "cases": [{"seq_len": 8, "world": 2, "expected": [[0, 1, 6, 7], [2, 3, 4, 5]]}],
    },
    "balancer_errors": {
        "source": "tests/test_core.py:70-74",
        "cases": [{"fn": "contiguous_indices", "seq_len": 7, "world": 2},
                  {"fn": "head_tail_indices", "seq_len": 8, "world": 3}],
    },
    "zigzag_shard_rank0_cp2_16": {
        "source": "tests/test_zigzag_shard.py:76-83",
        "seq_len": 16, "cp_rank": 0, "cp_size": 2,
        "expected_position_ids": [0, 1, 2, 3, 12, 13, 14, 15],
    },
    "zigzag_roundtrip_cases": {
        "source": "tests/test_zigzag_shard.py:15-43 (48 is not divisible by 2*8: pad path)",
        "cp_sizes": [2, 4, 8], "seq_lens": [32, 48],
    },
    "head_tail_global_positions": {
        "source": "tests/test_attention_masks_cp.py:13-29 (strategies/query_scaling.py:17-26)",
        "cp_rank": 1, "cp_size": 2, "local_len": 8,
        "expected": [4, 5, 6, 7, 8, 9, 10, 11],
    },
    "cu_seqlens_from_position_ids": {
        "source": "tests/test_varlen_cp.py:275-282",
        "position_ids": [[0, 1, 2, 3, 0, 1, 0, 1, 2, 3, 4]],
        "expected_cu": [0, 4, 6, 11], "expected_max": 5,
    },
    "varlen_packing_cases": {
        "source": "tests/test_varlen_cp.py:23-30",
        "cases": [[16, [6, 10], 2], [16, [4, 4, 4, 4], 2], [24, [5, 7, 12], 2],
                  [16, [16], 2], [32, [10, 9, 13], 4], [24, [3, 3, 6, 4, 8], 4]],
    },
    "zigzag_varlen_fwd_bwd_cases": {
        "source": "tests/test_varlen_cp.py:256-260 (H=4, d=8, fp64, tol 1e-6)",
        "cases": [[16, [6, 10], 2], [16, [5, 7, 4], 2], [32, [10, 9, 13], 4]],
    },
    "state_passing": {
        "source": "tests/test_state_passing.py:15-58 (batch=1, T=8, d=3, a in (0.05, 0.95), tol 1e-5)",
        "batch": 1, "T": 8, "d": 3, "a_lo": 0.05, "a_hi": 0.95, "world": 2, "tol": 1e-5,
    },
    "gated_linear_attention": {
        "source": "tests/test_state_passing.py:61-115 (T=8, dk=4, dv=5, fp64, tol 1e-5)",
        "T": 8, "dk": 4, "dv": 5, "world": 2, "tol": 1e-5,
    },
    "mamba2_prefix": {
        "source": "tests/test_mamba_cp.py:88-136 (b=1, T=16, H=2, d=3, G=1, n=4, dt in [0,0.1), "
                  "A in (-1, 0], fp64, tol 1e-6)",
        "b": 1, "T": 16, "H": 2, "d": 3, "G": 1, "n": 4, "worlds": [2, 4, 8], "tol": 1e-6,
    },
    "ring_cpu": {
        "source": "tests/test_ring_cpu.py:24-37,88-99 (b,h,S,d = 1,4,8,16; fp64; tol 1e-6)",
        "b": 1, "h": 4, "S": 8, "d": 16, "world": 2, "tol": 1e-6,
    },
    "flash_backward_probe": {
        "source": "tests/_flash_backward_probe.py:21-50 (GQA 4:2, S=128, D=32, seed 29; "
                  "out atol 0.015 rtol 0.04; grads atol 0.03 rtol 0.05)",
        "hq": 4, "hkv": 2, "S": 128, "D": 32, "seed": 29,
        "out_atol": 0.015, "out_rtol": 0.04, "grad_atol": 0.03, "grad_rtol": 0.05,
    },
}

if __name__ == "__main__":
    out = Path(__file__).with_name("reference_literals.json")
    out.write_text(json.dumps(LITERALS, indent=1) + "\n")
    print(out)
