"""CPU oracle for the ring-attention compute path — TEST INFRASTRUCTURE ONLY.

A restatement, in torch on the CPU, of the reference's algorithms for the path:
the ``math`` block provider, the online-softmax merge, the zigzag schedule with its
reverse-ring backward, document masks, the zigzag shard and the
context-parallel linear scan. Each function cites the reference file:line it
follows. It is the checker the HIP path is compared against; nothing in
``ringmaster_amd`` may import it. Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg use it.

Pinning (how each function is checked before it is trusted) lives in
``tests/test_oracle_*.py``: reference literal vectors (``tests/golden/``), fp64
brute force, torch SDPA, and invariants (ring == full causal attention, merge
associativity, disjoint shard cover, scan == sequential recurrence). Every
function here has at least one such check; none is "parity unpinned".
"""
