"""configs[0] CPU plumbing: the zigzag ring on a real 2-process gloo group.

Causal zigzag shard, B=1, H=8 (MHA), total S=4096 (2048 per rank as two 1024
chunks), D=64, fp32, q/k/v/dout ~ N(0,1) from seeds 1-4. Each rank runs the
distributed restatement (K/V and the dK/dV accumulators move by point-to-point
hops, oracle/dist_ring.py) and checks fwd out/lse and bwd dq/dk/dv against the
single-process emulation of the same ring (oracle/ring_math.py), which the GPU
path is tested against."""

import os
import socket

import torch
import torch.distributed as dist
import torch.multiprocessing as mp

B, S, H, D, WORLD = 1, 4096, 8, 64, 2


def _free_port():
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        return s.getsockname()[1]


def _worker(rank, port):
    os.environ["MASTER_ADDR"] = "127.0.0.1"
    os.environ["MASTER_PORT"] = str(port)
    torch.set_num_threads(2)
    dist.init_process_group("gloo", rank=rank, world_size=WORLD)
    try:
        from oracle import dist_ring
        from oracle import ring_math as rm

        def full(seed):
            return torch.randn(B, S, H, D, generator=torch.Generator().manual_seed(seed))

        q, k, v, do = full(1), full(2), full(3), full(4)
        half = S // (2 * WORLD)
        idx = [rm.zigzag_gidx(r, half, WORLD) for r in range(WORLD)]
        shard = lambda t, r: t[:, idx[r]].transpose(1, 2).contiguous()  # noqa: E731  [b,H,L,d]
        qs, ks, vs = ([shard(t, r) for r in range(WORLD)] for t in (q, k, v))
        dos = [do[:, idx[r]] for r in range(WORLD)]

        out, lse = dist_ring.zigzag_forward(qs[rank], ks[rank], vs[rank])
        dq, dk, dv = dist_ring.zigzag_backward(dos[rank], qs[rank], ks[rank], vs[rank], out, lse)

        ref_out, ref_lse = rm.zigzag_ring_forward(qs, ks, vs)
        rdq, rdk, rdv = rm.zigzag_ring_backward(dos, qs, ks, vs, ref_out, ref_lse)
        for name, got, ref in (("out", out, ref_out[rank]), ("lse", lse, ref_lse[rank]),
                               ("dq", dq, rdq[rank]), ("dk", dk, rdk[rank]),
                               ("dv", dv, rdv[rank])):
            err = (got - ref).abs().max().item()
            assert err < 1e-5, f"rank {rank} {name}: max-abs {err:.3e}"
        # every rank computes the same number of attended pairs (zigzag balance)
        L = S // WORLD
        assert out.shape == (B, L, H, D) and lse.shape == (B, H, L)
    finally:
        dist.destroy_process_group()


def test_zigzag_ring_gloo_world2():
    mp.spawn(_worker, args=(_free_port(),), nprocs=WORLD, join=True)
