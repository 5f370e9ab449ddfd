"""Writes the small golden fixtures of this directory from the (pinned) CPU oracle.

The reference commits no tensors for this path (its tests seed at run time),
so the fixtures are generated here, after tests/test_oracle_*.py pin the
oracle, and then serve as fixed data for the CPU regression check and the GPU
parity tests. Inputs follow the workload convention: torch.Generator(seed),
float32 N(0, 1) draws cast to fp16, order Q, K, V.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import decode as od  # noqa: E402
from oracle import splice as osp  # noqa: E402


def draw(seed, *shapes):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(*s, generator=g).half().numpy() for s in shapes]


def decode_fixture(name, seed, hkv, g, n, scale):
    q, k, v = draw(seed, (hkv, g, 128), (hkv, n, 128), (hkv, n, 128))
    qf, kf, vf = (x.astype(np.float32) for x in (q, k, v))
    o_part, lse = od.flash_decode_partial(qf, kf, vf, scale, split=256, block=16)
    out32 = od.flash_decode_combine(o_part, lse)
    np.savez_compressed(os.path.join(HERE, name), q=q, k=k, v=v, scale=np.float64(scale),
                        o_part=o_part, lse=lse, out32=out32, out16=out32.astype(np.float16),
                        out64=od.attention_f64(qf, kf, vf, scale))


def splice_fixture(name, seed, heads, n, a, c0, c, theta):
    k, v = draw(seed, (1, heads, n, 128), (1, heads, n, 128))
    inv = osp.default_inv_freq(theta, 128)
    cos, sin = osp.rope_table(-(c0 - a), inv)
    kb, vb, n2 = osp.splice_growing(k, v, n, a, c0, c, cos, sin)
    np.savez_compressed(os.path.join(HERE, name), k=k, v=v, split=np.array([a, c0, c]), theta=np.float64(theta),
                        inv_freq=inv.numpy(), cos=cos, sin=sin, k_out=kb, v_out=vb, n_out=np.int64(n2))


def main():
    decode_fixture("decode_g4_n300.npz", 1000, 2, 4, 300, 128 ** -0.5)
    decode_fixture("decode_g2_n77.npz", 1001, 2, 2, 77, 0.3)
    splice_fixture("splice_overlap_n40.npz", 1002, 2, 40, 10, 17, 20, 1e4)
    splice_fixture("splice_gap_n96.npz", 1003, 2, 96, 8, 60, 30, 1e6)
    print("fixtures written to", HERE)


if __name__ == "__main__":
    main()
