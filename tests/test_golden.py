"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle still reproduces every stored output (a regression test of the oracle).
GPU: the HIP kernels reproduce them (decode within 2e-3, splice bit-exact).
"""
import os

import numpy as np
import pytest
import torch

from oracle import decode as od
from oracle import splice as osp

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
DECODE = ["decode_g4_n300.npz", "decode_g2_n77.npz"]
SPLICE = ["splice_overlap_n40.npz", "splice_gap_n96.npz"]


def load(name):
    return np.load(os.path.join(HERE, name))


@pytest.mark.parametrize("name", DECODE)
def test_oracle_reproduces_decode_fixture(name):
    f = load(name)
    q, k, v = (f[x].astype(np.float32) for x in ("q", "k", "v"))
    o, lse = od.flash_decode_partial(q, k, v, float(f["scale"]))
    assert np.array_equal(o, f["o_part"]) and np.array_equal(lse, f["lse"])
    assert np.abs(od.attention_f64(q, k, v, float(f["scale"])) - f["out64"]).max() < 1e-12
    assert np.abs(f["out32"] - f["out64"]).max() < 2e-6


@pytest.mark.parametrize("name", SPLICE)
def test_oracle_reproduces_splice_fixture(name):
    f = load(name)
    a, c0, c = (int(x) for x in f["split"])
    cos, sin = osp.rope_table(-(c0 - a), torch.from_numpy(f["inv_freq"]))
    assert np.array_equal(cos, f["cos"]) and np.array_equal(sin, f["sin"])
    kb, vb, n = osp.splice_growing(f["k"], f["v"], f["k"].shape[2], a, c0, c, cos, sin)
    assert n == int(f["n_out"])
    assert np.array_equal(kb.view(np.uint16), f["k_out"].view(np.uint16))
    assert np.array_equal(vb.view(np.uint16), f["v_out"].view(np.uint16))


@pytest.mark.gpu
@pytest.mark.parametrize("name", DECODE)
def test_kernels_reproduce_decode_fixture(gpu, name):
    from threadcut_amd import flash_decode

    f = load(name)
    q = torch.from_numpy(f["q"]).to(gpu)
    k = torch.from_numpy(f["k"]).to(gpu)
    v = torch.from_numpy(f["v"]).to(gpu)
    out = flash_decode.decode_attention(q, k, v, float(f["scale"]), split=256)
    torch.cuda.synchronize()
    assert np.abs(out.float().cpu().numpy() - f["out64"]).max() <= 2e-3
    assert np.abs(out.float().cpu().numpy() - f["out16"].astype(np.float32)).max() <= 2e-3


@pytest.mark.gpu
@pytest.mark.parametrize("name", SPLICE)
def test_kernels_reproduce_splice_fixture(gpu, name):
    from threadcut_amd import kv
    from threadcut_amd.match import Split

    f = load(name)
    a, c0, c = (int(x) for x in f["split"])
    layer = kv.GrowingLayer()
    layer.update(torch.from_numpy(f["k"]).to(gpu), torch.from_numpy(f["v"]).to(gpu))
    layer.splice(Split(a, c0, c), torch.from_numpy(f["inv_freq"]))
    torch.cuda.synchronize()
    n = f["k"].shape[2]
    assert layer.n == int(f["n_out"])
    assert np.array_equal(layer.kbuf[:, :, :n].cpu().numpy().view(np.uint16), f["k_out"].view(np.uint16))
    assert np.array_equal(layer.vbuf[:, :, :n].cpu().numpy().view(np.uint16), f["v_out"].view(np.uint16))
