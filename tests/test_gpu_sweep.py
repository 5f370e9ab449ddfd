"""The 36-layer decode sweep (Qwen3-4B GQA shape, seed 2) through the entry points the benchmark times.

Every sweep length runs through ``decode_attention_batched`` (tc_decode_attention with the
tuned split plan) and ``DecodePlan.run()``, against the float64 closed form and fp32 torch
SDPA with the query heads folded (the reference's CPU path), at max-abs 2e-3 (fp16 output
after fp32 accumulation). The benchmark's step itself, 36 DecodePlan.run() calls captured as
one HIP graph, is replayed three times with eager work between the replays, and three
layers' outputs are checked against the oracle after every replay.
"""
import numpy as np
import pytest
import torch

from oracle import decode as od
from threadcut_amd import flash_decode, workloads

pytestmark = pytest.mark.gpu

TOL = 2e-3
SCALE = 128 ** -0.5


@pytest.mark.parametrize("n", workloads.SWEEP_TOKENS)
def test_sweep_length_through_timed_entry_points(gpu, n):
    q, k, v, _ = workloads.decode_inputs(2, n=n)
    qd = q.to(gpu).reshape(1, 8, 4, 128)
    kd, vd = k.to(gpu), v.to(gpu)
    plan_out = torch.full_like(qd, float("nan"))
    plan = flash_decode.DecodePlan(qd, kd, vd, SCALE, plan_out)
    print(f"case: sweep n={n} seed 2, {plan.splits} splits of {plan.split_tokens} tokens", flush=True)
    assert plan.splits == flash_decode.num_splits(1, 8, n) and plan.splits * plan.split_tokens >= n
    out = flash_decode.decode_attention_batched(qd, kd, vd, SCALE)
    plan.run()
    torch.cuda.synchronize()
    assert torch.equal(out, plan_out)
    got = out.float().cpu().numpy()
    ref64 = od.attention_f64(q.float().numpy().reshape(1, 8, 4, 128), k.float().numpy(), v.float().numpy(), SCALE)
    ref32 = od.folded_sdpa(q.float(), k.float(), v.float(), SCALE).numpy().reshape(1, 8, 4, 128)
    assert np.abs(got - ref64).max() <= TOL
    assert np.abs(got - ref32).max() <= TOL


def test_captured_36_layer_step_replays_match_oracle(gpu):
    n = 10240
    print(f"case: 36-layer graph at n={n} seed 2", flush=True)
    qs, ks, vs = workloads.sweep_layers(n, device=gpu)
    outs = [torch.empty_like(q) for q in qs]
    plans = [flash_decode.DecodePlan(q, k, v, SCALE, o) for q, k, v, o in zip(qs, ks, vs, outs)]

    def step():
        for p in plans:
            p.run()

    step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    checked = (0, 17, 35)
    refs = {l: od.attention_f64(qs[l].float().cpu().numpy(), ks[l].float().cpu().numpy(),
                                vs[l].float().cpu().numpy(), SCALE) for l in checked}
    for rep in range(3):
        for o in outs:
            o.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for l in checked:
            err = np.abs(outs[l].float().cpu().numpy() - refs[l]).max()
            assert err <= TOL, (rep, l, err)
        assert all(bool(torch.isfinite(o).all()) for o in outs)
