"""Seeded synthetic inputs of the decode and splice workloads (Qwen3-4B geometry).

Convention: one ``torch.Generator`` per workload, seeded; float32 N(0, 1)
draws cast to the storage dtype; draw order lengths (if any), then Q, then K,
then V. ``device="cpu"`` draws on the host generator (the parity tests'
inputs); a CUDA device draws on a seeded device generator (same distribution,
different values), which the benchmark uses for its multi-GB caches.

Workloads:
- single decode call: B=1, 32 query heads over 8 KV heads, D=128, 1536 tokens, seed 0;
- 36-layer suffix splice: 36 x [1, 8, 14336, 128], prune [2048, 8668), theta 1e6, seed 1;
- 36-layer decode sweep: 1536 / 4096 / 10240 / 14336 tokens, seed 2;
- ragged batch: 16 sequences, lengths U[1024, 32768], seed 3;
- long context: B = 1 and 4 at 131072 tokens, seed 4.
"""
import torch

from .match import Split

QWEN3_4B = dict(layers=36, q_heads=32, kv_heads=8, head_dim=128, rope_theta=1e6)

SPLICE_SPLIT = Split(2048, 8668, 5668)
SPLICE_TOKENS = 14336
SWEEP_TOKENS = (1536, 4096, 10240, 14336)


def _gen(seed, device):
    device = torch.device(device)
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def randn(shape, gen, dtype, device):
    return torch.randn(shape, generator=gen, dtype=torch.float32, device=device).to(dtype)


def decode_inputs(seed, batch=1, n=1536, q_heads=32, kv_heads=8, head_dim=128, dtype=torch.float16,
                  device="cpu", lens_range=None):
    """(query [B, Hq, 1, D], key [B, Hkv, n, D], value, lens or None)."""
    g = _gen(seed, device)
    lens = None
    if lens_range is not None:
        lo, hi = lens_range
        lens = torch.randint(lo, hi + 1, (batch,), generator=g, device=device, dtype=torch.int64).to(torch.int32)
    q = randn((batch, q_heads, 1, head_dim), g, dtype, device)
    k = randn((batch, kv_heads, n, head_dim), g, dtype, device)
    v = randn((batch, kv_heads, n, head_dim), g, dtype, device)
    return q, k, v, lens


def layer_caches(seed, layers, n, kv_heads=8, head_dim=128, batch=1, dtype=torch.float16, device="cpu"):
    """Per-layer (K, V) lists of [B, Hkv, n, D], each layer its own buffers."""
    g = _gen(seed, device)
    ks, vs = [], []
    for _ in range(layers):
        ks.append(randn((batch, kv_heads, n, head_dim), g, dtype, device))
        vs.append(randn((batch, kv_heads, n, head_dim), g, dtype, device))
    return ks, vs


def sweep_layers(n, layers=36, seed=2, device="cpu"):
    """The 36-layer decode sweep at n tokens: (queries, keys, values), per layer its own K/V
    [1, 8, n, 128] fp16 (drawn layer by layer, K then V) and its own query grouped as
    [1, 8, 4, 128] (the 4 query heads of each KV head), drawn afterwards from a second
    generator of the same seed."""
    ks, vs = layer_caches(seed, layers, n, device=device)
    g = _gen(seed, device)
    qs = [randn((1, 8, 4, 128), g, torch.float16, device) for _ in range(layers)]
    return qs, ks, vs


def inv_freq(theta=1e6, head_dim=128):
    """transformers' default RoPE inverse frequencies, float32 [head_dim / 2]."""
    return (1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))).float()


# Prefill: the engine runs new tokens in chunks of 2048 (threadcut/engine.py:46-48).
# After SPLICE_SPLIT the cache keeps a + c = 7716 tokens; the next chunk attends to them.
PREFILL_CHUNK = 2048
PREFILL_PAST = SPLICE_SPLIT.a + SPLICE_SPLIT.c


def prefill_inputs(seed, batch=1, q_len=PREFILL_CHUNK, n=PREFILL_PAST + PREFILL_CHUNK, q_heads=32, kv_heads=8,
                   head_dim=128, dtype=torch.float16, device="cpu"):
    """(query [B, Hq, q_len, D] as the transposed view of [B, q_len, Hq, D] that
    transformers hands over, key [B, Hkv, n, D], value)."""
    g = _gen(seed, device)
    q = randn((batch, q_len, q_heads, head_dim), g, dtype, device).transpose(1, 2)
    k = randn((batch, kv_heads, n, head_dim), g, dtype, device)
    v = randn((batch, kv_heads, n, head_dim), g, dtype, device)
    return q, k, v


def causal_mask(q_len, n, batch=1, device="cpu"):
    """Boolean [B, 1, q_len, n]: query t (at position n - q_len + t) sees keys <= its position,
    the mask transformers' sdpa_mask builds for a chunk on top of a cache."""
    t = torch.arange(q_len, device=device)[:, None] + (n - q_len)
    m = torch.arange(n, device=device)[None, :] <= t
    return m[None, None].expand(batch, 1, q_len, n)
