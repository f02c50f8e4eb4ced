"""Seeded synthetic inputs for the five BASELINE configurations (TEST INFRASTRUCTURE ONLY:
shared by the parity tests, smoke() and bench.py so all of them draw identical tensors).

Draws follow the configuration text: activations N(0, 1) (silu input N(0, 2), i.e. std 2),
norm weights N(1, 0.1), the embedding table N(0, 0.02), positions and ids uniform. All
draws come from a CPU torch.Generator, so they do not depend on the device.
"""

from __future__ import annotations

import torch


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def normal(shape, dtype, seed, mean=0.0, std=1.0) -> torch.Tensor:
    return (torch.randn(*shape, generator=gen(seed)) * std + mean).to(dtype)


def uniform_ints(n: int, high: int, seed: int) -> torch.Tensor:
    return torch.randint(0, high, (n,), generator=gen(seed), dtype=torch.int64)


def add_rmsnorm_inputs(tokens: int, hidden: int, dtype, seed: int = 0):
    """Configs 1 and 4c: x, residual N(0,1); weight N(1, 0.1)."""
    x = normal((tokens, hidden), dtype, seed)
    r = normal((tokens, hidden), dtype, seed + 1)
    w = normal((hidden,), dtype, seed + 2, mean=1.0, std=0.1)
    return x, r, w


def rope_inputs(tokens: int, hq: int, hk: int, d: int, max_pos: int, dtype, seed: int = 0):
    """Config 2: q [T, Hq, D], k [T, Hk, D] N(0,1); positions uniform in [0, max_pos)."""
    q = normal((tokens, hq, d), dtype, seed)
    k = normal((tokens, hk, d), dtype, seed + 1)
    pos = uniform_ints(tokens, max_pos, seed + 2)
    return q, k, pos


def silu_inputs(tokens: int, inter: int, dtype, seed: int = 0):
    """Config 3: fused gate/up [T, 2I] drawn N(0, 2) (std 2)."""
    return normal((tokens, 2 * inter), dtype, seed, std=2.0)


def gate_up_inputs(tokens: int, hidden: int, inter: int, dtype, seed: int = 0):
    """The dense MLP's input: activations N(0, 1) [T, H] and a gate_up weight [2I, H] drawn
    N(0, 1.5 / sqrt(H)), so the projections are about N(0, 1.5^2) as in a trained layer."""
    x = normal((tokens, hidden), dtype, seed)
    w = normal((2 * inter, hidden), dtype, seed + 1, std=1.5 / hidden ** 0.5)
    return x, w


def embedding_inputs(tokens: int, vocab: int, hidden: int, dtype, seed: int = 0):
    """Config 4a: table N(0, 0.02), ids uniform over the vocabulary."""
    w = normal((vocab, hidden), dtype, seed, std=0.02)
    ids = uniform_ints(tokens, vocab, seed + 1)
    return ids, w


def qkv_inputs(tokens: int, hq: int, hk: int, d: int, max_pos: int, dtype, seed: int = 0):
    """Config 4b: the fused qkv projection output [T, (Hq + 2 Hk) * D] N(0,1), per-head
    norm weights N(1, 0.1), positions uniform."""
    qkv = normal((tokens, (hq + 2 * hk) * d), dtype, seed)
    qw = normal((d,), dtype, seed + 1, mean=1.0, std=0.1)
    kw = normal((d,), dtype, seed + 2, mean=1.0, std=0.1)
    pos = uniform_ints(tokens, max_pos, seed + 3)
    return qkv, qw, kw, pos


def mla_inputs(tokens: int, heads: int, nope: int, rope_dim: int, rank: int, max_pos: int, dtype,
               seed: int = 0):
    """Config 5: kv_a [T, R + Dr] and q [T, H, Dn + Dr] N(0,1), weight N(1, 0.1),
    positions uniform."""
    kv_a = normal((tokens, rank + rope_dim), dtype, seed)
    q = normal((tokens, heads, nope + rope_dim), dtype, seed + 1)
    w = normal((rank,), dtype, seed + 2, mean=1.0, std=0.1)
    pos = uniform_ints(tokens, max_pos, seed + 3)
    return kv_a, q, w, pos


def decode_inputs(ctx_lens, hq: int, hkv: int, d: int, block: int, dtype, seed: int = 0,
                  spare_blocks: int = 1, table_width: int | None = None):
    """A paged decode step in the shape of the reference's decode tests and kernel bench
    (tests/test_paged_triton_gpu.py:50-87, scripts/bench_kernels.py:55-80): every cache
    block holds N(0, 1) K/V (stale blocks hold real data, so a wrong table read shows), each
    sequence's blocks are a random permutation of the pool (scrambled, non-contiguous
    tables), q ~ N(0, 1). Table padding entries are valid block ids (0), as the backend
    passes them (attn/paged_flash.py:91-96). Returns (q, k_cache, v_cache, block_tables
    int32, context_lens int32)."""
    ctx = [int(c) for c in ctx_lens]
    g = gen(seed)
    per = [-(-c // block) for c in ctx]
    num_blocks = sum(per) + spare_blocks
    width = max(1, max(per) if per else 1) if table_width is None else table_width
    k_cache = torch.randn(num_blocks, block, hkv, d, generator=g).to(dtype)
    v_cache = torch.randn(num_blocks, block, hkv, d, generator=g).to(dtype)
    perm = torch.randperm(num_blocks, generator=g).tolist()
    tables = torch.zeros(len(ctx), width, dtype=torch.int32)
    at = 0
    for i, n in enumerate(per):
        tables[i, :n] = torch.tensor(perm[at:at + n], dtype=torch.int32)
        at += n
    q = torch.randn(len(ctx), hq, d, generator=g).to(dtype)
    return q, k_cache, v_cache, tables, torch.tensor(ctx, dtype=torch.int32)


def mla_decode_inputs(ctx_lens, num_heads: int, dl: int, dr: int, block: int, dtype, seed: int = 0,
                      spare_blocks: int = 5, table_width: int | None = None, amp: float = 0.5):
    """An MLA decode step in the shape of the reference's kernel test
    (tests/test_mla_triton_gpu.py:27-37): a latent cache [num_blocks, block, DL + DR] of
    amp * N(0, 1) rows (stale blocks hold real data), scrambled non-contiguous tables with
    valid padding ids (0), q_abs = [q_c | q_pe] ~ amp * N(0, 1). Returns (q_abs [B, H, DL +
    DR], latent_cache, block_tables int32, context_lens int32)."""
    ctx = [int(c) for c in ctx_lens]
    g = gen(seed)
    per = [-(-c // block) for c in ctx]
    num_blocks = sum(per) + spare_blocks
    width = max(1, max(per) if per else 1) if table_width is None else table_width
    latent = (torch.randn(num_blocks, block, dl + dr, generator=g) * amp).to(dtype)
    perm = torch.randperm(num_blocks, generator=g).tolist()
    tables = torch.zeros(len(ctx), width, dtype=torch.int32)
    at = 0
    for i, n in enumerate(per):
        tables[i, :n] = torch.tensor(perm[at:at + n], dtype=torch.int32)
        at += n
    q_abs = (torch.randn(len(ctx), num_heads, dl + dr, generator=g) * amp).to(dtype)
    return q_abs, latent, tables, torch.tensor(ctx, dtype=torch.int32)
