"""CPU restatement of the reference's PyTorch-eager ops (TEST INFRASTRUCTURE ONLY).

Each function restates, op for op and in the same dtypes, the reference function named in
its docstring, so its rounding structure is the reference's by construction: it runs the
same PyTorch CPU kernels (torch 2.10 here; the reference pins torch>=2.2,
pyproject.toml:14). The reference defines these ops as "whatever torch-eager computes", so
torch CPU *is* the arithmetic being restated.

How each function is pinned (tests/test_oracle.py), beyond this restatement:
  rmsnorm, fused_add_rmsnorm   float64 closed form within 1 ulp of the storage dtype; a
                               constant row's closed form; exact invariance under
                               power-of-two scaling (eps = 0); the residual equals numpy's
                               IEEE float16 sum bit for bit (bf16: explicit RNE in numpy);
                               the reference's own test cases (shapes, seeds).
  rope, rope_tables            float64 complex-number rotation (the reference's own
                               closed-form test, tests/test_rope.py:17-27); identity at
                               position 0; norm preservation; relative-position invariance;
                               rotate_half on arange(6) (test_rope.py:31-32); the tables
                               against float64 cos/sin; Llama-3 scaling bands.
  silu_and_mul                 float64 g*sigmoid(g)*u within 2 ulp; silu(0) = 0.
  embedding                    numpy.take, bit-exact.
  qk_norm_rope, mla_latent_rope  float64 normalise-then-rotate closed forms; untouched
                               columns bit-exact.
  kv_cache_write, latent_cache_write  an explicit per-token loop of slice assignments
                               (slot by slot), bit-exact; untouched slots stay untouched.
  mixed_pack, mixed_unpack     a per-element Python definition on small inputs (slot by
                               slot, zero padding); unpack(pack(q)) == q for every mix.
  gather_batch, paged_decode   float64 brute force over the block table, key by key
                               (math.exp, Python sums); one key gives its V row; equal
                               keys give the mean of V; relocating blocks leaves the result
                               unchanged; GQA maps head h to KV head h // G; the per-sequence
                               causal_softmax_attention formulation (attn/base.py:105-128).
  mla_decode                   float64 brute force over the block table, key by key; one
                               key gives its c row; equal rows give the mean of c; block
                               relocation invariance; q_pe = 0 with k_pe = 0 reduces it to
                               MQA paged_decode over the c part; the non-absorbed per-head
                               form with random W_UK / W_UV equals the absorbed one
                               (mla_torch.py:1-17 derivation).
  gate_up_silu                 per-element float64 dot products (Python sums) rounded to
                               the dtype, then silu_and_mul, on small inputs; unit-vector
                               weight rows pick single x columns exactly; zero up rows give
                               zero; the gate and up halves map to rows [0, I) and [I, 2I).
  moe_gate_up_silu             every token routed to one expert equals gate_up_silu with
                               that expert's weight, row by row; rows follow the assignment
                               order t * k + c; experts are picked by index, not position.
  pack_gate_up_weight          an element-by-element index definition on a small weight.
  pack_moe_gate_up_weight      the same, per expert.
  moe_align                    the reference's own layout case (tests/test_moe_triton.py:
                               34-48) written out slot by slot; every assignment exactly once;
                               runs ascending and block-aligned; sizes; all-one-expert and
                               no-assignment cases in closed form.
No function is left unpinned.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """emberserve/model/ops.py:51-55 (rmsnorm_torch)."""
    xf = x.float()
    variance = xf.pow(2).mean(-1, keepdim=True)
    xf = xf * torch.rsqrt(variance + eps)
    return weight * xf.to(x.dtype)


def fused_add_rmsnorm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                      eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """emberserve/model/ops.py:58-63 (fused_add_rmsnorm_torch): (normed, new_residual)."""
    residual = residual + x
    return rmsnorm(residual, weight, eps), residual


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """emberserve/model/ops.py:66-68 (_rotate_half)."""
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def rope(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
         positions: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """emberserve/model/ops.py:71-81 (rope_torch): new tensors."""
    c = cos[positions][:, None, :]
    s = sin[positions][:, None, :]

    def rot(x: torch.Tensor) -> torch.Tensor:
        xf = x.float()
        return (xf * c + rotate_half(xf) * s).to(x.dtype)

    return rot(q), rot(k)


def silu_and_mul(x: torch.Tensor) -> torch.Tensor:
    """emberserve/model/ops.py:84-87 (silu_and_mul_torch)."""
    inter = x.shape[-1] // 2
    return F.silu(x[..., :inter]) * x[..., inter:]


def gate_up_silu(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """silu_and_mul(gate_up_proj(x)), Qwen2MLP.forward (emberserve/model/qwen2.py:60-61),
    weight [2I, H] = nn.Linear(H, 2I).weight (rows [0, I) gate, [I, 2I) up,
    qwen2.py:49-57). The linear layer's output is in x's dtype (rounded) before
    silu_and_mul; its dot products are formed in float64 here, so the only rounding before
    the activation's is the one to the dtype."""
    gate_up = (x.double() @ weight.double().T).to(x.dtype)
    return silu_and_mul(gate_up)


def pack_gate_up_weight(weight: torch.Tensor, num_workgroups: int) -> torch.Tensor:
    """The packed gate_up weight layout of this library's decode kernel for a grid of
    num_workgroups (no counterpart in the reference; a permutation of W [2I, H]). Units
    (slab, j) of 8192 elements, unit[h][wave][part][lane][8] = W[part I + 64 slab + 16 wave +
    lane % 16][64 j + 32 h + 8 (lane // 16) + e]; workgroup b runs units [b U // G, (b + 1) U
    // G) of the slab-major order, and the packed array lists the runs' units round by round:
    the first unit of every run in workgroup order, then the second, and so on."""
    two_i, h = weight.shape
    i = two_i // 2
    v = weight.reshape(2, i // 64, 4, 16, h // 64, 2, 4, 8)   # part, slab, wave, n, j, h, g, e
    units = v.permute(1, 4, 5, 2, 0, 6, 3, 7).reshape(-1, 8192)  # slab, j, h, wave, part, g, n, e
    total = units.shape[0]
    g = min(num_workgroups, total)
    runs = [list(range(b * total // g, (b + 1) * total // g)) for b in range(g)]
    order = [run[t] for t in range(max(len(r) for r in runs)) for run in runs if t < len(run)]
    return units[torch.tensor(order)].reshape(-1)


def pack_moe_gate_up_weight(w_gate_up: torch.Tensor) -> torch.Tensor:
    """The packed routed-expert gate_up layout of this library (no counterpart in the
    reference; a permutation of W [E, 2I, H]): per expert, units (j, slab) in j-major order,
    each unit[h][wave][part][lane][8] = W[e][part I + 64 slab + 16 wave + lane % 16]
    [64 j + 32 h + 8 (lane // 16) + e8]."""
    ne, two_i, h = w_gate_up.shape
    i = two_i // 2
    v = w_gate_up.reshape(ne, 2, i // 64, 4, 16, h // 64, 2, 4, 8)  # E, part, slab, wave, n, j, h, g, e8
    return v.permute(0, 5, 2, 6, 3, 1, 7, 4, 8).reshape(-1)        # E, j, slab, h, wave, part, g, n, e8


def moe_gate_up_silu(x: torch.Tensor, topk_ids: torch.Tensor, w_gate_up: torch.Tensor) -> torch.Tensor:
    """The routed experts' activations of fused_moe_forward (emberserve/model/moe_triton.py:
    332-341), defined per assignment as DeepseekMoE.expert computes them (moe.py:117-120):
    row t * k + c is silu_and_mul(x[t] @ w_gate_up[topk_ids[t, c]].T), the projection
    rounded to x's dtype (the grouped GEMM's output) before the activation."""
    n, k = topk_ids.shape
    rows = []
    for t in range(n):
        for c in range(k):
            rows.append(gate_up_silu(x[t:t + 1], w_gate_up[int(topk_ids[t, c])]))
    return torch.cat(rows, dim=0)


def moe_align(topk_ids: torch.Tensor, num_experts: int, block_m: int) -> tuple[list, list, int]:
    """The block-aligned expert layout that moe_align returns (emberserve/model/
    moe_triton.py:215-254, contract in its docstring :217-228), defined assignment by
    assignment: for experts in ascending order, the ids (token * k + choice) routed to the
    expert in ascending order, padded with num_valid to a multiple of block_m; num_valid up
    to max_padded = round_up(num_valid + E (block_m - 1), block_m) (:247); block b's expert
    is the expert whose padded run holds slot b * block_m, num_experts past the last run.
    Returns plain lists (sorted_ids, block_expert) and num_valid."""
    flat = [int(v) for v in topk_ids.reshape(-1).tolist()]
    num_valid = len(flat)
    max_padded = (num_valid + num_experts * (block_m - 1) + block_m - 1) // block_m * block_m
    sorted_ids, block_expert = [], []
    for e in range(num_experts):
        run = [i for i, v in enumerate(flat) if v == e]
        if not run:
            continue
        pad = -len(run) % block_m
        sorted_ids += run + [num_valid] * pad
        block_expert += [e] * ((len(run) + pad) // block_m)
    sorted_ids += [num_valid] * (max_padded - len(sorted_ids))
    block_expert += [num_experts] * (max_padded // block_m - len(block_expert))
    return sorted_ids, block_expert, num_valid


def embedding(ids: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """torch.nn.Embedding.forward as used at emberserve/model/qwen2.py:182."""
    return F.embedding(ids, weight)


def llama3_scale_inv_freq(inv_freq: torch.Tensor, scaling: dict) -> torch.Tensor:
    """emberserve/model/rope.py:36-51."""
    factor = float(scaling["factor"])
    low_freq_factor = float(scaling["low_freq_factor"])
    high_freq_factor = float(scaling["high_freq_factor"])
    old_context_len = float(scaling["original_max_position_embeddings"])
    low_freq_wavelen = old_context_len / low_freq_factor
    high_freq_wavelen = old_context_len / high_freq_factor
    wavelen = 2 * math.pi / inv_freq
    inv_freq_llama = torch.where(wavelen > low_freq_wavelen, inv_freq / factor, inv_freq)
    smooth = (old_context_len / wavelen - low_freq_factor) / (high_freq_factor - low_freq_factor)
    smoothed = (1 - smooth) * inv_freq_llama / factor + smooth * inv_freq_llama
    is_medium = ~(wavelen < high_freq_wavelen) & ~(wavelen > low_freq_wavelen)
    return torch.where(is_medium, smoothed, inv_freq_llama)


def rope_tables(head_dim: int, max_position_embeddings: int, base: float,
                rope_scaling: dict | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """emberserve/model/rope.py:68-82 (inv_freq + _build_tables), on the CPU: fp32
    cos/sin [max_pos, head_dim] with equal halves."""
    exponent = torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim
    inv = 1.0 / (float(base) ** exponent)
    if rope_scaling and rope_scaling.get("rope_type", rope_scaling.get("type")) == "llama3":
        inv = llama3_scale_inv_freq(inv, rope_scaling)
    positions = torch.arange(max_position_embeddings, dtype=torch.float32)
    freqs = torch.outer(positions, inv)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos(), emb.sin()


def qk_norm_rope(q: torch.Tensor, k: torch.Tensor, q_weight: torch.Tensor, k_weight: torch.Tensor,
                 eps: float, cos: torch.Tensor, sin: torch.Tensor,
                 positions: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """emberserve/model/qwen2.py:95-101: q_norm/k_norm on [n*heads, head_dim] rows (the
    reshape copies the split views), view back, then rotary_emb -> ops.rope."""
    n, h, d = q.shape
    hk = k.shape[1]
    qn = rmsnorm(q.reshape(n * h, d), q_weight, eps).view(n, h, d)
    kn = rmsnorm(k.reshape(n * hk, d), k_weight, eps).view(n, hk, d)
    return rope(qn, kn, cos, sin, positions)


def mla_latent_rope(c: torch.Tensor, k_pe: torch.Tensor, q_pe: torch.Tensor, weight: torch.Tensor,
                    eps: float, cos: torch.Tensor, sin: torch.Tensor,
                    positions: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """emberserve/model/deepseek.py:126-133 (rope_folded branch): c = kv_a_layernorm(c);
    q_pe, k_pe = rotary_emb(q_pe, k_pe.unsqueeze(1)); latent = cat([c, k_pe.squeeze(1)]).
    Returns (q_pe, latent)."""
    c = rmsnorm(c, weight, eps)
    q_pe, k_pe = rope(q_pe, k_pe.reshape(k_pe.shape[0], -1).unsqueeze(1), cos, sin, positions)
    latent = torch.cat([c, k_pe.squeeze(1)], dim=-1)
    return q_pe, latent


def kv_cache_write(k: torch.Tensor, v: torch.Tensor, slot_mapping: torch.Tensor,
                   k_cache: torch.Tensor, v_cache: torch.Tensor) -> None:
    """emberserve/kv/cache.py:54-61 (PagedKVCache.write) for one layer's caches
    [num_blocks, block_size, Hkv, D]: index_copy_ of k and v at the slots, in place."""
    slots = slot_mapping.to(device=k_cache.device, dtype=torch.long)
    flat = (-1, k.shape[1], k.shape[2])
    k_cache.view(flat).index_copy_(0, slots, k.to(k_cache.dtype))
    v_cache.view(flat).index_copy_(0, slots, v.to(v_cache.dtype))


def latent_cache_write(latent: torch.Tensor, slot_mapping: torch.Tensor, cache: torch.Tensor) -> None:
    """emberserve/kv/cache.py:152-157 (PagedLatentCache.write) for one layer's cache
    [num_blocks, block_size, latent_dim]."""
    slots = slot_mapping.to(device=cache.device, dtype=torch.long)
    cache.view(-1, latent.shape[-1]).index_copy_(0, slots, latent.to(cache.dtype))


def gather_batch(k_cache: torch.Tensor, v_cache: torch.Tensor, block_tables: torch.Tensor,
                 context_lens: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """emberserve/kv/cache.py:81-107 (PagedKVCache.gather_batch) for one layer's caches
    [num_blocks, block_size, Hkv, D]: padded K/V [B, max_ctx, Hkv, D] and the validity mask
    [B, max_ctx]; negative table entries are clamped to 0 as there."""
    bs = k_cache.shape[1]
    ctx = context_lens.to(dtype=torch.long)
    max_ctx = int(ctx.max())
    nb = -(-max_ctx // bs)
    idx = block_tables[:, :nb].to(dtype=torch.long).clamp_min(0)
    batch = idx.shape[0]

    def one(store: torch.Tensor) -> torch.Tensor:
        blocks = store[idx]
        return blocks.reshape(batch, nb * bs, store.shape[2], store.shape[3])[:, :max_ctx]

    valid = torch.arange(max_ctx)[None, :] < ctx[:, None]
    return one(k_cache), one(v_cache), valid


def paged_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                 block_tables: torch.Tensor, context_lens: torch.Tensor, scale: float) -> torch.Tensor:
    """emberserve/attn/paged_torch.py:87-98 (PagedTorchAttentionBackend._decode), the fp32
    definition every decode kernel of the reference is tested against: GQA-expanded fp32
    K/V, scores * scale, masked softmax, P.V; the result in q.dtype."""
    k, v, valid = gather_batch(k_cache, v_cache, block_tables, context_lens)
    groups = q.shape[1] // k_cache.shape[2]
    kf = k.float().repeat_interleave(groups, dim=2)
    vf = v.float().repeat_interleave(groups, dim=2)
    scores = torch.einsum("bhd,bkhd->bhk", q.float(), kf) * scale
    scores = scores.masked_fill(~valid[:, None, :], float("-inf"))
    probs = torch.softmax(scores, dim=-1)
    out = torch.einsum("bhk,bkhd->bhd", probs, vf)
    return out.to(q.dtype)


def paged_decode_prob_mass(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                           block_tables: torch.Tensor, context_lens: torch.Tensor,
                           scale: float) -> torch.Tensor:
    """sum_j p_j |v_j| per output element (fp32, [B, H, D]), the same softmax as
    paged_decode: the scale of the error that rounding the probabilities to the cache dtype
    before P.V (the reference's tl.dot variant, attn/paged_triton.py:163-167) can add."""
    k, v, valid = gather_batch(k_cache, v_cache, block_tables, context_lens)
    groups = q.shape[1] // k_cache.shape[2]
    kf = k.float().repeat_interleave(groups, dim=2)
    vf = v.float().repeat_interleave(groups, dim=2)
    scores = torch.einsum("bhd,bkhd->bhk", q.float(), kf) * scale
    scores = scores.masked_fill(~valid[:, None, :], float("-inf"))
    probs = torch.softmax(scores, dim=-1)
    return torch.einsum("bhk,bkhd->bhd", probs, vf.abs())


def gather_latent(latent_cache: torch.Tensor, block_table_row: torch.Tensor, n: int) -> torch.Tensor:
    """emberserve/kv/cache.py (PagedLatentCache.gather): the first n cache rows of one
    sequence, [n, DL + DR]."""
    bs = latent_cache.shape[1]
    idx = block_table_row[:-(-n // bs)].to(dtype=torch.long)
    return latent_cache[idx].reshape(-1, latent_cache.shape[2])[:n]


def mla_attention_absorbed(q_nope: torch.Tensor, q_pe: torch.Tensor, latent: torch.Tensor,
                           w_uk: torch.Tensor, w_uv: torch.Tensor, scale: float,
                           kv_lora_rank: int) -> torch.Tensor:
    """emberserve/attn/mla_torch.py:33-53: one sequence, q [Q, H, .] the last Q positions of
    a context of latent rows [T, DL + DR]; causal mask; fp32 math; the result in q_nope's
    dtype."""
    q_len, t_len = q_nope.shape[0], latent.shape[0]
    c = latent[:, :kv_lora_rank].float()
    k_pe = latent[:, kv_lora_rank:].float()
    q_c = torch.einsum("qhn,hnl->qhl", q_nope.float(), w_uk.float())
    scores = (torch.einsum("qhl,tl->hqt", q_c, c) + torch.einsum("qhr,tr->hqt", q_pe.float(), k_pe)) * scale
    pos = torch.arange(t_len - q_len, t_len)[:, None]
    mask = torch.arange(t_len)[None, :] > pos
    scores = scores.masked_fill(mask[None], float("-inf"))
    p = torch.softmax(scores, dim=-1)
    out_c = torch.einsum("hqt,tl->qhl", p, c)
    return torch.einsum("qhl,hvl->qhv", out_c, w_uv.float()).to(q_nope.dtype)


def mla_decode(q_c: torch.Tensor, q_pe: torch.Tensor, latent_cache: torch.Tensor,
               block_tables: torch.Tensor, context_lens: torch.Tensor, scale: float,
               kv_lora_rank: int) -> torch.Tensor:
    """The raw P.c output of the MLA decode kernel (attn/mla_triton.py:119-182) as the
    reference's tests define it (tests/test_mla_triton_gpu.py:40-49): per sequence, gather
    its rows and run mla_attention_absorbed with identity W_UK / W_UV on fp32 inputs.
    q_c [B, H, DL], q_pe [B, H, DR]; returns fp32 [B, H, DL]."""
    h = q_c.shape[1]
    eye = torch.eye(kv_lora_rank).expand(h, kv_lora_rank, kv_lora_rank)
    outs = []
    for b in range(q_c.shape[0]):
        rows = gather_latent(latent_cache, block_tables[b], int(context_lens[b]))
        outs.append(mla_attention_absorbed(q_c[b][None].float(), q_pe[b][None].float(), rows.float(),
                                           eye, eye, scale, kv_lora_rank)[0])
    return torch.stack(outs)


def mla_decode_prob_mass(q_c: torch.Tensor, q_pe: torch.Tensor, latent_cache: torch.Tensor,
                         block_tables: torch.Tensor, context_lens: torch.Tensor, scale: float,
                         kv_lora_rank: int) -> torch.Tensor:
    """sum_j p_j |c_j| per output element (fp32 [B, H, DL]) under mla_decode's softmax: the
    scale of the error that rounding the probabilities to the cache dtype before P.c (the
    reference kernel's tl.dot, attn/mla_triton.py:109) can add."""
    outs = []
    for b in range(q_c.shape[0]):
        rows = gather_latent(latent_cache, block_tables[b], int(context_lens[b])).float()
        c, k_pe = rows[:, :kv_lora_rank], rows[:, kv_lora_rank:]
        scores = (q_c[b].float() @ c.T + q_pe[b].float() @ k_pe.T) * scale
        outs.append(torch.softmax(scores, dim=-1) @ c.abs())
    return torch.stack(outs)


def mixed_rows(query_lens):
    """MixedPlan.build's row bookkeeping (emberserve/attn/paged_flash.py:127-150): packed
    start of each decode row (query_len == 1) and (start, n) of each prefill row."""
    dec, pre, start = [], [], 0
    for n in query_lens:
        if n == 1:
            dec.append(start)
        else:
            pre.append((start, n))
        start += n
    return dec, pre


def mixed_pack(q: torch.Tensor, query_lens):
    """The query side of PagedFlashAttentionBackend._prefill_kvcache (paged_flash.py:
    259-272): q.index_select(0, dec_tokens) for the decode rows; the prefill rows
    left-padded into q.new_zeros((P, max_q, H, D)). Returns (q_dec or None, qpad or None)."""
    dec, pre = mixed_rows(query_lens)
    q_dec = q.index_select(0, torch.tensor(dec, dtype=torch.long)) if dec else None
    qpad = None
    if pre:
        max_q = max(n for _, n in pre)
        qpad = q.new_zeros((len(pre), max_q) + tuple(q.shape[1:]))
        for i, (start, n) in enumerate(pre):
            qpad[i, max_q - n:] = q[start:start + n]
    return q_dec, qpad


def mixed_unpack(out: torch.Tensor, o_dec, o_pad, query_lens) -> torch.Tensor:
    """The output side (paged_flash.py:267, 276-277): out.index_copy_(0, dec_tokens, o_dec)
    and out[start:start + n] = o_pad[i, max_q - n:]. In place on out; returns it."""
    dec, pre = mixed_rows(query_lens)
    if dec:
        out.index_copy_(0, torch.tensor(dec, dtype=torch.long), o_dec.reshape((len(dec),) + tuple(out.shape[1:])))
    if pre:
        max_q = o_pad.shape[1]
        for i, (start, n) in enumerate(pre):
            out[start:start + n] = o_pad[i, max_q - n:]
    return out
