"""Fused per-layer elementwise ops on MI355X: the drop-in for emberserve/model/ops.py.

The public functions keep the reference's signatures and dispatch rule
(emberserve/model/ops.py:92-115): a GPU tensor runs the gfx950 HIP kernel of
libember_ops.so, a CPU tensor (or any tensor with `EMBERSERVE_FUSED_OPS=0`) runs the
PyTorch-eager form. Differences from the reference's dispatch, on purpose:

* there is no silent fallback: a GPU tensor with the fused path enabled raises
  RuntimeError when the HIP library is missing, instead of dropping to eager torch;
* three fused entry points are added for callers that want one pass instead of several:
  `qk_norm_rope` (qwen2.py:95-101), `mla_latent_rope` (deepseek.py:126-133) and
  `embedding` (nn.Embedding at qwen2.py:182).

The `*_hip` functions are the counterparts of the reference's `*_triton` wrappers
(ops_triton.py:90-134): same arguments, same output allocation (torch caching allocator on
the input's device), same in-place behaviour (rope and qk-norm rope rotate q/k in place and
return them), launched on torch's current stream with no host synchronisation, so they can
be recorded into a torch.cuda.graph.

Numerics (vs the reference's PyTorch ops on the same inputs): the residual of
fused_add_rmsnorm and the embedding gather are bit-exact; rope output is the same fp32
expression as the reference (separately rounded products and sum) and is bit-exact when the
cos/sin tables are equal; rmsnorm and silu differ only through fp32 reduction order and
exp/rsqrt implementations, within 2 ulp of the storage dtype.
"""

from __future__ import annotations

import os

import torch

from . import _lib
from .eager import (  # noqa: F401  (re-exported: the reference's names)
    _rotate_half,
    embedding_torch,
    fused_add_rmsnorm_torch,
    kv_cache_write_torch,
    latent_cache_write_torch,
    mla_latent_rope_torch,
    qk_norm_rope_torch,
    rmsnorm_torch,
    rope_torch,
    silu_and_mul_torch,
)

__all__ = [
    "fused_enabled", "rmsnorm", "fused_add_rmsnorm", "rope", "silu_and_mul", "embedding",
    "qk_norm_rope", "mla_latent_rope", "rmsnorm_hip", "fused_add_rmsnorm_hip", "rope_hip",
    "silu_and_mul_hip", "embedding_hip", "qk_norm_rope_hip", "mla_latent_rope_hip",
    "rmsnorm_torch", "fused_add_rmsnorm_torch", "rope_torch", "silu_and_mul_torch",
    "embedding_torch", "qk_norm_rope_torch", "mla_latent_rope_torch",
    "kv_cache_write", "latent_cache_write", "kv_cache_write_hip", "latent_cache_write_hip",
    "kv_cache_write_torch", "latent_cache_write_torch", "rope_kv_cache", "rope_kv_cache_hip",
    "mla_latent_rope_cache", "mla_latent_rope_cache_hip",
]


def fused_enabled(x: torch.Tensor) -> bool:
    """HIP path: a GPU tensor and `EMBERSERVE_FUSED_OPS` not "0" (ops.py:43-46). Whether
    the library is built does not enter: a missing library is an error, not a fallback."""
    return x.is_cuda and os.environ.get("EMBERSERVE_FUSED_OPS", "1") != "0"


def _check_indices() -> bool:
    return os.environ.get("EMBERSERVE_CHECK_INDICES", "0") == "1"


def _raise_index_errors() -> None:
    flags = _lib.read_errors(clear=True)
    if flags & _lib.ERR_EMBED_ID:
        raise IndexError("emberserve_amd.embedding: token id out of range")
    if flags & _lib.ERR_ROPE_POS:
        raise IndexError("emberserve_amd.rope: position out of range of the cos/sin table")
    if flags & _lib.ERR_KV_SLOT:
        raise IndexError("emberserve_amd.kv_cache_write: slot out of range of the cache")
    if flags & _lib.ERR_ROW_INDEX:
        raise IndexError("emberserve_amd.mixed: row index out of range")


_EALIGN = 2  # EMBER_EALIGN: a fused entry point refused misaligned operands, nothing ran


def _launch(what: str, fn, device: torch.device, *args, allow_unaligned: bool = False) -> bool:
    """Calls C-ABI entry point `fn(*args, stream)` with `device` current and torch's current
    stream on it (the capture stream while a torch.cuda.graph records), raising on a
    non-zero status. With allow_unaligned, EMBER_EALIGN is returned as False (the caller
    then runs the unfused ops) instead of raising. Uses torch's raw-handle accessors: this
    is on every op's hot path."""
    idx = device.index
    cur = torch._C._cuda_getDevice()
    if idx is None or idx == cur:
        st = fn(*args, torch._C._cuda_getCurrentRawStream(cur))
    else:
        with torch.cuda.device(idx):
            st = fn(*args, torch._C._cuda_getCurrentRawStream(idx))
    if st == _EALIGN and allow_unaligned:
        return False
    if st != 0:
        _lib.check(st, what)
    return True


def _require_device(what: str, *tensors: torch.Tensor) -> None:
    """Every operand of a HIP launch must live on the same GPU: a host pointer or another
    device's pointer handed to a kernel would fault the device, so it is refused here."""
    dev = tensors[0].device
    if dev.type != "cuda":
        raise ValueError(f"{what}: tensors must be on a GPU, got {dev}")
    for t in tensors[1:]:
        if t.device != dev:
            raise ValueError(f"{what}: all tensors must be on {dev}, got one on {t.device}")


def _rows2d(x: torch.Tensor) -> torch.Tensor:
    x2 = x.reshape(-1, x.shape[-1])
    if x2.shape[-1] > 1 and x2.stride(-1) != 1:
        x2 = x2.contiguous()
    return x2


def _weight_for(weight: torch.Tensor, x: torch.Tensor) -> tuple[torch.Tensor, int]:
    """The norm weight as the kernel reads it: x's dtype, or fp32 for any other dtype (an
    exact widening, which is what the reference's kernel does when it loads it)."""
    if weight.device != x.device:
        raise ValueError(f"weight on {weight.device}, activations on {x.device}")
    w = weight if weight.dtype in (x.dtype, torch.float32) else weight.float()
    if not w.is_contiguous():
        w = w.contiguous()
    return w, _lib.dtype_tag(w.dtype)


def _tables(cos: torch.Tensor, sin: torch.Tensor, positions: torch.Tensor, d: int):
    if cos.dtype != torch.float32:
        cos = cos.float()
    if sin.dtype != torch.float32:
        sin = sin.float()
    if cos.stride(-1) != 1:
        cos = cos.contiguous()
    if sin.stride(-1) != 1:
        sin = sin.contiguous()
    if cos.shape != sin.shape or cos.dim() != 2 or cos.shape[1] < d // 2 or cos.stride(0) != sin.stride(0):
        raise ValueError(f"cos/sin tables must both be [max_pos, >= {d // 2}] with equal strides")
    if positions.dtype != torch.int64:
        positions = positions.long()
    if not positions.is_contiguous():
        positions = positions.contiguous()
    return cos, sin, positions


# ---- HIP wrappers (the counterparts of ops_triton.py) ----------------------------------

def rmsnorm_hip(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """ops_triton.py:90-97."""
    _require_device("rmsnorm", x, weight)
    x2 = _rows2d(x)
    out = torch.empty(x2.shape, dtype=x.dtype, device=x.device)
    w, wtag = _weight_for(weight, x)
    if w.numel() != x2.shape[1]:
        raise ValueError(f"weight has {w.numel()} elements, rows have {x2.shape[1]}")
    _launch("ember_rmsnorm", _lib.load().ember_rmsnorm, x.device,
            x2.data_ptr(), x2.stride(0), w.data_ptr(), wtag, out.data_ptr(),
            out.stride(0), x2.shape[0], x2.shape[1], float(eps),
            _lib.dtype_tag(x.dtype))
    return out.view(x.shape)


def fused_add_rmsnorm_hip(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                          eps: float, *, out: torch.Tensor | None = None,
                          residual_out: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """ops_triton.py:100-110. Returns (normed, new_residual); the inputs are not modified.
    `out` / `residual_out` (2-D [rows, H], unit inner stride) receive the results instead of
    new tensors, for callers with static buffers (graph pieces); `residual_out` may be
    `residual` itself (each row is read whole before it is written)."""
    _require_device("fused_add_rmsnorm", x, residual, weight)
    if residual.dtype != x.dtype or residual.shape != x.shape:
        raise ValueError("x and residual must share shape and dtype")
    x2 = _rows2d(x)
    r2 = _rows2d(residual)
    for name, t in (("out", out), ("residual_out", residual_out)):
        if t is not None and (t.shape != x2.shape or t.dtype != x.dtype or t.stride(-1) != 1 or t.device != x.device):
            raise ValueError(f"fused_add_rmsnorm: {name} must be a {tuple(x2.shape)} {x.dtype} tensor on "
                             f"{x.device} with unit inner stride")
    out = torch.empty(x2.shape, dtype=x.dtype, device=x.device) if out is None else out
    new_res = torch.empty(r2.shape, dtype=x.dtype, device=x.device) if residual_out is None else residual_out
    w, wtag = _weight_for(weight, x)
    if w.numel() != x2.shape[1]:
        raise ValueError(f"weight has {w.numel()} elements, rows have {x2.shape[1]}")
    _launch("ember_fused_add_rmsnorm", _lib.load().ember_fused_add_rmsnorm, x.device,
            x2.data_ptr(), x2.stride(0), r2.data_ptr(), r2.stride(0), w.data_ptr(), wtag,
            out.data_ptr(), out.stride(0), new_res.data_ptr(), new_res.stride(0), x2.shape[0],
            x2.shape[1], float(eps), _lib.dtype_tag(x.dtype))
    return out.view(x.shape), new_res.view(residual.shape)


def rope_hip(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
             positions: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """ops_triton.py:113-124: in place on q [N, H, D] and k [N, Hkv, D] (unit stride in D,
    any other strides); returns (q, k)."""
    _require_device("rope", q, k, cos, sin, positions)
    n, h, d = q.shape
    hk = k.shape[1]
    if not (q.stride(2) == 1 and k.stride(2) == 1 and d % 2 == 0):
        raise AssertionError("rope: q/k need unit stride in the head dim and an even head_dim")
    if k.shape[0] != n or k.shape[2] != d or k.dtype != q.dtype:
        raise ValueError("rope: q and k must agree in tokens, head_dim and dtype")
    if n == 0:
        return q, k
    cos, sin, positions = _tables(cos, sin, positions, d)
    _launch("ember_rope", _lib.load().ember_rope, q.device,
            q.data_ptr(), q.stride(0), q.stride(1), h, k.data_ptr(), k.stride(0),
            k.stride(1), hk, d, cos.data_ptr(), sin.data_ptr(), cos.shape[0],
            cos.stride(0), positions.data_ptr(), n, _lib.dtype_tag(q.dtype))
    if _check_indices():
        _raise_index_errors()
    return q, k


def silu_and_mul_hip(x: torch.Tensor, *, out: torch.Tensor | None = None) -> torch.Tensor:
    """ops_triton.py:127-134. `out` ([rows, I], unit inner stride) receives the result
    instead of a new tensor."""
    _require_device("silu_and_mul", x)
    if x.shape[-1] % 2 != 0:  # the eager form fails the same way: halves of unequal size
        raise ValueError(f"silu_and_mul: last dim {x.shape[-1]} is not even")
    x2 = _rows2d(x)
    inter = x2.shape[-1] // 2
    if out is not None:
        if out.shape != (x2.shape[0], inter) or out.dtype != x.dtype or out.stride(-1) != 1 or out.device != x.device:
            raise ValueError(f"silu_and_mul: out must be a ({x2.shape[0]}, {inter}) {x.dtype} tensor on {x.device} "
                             "with unit inner stride")
    else:
        out = torch.empty((x2.shape[0], inter), dtype=x.dtype, device=x.device)
    if inter == 0 or x2.shape[0] == 0:
        return out.view(*x.shape[:-1], inter)
    _launch("ember_silu_and_mul", _lib.load().ember_silu_and_mul, x.device,
            x2.data_ptr(), x2.stride(0), out.data_ptr(), out.stride(0),
            x2.shape[0], inter, _lib.dtype_tag(x.dtype))
    return out.view(*x.shape[:-1], inter)


def stream_copy_hip(src: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """out <- src (contiguous, same byte size, 16-byte aligned) with the library's streaming
    copy: the bandwidth reference of the benchmark's copy-ceiling rows."""
    _require_device("stream_copy", src, out)
    nbytes = src.numel() * src.element_size()
    if (not src.is_contiguous() or not out.is_contiguous() or out.numel() * out.element_size() != nbytes
            or nbytes % 16 or src.data_ptr() % 16 or out.data_ptr() % 16):
        raise ValueError("stream_copy: contiguous, 16-byte aligned tensors of one size (a multiple of 16 bytes)")
    _launch("ember_stream_copy", _lib.load().ember_stream_copy, src.device, src.data_ptr(), out.data_ptr(), nbytes)
    return out


def embedding_hip(ids: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """nn.Embedding forward: out[..., :] = weight[ids[...], :], bit-exact."""
    _require_device("embedding", weight, ids)
    if weight.dim() != 2:
        raise ValueError("embedding weight must be [vocab, hidden]")
    if ids.dtype not in (torch.int64, torch.int32):
        raise TypeError(f"embedding ids must be int64 or int32, got {ids.dtype}")
    flat = ids.reshape(-1)
    if flat.dtype != torch.int64:
        flat = flat.long()
    if not flat.is_contiguous():
        flat = flat.contiguous()
    w = weight if weight.stride(1) == 1 else weight.contiguous()
    out = torch.empty((flat.shape[0], w.shape[1]), dtype=w.dtype, device=w.device)
    if flat.shape[0] == 0:
        return out.view(*ids.shape, w.shape[1])
    _launch("ember_embedding", _lib.load().ember_embedding, w.device,
            flat.data_ptr(), flat.shape[0], w.data_ptr(), w.shape[0], w.shape[1],
            w.stride(0), out.data_ptr(), out.stride(0), w.element_size())
    if _check_indices():
        _raise_index_errors()
    return out.view(*ids.shape, w.shape[1])


def qk_norm_rope_hip(q: torch.Tensor, k: torch.Tensor, q_weight: torch.Tensor,
                     k_weight: torch.Tensor, eps: float, cos: torch.Tensor, sin: torch.Tensor,
                     positions: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Qwen3 per-head RMSNorm of q and k, then neox rope, in place on the q/k views
    (qwen2.py:95-101 in one kernel); returns (q, k)."""
    _require_device("qk_norm_rope", q, k, q_weight, k_weight, cos, sin, positions)
    n, h, d = q.shape
    hk = k.shape[1]
    if not (q.stride(2) == 1 and k.stride(2) == 1 and d % 2 == 0):
        raise AssertionError("qk_norm_rope: q/k need unit stride in the head dim and an even head_dim")
    if k.shape[0] != n or k.shape[2] != d or k.dtype != q.dtype:
        raise ValueError("qk_norm_rope: q and k must agree in tokens, head_dim and dtype")
    if q_weight.numel() != d or k_weight.numel() != d:
        raise ValueError("qk_norm_rope: q/k norm weights must have head_dim elements")
    if n == 0:
        return q, k
    qw, qtag = _weight_for(q_weight, q)
    kw, ktag = _weight_for(k_weight, q)
    if qtag != ktag:
        qw, kw, qtag = qw.float(), kw.float(), _lib.F32
    cos, sin, positions = _tables(cos, sin, positions, d)
    _launch("ember_qk_norm_rope", _lib.load().ember_qk_norm_rope, q.device,
            q.data_ptr(), q.stride(0), q.stride(1), h, k.data_ptr(), k.stride(0),
            k.stride(1), hk, d, qw.data_ptr(), kw.data_ptr(), qtag, float(eps),
            cos.data_ptr(), sin.data_ptr(), cos.shape[0], cos.stride(0),
            positions.data_ptr(), n, _lib.dtype_tag(q.dtype))
    if _check_indices():
        _raise_index_errors()
    return q, k


def mla_latent_rope_hip(c: torch.Tensor, k_pe: torch.Tensor, q_pe: torch.Tensor,
                        weight: torch.Tensor, eps: float, cos: torch.Tensor, sin: torch.Tensor,
                        positions: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """MLA latent path (deepseek.py:126-133, rope folded into the weights): rmsnorm of the
    latent c [N, R], rope of the single key head k_pe [N, Dr] (or [N, 1, Dr]) into a new
    latent [N, R + Dr], and rope of q_pe [N, H, Dr] in place. c and k_pe are not modified.
    Returns (q_pe, latent)."""
    _require_device("mla_latent_rope", c, k_pe, q_pe, weight, cos, sin, positions)
    n, r = c.shape
    kp = k_pe.reshape(k_pe.shape[0], -1)
    nh, dr = q_pe.shape[1], q_pe.shape[2]
    if kp.shape != (n, dr) or q_pe.shape[0] != n:
        raise ValueError("mla_latent_rope: c [N, R], k_pe [N, Dr], q_pe [N, H, Dr] expected")
    if c.stride(1) != 1 or kp.stride(1) != 1 or q_pe.stride(2) != 1 or dr % 2 != 0:
        raise AssertionError("mla_latent_rope: unit innermost stride and an even rope dim required")
    if c.dtype != kp.dtype or c.dtype != q_pe.dtype:
        raise ValueError("mla_latent_rope: c, k_pe and q_pe must share a dtype")
    if weight.numel() != r:
        raise ValueError("mla_latent_rope: weight must have kv_lora_rank elements")
    latent = torch.empty((n, r + dr), dtype=c.dtype, device=c.device)
    if n == 0:
        return q_pe, latent
    w, wtag = _weight_for(weight, c)
    cos, sin, positions = _tables(cos, sin, positions, dr)
    _launch("ember_mla_latent_rope", _lib.load().ember_mla_latent_rope, c.device,
            c.data_ptr(), c.stride(0), r, kp.data_ptr(), kp.stride(0), q_pe.data_ptr(), q_pe.stride(0),
            q_pe.stride(1), nh, dr, w.data_ptr(), wtag, float(eps), cos.data_ptr(), sin.data_ptr(),
            cos.shape[0], cos.stride(0), positions.data_ptr(), n, latent.data_ptr(), latent.stride(0),
            _lib.dtype_tag(c.dtype))
    if _check_indices():
        _raise_index_errors()
    return q_pe, latent


def kv_cache_write_hip(k: torch.Tensor, v: torch.Tensor, slot_mapping: torch.Tensor,
                       k_cache: torch.Tensor, v_cache: torch.Tensor) -> None:
    """PagedKVCache.write (kv/cache.py:54-61) for one layer: k, v [N, Hkv, D] (any token
    and head strides, unit stride in D) scattered into k_cache / v_cache
    [num_blocks, block_size, Hkv, D] (or already flat [num_slots, Hkv, D]) at slot_mapping
    [N]. Bit-exact."""
    _require_device("kv_cache_write", k, v, slot_mapping, k_cache, v_cache)
    n, hk, d = k.shape
    if v.shape != k.shape or k.dtype != v.dtype or k_cache.dtype != k.dtype or v_cache.dtype != k.dtype:
        raise ValueError("kv_cache_write: k, v and the caches must agree in shape and dtype")
    if k_cache.shape != v_cache.shape or k_cache.stride() != v_cache.stride():
        raise ValueError("kv_cache_write: k_cache and v_cache must share a geometry")
    if tuple(k_cache.shape[-2:]) != (hk, d):
        raise ValueError(f"kv_cache_write: cache rows are {tuple(k_cache.shape[-2:])}, k rows ({hk}, {d})")
    if k.stride(2) != 1 or v.stride(2) != 1 or k_cache.stride(-1) != 1:
        raise AssertionError("kv_cache_write: unit stride in head_dim required")
    kc = k_cache.view(-1, hk, d)  # [num_slots, Hkv, D]; a view, so the write lands in the cache
    if slot_mapping.numel() != n:
        raise ValueError("kv_cache_write: one slot per token expected")
    slots = slot_mapping if slot_mapping.dtype == torch.int64 else slot_mapping.long()
    slots = slots.contiguous()
    if n == 0:
        return
    _launch("ember_kv_cache_write", _lib.load().ember_kv_cache_write, k.device,
            k.data_ptr(), k.stride(0), k.stride(1), v.data_ptr(), v.stride(0), v.stride(1), hk, d,
            slots.data_ptr(), n, k_cache.data_ptr(), v_cache.data_ptr(), kc.shape[0], kc.stride(0),
            kc.stride(1), k.element_size())
    if _check_indices():
        _raise_index_errors()


def latent_cache_write_hip(latent: torch.Tensor, slot_mapping: torch.Tensor, cache: torch.Tensor) -> None:
    """PagedLatentCache.write (kv/cache.py:152-157) for one layer: latent [N, L] rows
    scattered into cache [num_blocks, block_size, L] at slot_mapping [N]. Bit-exact."""
    _require_device("latent_cache_write", latent, slot_mapping, cache)
    n, dim = latent.shape
    if cache.dtype != latent.dtype or cache.shape[-1] != dim:
        raise ValueError("latent_cache_write: cache rows must match the latent rows")
    if latent.stride(1) != 1 or cache.stride(-1) != 1:
        raise AssertionError("latent_cache_write: unit innermost stride required")
    flat = cache.view(-1, dim)
    if slot_mapping.numel() != n:
        raise ValueError("latent_cache_write: one slot per token expected")
    slots = (slot_mapping if slot_mapping.dtype == torch.int64 else slot_mapping.long()).contiguous()
    if n == 0:
        return
    _launch("ember_latent_cache_write", _lib.load().ember_latent_cache_write, latent.device,
            latent.data_ptr(), latent.stride(0), dim, slots.data_ptr(), n, flat.data_ptr(), flat.shape[0],
            flat.stride(0), latent.element_size())
    if _check_indices():
        _raise_index_errors()


def rope_kv_cache_hip(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor,
                      sin: torch.Tensor, positions: torch.Tensor, slot_mapping: torch.Tensor,
                      k_cache: torch.Tensor, v_cache: torch.Tensor,
                      q_weight: torch.Tensor | None = None, k_weight: torch.Tensor | None = None,
                      eps: float = 1e-6) -> tuple[torch.Tensor, torch.Tensor]:
    """rope (after the Qwen3 q/k RMSNorm when q_weight/k_weight are given), in place on the
    q/k views, fused with the paged KV-cache write of the rotated k and of v: one kernel
    for qwen2.py:95-101 followed by PagedKVCache.write (kv/cache.py:54-61). Returns (q, k).
    Operands the fused kernel cannot take (misaligned views, odd head sizes) run the two
    unfused HIP ops, with the same result."""
    tensors = [q, k, v, cos, sin, positions, slot_mapping, k_cache, v_cache]
    norm = q_weight is not None
    if norm:
        if k_weight is None:
            raise ValueError("rope_kv_cache: k_weight is required with q_weight")
        tensors += [q_weight, k_weight]
    _require_device("rope_kv_cache", *tensors)
    n, h, d = q.shape
    hk = k.shape[1]
    if not (q.stride(2) == 1 and k.stride(2) == 1 and v.stride(2) == 1 and d % 2 == 0):
        raise AssertionError("rope_kv_cache: unit stride in the head dim and an even head_dim required")
    if k.shape != (n, hk, d) or v.shape != k.shape or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("rope_kv_cache: q [N, H, D], k and v [N, Hkv, D] of one dtype expected")
    if k_cache.dtype != q.dtype or v_cache.dtype != q.dtype or k_cache.shape != v_cache.shape \
            or k_cache.stride() != v_cache.stride() or tuple(k_cache.shape[-2:]) != (hk, d):
        raise ValueError("rope_kv_cache: k_cache and v_cache must be [..., Hkv, D] caches of q's dtype")
    if slot_mapping.numel() != n:
        raise ValueError("rope_kv_cache: one slot per token expected")
    if n == 0:
        return q, k
    cos, sin, positions = _tables(cos, sin, positions, d)
    slots = (slot_mapping if slot_mapping.dtype == torch.int64 else slot_mapping.long()).contiguous()
    kc = k_cache.view(-1, hk, d)
    wtag, qw_ptr, kw_ptr = 0, None, None
    if norm:
        if q_weight.numel() != d or k_weight.numel() != d:
            raise ValueError("rope_kv_cache: q/k norm weights must have head_dim elements")
        qw, wtag = _weight_for(q_weight, q)
        kw, ktag = _weight_for(k_weight, q)
        if ktag != wtag:
            qw, kw, wtag = qw.float(), kw.float(), _lib.F32
        qw_ptr, kw_ptr = qw.data_ptr(), kw.data_ptr()
    fused = _launch(
        "ember_rope_kv_cache", _lib.load().ember_rope_kv_cache, q.device,
        q.data_ptr(), q.stride(0), q.stride(1), h, k.data_ptr(), k.stride(0), k.stride(1), hk, v.data_ptr(),
        v.stride(0), v.stride(1), d, qw_ptr, kw_ptr, wtag, float(eps), cos.data_ptr(), sin.data_ptr(),
        cos.shape[0], cos.stride(0), positions.data_ptr(), slots.data_ptr(), n, k_cache.data_ptr(),
        v_cache.data_ptr(), kc.shape[0], kc.stride(0), kc.stride(1), _lib.dtype_tag(q.dtype),
        allow_unaligned=True)
    if not fused:  # misaligned operands: the unfused pair
        if norm:
            qk_norm_rope_hip(q, k, q_weight, k_weight, eps, cos, sin, positions)
        else:
            rope_hip(q, k, cos, sin, positions)
        kv_cache_write_hip(k, v, slots, k_cache, v_cache)
        return q, k
    if _check_indices():
        _raise_index_errors()
    return q, k


def mla_latent_rope_cache_hip(c: torch.Tensor, k_pe: torch.Tensor, q_pe: torch.Tensor, weight: torch.Tensor,
                              eps: float, cos: torch.Tensor, sin: torch.Tensor, positions: torch.Tensor,
                              slot_mapping: torch.Tensor, cache: torch.Tensor,
                              return_latent: bool = True) -> tuple[torch.Tensor, torch.Tensor | None]:
    """mla_latent_rope fused with PagedLatentCache.write (kv/cache.py:152-157): the latent
    rows go straight to cache[slot] (and to a new [N, R + Dr] tensor when return_latent,
    which the fresh-prefill attention reads). Returns (q_pe, latent or None)."""
    _require_device("mla_latent_rope_cache", c, k_pe, q_pe, weight, cos, sin, positions, slot_mapping, cache)
    n, r = c.shape
    kp = k_pe.reshape(k_pe.shape[0], -1)
    nh, dr = q_pe.shape[1], q_pe.shape[2]
    if kp.shape != (n, dr) or q_pe.shape[0] != n:
        raise ValueError("mla_latent_rope_cache: c [N, R], k_pe [N, Dr], q_pe [N, H, Dr] expected")
    if c.stride(1) != 1 or kp.stride(1) != 1 or q_pe.stride(2) != 1 or dr % 2 != 0:
        raise AssertionError("mla_latent_rope_cache: unit innermost stride and an even rope dim required")
    if c.dtype != kp.dtype or c.dtype != q_pe.dtype or cache.dtype != c.dtype:
        raise ValueError("mla_latent_rope_cache: c, k_pe, q_pe and the cache must share a dtype")
    if weight.numel() != r or cache.shape[-1] != r + dr or cache.stride(-1) != 1:
        raise ValueError("mla_latent_rope_cache: weight [R] and cache rows [R + Dr] expected")
    if slot_mapping.numel() != n:
        raise ValueError("mla_latent_rope_cache: one slot per token expected")
    latent = torch.empty((n, r + dr), dtype=c.dtype, device=c.device) if return_latent else None
    if n == 0:
        return q_pe, latent
    w, wtag = _weight_for(weight, c)
    cos, sin, positions = _tables(cos, sin, positions, dr)
    slots = (slot_mapping if slot_mapping.dtype == torch.int64 else slot_mapping.long()).contiguous()
    flat = cache.view(-1, r + dr)
    fused = _launch(
        "ember_mla_latent_rope_cache", _lib.load().ember_mla_latent_rope_cache, c.device,
        c.data_ptr(), c.stride(0), r, kp.data_ptr(), kp.stride(0), q_pe.data_ptr(), q_pe.stride(0),
        q_pe.stride(1), nh, dr, w.data_ptr(), wtag, float(eps), cos.data_ptr(), sin.data_ptr(), cos.shape[0],
        cos.stride(0), positions.data_ptr(), n, latent.data_ptr() if latent is not None else None,
        latent.stride(0) if latent is not None else 0, slots.data_ptr(), flat.data_ptr(), flat.shape[0],
        flat.stride(0), _lib.dtype_tag(c.dtype), allow_unaligned=True)
    if not fused:  # misaligned operands: the unfused pair
        q_pe, lat = mla_latent_rope_hip(c, k_pe, q_pe, weight, eps, cos, sin, positions)
        latent_cache_write_hip(lat, slots, cache)
        return q_pe, lat if return_latent else None
    if _check_indices():
        _raise_index_errors()
    return q_pe, latent


# ---- dispatch (ops.py:92-115 plus the fused additions) ----------------------------------

def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    if fused_enabled(x):
        return rmsnorm_hip(x, weight, eps)
    return rmsnorm_torch(x, weight, eps)


def fused_add_rmsnorm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                      eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    if fused_enabled(x):
        return fused_add_rmsnorm_hip(x, residual, weight, eps)
    return fused_add_rmsnorm_torch(x, residual, weight, eps)


def rope(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
         positions: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    if fused_enabled(q):
        return rope_hip(q, k, cos, sin, positions)
    return rope_torch(q, k, cos, sin, positions)


def silu_and_mul(x: torch.Tensor) -> torch.Tensor:
    if fused_enabled(x):
        return silu_and_mul_hip(x)
    return silu_and_mul_torch(x)


def embedding(ids: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    if fused_enabled(weight):
        return embedding_hip(ids, weight)
    return embedding_torch(ids, weight)


def qk_norm_rope(q: torch.Tensor, k: torch.Tensor, q_weight: torch.Tensor, k_weight: torch.Tensor,
                 eps: float, cos: torch.Tensor, sin: torch.Tensor,
                 positions: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    if fused_enabled(q):
        return qk_norm_rope_hip(q, k, q_weight, k_weight, eps, cos, sin, positions)
    return qk_norm_rope_torch(q, k, q_weight, k_weight, eps, cos, sin, positions)


def mla_latent_rope(c: torch.Tensor, k_pe: torch.Tensor, q_pe: torch.Tensor, weight: torch.Tensor,
                    eps: float, cos: torch.Tensor, sin: torch.Tensor,
                    positions: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    if fused_enabled(c):
        return mla_latent_rope_hip(c, k_pe, q_pe, weight, eps, cos, sin, positions)
    return mla_latent_rope_torch(c, k_pe, q_pe, weight, eps, cos, sin, positions)


def kv_cache_write(k: torch.Tensor, v: torch.Tensor, slot_mapping: torch.Tensor,
                   k_cache: torch.Tensor, v_cache: torch.Tensor) -> None:
    if fused_enabled(k):
        return kv_cache_write_hip(k, v, slot_mapping, k_cache, v_cache)
    return kv_cache_write_torch(k, v, slot_mapping, k_cache, v_cache)


def latent_cache_write(latent: torch.Tensor, slot_mapping: torch.Tensor, cache: torch.Tensor) -> None:
    if fused_enabled(latent):
        return latent_cache_write_hip(latent, slot_mapping, cache)
    return latent_cache_write_torch(latent, slot_mapping, cache)


def rope_kv_cache(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                  positions: torch.Tensor, slot_mapping: torch.Tensor, k_cache: torch.Tensor,
                  v_cache: torch.Tensor, q_weight: torch.Tensor | None = None,
                  k_weight: torch.Tensor | None = None, eps: float = 1e-6) -> tuple[torch.Tensor, torch.Tensor]:
    if fused_enabled(q):
        return rope_kv_cache_hip(q, k, v, cos, sin, positions, slot_mapping, k_cache, v_cache, q_weight,
                                 k_weight, eps)
    if q_weight is not None:
        q, k = qk_norm_rope_torch(q, k, q_weight, k_weight, eps, cos, sin, positions)
    else:
        q, k = rope_torch(q, k, cos, sin, positions)
    kv_cache_write_torch(k, v, slot_mapping, k_cache, v_cache)
    return q, k


def mla_latent_rope_cache(c: torch.Tensor, k_pe: torch.Tensor, q_pe: torch.Tensor, weight: torch.Tensor,
                          eps: float, cos: torch.Tensor, sin: torch.Tensor, positions: torch.Tensor,
                          slot_mapping: torch.Tensor, cache: torch.Tensor,
                          return_latent: bool = True) -> tuple[torch.Tensor, torch.Tensor | None]:
    if fused_enabled(c):
        return mla_latent_rope_cache_hip(c, k_pe, q_pe, weight, eps, cos, sin, positions, slot_mapping, cache,
                                         return_latent)
    q_pe, latent = mla_latent_rope_torch(c, k_pe, q_pe, weight, eps, cos, sin, positions)
    latent_cache_write_torch(latent, slot_mapping, cache)
    return q_pe, latent if return_latent else None
