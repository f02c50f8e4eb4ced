/*
 * ember_ops.h - C ABI of libember_ops.so, the gfx950 (MI355X) kernels behind emberserve's
 * fused per-layer elementwise ops.
 *
 * Every entry point takes raw device pointers, element counts and element strides
 * (int64), a dtype tag and an opaque stream handle (a hipStream_t, passed as void*; NULL
 * is the null stream). Nothing is allocated, nothing synchronises the host, and every
 * launch goes on the given stream, so all entry points are safe under stream/graph
 * capture. Strides are in elements of the tensor's own dtype; the innermost dimension is
 * always unit-stride.
 *
 * Return value: EMBER_OK (0) or one of the EMBER_E* codes below. Argument errors are
 * detected on the host before any launch; a failed launch returns EMBER_ELAUNCH.
 * ember_status_string() names a code.
 *
 * Index safety: positions, token ids and cache slots are checked on the device. An
 * out-of-range position leaves that token's rows untouched, an out-of-range id writes a
 * zero row, an out-of-range slot skips the token; each sets a bit in a per-device error
 * word that ember_read_errors() returns (and optionally clears). Reading it synchronises,
 * so callers read it only in debug paths.
 *
 * Reference interfaces replaced (paths relative to the emberserve repository):
 *   ember_rmsnorm             emberserve/model/ops.py:92-95  (rmsnorm) and
 *                             emberserve/model/ops_triton.py:90-97 (rmsnorm_triton)
 *   ember_fused_add_rmsnorm   emberserve/model/ops.py:98-102 (fused_add_rmsnorm) and
 *                             emberserve/model/ops_triton.py:100-110
 *   ember_rope                emberserve/model/ops.py:105-109 (rope) and
 *                             emberserve/model/ops_triton.py:113-124 (rope_triton)
 *   ember_silu_and_mul        emberserve/model/ops.py:112-115 (silu_and_mul) and
 *                             emberserve/model/ops_triton.py:127-134
 *   ember_embedding           torch.nn.Embedding.forward as used by
 *                             emberserve/model/qwen2.py:172,182 and deepseek.py:197,205
 *   ember_qk_norm_rope        the q_norm/k_norm + rotary_emb sequence of
 *                             emberserve/model/qwen2.py:95-101 (two rmsnorm + one rope)
 *   ember_mla_latent_rope     the kv_a_layernorm + rotary_emb + cat sequence of
 *                             emberserve/model/deepseek.py:124-133
 *   ember_kv_cache_write      PagedKVCache.write, emberserve/kv/cache.py:54-61
 *   ember_latent_cache_write  PagedLatentCache.write, emberserve/kv/cache.py:152-157
 *   ember_mla_latent_rope_cache  ember_mla_latent_rope followed by PagedLatentCache.write
 *                             (deepseek.py:124-133 then attn/mla_triton.py:235)
 *   ember_rope_kv_cache       rotary_emb (with the Qwen3 q/k norm when weights are given)
 *                             followed by PagedKVCache.write: qwen2.py:95-101 and the
 *                             backends' cache.write (attn/paged_triton.py:477)
 *   ember_paged_decode        paged_attention_decode, emberserve/attn/paged_triton.py:323-399
 *                             (kernels :95-209; fp32 definition attn/paged_torch.py:87-98)
 *   ember_paged_decode_workspace_bytes  the split-K scratch size (_Scratch,
 *                             attn/paged_triton.py:293-310)
 *   ember_gather_rows         the query pack of a mixed step: index_select + new_zeros +
 *                             padded copies, attn/paged_flash.py:259-275
 *   ember_scatter_rows2       the output unpack: index_copy_ + slice copies,
 *                             attn/paged_flash.py:267,276-277
 *   ember_gate_up_silu        silu_and_mul(gate_up_proj(x)) of Qwen2MLP.forward,
 *                             emberserve/model/qwen2.py:60-61 (decode-sized batches)
 *   ember_gate_up_silu_packed the same over a weight packed at load time
 *                             (ember_gate_up_silu_pack_weight); up to 64 tokens
 *   ember_gate_up_silu_gemm   the same at prefill sizes: an MFMA GEMM with the activation
 *                             in its epilogue (also _packed: over the packed weight)
 *   ember_moe_gate_up_silu    the routed experts' grouped gate_up GEMM + silu_and_mul of
 *                             fused_moe_forward, emberserve/model/moe_triton.py:332-345
 *                             (also _packed, _direct for decode batches, _gemm at prefill)
 *   ember_moe_align           moe_align, emberserve/model/moe_triton.py:215-254 (one
 *                             workgroup, or a count + place grid with a workspace)
 *   ember_mla_decode          mla_decode, emberserve/attn/mla_triton.py:119-182 (kernel
 *                             :49-116; fp32 definition attn/mla_torch.py:33-53)
 *   ember_mla_decode_workspace_bytes  its split-K scratch size (the _SCRATCH buffers,
 *                             attn/mla_triton.py:163-166)
 *   ember_stream_copy         no counterpart: the benchmark's same-size copy ceiling
 *   ember_paged_decode_noalloc  no counterpart: ember_paged_decode for callers that cannot
 *                             allocate (a library-owned scratch array)
 */
#ifndef EMBER_OPS_H
#define EMBER_OPS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype tags (activations and, where stated, weights) */
#define EMBER_F32 0
#define EMBER_F16 1
#define EMBER_BF16 2

/* status codes */
#define EMBER_OK 0
#define EMBER_EINVAL 1      /* bad shape, stride, dtype or pointer */
#define EMBER_EALIGN 2      /* a fused entry point's operands are not 16-byte aligned: run the unfused ops */
#define EMBER_ELAUNCH 3     /* the HIP launch itself failed */
#define EMBER_ENODEV 4      /* no HIP device / runtime call failed */
#define EMBER_ETOOBIG 5     /* a no-allocation entry point's call needs more scratch than it holds */

/* bits of the device error word */
#define EMBER_ERR_EMBED_ID 1u   /* a token id outside [0, vocab) */
#define EMBER_ERR_ROPE_POS 2u   /* a position outside [0, table_rows) */
#define EMBER_ERR_KV_SLOT 4u    /* a cache slot outside [0, num_slots) */
#define EMBER_ERR_DECODE_CTX 8u /* a context length outside [0, max_blocks * block_size] */
#define EMBER_ERR_BLOCK_ID 16u  /* a block-table entry outside [0, num_blocks) */
#define EMBER_ERR_ROW_INDEX 32u /* a row index past the end in ember_gather_rows / ember_scatter_rows2 */
#define EMBER_ERR_SYNC 64u      /* an in-kernel wave handshake timed out (a library fault, never input) */
#define EMBER_ERR_EXPERT_ID 128u /* an expert id outside [0, num_experts) in ember_moe_align */

/* ABI version, bumped when an entry point is added or its signature changes. */
int ember_abi_version(void);

/* Static description of a status code. */
const char* ember_status_string(int status);

/* Copies the current device's error word into *flags (if non-NULL) and, when clear != 0,
 * zeroes it. Synchronises the device. Returns EMBER_OK or EMBER_ENODEV. */
int ember_read_errors(uint32_t* flags, int clear);

/* RMSNorm of `rows` rows of `cols` elements:
 *   out = round(w * round(x * rsqrt(mean(x^2) + eps)))
 * fp32 math, rounding to `dtype` at the two points the reference rounds.
 * `weight` is [cols], contiguous, of dtype `weight_dtype` (== dtype, or EMBER_F32).
 * Replaces ops.py:92-95 / ops_triton.py:90-97 (_rmsnorm_kernel with HAS_RESIDUAL=0). */
int ember_rmsnorm(const void* x, int64_t x_row_stride,
                  const void* weight, int weight_dtype,
                  void* out, int64_t out_row_stride,
                  int64_t rows, int64_t cols, float eps, int dtype, void* stream);

/* Fused residual add + RMSNorm:
 *   residual_out = round(residual + x);  out = rmsnorm(residual_out)
 * Inputs are not modified (outputs may not alias them).
 * Replaces ops.py:98-102 / ops_triton.py:100-110 (_rmsnorm_kernel with HAS_RESIDUAL=1). */
int ember_fused_add_rmsnorm(const void* x, int64_t x_row_stride,
                            const void* residual, int64_t residual_row_stride,
                            const void* weight, int weight_dtype,
                            void* out, int64_t out_row_stride,
                            void* residual_out, int64_t residual_out_row_stride,
                            int64_t rows, int64_t cols, float eps, int dtype, void* stream);

/* Neox (rotate-half) rotary embedding, in place on q [tokens, num_q_heads, head_dim] and
 * k [tokens, num_k_heads, head_dim]:
 *   o[i]      = round(x[i] * c[i] - x[i + D/2] * s[i])
 *   o[i+D/2]  = round(x[i+D/2] * c[i] + x[i] * s[i])      for i < D/2
 * with c, s = cos/sin[positions[t]][i], fp32 tables of `table_rows` rows, row stride
 * `table_row_stride` floats, whose two halves are equal (RotaryEmbedding builds
 * cat(freqs, freqs)). Each product and the sum are rounded separately in fp32 (no FMA),
 * as the reference's element-wise tensor ops are. num_k_heads may be 0 (k unused).
 * Replaces ops.py:105-109 / ops_triton.py:113-124 (_rope_kernel). */
int ember_rope(void* q, int64_t q_token_stride, int64_t q_head_stride, int64_t num_q_heads,
               void* k, int64_t k_token_stride, int64_t k_head_stride, int64_t num_k_heads,
               int64_t head_dim,
               const float* cos_table, const float* sin_table,
               int64_t table_rows, int64_t table_row_stride,
               const int64_t* positions, int64_t num_tokens, int dtype, void* stream);

/* SwiGLU activation: out[r, j] = round(round(silu(x[r, j])) * x[r, inter + j]).
 * x is [rows, 2*inter] (row stride x_row_stride), out is [rows, inter].
 * Replaces ops.py:112-115 / ops_triton.py:127-134 (_silu_and_mul_kernel). */
int ember_silu_and_mul(const void* x, int64_t x_row_stride,
                       void* out, int64_t out_row_stride,
                       int64_t rows, int64_t inter, int dtype, void* stream);

/* Row gather: out[t, :] = weight[ids[t], :], a bit-exact copy of `hidden` elements of
 * `elem_bytes` bytes each (1, 2, 4 or 8). ids outside [0, vocab) give a zero row and set
 * EMBER_ERR_EMBED_ID. Replaces torch.nn.Embedding.forward (F.embedding) as called at
 * qwen2.py:182 / deepseek.py:205 / attn/piecewise_graphs.py:176. */
int ember_embedding(const int64_t* ids, int64_t num_tokens,
                    const void* weight, int64_t vocab, int64_t hidden, int64_t weight_row_stride,
                    void* out, int64_t out_row_stride, int64_t elem_bytes, void* stream);

/* Qwen3 per-head QK-RMSNorm fused with neox rope, in place on q and k (same layout rules
 * as ember_rope). Per head row: y = round(w * round(x * rsqrt(mean(x^2) + eps))), then
 * the rope of ember_rope applied to y. q_weight, k_weight are [head_dim] of weight_dtype.
 * Same result as rmsnorm on [tokens*heads, head_dim] followed by rope
 * (qwen2.py:95-101), in one pass over q and k. */
int ember_qk_norm_rope(void* q, int64_t q_token_stride, int64_t q_head_stride, int64_t num_q_heads,
                       void* k, int64_t k_token_stride, int64_t k_head_stride, int64_t num_k_heads,
                       int64_t head_dim,
                       const void* q_weight, const void* k_weight, int weight_dtype, float eps,
                       const float* cos_table, const float* sin_table,
                       int64_t table_rows, int64_t table_row_stride,
                       const int64_t* positions, int64_t num_tokens, int dtype, void* stream);

/* MLA latent path (deepseek.py:124-133 with the rope permutation folded into the
 * weights):
 *   latent[t, :R]      = rmsnorm(c[t, :R], weight, eps)            (R = kv_lora_rank)
 *   latent[t, R:R+Dr]  = rope(k_pe[t, :Dr])                         (one key head)
 *   q_pe[t, h, :Dr]    = rope(q_pe[t, h, :Dr])  in place, h < num_heads
 * c and k_pe are read only. q_pe is typically the rope slice of q [T, H, Dn+Dr] (head
 * stride Dn+Dr). Rope as in ember_rope, Dr = rope_dim. */
int ember_mla_latent_rope(const void* c, int64_t c_token_stride, int64_t kv_lora_rank,
                          const void* k_pe, int64_t k_pe_token_stride,
                          void* q_pe, int64_t q_token_stride, int64_t q_head_stride, int64_t num_heads,
                          int64_t rope_dim,
                          const void* weight, int weight_dtype, float eps,
                          const float* cos_table, const float* sin_table,
                          int64_t table_rows, int64_t table_row_stride,
                          const int64_t* positions, int64_t num_tokens,
                          void* latent, int64_t latent_token_stride, int dtype, void* stream);

/* Row gather with padding (the query pack of a mixed prefill + decode step, replacing
 * q.index_select(0, dec_tokens), q.new_zeros(...) and the per-sequence copies into it at
 * emberserve/attn/paged_flash.py:259-275): dst[t, :] = src[rows[t], :] for rows[t] in
 * [0, src_rows); a negative rows[t] is a padding row, written as zeros; rows[t] >= src_rows
 * writes zeros and sets EMBER_ERR_ROW_INDEX. Rows are row_elems elements of elem_bytes
 * bytes (1, 2, 4 or 8), strides in elements. Bit-exact. */
/* A streaming copy of `bytes` (a multiple of 16, both pointers 16-byte aligned, no overlap)
 * with non-temporal loads and stores: the bandwidth reference the benchmark's copy-ceiling
 * rows measure each op against. No counterpart in the reference. */
int ember_stream_copy(const void* src, void* dst, int64_t bytes, void* stream);

int ember_gather_rows(const void* src, int64_t src_rows, int64_t src_row_stride,
                      const int64_t* rows, int64_t num_rows,
                      void* dst, int64_t dst_row_stride,
                      int64_t row_elems, int64_t elem_bytes, void* stream);

/* Two-source row scatter (the output unpack of the same step, replacing
 * out.index_copy_(0, dec_tokens, o) and out[start:start + n] = o_pad[i, max_q - n:] at
 * paged_flash.py:267,276-277): packed row t < src0_rows is src0[t], row t >= src0_rows is
 * src1[t - src0_rows]; it is copied to dst[rows[t]]. A negative rows[t] is a padding row
 * and is dropped; rows[t] >= dst_rows is dropped and sets EMBER_ERR_ROW_INDEX. src0 or
 * src1 may be null when it has no rows. Bit-exact. */
int ember_scatter_rows2(const void* src0, int64_t src0_rows, int64_t src0_row_stride,
                        const void* src1, int64_t src1_rows, int64_t src1_row_stride,
                        const int64_t* rows, void* dst, int64_t dst_rows, int64_t dst_row_stride,
                        int64_t row_elems, int64_t elem_bytes, void* stream);

/* Paged KV-cache write (PagedKVCache.write, kv/cache.py:54-61, an index_copy_ per tensor):
 *   k_cache[slot_mapping[t], h, :] = k[t, h, :]
 *   v_cache[slot_mapping[t], h, :] = v[t, h, :]        t < num_tokens, h < num_kv_heads
 * Bit-exact copies of head_dim elements of elem_bytes bytes. Strides are in elements; the
 * caches are [num_slots, ...] with slot stride cache_slot_stride and head stride
 * cache_head_stride (both caches share the geometry). Slot -1 marks a padding row (a step
 * replayed at a larger token bucket) and is skipped silently; any other slot outside
 * [0, num_slots) skips that token and sets EMBER_ERR_KV_SLOT; with duplicate slots one writer wins, as with
 * index_copy_. */
int ember_kv_cache_write(const void* k, int64_t k_token_stride, int64_t k_head_stride,
                         const void* v, int64_t v_token_stride, int64_t v_head_stride,
                         int64_t num_kv_heads, int64_t head_dim,
                         const int64_t* slot_mapping, int64_t num_tokens,
                         void* k_cache, void* v_cache, int64_t num_slots,
                         int64_t cache_slot_stride, int64_t cache_head_stride,
                         int64_t elem_bytes, void* stream);

/* Paged latent-cache write (PagedLatentCache.write, kv/cache.py:152-157):
 *   cache[slot_mapping[t], :latent_dim] = latent[t, :latent_dim]
 * Same slot rules as ember_kv_cache_write. */
int ember_latent_cache_write(const void* latent, int64_t latent_token_stride, int64_t latent_dim,
                             const int64_t* slot_mapping, int64_t num_tokens,
                             void* cache, int64_t num_slots, int64_t cache_slot_stride,
                             int64_t elem_bytes, void* stream);

/* ember_mla_latent_rope fused with the paged latent-cache write that follows it
 * (PagedLatentCache.write): the latent rows are stored at cache[slot_mapping[t], :] (slot
 * stride cache_slot_stride; slot -1 skipped silently, other slots outside [0, num_slots)
 * skipped with EMBER_ERR_KV_SLOT)
 * and, when latent != NULL, also to latent[t, :]. Needs 16-byte aligned operands;
 * otherwise returns EMBER_EALIGN and does nothing. */
int ember_mla_latent_rope_cache(const void* c, int64_t c_token_stride, int64_t kv_lora_rank,
                                const void* k_pe, int64_t k_pe_token_stride,
                                void* q_pe, int64_t q_token_stride, int64_t q_head_stride, int64_t num_heads,
                                int64_t rope_dim,
                                const void* weight, int weight_dtype, float eps,
                                const float* cos_table, const float* sin_table,
                                int64_t table_rows, int64_t table_row_stride,
                                const int64_t* positions, int64_t num_tokens,
                                void* latent, int64_t latent_token_stride,
                                const int64_t* slot_mapping, void* cache, int64_t num_slots,
                                int64_t cache_slot_stride, int dtype, void* stream);

/* Rope (and, when q_weight != NULL, the Qwen3 per-head q/k RMSNorm before it) fused with
 * the paged KV-cache write that follows it: q and k are transformed in place exactly as by
 * ember_qk_norm_rope / ember_rope, then the transformed k rows and the v rows are stored
 * at slot_mapping[t] of k_cache / v_cache as ember_kv_cache_write stores them. v is
 * [tokens, num_kv_heads, head_dim] (read only). Needs 16-byte aligned operands and strides
 * and head_dim / 2 a power-of-two multiple of 16 bytes; otherwise returns EMBER_EALIGN and
 * does nothing, and the caller runs the two unfused entry points. */
int ember_rope_kv_cache(void* q, int64_t q_token_stride, int64_t q_head_stride, int64_t num_q_heads,
                        void* k, int64_t k_token_stride, int64_t k_head_stride, int64_t num_kv_heads,
                        const void* v, int64_t v_token_stride, int64_t v_head_stride,
                        int64_t head_dim,
                        const void* q_weight, const void* k_weight, int weight_dtype, float eps,
                        const float* cos_table, const float* sin_table,
                        int64_t table_rows, int64_t table_row_stride,
                        const int64_t* positions, const int64_t* slot_mapping, int64_t num_tokens,
                        void* k_cache, void* v_cache, int64_t num_slots,
                        int64_t cache_slot_stride, int64_t cache_head_stride,
                        int dtype, void* stream);

/* Bytes of workspace ember_paged_decode needs for num_splits > 1 (0 for one split), -1 for
 * invalid arguments: fp32 partials [splits][seqs][heads][head_dim + 2] and one uint32
 * arrival counter per (sequence, head). */
int64_t ember_paged_decode_workspace_bytes(int64_t num_seqs, int64_t num_heads, int64_t head_dim,
                                           int64_t num_splits);

/* One-query-per-sequence attention over a paged KV cache (paged_attention_decode):
 *   out[b, h, :] = softmax_j(scale * q[b, h] . k[b, j]) @ v[b, j],  j < context_lens[b],
 * key j of sequence b at block block_tables[b, j / block_size], slot j % block_size, KV head
 * h / (num_heads / num_kv_heads). q and out are [num_seqs, num_heads, head_dim] of q_dtype
 * (unit stride on the last dim); the caches are [num_blocks, block_size, num_kv_heads,
 * head_dim] of cache_dtype with the given element strides; block_tables int32
 * [num_seqs, >= max_blocks] (row stride block_table_stride); context_lens int32 [num_seqs].
 * block_size must be a multiple of 16 and head_dim <= 256. With num_splits > 1 each
 * sequence's context is cut into num_splits key ranges whose partial results are merged by
 * the last split to finish (or a second kernel) through `workspace`
 * (ember_paged_decode_workspace_bytes bytes, 16-byte aligned, zero-filled before its first
 * use; every call leaves it ready for the next, and calls that overlap on one workspace
 * race); the split count changes rounding only, never which keys are seen.
 * fp16/bf16 q and cache of the same dtype with head_dim 64 or 128 and 16-byte aligned
 * operands run on MFMA with the reference's tl.dot numerics (fp32 scores, probabilities
 * rounded to the cache dtype for P.V); every other case computes in fp32. Context lengths
 * outside [0, max_blocks * block_size] are clamped (EMBER_ERR_DECODE_CTX); block ids outside
 * [0, num_blocks) read block 0 (EMBER_ERR_BLOCK_ID). A zero context yields NaN rows, as the
 * reference kernel's 0/0 does. flags: 0, or EMBER_DECODE_FP32 to compute in fp32 whatever
 * the dtypes (the reference's "sum" variant). */
#define EMBER_DECODE_FP32 1
int ember_paged_decode(const void* q, int64_t q_seq_stride, int64_t q_head_stride, int q_dtype,
                       const void* k_cache, const void* v_cache, int64_t num_blocks, int64_t block_size,
                       int64_t num_kv_heads, int64_t head_dim,
                       int64_t k_block_stride, int64_t k_slot_stride, int64_t k_head_stride,
                       int64_t v_block_stride, int64_t v_slot_stride, int64_t v_head_stride,
                       int cache_dtype,
                       const int32_t* block_tables, int64_t block_table_stride, int64_t max_blocks,
                       const int32_t* context_lens, int64_t num_seqs, int64_t num_heads, float scale,
                       int64_t num_splits, int flags, void* workspace, int64_t workspace_bytes,
                       void* out, int64_t out_seq_stride, int64_t out_head_stride, void* stream);

/* ember_paged_decode without a workspace argument, for callers that cannot allocate (code
 * under HIP graph capture that may not call hipMalloc, tight serving loops, harnesses that
 * forbid allocation). No counterpart in the reference. The split-K partials and counters live
 * in a library-owned 16 MiB device array per GPU, held until the process ends; a call whose
 * ember_paged_decode_workspace_bytes(num_seqs, num_heads, head_dim, num_splits) exceeds
 * ember_paged_decode_noalloc_max_bytes() (15 MiB, the part left beside the counters), or
 * with more than 262144 (sequence, head) rows, returns EMBER_ETOOBIG and launches nothing. It calls no allocator. All calls on one GPU share
 * the array: calls that overlap on one GPU (two streams, concurrent graph replays) race.
 * Arguments and results are ember_paged_decode's. */
int64_t ember_paged_decode_noalloc_max_bytes(void);
int ember_paged_decode_noalloc(const void* q, int64_t q_seq_stride, int64_t q_head_stride, int q_dtype,
                               const void* k_cache, const void* v_cache, int64_t num_blocks, int64_t block_size,
                               int64_t num_kv_heads, int64_t head_dim, int64_t k_block_stride,
                               int64_t k_slot_stride, int64_t k_head_stride, int64_t v_block_stride,
                               int64_t v_slot_stride, int64_t v_head_stride, int cache_dtype,
                               const int32_t* block_tables, int64_t block_table_stride, int64_t max_blocks,
                               const int32_t* context_lens, int64_t num_seqs, int64_t num_heads, float scale,
                               int64_t num_splits, int flags, void* out, int64_t out_seq_stride,
                               int64_t out_head_stride, void* stream);

/* Bytes of workspace ember_mla_decode needs for num_splits > 1 (0 for one split), -1 for
 * invalid arguments: fp32 partials [splits][seqs][heads][kv_lora_rank + 2] and one uint32
 * arrival counter per (sequence, head). */
int64_t ember_mla_decode_workspace_bytes(int64_t num_seqs, int64_t num_heads, int64_t kv_lora_rank,
                                         int64_t num_splits);

/* Absorbed-form multi-head latent attention for one query per sequence (mla_decode):
 *   out[b, h, :] = softmax_j(scale * (q_c[b, h] . c[b, j] + q_pe[b, h] . k_pe[b, j])) @ c[b, j]
 * for j < context_lens[b], where cache row j of sequence b is latent_cache[block_tables[b,
 * j / block_size], j % block_size] = [c (kv_lora_rank) | k_pe (rope_dim)], one row shared by
 * all heads. q_c [num_seqs, num_heads, kv_lora_rank] and q_pe [num_seqs, num_heads, rope_dim]
 * of q_dtype (unit last stride; q_pe may point into the same rows as q_c, the reference's
 * single q_abs tensor); the cache [num_blocks, block_size, kv_lora_rank + rope_dim] of
 * cache_dtype with the given element strides (unit last stride); out [num_seqs, num_heads,
 * kv_lora_rank] of q_dtype. block_size must be a multiple of 16 and kv_lora_rank + rope_dim
 * <= 1024. Split-K, workspace, error bits and the zero-context NaN follow ember_paged_decode.
 * fp16/bf16 q and cache of one dtype at kv_lora_rank 512, rope_dim 64 (DeepSeek-V2/V3,
 * Moonlight) with 16-byte aligned operands run on MFMA with the reference kernel's tl.dot
 * numerics (fp32 scores, probabilities rounded to the cache dtype for P.V); every other case
 * computes in fp32. The MFMA path merges 2-3 splits in the last split to arrive and 4 or more
 * in a second launch spread over many workgroups. */
int ember_mla_decode(const void* q_c, int64_t qc_seq_stride, int64_t qc_head_stride,
                     const void* q_pe, int64_t qpe_seq_stride, int64_t qpe_head_stride, int q_dtype,
                     const void* latent_cache, int64_t num_blocks, int64_t block_size,
                     int64_t kv_lora_rank, int64_t rope_dim,
                     int64_t cache_block_stride, int64_t cache_slot_stride, int cache_dtype,
                     const int32_t* block_tables, int64_t block_table_stride, int64_t max_blocks,
                     const int32_t* context_lens, int64_t num_seqs, int64_t num_heads, float scale,
                     int64_t num_splits, void* workspace, int64_t workspace_bytes,
                     void* out, int64_t out_seq_stride, int64_t out_head_stride, void* stream);

/* Bytes of workspace ember_gate_up_silu needs with num_workgroups workgroups, -1 for invalid
 * arguments: fp32 partials [inter / 64][parts][4 x ceil(tokens / 16) x 2048] (parts = the
 * most workgroups that share one 64-column slab) and one uint32 arrival counter per slab. */
int64_t ember_gate_up_silu_workspace_bytes(int64_t tokens, int64_t hidden, int64_t inter,
                                           int64_t num_workgroups);

/* The dense MLP's gate_up projection with silu_and_mul as its epilogue, for 1..64 tokens:
 *   g = round(x[t] . w[j]),  u = round(x[t] . w[inter + j]),
 *   out[t, j] = round(round(g / (1 + exp(-g))) * u),  j < inter,
 * the composition silu_and_mul(gate_up_proj(x)) of Qwen2MLP.forward
 * (emberserve/model/qwen2.py:60-61; weight rows [0, inter) gate, [inter, 2 inter) up,
 * qwen2.py:49-57; silu_and_mul: ops.py:84-87), with fp32 dot products whose term order is
 * this kernel's own. x [tokens, hidden], w [2 inter, hidden], out [tokens, inter], fp16 or
 * bf16 (dtype), unit inner stride, 16-byte aligned, row strides in elements (x and w
 * multiples of 8, out of 4); hidden and inter multiples of 64. num_workgroups persistent
 * workgroups (at most one per 64-column x 64-k unit; one per CU is the intended size) split
 * the units evenly. The workspace (ember_gate_up_silu_workspace_bytes, zero-filled once)
 * holds partials and counters; the counters are left at zero. Other shapes return
 * EMBER_EINVAL (the caller keeps the unfused pair). */
int ember_gate_up_silu(const void* x, int64_t x_row_stride, const void* w, int64_t w_row_stride, int dtype,
                       int64_t tokens, int64_t hidden, int64_t inter, int64_t num_workgroups, void* workspace,
                       int64_t workspace_bytes, void* out, int64_t out_row_stride, void* stream);

/* The routed experts' gate_up projection with silu_and_mul as its epilogue, over the
 * moe_align layout (fused_moe_forward, emberserve/model/moe_triton.py:332-345: the first
 * _grouped_gemm and ops.silu_and_mul). sorted_ids [num_blocks * 16] int32 holds assignment
 * ids id = token * top_k + choice (>= num_valid: padding), block_expert [num_blocks] int32
 * the expert of each 16-row block (>= num_experts: unused block), as moe_align returns them
 * (moe_triton.py:215-254). For every assignment id in a block of expert e:
 *   out[id, j] = round(round(silu(g)) * u),  g = round(x[id / top_k] . w[e, j]),
 *   u = round(x[id / top_k] . w[e, inter + j]),  j < inter.
 * x [num_tokens, hidden], w [num_experts, 2 inter, hidden] (element strides; unit inner
 * stride), out [num_valid, inter]; fp16 or bf16, 16-byte aligned, hidden and inter
 * multiples of 64. A row id / top_k >= num_tokens reads row 0 and sets
 * EMBER_ERR_ROW_INDEX. num_splits (1..4, dividing hidden / 64 with >= 2 steps per split)
 * splits k across workgroups for small batches; with more than one it needs a zero-filled
 * workspace of ember_moe_gate_up_silu_workspace_bytes, whose counters it leaves at zero.
 * num_blocks <= 65535 (EMBER_EINVAL beyond). */
int ember_moe_gate_up_silu(const void* x, int64_t x_row_stride, int64_t num_tokens, const void* w,
                           int64_t w_expert_stride, int64_t w_row_stride, int dtype, int64_t num_experts,
                           int64_t hidden, int64_t inter, const int32_t* sorted_ids, const int32_t* block_expert,
                           int64_t num_blocks, int64_t num_valid, int64_t top_k, int64_t num_splits, void* workspace,
                           int64_t workspace_bytes, void* out, int64_t out_row_stride, void* stream);

/* Rearranges the routed experts' gate_up weights W [E, 2I, H] (element strides
 * w_expert_stride, w_row_stride; fp16 or bf16, 16-byte aligned; H and I multiples of 64)
 * into the layout ember_moe_gate_up_silu_packed reads: E * 2 I H elements, expert e at
 * e * 2 I H, and in it unit (j, slab) (j < H / 64, slab < I / 64) at (j * I / 64 + slab) *
 * 8192, holding
 *   unit[h][wave][part][lane][8] = W[e][part I + 64 slab + 16 wave + lane % 16]
 *                                   [64 j + 32 h + 8 (lane / 16) + 0..7]
 * (h < 2, wave < 4, part 0 gate / 1 up, lane < 64). A pure permutation, done once per
 * weight (at load time). No counterpart in the reference: the layout is this library's. */
int ember_moe_gate_up_silu_pack_weight(const void* w, int64_t w_expert_stride, int64_t w_row_stride, int dtype,
                                       int64_t num_experts, int64_t hidden, int64_t inter, void* packed,
                                       void* stream);

/* ember_moe_gate_up_silu over weights packed by ember_moe_gate_up_silu_pack_weight: the same
 * arguments less the weight strides, the same workspace, limits and errors, and the same
 * results bit for bit (the same products in the same order); replaces the same reference
 * calls (moe_triton.py:332-345). half_slabs = 1 (one split only) runs two-wave workgroups
 * over 32 output columns each instead of four-wave ones over 64: twice the workgroups,
 * for batches whose used blocks x slabs leave CUs idle. */
int ember_moe_gate_up_silu_packed(const void* x, int64_t x_row_stride, int64_t num_tokens, const void* packed_w,
                                  int dtype, int64_t num_experts, int64_t hidden, int64_t inter,
                                  const int32_t* sorted_ids, const int32_t* block_expert, int64_t num_blocks,
                                  int64_t num_valid, int64_t top_k, int64_t num_splits, int64_t half_slabs,
                                  void* workspace, int64_t workspace_bytes, void* out, int64_t out_row_stride,
                                  void* stream);

/* The gate_up projection + silu_and_mul at prefill sizes: an MFMA GEMM over token_tile x
 * (column_tile gate + column_tile up) tiles whose epilogue applies silu_and_mul, writing only
 * out [tokens, inter] (out[t, j] = round(round(silu(g)) * u), g and u the dot products
 * rounded to the dtype). x [tokens, hidden], w [2 inter, hidden] (gate rows, then up rows),
 * fp16 or bf16, 16-byte aligned, unit inner stride; hidden a multiple of 64, inter of
 * column_tile (of 16 for 96, whose last tile may be ragged). Tiles (token_tile,
 * column_tile): (256, 64), (256, 96), (256, 128) or (128, 128). No workspace. Each accumulator runs over k in order in one chain,
 * so a token's result equals ember_gate_up_silu_packed's over whole-slab runs bit for bit.
 * Replaces qwen2.py:60-61 (gate_up_proj, then silu_and_mul) without the [T, 2I] round trip. */
int ember_gate_up_silu_gemm(const void* x, int64_t x_row_stride, const void* w, int64_t w_row_stride, int dtype,
                            int64_t tokens, int64_t hidden, int64_t inter, int64_t token_tile, int64_t column_tile,
                            void* out, int64_t out_row_stride, void* stream);

/* The routed experts' gate_up projection with silu_and_mul as its epilogue at prefill sizes,
 * replacing the first _grouped_gemm of fused_moe_forward and the silu_and_mul after it
 * (emberserve/model/moe_triton.py:307-329, :339-340): the MFMA GEMM of
 * ember_gate_up_silu_gemm over a block-aligned layout of block_rows-row blocks
 * (ember_moe_align with block_m = block_rows: sorted_ids [num_blocks * block_rows],
 * block_expert [num_blocks]), one block per token tile. Block b multiplies the x rows
 * sorted_ids[block_rows b + r] / top_k (entries >= num_valid are padding) by expert
 * block_expert[b]'s W [2I, H] (at w + e * w_expert_stride, rows w_row_stride apart; blocks
 * with an expert >= num_experts are skipped) and writes out[sorted_ids[block_rows b + r]] =
 * silu(g) * u, rounded as ember_gate_up_silu does, for every real assignment: out
 * [num_valid, inter] in assignment order, the `act` of moe_triton.py:340. Every accumulator
 * runs over k in order, so a row's result is bit-identical to ember_moe_gate_up_silu's for
 * the same assignment. (block_rows, column_tile) as ember_gate_up_silu_gemm's tiles; inter a
 * multiple of column_tile, hidden of 64, fp16/bf16, 16-byte aligned operands. */
int ember_moe_gate_up_silu_gemm(const void* x, int64_t x_row_stride, int64_t num_tokens, const void* w,
                                int64_t w_expert_stride, int64_t w_row_stride, int dtype, int64_t num_experts,
                                int64_t hidden, int64_t inter, const int32_t* sorted_ids,
                                const int32_t* block_expert, int64_t num_blocks, int64_t block_rows,
                                int64_t num_valid, int64_t top_k, int64_t column_tile, void* out,
                                int64_t out_row_stride, void* stream);

/* The routed experts' gate_up + silu_and_mul over packed weights straight from the routing
 * ids, with no alignment: assignment a = token * top_k + choice (a < num_assignments <= 256,
 * topk_ids [num_assignments] int32 or int64 per id_bytes, row-major [tokens, top_k]) gets
 *   out[a, j] = round(round(silu(g)) * u) for expert topk_ids[a], as ember_moe_gate_up_silu
 * computes it, bit for bit. The grid has a workgroup per (assignment, slab): the
 * assignments of one expert form groups of 16 in assignment order, the workgroups of each
 * group's first assignment compute the group (one assignment per tile row) and the others
 * exit, so each expert's weights are read once per 16 of its assignments. For decode
 * batches, where it saves the ember_moe_align launch. An expert id outside [0, num_experts)
 * leaves its row unwritten and sets EMBER_ERR_EXPERT_ID. half_slabs as in
 * ember_moe_gate_up_silu_packed. No workspace. No counterpart in the reference's interface:
 * it replaces moe_align + the first grouped GEMM + silu_and_mul (moe_triton.py:332-345) for
 * decode steps. */
int ember_moe_gate_up_silu_direct(const void* x, int64_t x_row_stride, int64_t num_tokens, const void* packed_w,
                                  int dtype, int64_t num_experts, int64_t hidden, int64_t inter, const void* topk_ids,
                                  int id_bytes, int64_t num_assignments, int64_t top_k, int64_t half_slabs, void* out,
                                  int64_t out_row_stride, void* stream);

/* Rearranges a gate_up weight W [2I, H] (row stride w_row_stride elements, fp16 or bf16,
 * 16-byte aligned) into the layout ember_gate_up_silu_packed reads with num_workgroups
 * workgroups: 2 I H elements in units of 8192. Unit (slab, j) (slab < I / 64, j < H / 64) is
 *   unit[h][wave][part][lane][8] = W[part I + 64 slab + 16 wave + lane % 16]
 *                                   [64 j + 32 h + 8 (lane / 16) + 0..7]
 * (h < 2, wave < 4, part 0 gate / 1 up, lane < 64). With U = (I / 64)(H / 64) units and
 * G = min(num_workgroups, U), workgroup b owns units [floor(b U / G), floor((b + 1) U / G))
 * in slab-major order; its t-th unit is stored at unit position t G + b while t < U / G
 * (integer division), and the extra unit of a longer run after all of those, in workgroup
 * order. A pure permutation, done once per weight (at load time); H and I multiples of 64.
 * No counterpart in the reference: the layout is this library's, chosen so that the decode
 * kernel's grid reads the weights front to back. */
int ember_gate_up_silu_pack_weight(const void* w, int64_t w_row_stride, int dtype, int64_t hidden, int64_t inter,
                                   int64_t num_workgroups, void* packed, void* stream);

/* ember_gate_up_silu over a weight packed by ember_gate_up_silu_pack_weight: the same
 * results (bit-identical: the same products in the same order), the same workspace
 * (ember_gate_up_silu_workspace_bytes) and limits; replaces the same reference call
 * (qwen2.py:60-61). num_workgroups must be the value the weight was packed for (the
 * library cannot check it: another value reads the wrong units). */
int ember_gate_up_silu_packed(const void* x, int64_t x_row_stride, const void* packed_w, int dtype, int64_t tokens,
                              int64_t hidden, int64_t inter, int64_t num_workgroups, void* workspace,
                              int64_t workspace_bytes, void* out, int64_t out_row_stride, void* stream);

/* ember_gate_up_silu_gemm over a weight packed by ember_gate_up_silu_pack_weight for
 * num_workgroups decode workgroups: the same tiles without the 96-column one ((256, 64),
 * (256, 128), (128, 128); inter a multiple of column_tile), the same results bit for bit.
 * Each tile's weight operand is its 64-row slabs' packed 16 KiB units, read as contiguous
 * 1 KiB blocks. With it a model keeps one copy of the gate_up weight (the packed one) for
 * both the decode kernels and prefill. Replaces qwen2.py:60-61 (gate_up_proj, then
 * silu_and_mul); num_workgroups must be the value the weight was packed for. */
int ember_gate_up_silu_gemm_packed(const void* x, int64_t x_row_stride, const void* packed, int dtype,
                                   int64_t tokens, int64_t hidden, int64_t inter, int64_t num_workgroups,
                                   int64_t token_tile, int64_t column_tile, void* out, int64_t out_row_stride,
                                   void* stream);

/* ember_moe_gate_up_silu_gemm over experts packed by ember_moe_gate_up_silu_pack_weight
 * (tiles (256, 64), (256, 128), (128, 128); inter a multiple of column_tile): the same
 * results bit for bit. Each stage of a tile reads its slabs' adjacent 16 KiB units of the
 * expert's k-major packed array, contiguous memory instead of 128-byte pieces of 256
 * weight rows. Replaces the same reference calls (moe_triton.py:307-329, :339-340). */
int ember_moe_gate_up_silu_gemm_packed(const void* x, int64_t x_row_stride, int64_t num_tokens, const void* packed,
                                       int dtype, int64_t num_experts, int64_t hidden, int64_t inter,
                                       const int32_t* sorted_ids, const int32_t* block_expert, int64_t num_blocks,
                                       int64_t block_rows, int64_t num_valid, int64_t top_k, int64_t column_tile,
                                       void* out, int64_t out_row_stride, void* stream);

/* Bytes of workspace ember_moe_gate_up_silu needs for num_splits > 1 (0 for one split), -1
 * for invalid arguments: fp32 partials [num_splits][num_valid][2 inter] and one uint32
 * arrival counter per (block, 64-column slab). */
int64_t ember_moe_gate_up_silu_workspace_bytes(int64_t num_valid, int64_t inter, int64_t num_blocks,
                                               int64_t num_splits);

/* Slots of the block-aligned expert layout: round_up(num_valid + num_experts (block_m - 1),
 * block_m), -1 for invalid arguments (the max_padded of moe_triton.py:249). */
int64_t ember_moe_align_padded_size(int64_t num_valid, int64_t num_experts, int64_t block_m);

/* Bytes of workspace for the grid form of ember_moe_align at num_valid assignments (0 when
 * the one-workgroup form is used at that size), -1 for invalid arguments: an int32 count
 * table [segments][num_experts] over at most 64 segments of the assignments. */
int64_t ember_moe_align_workspace_bytes(int64_t num_valid, int64_t num_experts);

/* The routed experts' block-aligned layout, replacing moe_align of
 * emberserve/model/moe_triton.py:215-254 (its single-launch form is _moe_align_kernel,
 * :97-160). topk_ids: num_valid = tokens * top_k expert ids (id_bytes 4 or 8, contiguous,
 * assignment id = position). Writes
 *   sorted_ids [max_padded]: each expert's assignment ids in ascending order, its run padded
 *     with num_valid to a multiple of block_m, experts in ascending order, num_valid after
 *     the last run;
 *   block_expert [max_blocks = max_padded / block_m]: the expert of each block, num_experts
 *     past the last used block.
 * max_padded must equal ember_moe_align_padded_size(...). 1 <= num_experts <= 1024,
 * 0 <= num_valid <= INT32_MAX / 2. An id
 * outside [0, num_experts) is left out of the layout and sets EMBER_ERR_EXPERT_ID.
 * workspace (may be null) holds the grid form's count table: with at least
 * ember_moe_align_workspace_bytes(...) bytes, a count launch over up to 64 workgroups and a
 * placement launch over the same segments; otherwise (and always at num_valid <= 3072) one
 * workgroup in one launch. Both give the same layout. The workspace needs no clearing; no
 * host synchronisation, no memset: safe to capture in a HIP graph. */
int ember_moe_align(const void* topk_ids, int id_bytes, int64_t num_valid, int64_t num_experts, int64_t block_m,
                    int32_t* sorted_ids, int64_t max_padded, int32_t* block_expert, int64_t max_blocks,
                    void* workspace, int64_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* EMBER_OPS_H */
