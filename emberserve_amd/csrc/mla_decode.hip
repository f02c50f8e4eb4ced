// Multi-head latent attention decode for gfx950: the absorbed-form MLA kernel over the paged
// latent cache.
//
// Reference semantics (emberserve/attn/mla_triton.py:49-116 kernel, :119-182 launcher; the
// fp32 definition is mla_attention_absorbed, attn/mla_torch.py:33-53, with identity W_UK /
// W_UV as the reference's tests compare it):
//   out[b, h] = softmax_j(scale * (q_c[b, h] . c[b, j] + q_pe[b, h] . k_pe[b, j])) @ c[b, :]
// for j < context_lens[b], where cache row j of sequence b is latent[block_tables[b, j / bs],
// j % bs] = [c (DL) | k_pe (DR)]. Every query head attends to the same row (MQA over the
// latent), so each row is read from HBM once per (sequence, 16-head chunk).
//
// k_mla_mfma (fp16/bf16 q and cache of one dtype, DL = 512, DR = 64): a workgroup owns
// (sequence, 16-head chunk, split) and runs two tile streams (wave pairs); the streams walk
// alternate 32-key tiles of the split's range with their own online-softmax state and merge
// through LDS at the end. The two waves of a pair split every cache row by d: wave hw loads
// chunks [hw DL/2, (hw+1) DL/2) of the value part and half of the rope part (9 of the 18
// 32-element chunks, 72 registers per tile), so a wave holds 64 accumulators and the
// kernel runs two waves per SIMD and two workgroups (76 KB of LDS each) per CU. Per tile
// (v_mfma_f32_16x16x32):
//   S^T[16 keys, 16 heads] = R[16 keys, 576] . Q^T[576, 16 heads], each wave over its 9
//   chunks (2 halves x 9 MFMAs), the two partial sums exchanged through LDS:
//     A = R: lane (n, g) holds cache row n at e = chunk + 8g + [0, 8) (one dwordx4 load);
//     B = Q^T: lane (n, g) holds head n at the same e (registers, loaded once);
//     C: lane (n, g) gets head n's scores for keys 16s + 4g + i, i < 4.
//   O^T[16 d, 16 heads] += C^T[16 d, 32 kslots] . P^T[32 kslots, 16 heads], over the wave's
//   own d half (16 MFMAs): its value chunks, already in registers, go to a wave-private
//   LDS tile as they are (row-major, 16-byte stores) and come back transposed by
//   ds_read_b64_tr_b16, so the cache is read once; kslot 8g + 4s + i <-> key 16s + 4g + i,
//   so P^T is the lane's own 8 probabilities; C: lane (n, g) accumulates O[head n,
//   d0 + 16 dt + 4g + i].
//   The next tile's rows are requested as soon as this tile's scores and values are out of
//   the registers; block ids come from a per-pair window of 32 tiles read ahead.
//   Online softmax in base 2 with a lazy rescale: a head's reference max moves only when a
//   tile's max exceeds it by more than kLazy (probabilities stay <= 2^kLazy, far inside
//   fp16/bf16/fp32 range), so the accumulator rescale runs a few times per split instead of
//   on every growth. The final division by l uses the same reference max, so the result is
//   the softmax whatever the reference max was.
//   Numerics are the reference kernel's tl.dot ones: q and rows in storage dtype, fp32
//   scores, P rounded to the cache dtype before P.V, fp32 l and accumulators.
//
// k_mla_any (fp32, any other DL/DR, unaligned operands): one wave per (sequence, head,
// split), lane = key for the scores and lane = d for P.V, fp32 throughout.
//
// With num_splits > 1 the partial (m, l, acc) of each split goes to the workspace; the MFMA
// kernel's last split to finish merges them (an arrival counter per sequence and head
// chunk), k_mla_reduce does it for the fp32 kernel (paged_triton.py:188-209 semantics).
//
// Bad inputs never fault: a context length outside [0, max_blocks * block_size] is clamped
// (EMBER_ERR_DECODE_CTX); a block id outside [0, num_blocks) reads block 0
// (EMBER_ERR_BLOCK_ID). A zero context gives 0/0 = NaN rows, as the reference kernel does.
#include "ember_common.h"

namespace ember {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

template <typename T>
struct MlaMfma;
template <>
struct MlaMfma<_Float16> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x4 run(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};
template <>
struct MlaMfma<__bf16> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x4 run(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kTile = 32;      // keys per tile (one P.V MFMA deep)
constexpr int kVPad = 8;       // elements of padding per LDS value row (keeps 16-byte alignment)
constexpr float kLazy = 8.f;   // log2 headroom before the running max moves
constexpr int kMlaPairs = 2;       // tile streams (wave pairs) per workgroup
constexpr int kMlaPairsSmall = 4;  // ... when the grid fills at most half of the CUs
#ifndef EMBER_MLA_PAIR_SYNC
#define EMBER_MLA_PAIR_SYNC 1
#endif
constexpr bool kMlaPairSync = EMBER_MLA_PAIR_SYNC != 0;  // pair-local exchange handshake
#ifndef EMBER_MLA_STAGED
#define EMBER_MLA_STAGED 1
#endif
constexpr bool kMlaStaged = EMBER_MLA_STAGED != 0;  // small grids: rows staged through LDS
#ifndef EMBER_MLA_MERGE_APART
#define EMBER_MLA_MERGE_APART 4
#endif
// Split counts from which the MFMA kernels leave the split-K merge to k_mla_merge (a second
// launch spread over many workgroups) instead of the last split to arrive.
constexpr int kMlaMergeApart = EMBER_MLA_MERGE_APART;
constexpr int kMlaDL = 512;
constexpr int kMlaDR = 64;

struct MlaArgs {
  const void* qc;
  int64_t qc_sb, qc_sh;        // elements
  const void* qpe;
  int64_t qpe_sb, qpe_sh;
  void* out;
  int64_t o_sb, o_sh;
  const void* lat;
  int64_t l_sblk, l_sslot;
  const int32_t* bt;
  int64_t bt_sb;
  int32_t max_blocks;
  const int32_t* ctx;
  int32_t num_blocks;
  int32_t block_size;
  FastDiv bdiv;
  int32_t nseq, nh, hchunks;
  int32_t dl, dr;
  float scale2;                // scale * log2(e)
  int32_t splits;
  float* part_m;               // [splits][nseq][nh]
  float* part_l;
  float* part_o;               // [splits][nseq][nh][dl]
  uint32_t* counters;          // [nseq][nh] split arrivals (MFMA kernel), zero between launches
  int32_t merge_apart;         // MFMA kernels: publish the partials only, k_mla_merge merges
  uint32_t* err;
};

// s_waitcnt immediates (gfx9 encoding: vmcnt[3:0] and [15:14], expcnt[6:4], lgkmcnt[11:8]):
// vmcnt(0) alone, lgkmcnt(0) alone.
constexpr int kWaitVmcnt0 = 0x0F70;
constexpr int kWaitLgkm0 = 0xC07F;
constexpr int kWaitVmcnt18 = 0x4F72;  // vmcnt(18): 18 = 0b01'0010 -> [15:14] = 1, [3:0] = 2
constexpr int kSyncSpins = 1 << 15;  // s_sleep(1) polls before a pair wait gives up

__device__ __forceinline__ void store_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_agent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float shfl_xor_f(float v, int mask) { return __shfl_xor(v, mask, kWave); }

// One 16-byte-per-lane load from global memory straight to LDS: lane i's 16 bytes land at
// lds_base + 16 i. Only the device pass sees the builtin (the host pass drops the kernel's
// launch stub when it appears in a kernel body it does not generate code for).
__device__ __forceinline__ void load_to_lds16(const void* gptr, void* lds_base) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_global_load_lds(gptr, (__attribute__((address_space(3))) void*)(
                                             reinterpret_cast<uintptr_t>(lds_base)), 16, 0, 0);
#else
  (void)gptr;
  (void)lds_base;
#endif
}

__device__ __forceinline__ int seq_context(const MlaArgs& a, int b) {
  int c = a.ctx[b];
  const int cap = a.max_blocks * a.block_size;
  if (c < 0 || c > cap) {
    if (threadIdx.x == 0) atomicOr(a.err, EMBER_ERR_DECODE_CTX);
    c = c < 0 ? 0 : cap;
  }
  return c;
}

__device__ __forceinline__ int phys_block(const MlaArgs& a, const int32_t* btrow, int lb) {
  int p = btrow[lb];
  if (p < 0 || p >= a.num_blocks) {
    atomicOr(a.err, EMBER_ERR_BLOCK_ID);
    p = 0;
  }
  return p;
}

// Tile range [t0, t1) of split `split`: the real context is partitioned (mla_triton.py:82-85).
__device__ __forceinline__ void split_range(int ctx, int splits, int split, int& t0, int& t1) {
  const int nt = (ctx + kTile - 1) / kTile;
  const int per = (nt + splits - 1) / splits;
  t0 = split * per;
  t1 = min(t0 + per, nt);
}

// The end of an MFMA kernel's workgroup: the tile streams merge through LDS, then either
// the output rows are written (one split) or the split's partial is published and the last
// split to arrive merges all of them. m, lsum and o are the wave's online-softmax state;
// wave w of pair w / 2 holds d in [(w % 2) DL / 2, (w % 2 + 1) DL / 2).
template <typename T, int DL, int NP>
__device__ __forceinline__ void mla_finish(const MlaArgs& a, unsigned char* lds, float m, float lsum,
                                           const f32x4 (&o)[DL / 32], int b, int split, int head0,
                                           int nhc, bool poisoned = false) {
  constexpr int NDT = DL / 32;
  struct Combine {
    float m[NP][16];
    float l[NP][16];
    float o[NP][16][DL + 4];
  };
  const int lane = threadIdx.x & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int pr = w >> 1;
  const int hw = w & 1;
  const int n = lane & 15;
  const int g = lane >> 4;
  // merge the tile streams (the two waves of a pair hold the same m and l)
  lsum += shfl_xor_f(lsum, 16);
  lsum += shfl_xor_f(lsum, 32);
  // any poisoned wave (a handshake that ran out) poisons every row of the workgroup
  __shared__ int any_poisoned;
  if (threadIdx.x == 0) any_poisoned = 0;
  __syncthreads();
  if (poisoned && lane == 0) any_poisoned = 1;
  Combine& cb = *reinterpret_cast<Combine*>(lds);
  if (g == 0 && hw == 0) {
    cb.m[pr][n] = m;
    cb.l[pr][n] = lsum;
  }
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i) cb.o[pr][n][hw * (DL / 2) + 16 * dt + 4 * g + i] = o[dt][i];
  __syncthreads();

  // PARTS threads per head (16, or 32 with four streams); thread p of a head owns
  // d = 4p + 4 PARTS j + [0, 4), j < NJ, so each j of a head's threads is one contiguous run
  // of 4 PARTS floats: full lines for the partial stores and loads below, 8-byte output
  // stores that cover 8 PARTS contiguous bytes.
  constexpr int PARTS = NP * 2 * kWave / 16;
  constexpr int NJ = DL / (4 * PARTS);
  const int hh = threadIdx.x / PARTS;
  const int p4 = (threadIdx.x % PARTS) * 4;
  const bool mine = hh < nhc;
  const int head = head0 + hh;
  float mx = -INFINITY;
  float L = 0.f;
  f32x4 acc[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (mine) {
    float mw[NP];
#pragma unroll
    for (int v = 0; v < NP; ++v) {
      mw[v] = cb.m[v][hh];
      mx = fmaxf(mx, mw[v]);
    }
    if (any_poisoned) mx = __builtin_nanf("");
#pragma unroll
    for (int v = 0; v < NP; ++v) {
      const float wt = mw[v] == -INFINITY ? 0.f : exp2_fast(mw[v] - mx);
      L += wt * cb.l[v][hh];
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        acc[j] += wt * *reinterpret_cast<const f32x4*>(&cb.o[v][hh][p4 + 4 * PARTS * j]);
    }
  }
  T* orow = static_cast<T*>(a.out) + b * a.o_sb + head * a.o_sh + p4;
  auto store_out = [&](float l) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      Pack<T, 4> r;
#pragma unroll
      for (int e = 0; e < 4; ++e) r.v[e] = from_f32<T>(acc[j][e] / l);
      store_pack<T, 4>(orow + 4 * PARTS * j, r);
    }
  };
  if (a.splits == 1) {
    if (mine) store_out(L);
    return;
  }

  // Split-K: publish this split's partial with agent-coherent (sc1, written through) 16-byte
  // stores, count the arrival once they have completed, and let the last split to arrive
  // merge all of them with agent-coherent loads; it returns the counter to zero for the next
  // launch. The workgroup's 16 partial rows of one split are contiguous, so one buffer
  // resource (uniform base, exact size) addresses them.
  const int64_t stride = int64_t(a.nseq) * a.nh;
  const int64_t row0 = int64_t(b) * a.nh + head0;  // this chunk's first (sequence, head) row
  if (mine) {
    if (threadIdx.x % PARTS == 0) {
      store_agent(a.part_m + split * stride + row0 + hh, mx);
      store_agent(a.part_l + split * stride + row0 + hh, L);
    }
    const CoherentRsrc rs = coherent_rsrc(a.part_o + (split * stride + row0) * DL, nhc * DL);
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      store_coherent<4>(rs, (hh * DL + p4 + 4 * PARTS * j) * int(sizeof(float)), acc[j]);
  }
  if (a.merge_apart) return;
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  __shared__ int is_last;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t* cnt = a.counters + row0;
    const uint32_t prev = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    is_last = prev == static_cast<uint32_t>(a.splits - 1);
    if (is_last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!is_last) return;

  // The merge, online over chunks of kMergeChunk splits: each thread issues every load of a
  // chunk at once (the splits' max and sum of its head, its own d values of each split's
  // partial), so a chunk costs one round trip. The running max moves per chunk.
  const int hr = min(hh, nhc - 1);  // padded heads read a real row and store nothing
  const int roff = (hr * DL + p4) * int(sizeof(float));
  constexpr int kMergeChunk = NJ >= 8 ? 4 : 8;  // registers: kMergeChunk x (4 NJ + 2)
  float gm = -INFINITY;
  float gl = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int c0 = 0; c0 < a.splits; c0 += kMergeChunk) {
    const int cn = min(kMergeChunk, a.splits - c0);
    float ms[kMergeChunk], ls[kMergeChunk];
    f32x4 v[kMergeChunk][NJ];
#pragma unroll
    for (int u = 0; u < kMergeChunk; ++u) {
      ms[u] = -INFINITY;
      ls[u] = 0.f;
#pragma unroll
      for (int j = 0; j < NJ; ++j) v[u][j] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (u < cn) {  // uniform
        const int sp = c0 + u;
        ms[u] = load_agent(a.part_m + sp * stride + row0 + hr);
        ls[u] = load_agent(a.part_l + sp * stride + row0 + hr);
        const CoherentRsrc rs = coherent_rsrc(a.part_o + (sp * stride + row0) * DL, nhc * DL);
#pragma unroll
        for (int j = 0; j < NJ; ++j) v[u][j] = load_coherent<4>(rs, roff + 4 * PARTS * j * int(sizeof(float)));
      }
    }
    float cm = gm;
#pragma unroll
    for (int u = 0; u < kMergeChunk; ++u) cm = fmaxf(cm, ms[u]);
    const float alpha = gm == -INFINITY ? 0.f : exp2_fast(gm - cm);
    gl *= alpha;
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[j] *= alpha;
#pragma unroll
    for (int u = 0; u < kMergeChunk; ++u) {
      const float wt = ms[u] == -INFINITY ? 0.f : exp2_fast(ms[u] - cm);
      gl += wt * ls[u];
#pragma unroll
      for (int j = 0; j < NJ; ++j) acc[j] += wt * v[u][j];
    }
    gm = cm;
  }
  if (mine) store_out(gl);
}

// Poisons a wave's online-softmax state (running max, sum, accumulators) with NaN.
template <int NDT>
__device__ __forceinline__ void poison_state(float& m, float& lsum, f32x4 (&o)[NDT]) {
  m = __builtin_nanf("");
  lsum = __builtin_nanf("");
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) o[dt] = f32x4{m, m, m, m};
}

template <typename T, int DL, int DR, int NP, bool PSYNC>
__global__ void __launch_bounds__(NP * 2 * kWave, 2)
k_mla_mfma(MlaArgs a) {
  using M = MlaMfma<T>;
  using V8 = typename M::v8;
  constexpr int NV = DL / 64;         // value chunks (32 elements) per wave: its half of d
  constexpr int NR = DR / 64;         // rope chunks per wave
  constexpr int NC = NV + NR;         // chunks (16-byte loads per lane per row) per wave
  constexpr int NDT = DL / 32;        // 16-wide d tiles of P.V per wave
  constexpr int VS = DL / 2 + kVPad;  // LDS row stride of a wave's value tile (elements)
  static_assert(DL % 64 == 0 && DR % 64 == 0 && NR >= 1, "geometry");
  struct Combine {
    float m[NP][16];
    float l[NP][16];
    float o[NP][16][DL + 4];
  };
  constexpr int kVBytes = NP * 2 * kTile * VS * int(sizeof(T));
  constexpr int kXBytes = NP * 2 * 2 * kWave * 16;  // partial scores: [wave][half][lane] f32x4
  constexpr int kLoopBytes = kVBytes + kXBytes;
  constexpr int kLdsBytes = kLoopBytes > int(sizeof(Combine)) ? kLoopBytes : int(sizeof(Combine));
  static_assert(kLdsBytes <= (NP <= 2 ? 80 : 160) * 1024, "two workgroups per CU at two tile streams");
  __shared__ __attribute__((aligned(16))) unsigned char lds[kLdsBytes];

  const int lane = threadIdx.x & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int pr = w >> 1;  // tile stream (pair)
  const int hw = w & 1;   // which half of every row this wave loads: d in [hw DL/2, (hw+1) DL/2)
  const int n = lane & 15;
  const int g = lane >> 4;

  const int hc = blockIdx.x % a.hchunks;
  const int b = blockIdx.x / a.hchunks;
  const int split = blockIdx.y;
  const int head0 = hc * 16;
  const int nhc = min(16, a.nh - head0);

  const int ctx = seq_context(a, b);
  int t0, t1;
  split_range(ctx, a.splits, split, t0, t1);
  const int kend = min(t1 * kTile, ctx);

  // Element offset of this wave's chunk j within a row: NV value chunks of its d half,
  // then NR chunks of the rope part.
  auto chunk_e = [&](int j) { return j < NV ? (hw * NV + j) * 32 : DL + (hw * NR + (j - NV)) * 32; };

  // The pair's physical block ids, a window of 32 tiles at a time: lane 2k + s holds the
  // block of half s of the pair's k-th tile of the window, so a tile's row loads never wait
  // on a block-table read.
  const int32_t* btrow = a.bt + b * a.bt_sb;
  const int nloc = t1 > t0 + pr ? (t1 - t0 - pr + NP - 1) / NP : 0;  // tiles of this pair
  int blk_win = 0;
  auto load_window = [&](int k0w) {
    int hk = (t0 + pr + NP * (k0w + (lane >> 1))) * kTile + 16 * (lane & 1);
    if (hk >= ctx) hk = (ctx - 1) & ~15;
    if (hk < 0) hk = 0;
    const int lb = static_cast<int>(a.bdiv.div(static_cast<uint32_t>(hk)));
    blk_win = phys_block(a, btrow, lb);
  };
  // Half s of the pair's k-th tile: a half past the context still loads (from the last valid
  // half's block) so the loads stay unconditional; keys past the split's range are masked
  // after the scores.
  const T* lbase = static_cast<const T*>(a.lat) + 8 * g;
  Pack<T, 8> kr[2][NC];
  auto load_tile = [&](int k) {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      int hk0 = (t0 + pr + NP * k) * kTile + 16 * s;
      if (hk0 >= ctx) hk0 = (ctx - 1) & ~15;
      const int lb = static_cast<int>(a.bdiv.div(static_cast<uint32_t>(hk0)));
      const int pb = __builtin_amdgcn_readlane(blk_win, ((k & 31) << 1) | s);
      const T* rp = lbase + pb * a.l_sblk + (hk0 - lb * a.block_size + n) * a.l_sslot;
#pragma unroll
      for (int j = 0; j < NC; ++j) kr[s][j] = load_pack<T, 8>(rp + chunk_e(j));
    }
  };
  if (nloc > 0) {
    load_window(0);
    load_tile(0);
  }

  // Q^T operand of this wave's chunks: head n of this chunk of heads at e = chunk_e(j) +
  // 8g + [0, 8), zero for padded heads.
  V8 qv[NC];
  {
    const int hq = head0 + min(n, nhc - 1);
    const T* qc = static_cast<const T*>(a.qc) + b * a.qc_sb + int64_t(hq) * a.qc_sh + 8 * g;
    const T* qp = static_cast<const T*>(a.qpe) + b * a.qpe_sb + int64_t(hq) * a.qpe_sh + 8 * g;
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      const int e = chunk_e(j);
      V8 v = __builtin_bit_cast(V8, e < DL ? load_pack<T, 8>(qc + e) : load_pack<T, 8>(qp + (e - DL)));
      if (n >= nhc) v = V8{};
      qv[j] = v;
    }
  }

  float m = -INFINITY;
  float lsum = 0.f;
  f32x4 o[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  T* vl = reinterpret_cast<T*>(lds) + w * (kTile * VS);
  f32x4* xs = reinterpret_cast<f32x4*>(lds + kVBytes);  // [wave][half][lane]
  // ds_read_b64_tr_b16: lane (n, g) addresses row 16r + 4g + n/4 at d = 16dt + 4(n%4) and
  // receives C[16r + 4g + jj][16dt + n], jj < 4: the A operand's kslots 8g + 4r + jj.
  const T* vtr = vl + (4 * g + (n >> 2)) * VS + 4 * (n & 3);

  // The partner exchange. With PSYNC the two waves of a pair hand their partial scores over
  // through per-wave LDS counters (a pair runs at its own pace): wave w publishes tile k's
  // partial once its partner has read tile k-1's (rd of the partner >= k), then bumps its
  // own wr to k + 1; it reads the partner's partial once the partner's wr reaches k + 1,
  // then bumps its rd. Each counter has one writer and is written after the data it
  // covers has completed (s_waitcnt lgkmcnt(0)); LDS serves a CU's waves coherently. Waits
  // are bounded: a wait that runs out sets EMBER_ERR_SYNC and turns every later wait of
  // the wave off, so a broken handshake can corrupt a result but never hang the GPU.
  // Without PSYNC every wave runs the workgroup's trip count (pair 0's) and meets two
  // workgroup barriers per tile; a pair past its own tiles only takes part in them.
  __shared__ unsigned sync_wr[NP * 2];
  __shared__ unsigned sync_rd[NP * 2];
  bool sync_ok = true;
  auto pair_wait = [&](const unsigned* cnt, unsigned target) {
    if (!sync_ok) return;
    int spins = 0;
    while (__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < target) {
      __builtin_amdgcn_s_sleep(1);
      if (++spins > kSyncSpins) {
        sync_ok = false;
        if (lane == 0) atomicOr(a.err, EMBER_ERR_SYNC);
        break;
      }
    }
    asm volatile("" ::: "memory");
  };
  auto pair_post = [&](unsigned* cnt, unsigned v) {
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);  // the data this count covers has landed
    asm volatile("" ::: "memory");
    __hip_atomic_store(cnt, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  };
  if constexpr (PSYNC) {
    if (threadIdx.x < NP * 2) {
      sync_wr[threadIdx.x] = 0;
      sync_rd[threadIdx.x] = 0;
    }
    __syncthreads();
  }
  const int nwg = PSYNC ? nloc : (t1 > t0 ? (t1 - t0 + NP - 1) / NP : 0);
  for (int k = 0; k < nwg; ++k) {
    const bool active = PSYNC || k < nloc;  // uniform over the pair
    const int k0 = (t0 + pr + NP * k) * kTile;
    const bool partial = k0 + kTile > kend;
    const bool more = k + 1 < nloc;
    if (more && ((k + 1) & 31) == 0) load_window(k + 1);
    f32x4 sc[2];
    if (active) {
      // partial scores over this wave's chunks (two accumulation chains per half)
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        f32x4 c0 = f32x4{0.f, 0.f, 0.f, 0.f}, c1 = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < NC; j += 2) {
          c0 = M::run(__builtin_bit_cast(V8, kr[s][j]), qv[j], c0);
          if (j + 1 < NC) c1 = M::run(__builtin_bit_cast(V8, kr[s][j + 1]), qv[j + 1], c1);
        }
        sc[s] = c0 + c1;
      }
      // values of this wave's d half into its LDS tile (rows past the range stored as zero
      // so that stale cache contents cannot turn 0 * v into NaN), partial scores out
      if (partial) {
#pragma unroll
        for (int s = 0; s < 2; ++s)
          if (k0 + 16 * s + n >= kend)
#pragma unroll
            for (int j = 0; j < NV; ++j) kr[s][j] = Pack<T, 8>{};
      }
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int j = 0; j < NV; ++j) store_pack<T, 8>(vl + (16 * s + n) * VS + 32 * j + 8 * g, kr[s][j]);
      if constexpr (PSYNC) pair_wait(&sync_rd[w ^ 1], k);
      xs[(w * 2 + 0) * kWave + lane] = sc[0];
      xs[(w * 2 + 1) * kWave + lane] = sc[1];
      if constexpr (PSYNC) pair_post(&sync_wr[w], k + 1);
      asm volatile("" ::: "memory");
      // the registers take the pair's next tile while this one's exchange, softmax and P.V
      // run
      if (more) load_tile(k + 1);
    }
    if constexpr (PSYNC) pair_wait(&sync_wr[w ^ 1], k + 1);
    else __syncthreads();
    if (active) {
      sc[0] += xs[((w ^ 1) * 2 + 0) * kWave + lane];
      sc[1] += xs[((w ^ 1) * 2 + 1) * kWave + lane];
      if constexpr (PSYNC) pair_post(&sync_rd[w], k + 1);

      float x[8];
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int i = 0; i < 4; ++i) x[4 * s + i] = sc[s][i] * a.scale2;
      if (partial) {
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (k0 + 16 * s + 4 * g + i >= kend) x[4 * s + i] = -INFINITY;
      }
      float mt = x[0];
#pragma unroll
      for (int j = 1; j < 8; ++j) mt = fmaxf(mt, x[j]);
      mt = fmaxf(mt, shfl_xor_f(mt, 16));
      mt = fmaxf(mt, shfl_xor_f(mt, 32));
      if (__any(mt > m + kLazy)) {
        const float mn = fmaxf(m, mt);
        const float alpha = exp2_fast(m - mn);
        m = mn;
        lsum *= alpha;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) o[dt] *= alpha;
      }
      V8 pb;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float p = exp2_fast(x[j] - m);
        lsum += p;
        pb[j] = from_f32<T>(p);
      }
      // P.V over this wave's d half in groups of PVB d tiles: the group's transposed reads
      // are issued together, then its MFMAs
      constexpr int PVB = 8;
      typedef short v4s __attribute__((ext_vector_type(4)));
      typedef short v8s __attribute__((ext_vector_type(8)));
      typedef __attribute__((address_space(3))) v4s* lds_v4s;
#pragma unroll
      for (int d0 = 0; d0 < NDT; d0 += PVB) {
        v8s va[PVB];
#pragma unroll
        for (int kk = 0; kk < PVB; ++kk) {
          const T* src = vtr + 16 * (d0 + kk);
          const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(src));
          const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(src + 16 * VS));
          va[kk] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        }
#pragma unroll
        for (int kk = 0; kk < PVB; ++kk) o[d0 + kk] = M::run(__builtin_bit_cast(V8, va[kk]), pb, o[d0 + kk]);
      }
    }
    // the partner has read this tile's partial scores before the next tile's land
    if constexpr (!PSYNC) __syncthreads();
  }

  // A wave whose handshake ran out has read stale partner scores: its state is poisoned, so
  // the output rows of this workgroup (or the merge of its split) come out NaN instead of a
  // plausible wrong value, next to the EMBER_ERR_SYNC bit.
  if (!sync_ok) poison_state(m, lsum, o);
  mla_finish<T, DL, NP>(a, lds, m, lsum, o, b, split, head0, nhc, !sync_ok);
}

// k_mla_lds: the small-grid form of k_mla_mfma (same work split: two wave pairs per
// workgroup, each pair splitting every row by d; same exchange, softmax and merge). A lone
// sequence's tile time is set by how many row-load instructions one CU issues, and a
// register-operand load covers 16 rows x 64 bytes (16 half lines). Here each wave's rows go
// straight to LDS (global_load_lds_dwordx4), 8 rows x one 128-byte line per instruction,
// double-buffered: the next tile's loads are in flight while this tile's scores and P.V
// read the staged rows. A 1 KiB block of 8 rows keeps 16-byte unit u of row r at slot
// 8r + (u ^ r), so both the score operands (one row per lane) and the transposed value
// reads spread over the banks. Rows past the context are zeroed in LDS before P.V (stale
// cache bytes cannot turn 0 * v into NaN); their scores are masked as in k_mla_mfma.
template <typename T, int DL, int DR>
__global__ void __launch_bounds__(4 * kWave)
k_mla_lds(MlaArgs a) {
  using M = MlaMfma<T>;
  using V8 = typename M::v8;
  constexpr int NP = 2;
  constexpr int LW = DL / 128;         // value lines (64 elements) per wave
  constexpr int NV = 2 * LW;           // value chunks (32 elements) per wave
  constexpr int NC = NV + 1;           // + the wave's rope chunk
  constexpr int NDT = DL / 32;         // 16-wide d tiles of P.V per wave
  static_assert(DL % 128 == 0 && DR == 64, "geometry");
  constexpr int kRope = 2 * LW * 2 * 1024;           // rope blocks after the value blocks
  constexpr int kWaveStage = kRope + 2 * 1024;       // one wave's rows of one tile
  constexpr int kStageBytes = 2 * 2 * NP * kWaveStage;
  constexpr int kXBytes = 2 * NP * 2 * kWave * 16;
  constexpr int kCombineBytes = NP * 16 * 4 * 2 + NP * 16 * (DL + 4) * 4;
  constexpr int kLoop = kStageBytes + kXBytes;
  constexpr int kLdsBytes = kLoop > kCombineBytes ? kLoop : kCombineBytes;
  static_assert(kLdsBytes <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(16))) unsigned char lds[kLdsBytes];

  const int lane = threadIdx.x & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int pr = w >> 1;
  const int hw = w & 1;
  const int n = lane & 15;
  const int g = lane >> 4;

  const int hc = blockIdx.x % a.hchunks;
  const int b = blockIdx.x / a.hchunks;
  const int split = blockIdx.y;
  const int head0 = hc * 16;
  const int nhc = min(16, a.nh - head0);

  const int ctx = seq_context(a, b);
  int t0, t1;
  split_range(ctx, a.splits, split, t0, t1);
  const int kend = min(t1 * kTile, ctx);

  const int32_t* btrow = a.bt + b * a.bt_sb;
  const int nloc = t1 > t0 + pr ? (t1 - t0 - pr + NP - 1) / NP : 0;
  int blk_win = 0;
  auto load_window = [&](int k0w) {
    int hk = (t0 + pr + NP * (k0w + (lane >> 1))) * kTile + 16 * (lane & 1);
    if (hk >= ctx) hk = (ctx - 1) & ~15;
    if (hk < 0) hk = 0;
    const int lb = static_cast<int>(a.bdiv.div(static_cast<uint32_t>(hk)));
    blk_win = phys_block(a, btrow, lb);
  };
  // staged rows of tile buffer `buf` for this wave: value block (s, q, rb) = rows 8rb..8rb+7
  // of half s, the wave's value line q; rope block s = the wave's rope chunk of half s
  auto stage = [&](int buf) { return lds + (buf * 2 * NP + w) * kWaveStage; };
  auto vblock = [&](int s, int q, int rb) { return ((s * LW + q) * 2 + rb) * 1024; };
  const T* lat = static_cast<const T*>(a.lat);
  auto load_tile = [&](int k, int buf) {
    unsigned char* st = stage(buf);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      int hk0 = (t0 + pr + NP * k) * kTile + 16 * s;
      if (hk0 >= ctx) hk0 = (ctx - 1) & ~15;
      const int lb = static_cast<int>(a.bdiv.div(static_cast<uint32_t>(hk0)));
      const int pb = __builtin_amdgcn_readlane(blk_win, ((k & 31) << 1) | s);
      const T* rows = lat + pb * a.l_sblk + (hk0 - lb * a.block_size) * a.l_sslot;
      const int rr = lane >> 3;
      const int u = (lane & 7) ^ rr;
#pragma unroll
      for (int q = 0; q < LW; ++q)
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
          load_to_lds16(rows + (8 * rb + rr) * a.l_sslot + (LW * hw + q) * 64 + 8 * u, st + vblock(s, q, rb));
      load_to_lds16(rows + n * a.l_sslot + DL + 32 * hw + 8 * g, st + kRope + s * 1024);
    }
  };
  if (nloc > 0) {
    load_window(0);
    load_tile(0, 0);
  }

  // Q^T operand of this wave's chunks: value chunk j covers elements 64 (LW hw + j / 2) +
  // 32 (j % 2) + 8g + [0, 8) of head n, the rope chunk DL + 32 hw + 8g + [0, 8).
  V8 qv[NC];
  {
    const int hq = head0 + min(n, nhc - 1);
    const T* qc = static_cast<const T*>(a.qc) + b * a.qc_sb + int64_t(hq) * a.qc_sh + 8 * g;
    const T* qp = static_cast<const T*>(a.qpe) + b * a.qpe_sb + int64_t(hq) * a.qpe_sh + 8 * g;
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      V8 v = __builtin_bit_cast(V8, j < NV ? load_pack<T, 8>(qc + 64 * (LW * hw + j / 2) + 32 * (j % 2))
                                           : load_pack<T, 8>(qp + 32 * hw));
      if (n >= nhc) v = V8{};
      qv[j] = v;
    }
  }

  float m = -INFINITY;
  float lsum = 0.f;
  f32x4 o[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  f32x4* xs = reinterpret_cast<f32x4*>(lds + kStageBytes);  // [wave][half][lane]
  __shared__ unsigned sync_wr[NP * 2];
  __shared__ unsigned sync_rd[NP * 2];
  bool sync_ok = true;
  auto pair_wait = [&](const unsigned* cnt, unsigned target) {
    if (!sync_ok) return;
    int spins = 0;
    while (__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < target) {
      __builtin_amdgcn_s_sleep(1);
      if (++spins > kSyncSpins) {
        sync_ok = false;
        if (lane == 0) atomicOr(a.err, EMBER_ERR_SYNC);
        break;
      }
    }
    asm volatile("" ::: "memory");
  };
  auto pair_post = [&](unsigned* cnt, unsigned v) {
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    asm volatile("" ::: "memory");
    __hip_atomic_store(cnt, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  };
  if (threadIdx.x < NP * 2) {
    sync_wr[threadIdx.x] = 0;
    sync_rd[threadIdx.x] = 0;
  }
  __syncthreads();

  // per-lane parts of the staged-row addresses: score operands read row n of their half,
  // value reads row 4g + n/4 of each half at d = 16 dt + 4 (n % 4)
  const int srb = n >> 3, srr = n & 7;
  const int vn = 4 * g + (n >> 2);
  const int vrb = vn >> 3, vrr = vn & 7;

  for (int k = 0; k < nloc; ++k) {
    const int buf = k & 1;
    const int k0 = (t0 + pr + NP * k) * kTile;
    const bool partial = k0 + kTile > kend;
    if (k + 1 < nloc) {
      if (((k + 1) & 31) == 0) load_window(k + 1);
      __builtin_amdgcn_s_waitcnt(kWaitLgkm0);  // the other buffer's reads (tile k - 1) are done
      asm volatile("" ::: "memory");
      load_tile(k + 1, buf ^ 1);
      __builtin_amdgcn_s_waitcnt(kWaitVmcnt18);  // all but the 18 just issued: tile k is staged
    } else {
      __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    }
    asm volatile("" ::: "memory");
    unsigned char* st = stage(buf);
    if (partial) {
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
          if (k0 + 16 * s + 8 * rb + (lane >> 3) >= kend)
#pragma unroll
            for (int q = 0; q < LW; ++q) store_pack<T, 8>(reinterpret_cast<T*>(st + vblock(s, q, rb)) + 8 * lane, Pack<T, 8>{});
      asm volatile("" ::: "memory");
    }

    // partial scores over this wave's chunks
    f32x4 sc[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      f32x4 c0 = f32x4{0.f, 0.f, 0.f, 0.f}, c1 = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < NC; ++j) {
        const unsigned char* src =
            j < NV ? st + vblock(s, j / 2, srb) + (8 * srr + ((4 * (j % 2) + g) ^ srr)) * 16
                   : st + kRope + s * 1024 + 16 * lane;
        const V8 kv = __builtin_bit_cast(V8, *reinterpret_cast<const Pack<T, 8>*>(src));
        if (j % 2 == 0) c0 = M::run(kv, qv[j], c0);
        else c1 = M::run(kv, qv[j], c1);
      }
      sc[s] = c0 + c1;
    }
    pair_wait(&sync_rd[w ^ 1], k);
    xs[(w * 2 + 0) * kWave + lane] = sc[0];
    xs[(w * 2 + 1) * kWave + lane] = sc[1];
    pair_post(&sync_wr[w], k + 1);
    pair_wait(&sync_wr[w ^ 1], k + 1);
    sc[0] += xs[((w ^ 1) * 2 + 0) * kWave + lane];
    sc[1] += xs[((w ^ 1) * 2 + 1) * kWave + lane];
    pair_post(&sync_rd[w], k + 1);

    float x[8];
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int i = 0; i < 4; ++i) x[4 * s + i] = sc[s][i] * a.scale2;
    if (partial) {
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (k0 + 16 * s + 4 * g + i >= kend) x[4 * s + i] = -INFINITY;
    }
    float mt = x[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) mt = fmaxf(mt, x[j]);
    mt = fmaxf(mt, shfl_xor_f(mt, 16));
    mt = fmaxf(mt, shfl_xor_f(mt, 32));
    if (__any(mt > m + kLazy)) {
      const float mn = fmaxf(m, mt);
      const float alpha = exp2_fast(m - mn);
      m = mn;
      lsum *= alpha;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) o[dt] *= alpha;
    }
    V8 pb;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float p = exp2_fast(x[j] - m);
      lsum += p;
      pb[j] = from_f32<T>(p);
    }
    constexpr int PVB = 8;
    typedef short v4s __attribute__((ext_vector_type(4)));
    typedef short v8s __attribute__((ext_vector_type(8)));
    typedef __attribute__((address_space(3))) v4s* lds_v4s;
#pragma unroll
    for (int d0 = 0; d0 < NDT; d0 += PVB) {
      v8s va[PVB];
#pragma unroll
      for (int kk = 0; kk < PVB; ++kk) {
        const int dt = d0 + kk;
        const int slot = 8 * vrr + ((2 * (dt & 3) + ((n & 3) >> 1)) ^ vrr);
        const unsigned char* lo_p = st + vblock(0, dt >> 2, vrb) + 16 * slot + 8 * (n & 1);
        const unsigned char* hi_p = st + vblock(1, dt >> 2, vrb) + 16 * slot + 8 * (n & 1);
        const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(reinterpret_cast<uintptr_t>(lo_p)));
        const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(reinterpret_cast<uintptr_t>(hi_p)));
        va[kk] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      }
#pragma unroll
      for (int kk = 0; kk < PVB; ++kk) o[d0 + kk] = M::run(__builtin_bit_cast(V8, va[kk]), pb, o[d0 + kk]);
    }
  }
  // A wave whose handshake ran out has read stale partner scores: its state is poisoned, so
  // the output rows of this workgroup (or the merge of its split) come out NaN instead of a
  // plausible wrong value, next to the EMBER_ERR_SYNC bit.
  if (!sync_ok) poison_state(m, lsum, o);
  mla_finish<T, DL, NP>(a, lds, m, lsum, o, b, split, head0, nhc, !sync_ok);
}

constexpr int kAnyMaxD = 1024;          // DL + DR of the fp32 kernel
constexpr int kAnyPer = 1024 / kWave;   // value elements per lane (DL <= 1024)

// Any geometry: one wave per (sequence, head, split), fp32 math.
template <typename TQ, typename TC>
__global__ void __launch_bounds__(kWave)
k_mla_any(MlaArgs a) {
  __shared__ float qs[kAnyMaxD];
  __shared__ float ps[kWave];
  __shared__ int64_t rows[kWave];
  const int lane = threadIdx.x;
  const int h = blockIdx.x % a.nh;
  const int b = blockIdx.x / a.nh;
  const int split = blockIdx.y;
  const int DL = a.dl;
  const int D = a.dl + a.dr;
  const int ctx = seq_context(a, b);
  int t0, t1;
  split_range(ctx, a.splits, split, t0, t1);
  const int kbeg = t0 * kTile;
  const int kend = min(t1 * kTile, ctx);

  const TQ* qc = static_cast<const TQ*>(a.qc) + b * a.qc_sb + h * a.qc_sh;
  const TQ* qp = static_cast<const TQ*>(a.qpe) + b * a.qpe_sb + h * a.qpe_sh;
  for (int e = lane; e < D; e += kWave) qs[e] = to_f32(e < DL ? qc[e] : qp[e - DL]) * a.scale2;
  __syncthreads();

  const TC* lat = static_cast<const TC*>(a.lat);
  const int32_t* btrow = a.bt + b * a.bt_sb;
  float m = -INFINITY, l = 0.f;
  float acc[kAnyPer];
#pragma unroll
  for (int j = 0; j < kAnyPer; ++j) acc[j] = 0.f;
  for (int kk = kbeg; kk < kend; kk += kWave) {
    const int key = kk + lane;
    const bool valid = key < kend;
    float s = -INFINITY;
    int64_t row = 0;
    if (valid) {
      const int lb = static_cast<int>(a.bdiv.div(static_cast<uint32_t>(key)));
      const int pb = phys_block(a, btrow, lb);
      row = pb * a.l_sblk + (key - lb * a.block_size) * a.l_sslot;
      float dot = 0.f;
      for (int e = 0; e < D; ++e) dot += qs[e] * to_f32(lat[row + e]);
      s = dot;
    }
    float mt = s;
    for (int off = 32; off >= 1; off >>= 1) mt = fmaxf(mt, shfl_xor_f(mt, off));
    const float mn = fmaxf(m, mt);
    const float alpha = exp2_fast(m - mn);
    m = mn;
    const float p = valid ? exp2_fast(s - mn) : 0.f;
    float psum = p;
    for (int off = 32; off >= 1; off >>= 1) psum += shfl_xor_f(psum, off);
    l = l * alpha + psum;
    __syncthreads();
    ps[lane] = p;
    rows[lane] = row;
    __syncthreads();
    const int nk = min(kWave, kend - kk);
#pragma unroll
    for (int j = 0; j < kAnyPer; ++j) acc[j] *= alpha;
    for (int r = 0; r < nk; ++r) {
      const float pr = ps[r];
      const TC* rp = lat + rows[r];
#pragma unroll
      for (int j = 0; j < kAnyPer; ++j) {
        const int e = lane + kWave * j;
        if (e < DL) acc[j] += pr * to_f32(rp[e]);
      }
    }
  }
  if (a.splits == 1) {
    TQ* op = static_cast<TQ*>(a.out) + b * a.o_sb + h * a.o_sh;
#pragma unroll
    for (int j = 0; j < kAnyPer; ++j) {
      const int e = lane + kWave * j;
      if (e < DL) op[e] = from_f32<TQ>(acc[j] / l);
    }
  } else {
    const int64_t row = (int64_t(split) * a.nseq + b) * a.nh + h;
    if (lane == 0) {
      a.part_m[row] = m;
      a.part_l[row] = l;
    }
#pragma unroll
    for (int j = 0; j < kAnyPer; ++j) {
      const int e = lane + kWave * j;
      if (e < DL) a.part_o[row * DL + e] = acc[j];
    }
  }
}

// Merge of the fp32 kernel's split-K partials: one wave per (sequence, head).
template <typename TO>
__global__ void __launch_bounds__(256)
k_mla_reduce(MlaArgs a) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.nseq * a.nh) return;
  const int lane = threadIdx.x & (kWave - 1);
  const int b = row / a.nh;
  const int h = row - b * a.nh;
  const int64_t stride = int64_t(a.nseq) * a.nh;
  float mx = -INFINITY;
  for (int s = 0; s < a.splits; ++s) mx = fmaxf(mx, a.part_m[s * stride + row]);
  float L = 0.f;
  float acc[kAnyPer];
#pragma unroll
  for (int j = 0; j < kAnyPer; ++j) acc[j] = 0.f;
  for (int s = 0; s < a.splits; ++s) {
    const int64_t r = s * stride + row;
    const float ms = a.part_m[r];
    const float wt = ms == -INFINITY ? 0.f : exp2_fast(ms - mx);
    L += wt * a.part_l[r];
#pragma unroll
    for (int j = 0; j < kAnyPer; ++j) {
      const int e = lane + kWave * j;
      if (e < a.dl) acc[j] += wt * a.part_o[r * a.dl + e];
    }
  }
  TO* op = static_cast<TO*>(a.out) + b * a.o_sb + h * a.o_sh;
#pragma unroll
  for (int j = 0; j < kAnyPer; ++j) {
    const int e = lane + kWave * j;
    if (e < a.dl) op[e] = from_f32<TO>(acc[j] / L);
  }
}

// The split-K merge of the MFMA kernels as its own launch: one thread per 4 contiguous d of
// a (sequence, head) row, all of whose splits' partials it merges online, eight splits'
// loads in flight at a time. One 64-lane workgroup per 256 output floats spreads a lone
// sequence's partials (16 heads x 512 floats per split) over 32 CUs.
template <typename TO, int DL>
__global__ void __launch_bounds__(kWave)
k_mla_merge(MlaArgs a) {
  constexpr int TPR = DL / 4;
  constexpr int kChunk = 8;
  const int t = blockIdx.x * kWave + threadIdx.x;
  const int row = t / TPR;  // sequence * nh + head
  if (row >= a.nseq * a.nh) return;
  const int d = (t % TPR) * 4;
  const int64_t stride = int64_t(a.nseq) * a.nh;
  float gm = -INFINITY, gl = 0.f;
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int c0 = 0; c0 < a.splits; c0 += kChunk) {
    float ms[kChunk], ls[kChunk];
    f32x4 v[kChunk];
#pragma unroll
    for (int u = 0; u < kChunk; ++u) {
      ms[u] = -INFINITY;
      ls[u] = 0.f;
      v[u] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (c0 + u < a.splits) {
        const int64_t r = (c0 + u) * stride + row;
        ms[u] = a.part_m[r];
        ls[u] = a.part_l[r];
        // part_o starts 8 bytes past a 16-byte boundary when splits x rows is odd
        const float2 lo = *reinterpret_cast<const float2*>(a.part_o + r * DL + d);
        const float2 hi = *reinterpret_cast<const float2*>(a.part_o + r * DL + d + 2);
        v[u] = f32x4{lo.x, lo.y, hi.x, hi.y};
      }
    }
    float cm = gm;
#pragma unroll
    for (int u = 0; u < kChunk; ++u) cm = fmaxf(cm, ms[u]);
    const float alpha = gm == -INFINITY ? 0.f : exp2_fast(gm - cm);
    gl *= alpha;
    acc *= alpha;
#pragma unroll
    for (int u = 0; u < kChunk; ++u) {
      const float wt = ms[u] == -INFINITY ? 0.f : exp2_fast(ms[u] - cm);
      gl += wt * ls[u];
      acc += wt * v[u];
    }
    gm = cm;
  }
  const int b = row / a.nh;
  const int h = row - b * a.nh;
  Pack<TO, 4> r;
#pragma unroll
  for (int e = 0; e < 4; ++e) r.v[e] = from_f32<TO>(acc[e] / gl);
  store_pack<TO, 4>(static_cast<TO*>(a.out) + b * a.o_sb + h * a.o_sh + d, r);
}

template <typename TQ>
int launch_any_q(int cdt, const MlaArgs& a, dim3 grid, hipStream_t st) {
  switch (cdt) {
    case EMBER_F32: k_mla_any<TQ, float><<<grid, kWave, 0, st>>>(a); break;
    case EMBER_F16: k_mla_any<TQ, _Float16><<<grid, kWave, 0, st>>>(a); break;
    case EMBER_BF16: k_mla_any<TQ, __bf16><<<grid, kWave, 0, st>>>(a); break;
    default: return EMBER_EINVAL;
  }
  return EMBER_OK;
}

template <typename TO>
void launch_reduce(const MlaArgs& a, hipStream_t st) {
  const int rows = a.nseq * a.nh;
  k_mla_reduce<TO><<<(rows + 3) / 4, 256, 0, st>>>(a);
}

}  // namespace
}  // namespace ember

using namespace ember;

extern "C" {

int64_t ember_mla_decode_workspace_bytes(int64_t num_seqs, int64_t num_heads, int64_t kv_lora_rank,
                                         int64_t num_splits) {
  if (num_seqs < 0 || num_heads < 0 || kv_lora_rank < 0 || num_splits < 1) return -1;
  if (num_splits == 1) return 0;
  const int64_t partials = num_splits * num_seqs * num_heads * (kv_lora_rank + 2) * int64_t(sizeof(float));
  return partials + (num_seqs * num_heads * int64_t(sizeof(uint32_t)) + 15) / 16 * 16;
}

int ember_mla_decode(const void* q_c, int64_t qc_seq_stride, int64_t qc_head_stride, const void* q_pe,
                     int64_t qpe_seq_stride, int64_t qpe_head_stride, int q_dtype, const void* latent_cache,
                     int64_t num_blocks, int64_t block_size, int64_t kv_lora_rank, int64_t rope_dim,
                     int64_t cache_block_stride, int64_t cache_slot_stride, int cache_dtype,
                     const int32_t* block_tables, int64_t block_table_stride, int64_t max_blocks,
                     const int32_t* context_lens, int64_t num_seqs, int64_t num_heads, float scale,
                     int64_t num_splits, void* workspace, int64_t workspace_bytes, void* out,
                     int64_t out_seq_stride, int64_t out_head_stride, void* stream) {
  const int qsz = dtype_size(q_dtype);
  const int csz = dtype_size(cache_dtype);
  if (qsz == 0 || csz == 0) return EMBER_EINVAL;
  if (num_seqs < 0 || num_heads < 1 || kv_lora_rank < 1 || rope_dim < 0) return EMBER_EINVAL;
  if (kv_lora_rank > kAnyMaxD || kv_lora_rank + rope_dim > kAnyMaxD) return EMBER_EINVAL;
  if (block_size < 16 || block_size % 16 != 0) return EMBER_EINVAL;
  if (num_blocks < 1 || max_blocks < 1 || num_splits < 1 || num_splits > 1024) return EMBER_EINVAL;
  if (max_blocks * block_size > INT32_MAX || num_blocks > INT32_MAX) return EMBER_EINVAL;
  if (num_seqs == 0) return EMBER_OK;
  if (!q_c || (rope_dim > 0 && !q_pe) || !latent_cache || !block_tables || !context_lens || !out)
    return EMBER_EINVAL;
  if (num_seqs * num_heads > INT32_MAX / 2) return EMBER_EINVAL;
  const int64_t need = ember_mla_decode_workspace_bytes(num_seqs, num_heads, kv_lora_rank, num_splits);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need || (reinterpret_cast<uintptr_t>(workspace) & 15)))
    return EMBER_EINVAL;
  uint32_t* err = device_error_word();
  if (err == nullptr) return EMBER_ENODEV;

  MlaArgs a{};
  a.qc = q_c;
  a.qc_sb = qc_seq_stride;
  a.qc_sh = qc_head_stride;
  a.qpe = rope_dim > 0 ? q_pe : q_c;
  a.qpe_sb = qpe_seq_stride;
  a.qpe_sh = qpe_head_stride;
  a.out = out;
  a.o_sb = out_seq_stride;
  a.o_sh = out_head_stride;
  a.lat = latent_cache;
  a.l_sblk = cache_block_stride;
  a.l_sslot = cache_slot_stride;
  a.bt = block_tables;
  a.bt_sb = block_table_stride;
  a.max_blocks = static_cast<int32_t>(max_blocks);
  a.ctx = context_lens;
  a.num_blocks = static_cast<int32_t>(num_blocks);
  a.block_size = static_cast<int32_t>(block_size);
  a.bdiv = FastDiv::make(static_cast<uint32_t>(block_size));
  a.nseq = static_cast<int32_t>(num_seqs);
  a.nh = static_cast<int32_t>(num_heads);
  a.hchunks = static_cast<int32_t>(cdiv(num_heads, 16));
  a.dl = static_cast<int32_t>(kv_lora_rank);
  a.dr = static_cast<int32_t>(rope_dim);
  a.scale2 = scale * kLog2e;
  a.splits = static_cast<int32_t>(num_splits);
  if (need > 0) {
    float* ws = static_cast<float*>(workspace);
    const int64_t rows = num_splits * num_seqs * num_heads;
    a.part_m = ws;
    a.part_l = ws + rows;
    a.part_o = ws + 2 * rows;
    a.counters = reinterpret_cast<uint32_t*>(ws + rows * (kv_lora_rank + 2));
  }
  a.err = err;
  hipStream_t st = static_cast<hipStream_t>(stream);

  // The MFMA kernel's 16-byte q / row loads and 16-byte output stores need that alignment;
  // anything else runs the fp32 kernel.
  const bool same = q_dtype == cache_dtype && q_dtype != EMBER_F32;
  const bool geom = kv_lora_rank == kMlaDL && rope_dim == kMlaDR;
  const bool aligned = aligned16(q_c) && aligned16(q_pe) && aligned16(latent_cache) && aligned16(out) &&
                       qc_seq_stride % 8 == 0 && qc_head_stride % 8 == 0 && qpe_seq_stride % 8 == 0 &&
                       qpe_head_stride % 8 == 0 && cache_block_stride % 8 == 0 && cache_slot_stride % 8 == 0 &&
                       out_seq_stride % 8 == 0 && out_head_stride % 8 == 0;
  const bool mfma = same && geom && aligned;
  int rc = EMBER_OK;
  if (mfma) {
    const int64_t progs = num_seqs * a.hchunks;
    if (progs > INT32_MAX) return EMBER_EINVAL;
    dim3 grid(static_cast<uint32_t>(progs), static_cast<uint32_t>(num_splits));
    // A grid that fills at most half of the CUs (one or a few sequences) runs four tile
    // streams per workgroup: half the serial tiles per stream, one workgroup per CU.
    const int ncu = device_cu_count();
    const bool small = ncu > 0 && progs * num_splits * 2 <= ncu;
    a.merge_apart = num_splits >= kMlaMergeApart ? 1 : 0;
    if (q_dtype == EMBER_F16) {
      if (small && kMlaStaged)
        k_mla_lds<_Float16, kMlaDL, kMlaDR><<<grid, 4 * kWave, 0, st>>>(a);
      else if (small)
        k_mla_mfma<_Float16, kMlaDL, kMlaDR, kMlaPairsSmall, kMlaPairSync><<<grid, kMlaPairsSmall * 2 * kWave, 0, st>>>(a);
      else
        k_mla_mfma<_Float16, kMlaDL, kMlaDR, kMlaPairs, kMlaPairSync><<<grid, kMlaPairs * 2 * kWave, 0, st>>>(a);
    } else {
      if (small && kMlaStaged)
        k_mla_lds<__bf16, kMlaDL, kMlaDR><<<grid, 4 * kWave, 0, st>>>(a);
      else if (small)
        k_mla_mfma<__bf16, kMlaDL, kMlaDR, kMlaPairsSmall, kMlaPairSync><<<grid, kMlaPairsSmall * 2 * kWave, 0, st>>>(a);
      else
        k_mla_mfma<__bf16, kMlaDL, kMlaDR, kMlaPairs, kMlaPairSync><<<grid, kMlaPairs * 2 * kWave, 0, st>>>(a);
    }
    if (a.merge_apart) {
      const int64_t threads = num_seqs * num_heads * (kMlaDL / 4);
      const uint32_t blocks = static_cast<uint32_t>((threads + kWave - 1) / kWave);
      if (q_dtype == EMBER_F16)
        k_mla_merge<_Float16, kMlaDL><<<blocks, kWave, 0, st>>>(a);
      else
        k_mla_merge<__bf16, kMlaDL><<<blocks, kWave, 0, st>>>(a);
    }
  } else {
    dim3 grid(static_cast<uint32_t>(num_seqs * num_heads), static_cast<uint32_t>(num_splits));
    switch (q_dtype) {
      case EMBER_F32: rc = launch_any_q<float>(cache_dtype, a, grid, st); break;
      case EMBER_F16: rc = launch_any_q<_Float16>(cache_dtype, a, grid, st); break;
      default: rc = launch_any_q<__bf16>(cache_dtype, a, grid, st); break;
    }
    if (rc != EMBER_OK) return rc;
    if (num_splits > 1) {
      switch (q_dtype) {
        case EMBER_F32: launch_reduce<float>(a, st); break;
        case EMBER_F16: launch_reduce<_Float16>(a, st); break;
        default: launch_reduce<__bf16>(a, st); break;
      }
    }
  }
  return launch_status();
}

}  // extern "C"
