// Paged decode attention for gfx950: one query token per sequence against its paged K/V.
//
// Reference semantics (emberserve/attn/paged_triton.py:95-209 kernels, :323-399 launcher;
// the fp32 definition is PagedTorchAttentionBackend._decode, attn/paged_torch.py:87-98):
//   out[b, h] = softmax_j(scale * q[b, h] . K[b, j, h/G]) @ V[b, :, h/G],  j < context_lens[b]
// where key j of sequence b lives in cache slot (block_tables[b, j / bs], j % bs) and G =
// H / Hkv query heads share one KV head. Every key is read from HBM once per KV head.
//
// Two kernels compute the attention; both write either the final row or, with split-K,
// the unnormalised partial (m, l, acc) of their key range. The MFMA kernel merges the
// partials in the epilogue of the last split to finish (an arrival counter per sequence
// and head chunk); the fp32 kernel's partials are merged by k_decode_reduce.
//
// k_decode_mfma (fp16/bf16 q and cache of one dtype, D in {64, 128}): the "dot" numerics of
// the reference (q in storage dtype, fp32 scores, P rounded to the V dtype before P.V; l in
// fp32). A workgroup owns (sequence, KV head, 16-head chunk, split); each of its 4 waves
// walks every 4th 32-key tile of the split's range with its own online-softmax state, and
// the waves merge through LDS at the end. Per tile (32 keys, v_mfma_f32_16x16x32):
//   S^T[16 keys, 16 heads] = K[16 keys, D] . Q^T[D, 16 heads]       (2 halves x D/32 MFMAs)
//     A = K: lane (n, g) holds key row n, d = 32c + 8g + [0, 8) for MFMA c, so one
//            dwordx4 load instruction covers 64 contiguous bytes of 16 key rows;
//     B = Q^T: lane (n, g) holds head n at the same d (zero for padded heads);
//     C: lane (n, g) gets head n's scores for keys 16s + 4g + i, i < 4.
//   O^T[16 d, 16 heads] += V^T[16 d, 32 kslots] . P^T[32 kslots, 16 heads]   (D/16 MFMAs)
//     kslot 8g + 4s + i <-> key 16s + 4g + i, so B = P^T is exactly the lane's own 8
//     probabilities (head n) in register order; A = V^T needs 8 keys of one d per lane,
//     which a wave-private LDS tile Vt[d][kslot] provides (V goes in as 2-byte scatters,
//     comes out as one 16-byte read per d tile);
//     C: lane (n, g) accumulates O[head n, 16 dt + 4g + i]: the head is the lane's own, so
//     the online-softmax rescale needs no cross-lane traffic.
//   The row max of a head is over its 4 lane groups (two xor shuffles per tile); the row
//   sum stays per lane until the end.
//
// k_decode_any (every other geometry and dtype mix, including fp32 caches): one wave per
// (sequence, query head, split), lane = key for the scores and lane = d for P.V, fp32 all
// the way (the reference's "sum" variant numerics).
//
// Bad inputs never fault: a context length outside [0, max_blocks * block_size] is clamped
// and sets EMBER_ERR_DECODE_CTX; a block id outside [0, num_blocks) reads block 0 and sets
// EMBER_ERR_BLOCK_ID. A zero context gives 0/0 = NaN rows, as the reference kernel does.
#include <atomic>
#include <mutex>

#include "ember_common.h"

namespace ember {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

template <typename T>
struct Mfma;
template <>
struct Mfma<_Float16> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x4 run(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mfma<__bf16> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x4 run(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kTile = 32;      // keys per tile (one P.V MFMA deep)
constexpr int kVtPad = 8;      // elements of padding per Vt row (keeps 16-byte alignment)

struct DecodeArgs {
  const void* q;
  int64_t q_sb, q_sh;          // elements
  void* out;
  int64_t o_sb, o_sh;
  const void* kc;
  const void* vc;
  int64_t k_sblk, k_sslot, k_sh;
  int64_t v_sblk, v_sslot, v_sh;
  const int32_t* bt;
  int64_t bt_sb;
  int32_t max_blocks;
  const int32_t* ctx;
  int32_t num_blocks;
  int32_t block_size;
  FastDiv bdiv;                // division by block_size
  int32_t nseq, nh, nkv, grp, hchunks;
  int32_t d;
  float scale2;                // scale * log2(e)
  int32_t splits;
  float* part_m;               // [splits][nseq][nh]
  float* part_l;
  float* part_o;               // [splits][nseq][nh][d]
  uint32_t* counters;          // [nseq][nh] split arrivals (MFMA kernel), zero between launches
  uint32_t* err;
};

#ifndef EMBER_DECODE_NT
#define EMBER_DECODE_NT 0
#endif

// K/V loads. Measured on MI355X (128 x 2048 keys, 8 KV heads, D=128): ordinary loads
// 5.4 TB/s, streaming (nt) loads 4.9 TB/s: the four dwordx4 instructions that cover one
// key row's 128-byte lines merge in the cache only when the lines are allocated.
template <typename T>
__device__ __forceinline__ Pack<T, 8> load_kv(const T* p) {
  if constexpr (EMBER_DECODE_NT) return load_stream<T, 8>(p);
  else return load_pack<T, 8>(p);
}

// s_waitcnt immediate for vmcnt(0) with expcnt and lgkmcnt left unconstrained (gfx9
// encoding: vmcnt[3:0] and [15:14], expcnt[6:4], lgkmcnt[11:8]).
constexpr int kWaitVmcnt0 = 0x0F70;

__device__ __forceinline__ void store_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_agent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float shfl_xor_f(float v, int mask) { return __shfl_xor(v, mask, kWave); }

// The context length of sequence b, clamped to what its block-table row can address.
__device__ __forceinline__ int seq_context(const DecodeArgs& a, int b) {
  int c = a.ctx[b];
  const int cap = a.max_blocks * a.block_size;
  if (c < 0 || c > cap) {
    if (threadIdx.x == 0) atomicOr(a.err, EMBER_ERR_DECODE_CTX);
    c = c < 0 ? 0 : cap;
  }
  return c;
}

// Physical block of logical block lb of sequence b (lb < max_blocks), checked.
__device__ __forceinline__ int phys_block(const DecodeArgs& a, const int32_t* btrow, int lb) {
  int p = btrow[lb];
  if (p < 0 || p >= a.num_blocks) {
    atomicOr(a.err, EMBER_ERR_BLOCK_ID);
    p = 0;
  }
  return p;
}

// Key-tile range [t0, t1) of split `split` (tiles of kTile keys), as every kernel here
// partitions it: the real context, not the table width, is split.
__device__ __forceinline__ void split_range(int ctx, int splits, int split, int& t0, int& t1) {
  const int nt = (ctx + kTile - 1) / kTile;
  const int per = (nt + splits - 1) / splits;
  t0 = split * per;
  t1 = min(t0 + per, nt);
}

// Tiles per loop iteration (KT) and next-iteration prefetch (PF) per head dim. Measured on
// MI355X: prefetch lifts D=128 from 5.35 to 5.6 TB/s (128 x 2048 keys, 8 KV heads).
#ifndef EMBER_DECODE_KT64
#define EMBER_DECODE_KT64 1
#endif
#ifndef EMBER_DECODE_PF64
#define EMBER_DECODE_PF64 1
#endif
#ifndef EMBER_DECODE_KT128
#define EMBER_DECODE_KT128 1
#endif
#ifndef EMBER_DECODE_PF128
#define EMBER_DECODE_PF128 1
#endif
#ifndef EMBER_DECODE_NW64
#define EMBER_DECODE_NW64 8
#endif
#ifndef EMBER_DECODE_NW128
#define EMBER_DECODE_NW128 4
#endif
// Waves per workgroup (each streams its own tiles of the workgroup's key range). At
// head_dim 128 a grid of at most half as many workgroups as CUs (a single sequence, a few
// KV heads) runs 8 waves per workgroup instead: twice the tile streams in flight per
// workgroup. Measured on MI355X, B = 1, 32q/8kv, ctx 8192, 16 splits (128 workgroups):
// 28.8 us with 4 waves, 24.6 us with 8 (16: 29.6). Full grids keep 4 (B = 8: 55.2 vs 56.5;
// B = 64: 188.5 vs 192.9).
constexpr int kWaves64 = EMBER_DECODE_NW64;
constexpr int kWaves128 = EMBER_DECODE_NW128;
constexpr int kWaves128Small = 8;

template <typename T, int D, int KT, bool PF, int NW>
__global__ void __launch_bounds__(NW * kWave)
k_decode_mfma(DecodeArgs a) {
  using M = Mfma<T>;
  using V8 = typename M::v8;
  constexpr int NP = D / 32;       // 16-byte packs per lane per key row (= QK MFMAs per half)
  constexpr int NDT = D / 16;      // d tiles of P.V
  constexpr int VS = D + kVtPad;   // LDS row stride of the V tile (elements)
  constexpr int CH = KT * NW;      // tiles between two chunks of one wave
  struct Combine {
    float m[NW][16];
    float l[NW][16];
    float o[NW][16][D + 4];
  };
  constexpr int kVtBytes = NW * KT * kTile * VS * int(sizeof(T));
  constexpr int kLdsBytes = kVtBytes > int(sizeof(Combine)) ? kVtBytes : int(sizeof(Combine));
  __shared__ __attribute__((aligned(16))) unsigned char lds[kLdsBytes];

  const int lane = threadIdx.x & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15;
  const int g = lane >> 4;

  int pid = blockIdx.x;
  const int hc = pid % a.hchunks;
  pid /= a.hchunks;
  const int kvh = pid % a.nkv;
  const int b = pid / a.nkv;
  const int split = blockIdx.y;
  const int head0 = kvh * a.grp + hc * 16;
  const int nhc = min(16, a.grp - hc * 16);

  const int ctx = seq_context(a, b);
  int t0, t1;
  split_range(ctx, a.splits, split, t0, t1);
  const int kend = min(t1 * kTile, ctx);  // keys of this split: [t0 * kTile, kend)

  // Q^T operand: head n of this chunk, d = 32c + 8g + [0, 8).
  V8 qv[NP];
  {
    const T* qp = static_cast<const T*>(a.q) + b * a.q_sb + int64_t(head0 + min(n, nhc - 1)) * a.q_sh + 8 * g;
#pragma unroll
    for (int c = 0; c < NP; ++c) {
      V8 v = __builtin_bit_cast(V8, load_pack<T, 8>(qp + 32 * c));
      if (n >= nhc) v = V8{};
      qv[c] = v;
    }
  }

  float m = -INFINITY;
  float lsum = 0.f;
  f32x4 o[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // The wave's V tiles: KT * 32 key rows (relative key order), row stride VS.
  T* vl = reinterpret_cast<T*>(lds) + w * (KT * kTile * VS);
  const T* kbase = static_cast<const T*>(a.kc) + kvh * a.k_sh + 8 * g;
  const T* vbase = static_cast<const T*>(a.vc) + kvh * a.v_sh + 8 * g;
  const int32_t* btrow = a.bt + b * a.bt_sb;
  // ds_read_b64_tr_b16 gives lane 4a+e of a 16-lane group element e of the 8 bytes that
  // lanes a, a+4, a+8, a+12 address. Lane n (a = n%4, jj = n/4) of group g therefore
  // addresses key row 16r + 4g + jj at d = 16dt + 4a, and lane (n, g) receives
  // V[16r + 4g + jj][16dt + n] for jj < 4: the A operand's kslots 8g + 4r + jj.
  const T* vtr = vl + (4 * g + (n >> 2)) * VS + 4 * (n & 3);

  // The wave's physical block ids, a window of WIN chunks at a time: lane 2(KT kk + u) + s
  // holds the block of half s of tile u of the wave's chunk kk of the window, so a chunk's
  // row loads never wait on a block-table read (one table read per WIN chunks instead of
  // one per chunk, which at a single sequence put two dependent round trips on every
  // chunk). Halves past the context point at the last valid half's block, as the row loads
  // below do; a wave without tiles reads no table entry.
  constexpr int WIN = kWave / (2 * KT);
  int blk_win = 0;
  auto load_window = [&](int k0w) {
    const int slot = lane >> 1;
    int hk = (t0 + KT * w + CH * (k0w + slot / KT) + slot % KT) * kTile + 16 * (lane & 1);
    if (hk >= ctx) hk = (ctx - 1) & ~15;
    if (hk < 0) hk = 0;
    const int lb = static_cast<int>(a.bdiv.div(static_cast<uint32_t>(hk)));
    blk_win = phys_block(a, btrow, lb);
  };

  // Loads of the wave's chunk k (KT tiles from tile tc): a half past the context still
  // loads (from the last valid half's block) so the loads stay unconditional; keys past the
  // split's range are masked after the scores.
  Pack<T, 8> kr[KT][2][NP];
  Pack<T, 8> vr[KT][2][NP];
  auto load_chunk = [&](int tc, int k) {
#pragma unroll
    for (int u = 0; u < KT; ++u)
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        int hk0 = (tc + u) * kTile + 16 * s;
        if (hk0 >= ctx) hk0 = (ctx - 1) & ~15;
        const int lb = static_cast<int>(a.bdiv.div(static_cast<uint32_t>(hk0)));
        const int pb = __builtin_amdgcn_readlane(blk_win, (((k % WIN) * KT + u) << 1) | s);
        const int slot = hk0 - lb * a.block_size + n;
        const T* kp = kbase + pb * a.k_sblk + slot * a.k_sslot;
        const T* vp = vbase + pb * a.v_sblk + slot * a.v_sslot;
#pragma unroll
        for (int c = 0; c < NP; ++c) kr[u][s][c] = load_kv<T>(kp + 32 * c);
#pragma unroll
        for (int c = 0; c < NP; ++c) vr[u][s][c] = load_kv<T>(vp + 32 * c);
      }
  };

  int tc = t0 + KT * w;
  int kc = 0;  // the wave's chunk index
  if (tc < t1) {
    load_window(0);
    if (PF) load_chunk(tc, 0);
  }
  for (; tc < t1; tc += CH, ++kc) {
    if (!PF) {
      if (kc > 0 && kc % WIN == 0) load_window(kc);
      load_chunk(tc, kc);
    }
    const int k0 = tc * kTile;
    const bool partial = k0 + KT * kTile > kend;  // wave-uniform

    // scores
    f32x4 sc[KT][2];
#pragma unroll
    for (int u = 0; u < KT; ++u)
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        sc[u][s] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NP; ++c) sc[u][s] = M::run(__builtin_bit_cast(V8, kr[u][s][c]), qv[c], sc[u][s]);
      }
    // V rows into the wave's tiles; rows past the split's range are stored as zero so that
    // stale cache contents cannot turn 0 * v into NaN.
    if (partial) {
#pragma unroll
      for (int u = 0; u < KT; ++u)
#pragma unroll
        for (int s = 0; s < 2; ++s)
          if (k0 + kTile * u + 16 * s + n >= kend)
#pragma unroll
            for (int c = 0; c < NP; ++c) vr[u][s][c] = Pack<T, 8>{};
    }
#pragma unroll
    for (int u = 0; u < KT; ++u)
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int c = 0; c < NP; ++c)
          store_pack<T, 8>(vl + (kTile * u + 16 * s + n) * VS + 32 * c + 8 * g, vr[u][s][c]);
    asm volatile("" ::: "memory");
    // K and V of this chunk are consumed (scores issued, V in LDS): the registers take the
    // wave's next chunk while this one's softmax and P.V run.
    if (PF && tc + CH < t1) {
      if ((kc + 1) % WIN == 0) load_window(kc + 1);
      load_chunk(tc + CH, kc + 1);
    }

    float x[KT][8];
#pragma unroll
    for (int u = 0; u < KT; ++u)
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int i = 0; i < 4; ++i) x[u][4 * s + i] = sc[u][s][i] * a.scale2;
    if (partial) {
#pragma unroll
      for (int u = 0; u < KT; ++u)
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (k0 + kTile * u + 16 * s + 4 * g + i >= kend) x[u][4 * s + i] = -INFINITY;
    }
    float mt = x[0][0];
#pragma unroll
    for (int u = 0; u < KT; ++u)
#pragma unroll
      for (int j = 0; j < 8; ++j) mt = fmaxf(mt, x[u][j]);
    mt = fmaxf(mt, shfl_xor_f(mt, 16));
    mt = fmaxf(mt, shfl_xor_f(mt, 32));
    // Rescale only when some head's running max grew (alpha = 1 exactly otherwise).
    if (__any(mt > m)) {
      const float mn = fmaxf(m, mt);
      const float alpha = exp2_fast(m - mn);
      m = mn;
      lsum *= alpha;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) o[dt] *= alpha;
    }
#pragma unroll
    for (int u = 0; u < KT; ++u) {
      V8 pb;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float p = exp2_fast(x[u][j] - m);
        lsum += p;
        pb[j] = from_f32<T>(p);
      }
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        typedef short v4s __attribute__((ext_vector_type(4)));
        typedef __attribute__((address_space(3))) v4s* lds_v4s;
        const T* src = vtr + kTile * u * VS + 16 * dt;
        const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(src));
        const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(src + 16 * VS));
        typedef short v8s __attribute__((ext_vector_type(8)));
        const v8s va = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        o[dt] = M::run(__builtin_bit_cast(V8, va), pb, o[dt]);
      }
    }
    asm volatile("" ::: "memory");
  }

  // merge the waves
  lsum += shfl_xor_f(lsum, 16);
  lsum += shfl_xor_f(lsum, 32);
  __syncthreads();
  Combine& cb = *reinterpret_cast<Combine*>(lds);
  if (g == 0) {
    cb.m[w][n] = m;
    cb.l[w][n] = lsum;
  }
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i) cb.o[w][n][16 * dt + 4 * g + i] = o[dt][i];
  __syncthreads();

  // PARTS threads per head; thread p of a head owns d = VEC p + VEC PARTS j + [0, VEC),
  // j < NJ, so each j of a head's threads is one contiguous run of VEC PARTS floats: whole
  // lines for the partial stores and loads below.
  constexpr int PARTS = NW * kWave / 16;
  constexpr int PER = D / PARTS;           // d values per thread
  constexpr int VEC = PER < 4 ? PER : 4;   // floats per access
  constexpr int NJ = PER / VEC;
  static_assert(VEC == 2 || VEC == 4, "merge layout");
  using FV = typename FloatVec<VEC>::type;
  const int hh = threadIdx.x / PARTS;
  const int pv = (threadIdx.x % PARTS) * VEC;
  const bool mine = hh < nhc;
  const int head = head0 + hh;
  float mx = -INFINITY;
  float L = 0.f;
  FV acc[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) acc[j] = FV{};
  if (mine) {
    float mw[NW];
#pragma unroll
    for (int v = 0; v < NW; ++v) {
      mw[v] = cb.m[v][hh];
      mx = fmaxf(mx, mw[v]);
    }
#pragma unroll
    for (int v = 0; v < NW; ++v) {
      const float wt = mw[v] == -INFINITY ? 0.f : exp2_fast(mw[v] - mx);
      L += wt * cb.l[v][hh];
#pragma unroll
      for (int j = 0; j < NJ; ++j) acc[j] += wt * *reinterpret_cast<const FV*>(&cb.o[v][hh][pv + VEC * PARTS * j]);
    }
  }
  T* orow = static_cast<T*>(a.out) + b * a.o_sb + head * a.o_sh + pv;
  auto store_out = [&](float l) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      Pack<T, VEC> r;
#pragma unroll
      for (int e = 0; e < VEC; ++e) r.v[e] = from_f32<T>(acc[j][e] / l);
      store_pack<T, VEC>(orow + VEC * PARTS * j, r);
    }
  };
  if (a.splits == 1) {
    if (mine) store_out(L);
    return;
  }

  // Split-K: publish this split's partial, then the last split of this (sequence, head
  // chunk) to arrive merges all of them (paged_triton.py:188-209 as a kernel epilogue, so
  // no second launch). The arrival counter returns to zero for the next launch.
  // Coherence across the XCDs' separate L2s without writing back whole caches: partials
  // go out as agent-coherent (sc1, written-through) stores, the counter is bumped only
  // after they have completed (s_waitcnt vmcnt(0)), and the merging workgroup reads them
  // with agent-coherent loads. The chunk's partial rows of one split are contiguous, so one
  // buffer resource (uniform base, exact size) addresses them.
  const int64_t stride = int64_t(a.nseq) * a.nh;
  const int64_t row0 = int64_t(b) * a.nh + head0;
  if (mine) {
    if (threadIdx.x % PARTS == 0) {
      store_agent(a.part_m + split * stride + row0 + hh, mx);
      store_agent(a.part_l + split * stride + row0 + hh, L);
    }
    const CoherentRsrc rs = coherent_rsrc(a.part_o + (split * stride + row0) * D, nhc * D);
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      store_coherent<VEC>(rs, (hh * D + pv + VEC * PARTS * j) * int(sizeof(float)), acc[j]);
  }
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
  // partial), so a chunk costs one round trip. The running max moves per chunk; with one
  // chunk the sums are formed in the same order as a two-pass merge.
  const int hr = min(hh, nhc - 1);  // padded heads read a real row and store nothing
  const int roff = (hr * D + pv) * int(sizeof(float));
  // 8 splits per chunk: a 16-split chunk's registers (16 x (2 + floats per split)) raised
  // the D = 64 kernel from 97 to 141 VGPRs and cut its occupancy (B = 128 x 2048 at 32
  // splits: 75.5 -> 126.6 us)
  constexpr int kMergeChunk = 8;
  float gm = -INFINITY;
  float gl = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; ++j) acc[j] = FV{};
  for (int c0 = 0; c0 < a.splits; c0 += kMergeChunk) {
    const int cn = min(kMergeChunk, a.splits - c0);
    float ms[kMergeChunk], ls[kMergeChunk];
    FV v[kMergeChunk][NJ];
#pragma unroll
    for (int u = 0; u < kMergeChunk; ++u) {
      ms[u] = -INFINITY;
      ls[u] = 0.f;
#pragma unroll
      for (int j = 0; j < NJ; ++j) v[u][j] = FV{};
      if (u < cn) {  // uniform
        const int sp = c0 + u;
        const int64_t r = sp * stride + row0 + hr;
        ms[u] = load_agent(a.part_m + r);
        ls[u] = load_agent(a.part_l + r);
        const CoherentRsrc rs = coherent_rsrc(a.part_o + (sp * stride + row0) * D, nhc * D);
#pragma unroll
        for (int j = 0; j < NJ; ++j) v[u][j] = load_coherent<VEC>(rs, roff + VEC * PARTS * j * int(sizeof(float)));
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

// Any geometry: one wave per (sequence, query head, split), fp32 math.
template <typename TQ, typename TC>
__global__ void __launch_bounds__(kWave)
k_decode_any(DecodeArgs a) {
  __shared__ float qs[256];
  __shared__ float ps[kWave];
  __shared__ int64_t rows[kWave];
  const int lane = threadIdx.x;
  int pid = blockIdx.x;
  const int h = pid % a.nh;
  const int b = pid / a.nh;
  const int split = blockIdx.y;
  const int kvh = h / a.grp;
  const int D = a.d;
  const int ctx = seq_context(a, b);
  int t0, t1;
  split_range(ctx, a.splits, split, t0, t1);
  const int kbeg = t0 * kTile;
  const int kend = min(t1 * kTile, ctx);

  const TQ* qp = static_cast<const TQ*>(a.q) + b * a.q_sb + h * a.q_sh;
  for (int e = lane; e < D; e += kWave) qs[e] = to_f32(qp[e]) * a.scale2;
  __syncthreads();

  const TC* kc = static_cast<const TC*>(a.kc) + kvh * a.k_sh;
  const TC* vc = static_cast<const TC*>(a.vc) + kvh * a.v_sh;
  const int32_t* btrow = a.bt + b * a.bt_sb;
  float m = -INFINITY, l = 0.f;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};  // d = lane + 64 j
  for (int kk = kbeg; kk < kend; kk += kWave) {
    const int key = kk + lane;
    const bool valid = key < kend;
    float s = -INFINITY;
    int64_t krow = 0, vrow = 0;
    if (valid) {
      const int lb = static_cast<int>(a.bdiv.div(static_cast<uint32_t>(key)));
      const int pb = phys_block(a, btrow, lb);
      const int slot = key - lb * a.block_size;
      krow = pb * a.k_sblk + slot * a.k_sslot;
      vrow = pb * a.v_sblk + slot * a.v_sslot;
      float dot = 0.f;
      for (int e = 0; e < D; ++e) dot += qs[e] * to_f32(kc[krow + e]);
      s = dot;
    }
    float mt = s;
    for (int off = 32; off >= 1; off >>= 1) mt = fmaxf(mt, shfl_xor_f(mt, off));
    const float mn = fmaxf(m, mt);
    const float alpha = exp2_fast(m - mn);
    m = mn;
    const float p = valid ? exp2_fast(s - mn) : 0.f;
    float ps_sum = p;
    for (int off = 32; off >= 1; off >>= 1) ps_sum += shfl_xor_f(ps_sum, off);
    l = l * alpha + ps_sum;
    __syncthreads();
    ps[lane] = p;
    rows[lane] = vrow;
    __syncthreads();
    const int nk = min(kWave, kend - kk);
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] *= alpha;
    for (int r = 0; r < nk; ++r) {
      const float pr = ps[r];
      const TC* vrp = vc + rows[r];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int e = lane + kWave * j;
        if (e < D) acc[j] += pr * to_f32(vrp[e]);
      }
    }
  }
  if (a.splits == 1) {
    TQ* op = static_cast<TQ*>(a.out) + b * a.o_sb + h * a.o_sh;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = lane + kWave * j;
      if (e < D) op[e] = from_f32<TQ>(acc[j] / l);
    }
  } else {
    const int64_t row = (int64_t(split) * a.nseq + b) * a.nh + h;
    if (lane == 0) {
      a.part_m[row] = m;
      a.part_l[row] = l;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = lane + kWave * j;
      if (e < D) a.part_o[row * D + e] = acc[j];
    }
  }
}

// Merge of the split-K partials (paged_triton.py:188-209): one wave per (sequence, head).
template <typename TO>
__global__ void __launch_bounds__(256)
k_decode_reduce(const float* __restrict__ pm, const float* __restrict__ pl, const float* __restrict__ po,
                int splits, int nseq, int nh, int d, TO* __restrict__ out, int64_t o_sb, int64_t o_sh) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= nseq * nh) return;
  const int lane = threadIdx.x & (kWave - 1);
  const int b = row / nh;
  const int h = row - b * nh;
  float mx = -INFINITY;
  for (int s = 0; s < splits; ++s) mx = fmaxf(mx, pm[int64_t(s) * nseq * nh + row]);
  float L = 0.f;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < splits; ++s) {
    const int64_t r = int64_t(s) * nseq * nh + row;
    const float ms = pm[r];
    const float wt = ms == -INFINITY ? 0.f : exp2_fast(ms - mx);
    L += wt * pl[r];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = lane + kWave * j;
      if (e < d) acc[j] += wt * po[r * d + e];
    }
  }
  TO* op = out + b * o_sb + h * o_sh;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = lane + kWave * j;
    if (e < d) op[e] = from_f32<TO>(acc[j] / L);
  }
}

template <typename TQ>
int launch_any_q(int cdt, const DecodeArgs& a, dim3 grid, hipStream_t st) {
  switch (cdt) {
    case EMBER_F32: k_decode_any<TQ, float><<<grid, kWave, 0, st>>>(a); break;
    case EMBER_F16: k_decode_any<TQ, _Float16><<<grid, kWave, 0, st>>>(a); break;
    case EMBER_BF16: k_decode_any<TQ, __bf16><<<grid, kWave, 0, st>>>(a); break;
    default: return EMBER_EINVAL;
  }
  return EMBER_OK;
}

template <typename T>
int launch_mfma(int d, int nw, const DecodeArgs& a, dim3 grid, hipStream_t st) {
  if (d == 64) {
    k_decode_mfma<T, 64, EMBER_DECODE_KT64, EMBER_DECODE_PF64 != 0, kWaves64>
        <<<grid, kWaves64 * kWave, 0, st>>>(a);
  } else if (nw == kWaves128Small) {
    k_decode_mfma<T, 128, EMBER_DECODE_KT128, EMBER_DECODE_PF128 != 0, kWaves128Small>
        <<<grid, kWaves128Small * kWave, 0, st>>>(a);
  } else {
    k_decode_mfma<T, 128, EMBER_DECODE_KT128, EMBER_DECODE_PF128 != 0, kWaves128>
        <<<grid, kWaves128 * kWave, 0, st>>>(a);
  }
  return EMBER_OK;
}

template <typename TO>
void launch_reduce(const DecodeArgs& a, hipStream_t st) {
  const int rows = a.nseq * a.nh;
  k_decode_reduce<TO><<<(rows + 3) / 4, 256, 0, st>>>(a.part_m, a.part_l, a.part_o, a.splits, a.nseq, a.nh, a.d,
                                                      static_cast<TO*>(a.out), a.o_sb, a.o_sh);
}

}  // namespace
}  // namespace ember

using namespace ember;

extern "C" {

int64_t ember_paged_decode_workspace_bytes(int64_t num_seqs, int64_t num_heads, int64_t head_dim,
                                           int64_t num_splits) {
  if (num_seqs < 0 || num_heads < 0 || head_dim < 0 || num_splits < 1) return -1;
  if (num_splits == 1) return 0;
  const int64_t partials = num_splits * num_seqs * num_heads * (head_dim + 2) * int64_t(sizeof(float));
  return partials + (num_seqs * num_heads * int64_t(sizeof(uint32_t)) + 15) / 16 * 16;
}

}  // extern "C"

namespace ember {
namespace {

// ember_paged_decode's body. `counters` (when non-null) replaces the arrival counters at the
// end of the workspace: the no-allocation entry point keeps them at a fixed place, so that
// calls of different shapes always find them at zero.
int paged_decode_core(const void* q, int64_t q_seq_stride, int64_t q_head_stride, int q_dtype,
                      const void* k_cache, const void* v_cache, int64_t num_blocks, int64_t block_size,
                      int64_t num_kv_heads, int64_t head_dim, int64_t k_block_stride, int64_t k_slot_stride,
                      int64_t k_head_stride, int64_t v_block_stride, int64_t v_slot_stride,
                      int64_t v_head_stride, int cache_dtype, const int32_t* block_tables,
                      int64_t block_table_stride, int64_t max_blocks, const int32_t* context_lens,
                      int64_t num_seqs, int64_t num_heads, float scale, int64_t num_splits, int flags,
                      void* workspace, int64_t workspace_bytes, uint32_t* counters, void* out,
                      int64_t out_seq_stride, int64_t out_head_stride, void* stream) {
  const int qsz = dtype_size(q_dtype);
  const int csz = dtype_size(cache_dtype);
  if (qsz == 0 || csz == 0) return EMBER_EINVAL;
  if (num_seqs < 0 || num_heads < 1 || num_kv_heads < 1 || num_heads % num_kv_heads != 0) return EMBER_EINVAL;
  if ((flags & ~EMBER_DECODE_FP32) != 0) return EMBER_EINVAL;
  if (head_dim < 1 || head_dim > 256 || block_size < 16 || block_size % 16 != 0) return EMBER_EINVAL;
  if (num_blocks < 1 || max_blocks < 1 || num_splits < 1 || num_splits > 1024) return EMBER_EINVAL;
  if (max_blocks * block_size > INT32_MAX || num_blocks > INT32_MAX) return EMBER_EINVAL;
  if (num_seqs == 0) return EMBER_OK;
  if (!q || !k_cache || !v_cache || !block_tables || !context_lens || !out) return EMBER_EINVAL;
  if (num_seqs * num_heads > INT32_MAX / 2) return EMBER_EINVAL;
  const int64_t need = ember_paged_decode_workspace_bytes(num_seqs, num_heads, head_dim, num_splits);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need || (reinterpret_cast<uintptr_t>(workspace) & 15)))
    return EMBER_EINVAL;
  uint32_t* err = device_error_word();
  if (err == nullptr) return EMBER_ENODEV;

  DecodeArgs a{};
  a.q = q;
  a.q_sb = q_seq_stride;
  a.q_sh = q_head_stride;
  a.out = out;
  a.o_sb = out_seq_stride;
  a.o_sh = out_head_stride;
  a.kc = k_cache;
  a.vc = v_cache;
  a.k_sblk = k_block_stride;
  a.k_sslot = k_slot_stride;
  a.k_sh = k_head_stride;
  a.v_sblk = v_block_stride;
  a.v_sslot = v_slot_stride;
  a.v_sh = v_head_stride;
  a.bt = block_tables;
  a.bt_sb = block_table_stride;
  a.max_blocks = static_cast<int32_t>(max_blocks);
  a.ctx = context_lens;
  a.num_blocks = static_cast<int32_t>(num_blocks);
  a.block_size = static_cast<int32_t>(block_size);
  a.bdiv = FastDiv::make(static_cast<uint32_t>(block_size));
  a.nseq = static_cast<int32_t>(num_seqs);
  a.nh = static_cast<int32_t>(num_heads);
  a.nkv = static_cast<int32_t>(num_kv_heads);
  a.grp = static_cast<int32_t>(num_heads / num_kv_heads);
  a.hchunks = static_cast<int32_t>(cdiv(a.grp, 16));
  a.d = static_cast<int32_t>(head_dim);
  a.scale2 = scale * kLog2e;
  a.splits = static_cast<int32_t>(num_splits);
  if (need > 0) {
    float* ws = static_cast<float*>(workspace);
    const int64_t rows = num_splits * num_seqs * num_heads;
    a.part_m = ws;
    a.part_l = ws + rows;
    a.part_o = ws + 2 * rows;
    a.counters = counters != nullptr ? counters : reinterpret_cast<uint32_t*>(ws + rows * (head_dim + 2));
  }
  a.err = err;
  hipStream_t st = static_cast<hipStream_t>(stream);

  // The MFMA kernel's 16-byte q/K/V loads and D/16-element output stores need the
  // corresponding alignment; anything else runs the fp32 kernel.
  const bool same = q_dtype == cache_dtype && q_dtype != EMBER_F32 && !(flags & EMBER_DECODE_FP32);
  const bool dok = head_dim == 64 || head_dim == 128;
  const int64_t progs = num_seqs * num_kv_heads * a.hchunks;
  const int ncu = device_cu_count();
  const bool small_grid = head_dim == 128 && ncu > 0 && progs * num_splits * 2 <= ncu;
  const int nw = head_dim == 64 ? kWaves64 : (small_grid ? kWaves128Small : kWaves128);
  const int64_t out_align_elems = std::min<int64_t>(4, head_dim / (nw * kWave / 16));  // the merge's store width
  const bool aligned = aligned16(q) && aligned16(k_cache) && aligned16(v_cache) && q_seq_stride % 8 == 0 &&
                       q_head_stride % 8 == 0 && k_block_stride % 8 == 0 && k_slot_stride % 8 == 0 &&
                       k_head_stride % 8 == 0 && v_block_stride % 8 == 0 && v_slot_stride % 8 == 0 &&
                       v_head_stride % 8 == 0 &&
                       (reinterpret_cast<uintptr_t>(out) % (out_align_elems * 2)) == 0 &&
                       out_seq_stride % out_align_elems == 0 && out_head_stride % out_align_elems == 0;
  int rc = EMBER_OK;
  const bool mfma = same && dok && aligned;
  if (mfma) {
    if (progs > INT32_MAX) return EMBER_EINVAL;
    dim3 grid(static_cast<uint32_t>(progs), static_cast<uint32_t>(num_splits));
    rc = q_dtype == EMBER_F16 ? launch_mfma<_Float16>(a.d, nw, a, grid, st)
                              : launch_mfma<__bf16>(a.d, nw, a, grid, st);
  } else {
    dim3 grid(static_cast<uint32_t>(num_seqs * num_heads), static_cast<uint32_t>(num_splits));
    switch (q_dtype) {
      case EMBER_F32: rc = launch_any_q<float>(cache_dtype, a, grid, st); break;
      case EMBER_F16: rc = launch_any_q<_Float16>(cache_dtype, a, grid, st); break;
      default: rc = launch_any_q<__bf16>(cache_dtype, a, grid, st); break;
    }
  }
  if (rc != EMBER_OK) return rc;
  if (num_splits > 1 && !mfma) {
    switch (q_dtype) {
      case EMBER_F32: launch_reduce<float>(a, st); break;
      case EMBER_F16: launch_reduce<_Float16>(a, st); break;
      default: launch_reduce<__bf16>(a, st); break;
    }
  }
  return launch_status();
}

}  // namespace
}  // namespace ember

extern "C" {

int ember_paged_decode(const void* q, int64_t q_seq_stride, int64_t q_head_stride, int q_dtype,
                       const void* k_cache, const void* v_cache, int64_t num_blocks, int64_t block_size,
                       int64_t num_kv_heads, int64_t head_dim, int64_t k_block_stride, int64_t k_slot_stride,
                       int64_t k_head_stride, int64_t v_block_stride, int64_t v_slot_stride,
                       int64_t v_head_stride, int cache_dtype, const int32_t* block_tables,
                       int64_t block_table_stride, int64_t max_blocks, const int32_t* context_lens,
                       int64_t num_seqs, int64_t num_heads, float scale, int64_t num_splits, int flags,
                       void* workspace, int64_t workspace_bytes, void* out, int64_t out_seq_stride,
                       int64_t out_head_stride, void* stream) {
  return paged_decode_core(q, q_seq_stride, q_head_stride, q_dtype, k_cache, v_cache, num_blocks, block_size,
                           num_kv_heads, head_dim, k_block_stride, k_slot_stride, k_head_stride, v_block_stride,
                           v_slot_stride, v_head_stride, cache_dtype, block_tables, block_table_stride, max_blocks,
                           context_lens, num_seqs, num_heads, scale, num_splits, flags, workspace, workspace_bytes,
                           nullptr, out, out_seq_stride, out_head_stride, stream);
}

}  // extern "C"

// ---------------------------------------------------------------- the no-allocation variant
//
// ember_paged_decode_noalloc keeps its split-K partials and arrival counters in `scratch`, a
// file-scope device array of kNoAllocScratchBytes that every GPU the library runs on holds
// until the process ends. The host-side name of the array is not a device address: its
// address on each device comes from hipGetSymbolAddress, resolved once per device with that
// device current, and only that address reaches kernels. The arrival counters sit at the
// array's start, at the same place for every shape, and the partials after them. The array
// is cleared by a fill kernel once per device (the counters must start at zero); every call
// leaves the counters it used at zero again, and calls that overlap on one GPU share the
// array and race.
namespace ember {
namespace {

constexpr int64_t kNoAllocScratchBytes = int64_t(16) << 20;
constexpr int64_t kNoAllocCounterBytes = int64_t(1) << 20;  // arrival counters: 256 Ki (sequence, head) rows
constexpr int kNoAllocMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

std::atomic<void*> g_scratch_addr[kNoAllocMaxDevices];
std::mutex g_scratch_init;

__global__ void __launch_bounds__(256) k_zero_words(uint32_t* p, int64_t n) {
  for (int64_t i = blockIdx.x * int64_t(256) + threadIdx.x; i < n; i += int64_t(gridDim.x) * 256) p[i] = 0u;
}

// The current device's address of `scratch`, cleared on first use (on `st`); null on failure.
void* scratch_address(hipStream_t st) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kNoAllocMaxDevices) return nullptr;
  void* p = g_scratch_addr[dev].load(std::memory_order_acquire);
  if (p != nullptr) return p;
  std::lock_guard<std::mutex> lock(g_scratch_init);
  p = g_scratch_addr[dev].load(std::memory_order_acquire);
  if (p != nullptr) return p;
  void* addr = nullptr;
  if (hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch)) != hipSuccess || addr == nullptr) return nullptr;
  k_zero_words<<<1024, 256, 0, st>>>(static_cast<uint32_t*>(addr), kNoAllocScratchBytes / 4);
  if (hipGetLastError() != hipSuccess) return nullptr;
  g_scratch_addr[dev].store(addr, std::memory_order_release);
  return addr;
}

}  // namespace
}  // namespace ember

extern "C" {

int64_t ember_paged_decode_noalloc_max_bytes(void) {
  return ember::kNoAllocScratchBytes - ember::kNoAllocCounterBytes;
}

int ember_paged_decode_noalloc(const void* q, int64_t q_seq_stride, int64_t q_head_stride, int q_dtype,
                               const void* k_cache, const void* v_cache, int64_t num_blocks, int64_t block_size,
                               int64_t num_kv_heads, int64_t head_dim, int64_t k_block_stride,
                               int64_t k_slot_stride, int64_t k_head_stride, int64_t v_block_stride,
                               int64_t v_slot_stride, int64_t v_head_stride, int cache_dtype,
                               const int32_t* block_tables, int64_t block_table_stride, int64_t max_blocks,
                               const int32_t* context_lens, int64_t num_seqs, int64_t num_heads, float scale,
                               int64_t num_splits, int flags, void* out, int64_t out_seq_stride,
                               int64_t out_head_stride, void* stream) {
  const int64_t need = ember_paged_decode_workspace_bytes(num_seqs, num_heads, head_dim, num_splits);
  if (need < 0) return EMBER_EINVAL;
  // counters at the array's start (fixed, whatever the shape), partials after them
  if (need > ember::kNoAllocScratchBytes - ember::kNoAllocCounterBytes ||
      num_seqs * num_heads * int64_t(sizeof(uint32_t)) > ember::kNoAllocCounterBytes)
    return EMBER_ETOOBIG;
  unsigned char* base = nullptr;
  if (need > 0 && num_seqs > 0) {
    base = static_cast<unsigned char*>(ember::scratch_address(static_cast<hipStream_t>(stream)));
    if (base == nullptr) return EMBER_ENODEV;
  }
  return ember::paged_decode_core(
      q, q_seq_stride, q_head_stride, q_dtype, k_cache, v_cache, num_blocks, block_size, num_kv_heads, head_dim,
      k_block_stride, k_slot_stride, k_head_stride, v_block_stride, v_slot_stride, v_head_stride, cache_dtype,
      block_tables, block_table_stride, max_blocks, context_lens, num_seqs, num_heads, scale, num_splits, flags,
      base != nullptr ? base + ember::kNoAllocCounterBytes : nullptr,
      base != nullptr ? ember::kNoAllocScratchBytes - ember::kNoAllocCounterBytes : 0,
      reinterpret_cast<uint32_t*>(base), out, out_seq_stride, out_head_stride, stream);
}

}  // extern "C"
