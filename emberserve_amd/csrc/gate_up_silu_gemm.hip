// Prefill-size gate_up projection with silu_and_mul as its epilogue, for gfx950:
//   out[t, j] = round(round(silu(g)) * u),  g = round(x[t] . W[j]),  u = round(x[t] . W[I + j])
// for t < T, j < I, with W [2I, H] the nn.Linear(H, 2I) weight (gate rows, then up rows).
//
// Reference: Qwen2MLP.forward, emberserve/model/qwen2.py:60-61 (gate_up_proj, then
// ops.silu_and_mul), where the [T, 2I] projection is written and read back. Here it never
// leaves the chip: each workgroup computes a BM-token x (BNG gate + BNG up) column tile with
// bf16/fp16 MFMA (v_mfma_f32_16x16x32) and writes only the [BM, BNG] activation tile. Tiles:
// 256 x 64, 256 x 96 (the last one ragged when 96 does not divide I), 256 x 128, 128 x 128.
//
// Structure:
//   * 8 waves in BM / 64 token groups x 8 / (BM / 64) column groups: each owns 64 tokens of
//     the tile and WC = BNG BM / 512 columns of both the gate and the up half, so it holds
//     (2 WC / 16) x 4 accumulator tiles of 16 x 16;
//   * the tile's operands stream through an LDS ring of "double stages" of 64 k (three for
//     the 256 x 64 and 128 x 128 tiles; for 256 x 96 and 256 x 128, where three would not fit, separate
//     rings of three weight and two x buffers, 160 KiB: 94 instead of 102 us for Qwen3-8B
//     at 256 tokens, the same at 8192): rows of 128
//     bytes (one 64-k line per row), so each direct-to-LDS load (global_load_lds_dwordx4)
//     moves 8 rows x 128 B; 16-byte chunks XOR-swizzled by row & 7 so the fragment reads
//     (one row per lane) spread over the banks. At 256 tokens each workgroup streams its
//     weight rows from HBM once, and the third buffer (two double stages in flight) took the
//     Qwen3-8B call from 91.7 to 70.0 us;
//   * ping-pong: the two waves of each SIMD belong to different groups (grp), and group 1
//     starts one barrier late, so between two barriers one group reads fragments and issues
//     loads while the other runs its MFMAs;
//   * XCD-aware tile order: consecutive workgroups land on different XCDs (round robin), so
//     the order is remapped to give each XCD a contiguous range of tiles, grouped GROUP_M
//     token tiles at a time over a band of column tiles (their weight rows stay in that
//     XCD's L2).
// The k order of every accumulator is the decode kernels' (32-k steps in order, one chain),
// so a token's result is bit-identical to ember_gate_up_silu_packed over whole-slab runs.
// The epilogue is the decode kernels' exact one (expf and a division); v_exp_f32 / v_rcp_f32
// measured 3% faster at 8192 tokens and would give up that identity.
//
// Measured on MI355X (bf16, µs; this kernel at the better column tile / hipBLASLt +
// silu_and_mul): Qwen3-8B 256 tokens 70.0 / 72.6, 8192 tokens 1286 / 1235; Qwen2.5-7B 256
// tokens 110 / 88.5, 8192 tokens 1791 / 1834. The library therefore keeps the unfused pair
// by default at these sizes and runs this kernel when the fused form is asked for.
#include "ember_common.h"

#ifndef EMBER_GEMM_GROUP_M
#define EMBER_GEMM_GROUP_M 8
#endif
// Double-stage buffers of the 64-column tile (the 128-column tile's two fill 128 KiB).
#ifndef EMBER_GEMM_SPLIT_RING
#define EMBER_GEMM_SPLIT_RING 1
#endif
#ifndef EMBER_GEMM_NBUF64
#define EMBER_GEMM_NBUF64 3
#endif

namespace ember {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

template <typename T>
struct GemmMfma;
template <>
struct GemmMfma<_Float16> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x4 run(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};
template <>
struct GemmMfma<__bf16> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x4 run(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

constexpr int kGemmRowB = 128;  // LDS row: 64 k of one operand row

__device__ __forceinline__ void gemm_load_lds16(const void* gptr, void* lds_base) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_global_load_lds(gptr, (__attribute__((address_space(3))) void*)(
                                             reinterpret_cast<uintptr_t>(lds_base)), 16, 0, 0);
#else
  (void)gptr;
  (void)lds_base;
#endif
}

// s_waitcnt vmcnt(N) / lgkmcnt(0) alone (gfx9 encoding).
template <int N>
__device__ __forceinline__ void gemm_wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
__device__ __forceinline__ void gemm_wait_vm0() { gemm_wait_vm<0>(); }
__device__ __forceinline__ void gemm_wait_lgkm0() { __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4)); }

// A workgroup barrier with no fence (the waits above are explicit); the asm clobbers keep
// the compiler from moving LDS accesses across it.
__device__ __forceinline__ void gemm_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

struct GemmArgs {
  const void* x;
  int64_t xs;
  const void* w;
  int64_t ws;
  void* out;
  int64_t os;
  int T, H, I;
  // routed experts (MOE kernels only): token tiles are BM-assignment blocks of the
  // block-aligned layout; block b's rows are assignments sorted_ids[b BM + r] (padding:
  // >= num_valid) of expert block_expert[b], x row = assignment / top_k, output row = the
  // assignment; wes = elements between experts' [2I, H] weights
  const int32_t* sorted_ids;
  const int32_t* block_expert;
  int num_valid, top_k, E, ntok;
  int64_t wes;
  uint32_t* err;  // MOE: EMBER_ERR_ROW_INDEX for a valid assignment whose token is >= ntok
  // packed weights (PK kernels only): w is the decode kernels' packed array for a grid of
  // pk_G workgroups over pk_total units (pk_total = (I / 64) (H / 64))
  int64_t pk_total, pk_G;
};

// Walks the packed units of one 64-row slab, u = slab * nk + j for j = 0, 1, ...: the unit's
// place in the packed array, tracking its owner workgroup b and b's run [start, next)
// incrementally (a division only where the walk crosses into the next run).
struct PackedSlabWalk {
  int64_t u, last, b, start, next, q, total, G;
  __device__ void init(int64_t slab, int64_t nk, int64_t total_, int64_t G_) {
    total = total_;
    G = G_;
    q = total / G;
    u = slab * nk;
    last = u + nk - 1;
    b = gu_owner(u, total, G);
    start = gu_start(b, total, G);
    next = gu_start(b + 1, total, G);
  }
  // the unit's element offset (16 KiB units)
  template <typename T>
  __device__ int64_t elem_offset() const {
    const int64_t t = u - start;
    const int64_t pos = t < q ? t * G + b : q * G + (start - b * q);
    return pos * (16384 / static_cast<int64_t>(sizeof(T)));
  }
  __device__ void advance() {  // past the slab's last unit it stays there
    if (u == last) return;
    ++u;
    if (u >= next) {
      ++b;
      start = next;
      next = gu_start(b + 1, total, G);
    }
  }
};

template <typename T, int BNG, int BM, bool MOE, bool PK = false>
__global__ void __launch_bounds__(512, 1)
k_gate_up_silu_gemm(GemmArgs a) {
  static_assert(!PK || BNG % 64 == 0, "packed tiles are whole 64-row slabs");
  using M = GemmMfma<T>;
  using V8 = typename M::v8;
  static_assert((BM == 256 && (BNG == 64 || BNG == 96 || BNG == 128)) || (BM == 128 && BNG == 128), "tile");
  constexpr int TG = BM / 64;                  // token groups of 64
  constexpr int WC = BNG * TG / 8;             // gate (and up) columns per wave
  constexpr int NT = 2 * WC / 16;              // row tiles per wave: NT / 2 gate, NT / 2 up
  constexpr int WREG = 2 * BNG * kGemmRowB;    // weight region of a double stage
  constexpr int XREG = BM * kGemmRowB;         // x region
  constexpr int DST = WREG + XREG;             // one double stage (64 k)
  constexpr int LOADS = (2 * BNG + BM) / 8 / 8;  // 1 KiB load instructions per wave per double stage
  // Double-stage buffers: NBUF - 1 double stages of loads in flight while one is consumed.
  constexpr int NBUF = 3 * DST <= 160 * 1024 ? EMBER_GEMM_NBUF64 : 2;
  // SPLIT: when three double stages do not fit, the operands get rings of their own: three
  // weight buffers (HBM latency) and two x buffers (mostly L2 hits), 160 KiB in all. Each
  // wave then loads WL weight blocks and LOADS - WL x blocks per double stage.
  constexpr bool SPLIT = EMBER_GEMM_SPLIT_RING != 0 && NBUF == 2 && 3 * WREG + 2 * XREG <= 160 * 1024;
  constexpr int WL = SPLIT ? 2 * BNG / 8 / 8 : 0;
  constexpr int LDS_BYTES = SPLIT ? 3 * WREG + 2 * XREG : NBUF * DST;
  static_assert(LDS_BYTES <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(1024))) unsigned char lds[LDS_BYTES];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = w >> 2;    // ping-pong group: waves w and w + 4 share a SIMD
  const int q = w % TG;      // token group
  const int cg = w / TG;     // column group
  const int n = lane & 15, g = lane >> 4;

  // XCD-aware tile order, then GROUP_M token tiles per band of column tiles
  int mtiles = (a.T + BM - 1) / BM;
  const int ntiles = (a.I + BNG - 1) / BNG;  // the last one ragged when BNG does not divide I
  int pid = blockIdx.x;
  int nb = gridDim.x;
  if (MOE) {
    // The grid covers every block the layout may use, but only the blocks before the first
    // one past the last expert hold work (block_expert is ascending, num_experts after the
    // used blocks). Counted here (one coalesced read of the small table, the same for every
    // workgroup) so that the XCD ranges below split the real tiles evenly instead of
    // leaving the unused blocks' share of the chip idle.
    int used = 0;
    for (int i0 = 0; i0 < mtiles; i0 += kWave) {
      const int i = i0 + lane;
      const bool u = i < mtiles && a.block_expert[i] < a.E;
      used += __builtin_popcountll(__ballot(u));
    }
    mtiles = used;
    nb = used * ntiles;
  }
  {
    const int per = (nb + 7) / 8;
    const int xcd = pid % 8, idx = pid / 8;
    const int full = nb % 8 == 0 ? 8 : nb % 8;
    if (MOE && idx >= (xcd < full ? per : per - 1)) return;  // past this XCD's share of the real tiles
    pid = xcd < full ? xcd * per + idx : full * per + (xcd - full) * (per - 1) + idx;
  }
  constexpr int GM = EMBER_GEMM_GROUP_M;
  const int group = pid / (GM * ntiles);
  const int first_m = group * GM;
  const int gsize = min(mtiles - first_m, GM);
  const int mt = first_m + (pid % (GM * ntiles)) % gsize;
  const int nt = (pid % (GM * ntiles)) / gsize;
  const int m0 = mt * BM, n0 = nt * BNG;

  const T* X = static_cast<const T*>(a.x);
  const T* W = static_cast<const T*>(a.w);
  if (MOE) {
    const int e = a.block_expert[mt];  // uniform
    if (e < 0 || e >= a.E) return;     // past the layout's used blocks
    W += static_cast<int64_t>(e) * a.wes;
  }
  // This wave's load instructions of a double stage: instruction ins moves rows
  // 8 (ins % 32) + lane / 8 of region ins / 32-ish (weight rows first, then x rows); lane l
  // loads 16-byte chunk (l % 8) ^ (row % 8) of its row into slot l of the 1 KiB block.
  const T* src[LOADS];
  int dst[LOADS];
  auto x_src = [&](int xr, int c) {
    int64_t xrow;
    if (MOE) {  // padding assignments read token 0 and store nothing
      const int id = a.sorted_ids[m0 + xr];
      xrow = id >= 0 && id < a.num_valid ? id / a.top_k : 0;
      if (xrow >= a.ntok) {  // a corrupt layout: flag it, read token 0 (the row is stored)
        atomicOr(a.err, EMBER_ERR_ROW_INDEX);
        xrow = 0;
      }
    } else {
      xrow = min(m0 + xr, a.T - 1);  // padded tokens: the last real one
    }
    return X + xrow * a.xs + 8 * c;
  };
  auto w_src = [&](int row, int c) {
    // columns past I (a ragged last tile) read the last real row and store nothing
    const int wr = row < BNG ? min(n0 + row, a.I - 1) : a.I + min(n0 + row - BNG, a.I - 1);
    return W + static_cast<int64_t>(wr) * a.ws + 8 * c;
  };
  // Packed weights: the tile's weight region is its S slabs' 16 KiB units side by side, in
  // the units' own fragment order (1 KiB block ins of slab ins / 16 is bytes
  // [1024 (ins % 16), +1024) of the slab's unit), so every load is 1 KiB of contiguous
  // memory and the fragment reads need no swizzle.
  constexpr int S = PK ? BNG / 64 : 1;
  bool isw[LOADS];  // a weight load (uniform)
  int wsl[LOADS];   // PK: the slab of a weight load
  auto pk_src = [&](int ins) { return W + (ins % 16) * 512 + 8 * lane; };
#pragma unroll
  for (int i = 0; i < LOADS; ++i) {
    if (SPLIT) {  // block offsets within the operand's own buffer
      const int ins = i < WL ? WL * w + i : (LOADS - WL) * w + (i - WL);
      const int row = 8 * ins + (lane >> 3);
      const int c = (lane & 7) ^ (row & 7);
      isw[i] = i < WL;
      wsl[i] = ins / 16;
      src[i] = i < WL ? (PK ? pk_src(ins) : w_src(row, c)) : x_src(row, c);
      dst[i] = ins * 1024;
    } else {
      const int ins = LOADS * w + i;  // 0 .. 2 BNG / 8 + BM / 8 - 1
      const int row = 8 * ins + (lane >> 3);
      const int c = (lane & 7) ^ (row & 7);
      isw[i] = row < 2 * BNG;  // whole blocks: uniform
      wsl[i] = ins / 16;
      src[i] = isw[i] ? (PK ? pk_src(ins) : w_src(row, c)) : x_src(row - 2 * BNG, c);
      dst[i] = ins * 1024;  // the weight region is rows 0 .. 2 BNG - 1, the x region follows
    }
  }
  const int nd = a.H / 64;  // double stages
  // Dense packed weights: a unit's place depends on the decode grid it was packed for, so
  // each slab's units are walked in k order. Routed experts' packed weights are per expert
  // k-major (unit j * slabs + slab of the expert's array), so a stage's S units are adjacent.
  PackedSlabWalk walk[S];
  if (PK && !MOE) {
#pragma unroll
    for (int ss = 0; ss < S; ++ss) walk[ss].init(n0 / 64 + ss, nd, a.pk_total, a.pk_G);
  }
  // element offsets of double stage d's weight units (PK)
  int64_t wofs[S];
  auto next_units = [&](int d) {
    constexpr int64_t kUnitElems = 16384 / static_cast<int64_t>(sizeof(T));
#pragma unroll
    for (int ss = 0; ss < S; ++ss) {
      if (MOE) {
        wofs[ss] = (static_cast<int64_t>(min(d, nd - 1)) * (a.I / 64) + n0 / 64 + ss) * kUnitElems;
      } else {
        wofs[ss] = walk[ss].template elem_offset<T>();
        walk[ss].advance();
      }
    }
  };
  auto wk = [&](int i, int kk) -> int64_t { return PK ? wofs[wsl[i]] : kk; };
  auto wbuf = [&](int d) { return lds + (SPLIT ? (d % 3) * WREG : (d % NBUF) * DST); };
  auto xbuf = [&](int d) { return lds + (SPLIT ? 3 * WREG + (d % 2) * XREG : (d % NBUF) * DST + WREG); };
  auto issue = [&](int d) {
    const int kk = min(d, nd - 1) * 64;
    if (PK) next_units(d);
    unsigned char* st = lds + (d % NBUF) * DST;
#pragma unroll
    for (int i = 0; i < LOADS; ++i) gemm_load_lds16(src[i] + (isw[i] ? wk(i, kk) : kk), st + dst[i]);
  };
  auto issue_w = [&](int d) {
    const int kk = min(d, nd - 1) * 64;
    if (PK) next_units(d);
#pragma unroll
    for (int i = 0; i < WL; ++i) gemm_load_lds16(src[i] + wk(i, kk), wbuf(d) + dst[i]);
  };
  auto issue_x = [&](int d) {
    const int kk = min(d, nd - 1) * 64;
#pragma unroll
    for (int i = WL; i < LOADS; ++i) gemm_load_lds16(src[i] + kk, xbuf(d) + dst[i]);
  };
  int woff[NT], xoff[4];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    if (PK) {  // slab c / 64, fragment (row tile (c % 64) / 16, part) of the unit's first k32 half
      const int c = WC * cg + 16 * (t % (NT / 2));
      woff[t] = (c / 64) * 16384 + (((c % 64) / 16) * 2 + (t < NT / 2 ? 0 : 1)) * 1024 + 16 * lane;
    } else {
      woff[t] = ((t < NT / 2 ? 0 : BNG) + WC * cg + 16 * (t % (NT / 2)) + n) * kGemmRowB;
    }
  }
#pragma unroll
  for (int u = 0; u < 4; ++u) xoff[u] = (64 * q + 16 * u + n) * kGemmRowB;
  const int sw = n & 7;  // row % 8 of every fragment row

  f32x4 acc[NT][4];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[t][u] = f32x4{0.f, 0.f, 0.f, 0.f};
  V8 fw[NT], fx[4];

  // vmcnt after which the next double stage has landed: split rings issue x(j + 1), then
  // w(j + 2) at each even step, so all but the last WL loads
  constexpr int kNextLanded = SPLIT ? WL : (NBUF - 2) * LOADS;
  if (SPLIT) {
    issue_w(0);
    issue_x(0);
    issue_w(1);
  } else {
#pragma unroll
    for (int d = 0; d < NBUF - 1; ++d) issue(d);
  }
  gemm_wait_vm<kNextLanded>();
  gemm_barrier();
  // M(s): at an even 32-k stage issue the next loads into free buffers; read this stage's
  // fragments; at an odd stage wait for the next double stage's loads.
  auto mphase = [&](int s, bool even) {
    const int j = s >> 1;
    if (even) {
      if (SPLIT) {
        issue_x(j + 1);
        issue_w(j + 2);
      } else {
        issue(j + NBUF - 1);
      }
    }
    const unsigned char* sw_ = wbuf(j);
    const unsigned char* sx_ = xbuf(j);
    const int co = ((4 * (s & 1) + g) ^ sw) << 4;
#pragma unroll
    for (int t = 0; t < NT; ++t)
      fw[t] = *reinterpret_cast<const V8*>(sw_ + woff[t] + (PK ? (s & 1) * 8192 : co));
#pragma unroll
    for (int u = 0; u < 4; ++u) fx[u] = *reinterpret_cast<const V8*>(sx_ + xoff[u] + co);
    if (!even) gemm_wait_vm<kNextLanded>();  // the next double stage has landed
    gemm_wait_lgkm0();
  };
  // Routed experts: an expert's run is padded to whole blocks at its end, so a wave whose
  // 64 rows start with a padding assignment holds padding only; it still loads its share
  // of the tiles and keeps the barriers, but skips the MFMAs (nothing of it is stored).
  bool live = true;
  if (MOE) {
    const int id0 = a.sorted_ids[m0 + 64 * q];
    live = __builtin_amdgcn_readfirstlane(id0 >= 0 && id0 < a.num_valid ? 1 : 0) != 0;
  }
  auto cphase = [&]() {
    if (MOE && !live) return;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int u = 0; u < 4; ++u) acc[t][u] = M::run(fw[t], fx[u], acc[t][u]);
  };
  const int nk = 2 * nd;
  if (grp == 1) gemm_barrier();
  for (int s = 0; s < nk; s += 2) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      mphase(s + h, h == 0);
      gemm_barrier();
      cphase();
      gemm_barrier();
    }
  }
  if (grp == 0) gemm_barrier();
  gemm_wait_vm0();

  // Epilogue: lane (n, g) holds rows 4g + r of each 16-row tile for token 16 u + n.
  T* out = static_cast<T*>(a.out);
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    int tok = m0 + 64 * q + 16 * u + n;
    bool real = tok < a.T;
    if (MOE) {  // the assignment's own output row
      tok = a.sorted_ids[tok];
      real = tok >= 0 && tok < a.num_valid;
    }
    if (real) {
#pragma unroll
      for (int t = 0; t < NT / 2; ++t) {
        const int col = n0 + WC * cg + 16 * t + 4 * g;
        if (col >= a.I) continue;  // a ragged last tile (I a multiple of 16)
        Pack<T, 4> o;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float gf = round_to<T>(acc[t][u][r]);
          const float uf = round_to<T>(acc[t + NT / 2][u][r]);
          const float act = round_to<T>(gf / (1.0f + expf(-gf)));
          o.v[r] = half_product<T>(act, uf);
        }
        store_pack<T, 4>(out + static_cast<int64_t>(tok) * a.os + col, o);
      }
    }
  }
}

template <typename T, int BNG, int BM = 256, bool MOE = false, bool PK = false>
int launch_gemm(const GemmArgs& a, hipStream_t st) {
  const int64_t grid = cdiv(a.T, BM) * cdiv(a.I, BNG);
  if (grid > 0x7fffffffLL) return EMBER_EINVAL;
  hipLaunchKernelGGL((k_gate_up_silu_gemm<T, BNG, BM, MOE, PK>), dim3(static_cast<uint32_t>(grid)), dim3(512), 0, st,
                     a);
  return launch_status();
}

// The tile shapes: (tokens, gate columns) of 256 x 64, 256 x 96, 256 x 128 or 128 x 128;
// every one gives each of the 8 waves 64 tokens x (WC gate + WC up) columns. 96-column
// tiles need I only a multiple of 16 (the last tile may be ragged), the others I a
// multiple of the tile.
template <typename T, bool MOE>
int launch_tile(const GemmArgs& a, int64_t token_tile, int64_t column_tile, hipStream_t st) {
  if (token_tile == 128) return launch_gemm<T, 128, 128, MOE>(a, st);
  if (column_tile == 96) return launch_gemm<T, 96, 256, MOE>(a, st);
  return column_tile == 64 ? launch_gemm<T, 64, 256, MOE>(a, st) : launch_gemm<T, 128, 256, MOE>(a, st);
}

bool gemm_tile_ok(int64_t token_tile, int64_t column_tile, int64_t inter) {
  const bool shape = (token_tile == 256 && (column_tile == 64 || column_tile == 96 || column_tile == 128)) ||
                     (token_tile == 128 && column_tile == 128);
  return shape && inter >= column_tile && inter % (column_tile == 96 ? 16 : column_tile) == 0;
}

}  // namespace
}  // namespace ember

extern "C" int ember_gate_up_silu_gemm(const void* x, int64_t x_row_stride, const void* w, int64_t w_row_stride,
                                       int dtype, int64_t tokens, int64_t hidden, int64_t inter, int64_t token_tile,
                                       int64_t column_tile, void* out, int64_t out_row_stride, void* stream) {
  using namespace ember;
  if (tokens == 0) return EMBER_OK;
  if (tokens < 0 || tokens > (int64_t(1) << 24) || hidden < 64 || hidden % 64 != 0 || hidden > (int64_t(1) << 20) ||
      !gemm_tile_ok(token_tile, column_tile, inter) || inter > (int64_t(1) << 28))
    return EMBER_EINVAL;
  if (dtype != EMBER_F16 && dtype != EMBER_BF16) return EMBER_EINVAL;
  if (x == nullptr || w == nullptr || out == nullptr || !aligned16(x) || !aligned16(w) || !aligned16(out))
    return EMBER_EINVAL;
  if (x_row_stride < hidden || w_row_stride < hidden || out_row_stride < inter || x_row_stride % 8 != 0 ||
      w_row_stride % 8 != 0 || out_row_stride % 4 != 0)
    return EMBER_EINVAL;
  GemmArgs a{x, x_row_stride, w, w_row_stride, out, out_row_stride, static_cast<int>(tokens),
             static_cast<int>(hidden), static_cast<int>(inter), nullptr, nullptr, 0, 1, 0, 0, 0};
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == EMBER_F16) return launch_tile<_Float16, false>(a, token_tile, column_tile, st);
  return launch_tile<__bf16, false>(a, token_tile, column_tile, st);
}

extern "C" int ember_moe_gate_up_silu_gemm(const void* x, int64_t x_row_stride, int64_t num_tokens, const void* w,
                                           int64_t w_expert_stride, int64_t w_row_stride, int dtype,
                                           int64_t num_experts, int64_t hidden, int64_t inter,
                                           const int32_t* sorted_ids, const int32_t* block_expert, int64_t num_blocks,
                                           int64_t block_rows, int64_t num_valid, int64_t top_k, int64_t column_tile,
                                           void* out, int64_t out_row_stride, void* stream) {
  using namespace ember;
  if (num_blocks == 0 || num_valid == 0) return EMBER_OK;
  if (num_blocks < 0 || num_valid < 0 || num_tokens < 1 || top_k < 1 || num_experts < 1 || num_blocks > (1 << 22) ||
      num_valid > INT32_MAX / 2 || num_tokens > INT32_MAX || hidden < 64 || hidden % 64 != 0 ||
      hidden > (int64_t(1) << 20) || !gemm_tile_ok(block_rows, column_tile, inter) || inter > (int64_t(1) << 28))
    return EMBER_EINVAL;
  if (dtype != EMBER_F16 && dtype != EMBER_BF16) return EMBER_EINVAL;
  if (x == nullptr || w == nullptr || out == nullptr || sorted_ids == nullptr || block_expert == nullptr ||
      !aligned16(x) || !aligned16(w) || !aligned16(out))
    return EMBER_EINVAL;
  if (x_row_stride < hidden || w_row_stride < hidden || w_expert_stride < 2 * inter * w_row_stride ||
      out_row_stride < inter || x_row_stride % 8 != 0 || w_row_stride % 8 != 0 || w_expert_stride % 8 != 0 ||
      out_row_stride % 4 != 0)
    return EMBER_EINVAL;
  GemmArgs a{x, x_row_stride, w, w_row_stride, out, out_row_stride, static_cast<int>(num_blocks * block_rows),
             static_cast<int>(hidden), static_cast<int>(inter), sorted_ids, block_expert,
             static_cast<int>(num_valid), static_cast<int>(top_k), static_cast<int>(num_experts),
             static_cast<int>(num_tokens), w_expert_stride, device_error_word()};
  if (a.err == nullptr) return EMBER_ENODEV;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == EMBER_F16) return launch_tile<_Float16, true>(a, block_rows, column_tile, st);
  return launch_tile<__bf16, true>(a, block_rows, column_tile, st);
}

extern "C" int ember_gate_up_silu_gemm_packed(const void* x, int64_t x_row_stride, const void* packed, int dtype,
                                              int64_t tokens, int64_t hidden, int64_t inter, int64_t num_workgroups,
                                              int64_t token_tile, int64_t column_tile, void* out,
                                              int64_t out_row_stride, void* stream) {
  using namespace ember;
  if (tokens == 0) return EMBER_OK;
  if (tokens < 0 || tokens > (int64_t(1) << 24) || hidden < 64 || hidden % 64 != 0 || hidden > (int64_t(1) << 20) ||
      inter < 64 || inter % 64 != 0 || inter > (int64_t(1) << 28) || num_workgroups < 1)
    return EMBER_EINVAL;
  const bool shape = (token_tile == 256 && (column_tile == 64 || column_tile == 128)) ||
                     (token_tile == 128 && column_tile == 128);
  if (!shape || inter % column_tile != 0) return EMBER_EINVAL;
  if (dtype != EMBER_F16 && dtype != EMBER_BF16) return EMBER_EINVAL;
  if (x == nullptr || packed == nullptr || out == nullptr || !aligned16(x) || !aligned16(packed) || !aligned16(out))
    return EMBER_EINVAL;
  if (x_row_stride < hidden || out_row_stride < inter || x_row_stride % 8 != 0 || out_row_stride % 4 != 0)
    return EMBER_EINVAL;
  const int64_t total = (inter / 64) * (hidden / 64);
  GemmArgs a{x, x_row_stride, packed, 0, out, out_row_stride, static_cast<int>(tokens),
             static_cast<int>(hidden), static_cast<int>(inter), nullptr, nullptr, 0, 1, 0, 0, 0, nullptr,
             total, num_workgroups < total ? num_workgroups : total};  // the packing's grid
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == EMBER_F16) {
    if (token_tile == 128) return launch_gemm<_Float16, 128, 128, false, true>(a, st);
    return column_tile == 64 ? launch_gemm<_Float16, 64, 256, false, true>(a, st)
                             : launch_gemm<_Float16, 128, 256, false, true>(a, st);
  }
  if (token_tile == 128) return launch_gemm<__bf16, 128, 128, false, true>(a, st);
  return column_tile == 64 ? launch_gemm<__bf16, 64, 256, false, true>(a, st)
                           : launch_gemm<__bf16, 128, 256, false, true>(a, st);
}

extern "C" int ember_moe_gate_up_silu_gemm_packed(const void* x, int64_t x_row_stride, int64_t num_tokens,
                                                  const void* packed, int dtype, int64_t num_experts, int64_t hidden,
                                                  int64_t inter, const int32_t* sorted_ids,
                                                  const int32_t* block_expert, int64_t num_blocks, int64_t block_rows,
                                                  int64_t num_valid, int64_t top_k, int64_t column_tile, void* out,
                                                  int64_t out_row_stride, void* stream) {
  using namespace ember;
  if (num_blocks == 0 || num_valid == 0) return EMBER_OK;
  if (num_blocks < 0 || num_valid < 0 || num_tokens < 1 || top_k < 1 || num_experts < 1 || num_blocks > (1 << 22) ||
      num_valid > INT32_MAX / 2 || num_tokens > INT32_MAX || hidden < 64 || hidden % 64 != 0 ||
      hidden > (int64_t(1) << 20) || inter < 64 || inter > (int64_t(1) << 28))
    return EMBER_EINVAL;
  const bool shape = (block_rows == 256 && (column_tile == 64 || column_tile == 128)) ||
                     (block_rows == 128 && column_tile == 128);
  if (!shape || inter % column_tile != 0) return EMBER_EINVAL;
  if (dtype != EMBER_F16 && dtype != EMBER_BF16) return EMBER_EINVAL;
  if (x == nullptr || packed == nullptr || out == nullptr || sorted_ids == nullptr || block_expert == nullptr ||
      !aligned16(x) || !aligned16(packed) || !aligned16(out))
    return EMBER_EINVAL;
  if (x_row_stride < hidden || out_row_stride < inter || x_row_stride % 8 != 0 || out_row_stride % 4 != 0)
    return EMBER_EINVAL;
  GemmArgs a{x, x_row_stride, packed, 0, out, out_row_stride, static_cast<int>(num_blocks * block_rows),
             static_cast<int>(hidden), static_cast<int>(inter), sorted_ids, block_expert,
             static_cast<int>(num_valid), static_cast<int>(top_k), static_cast<int>(num_experts),
             static_cast<int>(num_tokens), 2 * inter * hidden, device_error_word(), 0, 1};
  if (a.err == nullptr) return EMBER_ENODEV;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == EMBER_F16) {
    if (block_rows == 128) return launch_gemm<_Float16, 128, 128, true, true>(a, st);
    return column_tile == 64 ? launch_gemm<_Float16, 64, 256, true, true>(a, st)
                             : launch_gemm<_Float16, 128, 256, true, true>(a, st);
  }
  if (block_rows == 128) return launch_gemm<__bf16, 128, 128, true, true>(a, st);
  return column_tile == 64 ? launch_gemm<__bf16, 64, 256, true, true>(a, st)
                           : launch_gemm<__bf16, 128, 256, true, true>(a, st);
}
