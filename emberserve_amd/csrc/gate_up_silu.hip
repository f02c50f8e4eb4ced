// The dense MLP's gate_up projection with SiLU-and-mul as its epilogue, for decode-sized
// batches (T <= 64 tokens) on gfx950.
//
// Reference: Qwen2MLP.forward (emberserve/model/qwen2.py:60-61),
//   silu_and_mul(gate_up_proj(x)),  gate_up_proj = nn.Linear(H, 2I, bias=False),
// weight rows [0, I) gate and [I, 2I) up (qwen2.py:49-57), then ops.silu_and_mul
// (ops.py:84-87). The linear layer's output is rounded to the activation dtype before the
// activation reads it, so per output element
//   g = round(x . W[j]),  u = round(x . W[I + j]),  out[t, j] = round(round(silu(g)) * u)
// with fp32 dot products (MFMA accumulation; the order of the k terms is this kernel's
// own, so results agree with another GEMM to within the dot product's rounding).
//
// Why a kernel of its own: at T <= 64 the projection is a stream over the weights
// (2 I H elements, 201 MB at Qwen3-8B) and the unfused pair also writes and rereads the
// [T, 2I] projection and pays a second launch. The library GEMM streams the weights at
// 4.3-5.2 TB/s at these sizes.
//
// Work split. The work is (slab, k step) units: a slab is 64 output columns (wave w of a
// workgroup: gate rows 16w.. and the matching up rows, so the epilogue pairs them in
// registers), a k step 64 elements of H. A persistent grid (one or two workgroups per CU)
// takes equal contiguous runs of the slab-major unit order, so every CU streams the same
// number of weight bytes and its load ring runs on across slab boundaries. Per unit every
// wave moves its 32 weight rows, and the workgroup the unit's x rows, straight from HBM to
// LDS (global_load_lds_dwordx4: 8 rows x one 128-byte line per instruction, the cheapest
// load issue per byte on a CU) in a ring of NS stages, then forms D[weight row][token] with
// v_mfma_f32_16x16x32 (A = weight rows, B = tokens). A 1 KiB LDS block of 8 rows keeps
// 16-byte unit c of row r at slot 8r + (c ^ r), so the operand reads (one row per lane)
// spread over the banks.
//
// A workgroup that covers a slab's whole k range writes its output directly. Otherwise each
// workgroup that covers part of it leaves an agent-coherent partial; at the end of its run a
// workgroup counts its partials in (one per-slab arrival counter) and the last to arrive
// sums the slab's partials in k order (so results do not depend on arrival order), applies
// the epilogue and returns the counter to zero for the next launch.
#include <algorithm>

#include "ember_common.h"

#ifndef EMBER_GU_STAGES
#define EMBER_GU_STAGES 3
#endif
// Register ring stages of the packed-weight dense kernel. Measured on MI355X at Qwen3-8B and
// Qwen2.5-7B, 1 and 16 tokens: 3 and 4 stages tie, 6 and 8 are 1-5% slower.
#ifndef EMBER_GU_PACKED_STAGES
#define EMBER_GU_PACKED_STAGES 3
#endif
// 1-16 tokens: x resident in LDS for the whole run (0: per-wave loads from L2).
#ifndef EMBER_GU_PACKED_XR
#define EMBER_GU_PACKED_XR 1
#endif
// Token tiles up to which the packed kernel loads x per wave from L2 (above: shared in LDS).
#ifndef EMBER_GU_PACKED_PRIVX_MT
#define EMBER_GU_PACKED_PRIVX_MT 1
#endif
// Ring stages of the routed-expert kernel (one workgroup per block and slab, not persistent).
// Measured at Moonlight's geometry: 2 stages (48 KB of LDS, three workgroups per CU) are
// 5-10% slower than 3 at 1-64 tokens (8 tokens: 98.8 vs 89.6 us).
#ifndef EMBER_MOE_STAGES
#define EMBER_MOE_STAGES 3
#endif
// Token tiles (of 16) up to which every wave loads its own copy of x. Measured on MI355X
// (persistent grid, one workgroup per CU): private and shared copies tie at 1-16 tokens;
// at 32 tokens the shared copy is faster (Qwen3-8B 41.2 vs 41.9 us, Qwen2.5-7B 59.2 vs 61.4).
// Register ring stages of the packed routed-expert kernel.
#ifndef EMBER_MOE_PACKED_STAGES
#define EMBER_MOE_PACKED_STAGES 3
#endif
#ifndef EMBER_GU_PRIVX_MT
#define EMBER_GU_PRIVX_MT 1
#endif

namespace ember {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

template <typename T>
struct GuMfma;
template <>
struct GuMfma<_Float16> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x4 run(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};
template <>
struct GuMfma<__bf16> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x4 run(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

constexpr int kGuWaves = 4;
constexpr int kGuRows = 16;                   // gate (and up) rows per wave
constexpr int kGuSlab = kGuWaves * kGuRows;   // output columns per workgroup
constexpr int kGuBK = 64;                     // k per stage: one 128-byte line per row
constexpr int kGuMaxTokens = 64;

struct GuArgs {
  const void* x;
  int64_t xs;
  const void* w;
  int64_t ws;
  void* out;
  int64_t os;
  int T, H, I;
  int64_t max_parts;  // partial slots per slab
  float* part;
  uint32_t* counters;
};

// One 16-byte-per-lane load from global memory straight to LDS: lane i's 16 bytes land at
// lds_base + 16 i. Only the device pass sees the builtin (the host pass drops the kernel's
// launch stub when it appears in a kernel body it does not generate code for).
__device__ __forceinline__ void gu_load_lds16(const void* gptr, void* lds_base) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_global_load_lds(gptr, (__attribute__((address_space(3))) void*)(
                                             reinterpret_cast<uintptr_t>(lds_base)), 16, 0, 0);
#else
  (void)gptr;
  (void)lds_base;
#endif
}

// s_waitcnt vmcnt(n) (gfx9 encoding, expcnt and lgkmcnt left alone).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// A workgroup barrier that waits for this wave's LDS reads but not for its global loads
// (__syncthreads() carries a workgroup fence, which waits for every outstanding load and
// would drain the load ring each step). The asm clobbers keep the compiler from moving
// memory accesses across it.
__device__ __forceinline__ void gu_barrier() {
  __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));  // lgkmcnt(0)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Slabs a run leaves partials for: only its first and last (it emits every slab it covers
// whole), so two.
constexpr int kGuMaxFlush = 2;

// The part of a dense run shared by both load paths: the per-unit bookkeeping of the
// persistent run (slab ends, partials of slabs shared with other workgroups), the epilogue,
// and the end-of-run merge of shared slabs by their last contributor.
template <typename T, int MT>
struct GuRun {
  static constexpr int kFloats = kGuWaves * MT * 2 * kWave * 4;  // one partial of a slab
  const GuArgs& a;
  int w, lane, n, g;
  int64_t nk, total, G;
  int64_t flushed0 = 0, flushed1 = 0;  // scalars, not an array: an indexed member array goes to scratch
  int nflush = 0;
  int64_t cur_slab, cur_k, cur_first;  // the current unit; first k step of its slab in this run

  __device__ __forceinline__ GuRun(const GuArgs& args, int64_t u0) : a(args) {
    lane = threadIdx.x & (kWave - 1);
    w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    n = lane & 15;
    g = lane >> 4;
    nk = a.H / kGuBK;
    total = static_cast<int64_t>(a.I / kGuSlab) * nk;
    G = gridDim.x;
    cur_slab = u0 / nk;
    cur_k = u0 - cur_slab * nk;
    cur_first = cur_k;
  }

  // Epilogue of slab `sl` from sums `v`: lane (n, g) holds D[row 4g + i][token 16 mt + n]
  // of its wave's gate and up tiles, so output columns sl * 64 + 16 w + 4g + [0, 4).
  __device__ __forceinline__ void emit(int64_t sl, const f32x4 (&v)[MT][2]) {
    T* out = static_cast<T*>(a.out);
    const int64_t col = sl * kGuSlab + w * kGuRows + 4 * g;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int tok = 16 * mt + n;
      if (tok < a.T) {
        Pack<T, 4> o;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float gf = round_to<T>(v[mt][0][i]);
          const float uf = round_to<T>(v[mt][1][i]);
          const float act = round_to<T>(gf / (1.0f + expf(-gf)));
          o.v[i] = half_product<T>(act, uf);
        }
        store_pack<T, 4>(out + static_cast<int64_t>(tok) * a.os + col, o);
      }
    }
  }
  // Where a slab's partials live: part p of slab sl (p = contributing workgroup's order).
  __device__ __forceinline__ CoherentRsrc part_rsrc(int64_t sl, int64_t p) const {
    return coherent_rsrc(a.part + (sl * a.max_parts + p) * kFloats, kFloats);
  }
  __device__ __forceinline__ int part_off(int mt, int gu) const {
    return (((w * MT + mt) * 2 + gu) * kWave + lane) * 16;
  }

  // After unit j of nu: at a slab end, emit the slab (whole k range here) or leave its
  // partial, and clear the sums. DRAIN: then wait for the stores (and everything else) in the
  // same block, so no path into the next unit carries a pending store.
  template <bool DRAIN = false>
  __device__ __forceinline__ void end_unit(int j, int nu, f32x4 (&acc)[MT][2]) {
    const bool slab_end = cur_k == nk - 1 || j == nu - 1;
    if (!slab_end) {
      ++cur_k;
      return;
    }
    if (cur_first == 0 && cur_k == nk - 1) {
      emit(cur_slab, acc);
    } else {
      const int64_t p = gu_owner(cur_slab * nk + cur_first, total, G) - gu_owner(cur_slab * nk, total, G);
      const CoherentRsrc rs = part_rsrc(cur_slab, p);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int gu = 0; gu < 2; ++gu) store_coherent<4>(rs, part_off(mt, gu), acc[mt][gu]);
      if (nflush == 0) {
        flushed0 = cur_slab;
        nflush = 1;
      } else if (nflush == 1) {
        flushed1 = cur_slab;
        nflush = 2;
      }
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt][0] = acc[mt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    ++cur_slab;
    cur_k = 0;
    cur_first = 0;
    if (DRAIN) __builtin_amdgcn_s_waitcnt(0);
  }

  // Count this workgroup's partials in; the last contributor of a slab sums its partials in
  // k order (so results do not depend on arrival order), emits it and returns the counter
  // to zero for the next launch.
  __device__ __forceinline__ void merge(int* last_flags) {
    if (nflush == 0) return;  // uniform
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x < nflush) {
      const int64_t sl = threadIdx.x == 0 ? flushed0 : flushed1;
      const uint32_t parts =
          static_cast<uint32_t>(gu_owner(sl * nk + nk - 1, total, G) - gu_owner(sl * nk, total, G) + 1);
      uint32_t* cnt = a.counters + sl;
      const uint32_t prev = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const bool last = prev == parts - 1;
      if (last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last_flags[threadIdx.x] = last;
    }
    __syncthreads();
    for (int f = 0; f < nflush; ++f) {
      if (!last_flags[f]) continue;  // uniform
      const int64_t sl = f == 0 ? flushed0 : flushed1;
      const int64_t parts = gu_owner(sl * nk + nk - 1, total, G) - gu_owner(sl * nk, total, G) + 1;
      f32x4 sum[MT][2];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) sum[mt][0] = sum[mt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
      constexpr int SB = MT <= 4 ? 4 : (MT <= 8 ? 2 : 1);  // partials per batch of loads (registers)
      for (int64_t p0 = 0; p0 < parts; p0 += SB) {
        f32x4 v[SB][MT][2];
#pragma unroll
        for (int u = 0; u < SB; ++u) {
          const CoherentRsrc rs = part_rsrc(sl, min<int64_t>(p0 + u, parts - 1));
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int gu = 0; gu < 2; ++gu)
              v[u][mt][gu] = p0 + u < parts ? load_coherent<4>(rs, part_off(mt, gu)) : f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int u = 0; u < SB; ++u)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int gu = 0; gu < 2; ++gu) sum[mt][gu] += v[u][mt][gu];
      }
      emit(sl, sum);
    }
  }
};

// PRIVX: every wave loads its own copy of a step's x rows (2 KiB per 16 tokens, from L2),
// so the waves never wait for each other; otherwise the four waves share one copy and
// meet at a barrier every step. Private copies cost XB load instructions per wave per
// step, affordable for up to 32 tokens.
template <typename T, int MT, int NS, bool PRIVX>
__global__ void __launch_bounds__(kGuWaves * kWave, 1)
k_gate_up_silu(GuArgs a) {
  using M = GuMfma<T>;
  using V8 = typename M::v8;
  constexpr int XB = 2 * MT;                                // 8-token blocks of x per stage
  constexpr int XBW = PRIVX ? XB : (XB + kGuWaves - 1) / kGuWaves;  // x blocks each wave loads
  constexpr int WB = 4;                                     // weight blocks per wave per stage
  constexpr int WBYTES = kGuWaves * WB * 1024;
  constexpr int STAGE = WBYTES + (PRIVX ? kGuWaves : 1) * XB * 1024;
  constexpr int LPS = WB + XBW;                             // direct loads per wave per stage
  static_assert(NS >= 2 && NS <= 4 && LPS * (NS - 1) < 64, "stages");
  __shared__ __attribute__((aligned(16))) unsigned char lds[NS * STAGE];
  __shared__ int last_flags[kGuMaxFlush];

  const int lane = threadIdx.x & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15;
  const int g = lane >> 4;
  const int64_t nk = a.H / kGuBK;                 // k steps per slab
  const int64_t total = static_cast<int64_t>(a.I / kGuSlab) * nk;
  const int64_t G = gridDim.x;
  const int64_t u0 = gu_start(blockIdx.x, total, G);
  const int nu = static_cast<int>(gu_start(blockIdx.x + 1, total, G) - u0);  // >= 1 (G <= total)

  // Direct-load lanes: lane l moves row l / 8 of an 8-row block, global 16-byte unit
  // (l % 8) ^ (l / 8), into slot l of the block.
  const int lr = lane >> 3;
  const int lc = (lane & 7) ^ lr;
  const T* xg = static_cast<const T*>(a.x);
  const T* wg = static_cast<const T*>(a.w);
  int64_t wrow[WB];  // element offsets of this lane's weight rows in slab 0
#pragma unroll
  for (int q = 0; q < WB; ++q)
    wrow[q] = static_cast<int64_t>((q < 2 ? 0 : a.I) + w * kGuRows + 8 * (q & 1) + lr) * a.ws + 8 * lc;
  const int64_t slab_stride = static_cast<int64_t>(kGuSlab) * a.ws;
  const T* xsrc[XBW];
  int xdst[XBW];
#pragma unroll
  for (int j = 0; j < XBW; ++j) {
    // shared: past the last block a wave loads it again (identical bytes)
    const int blk = PRIVX ? j : min(w + kGuWaves * j, XB - 1);
    const int tok = min(8 * blk + lr, a.T - 1);  // padded tokens read the last real one
    xsrc[j] = xg + static_cast<int64_t>(tok) * a.xs + 8 * lc;
    xdst[j] = WBYTES + (PRIVX ? w * XB * 1024 : 0) + blk * 1024;
  }
  // The issue position walks the units in order: (slab, k step) of the next unit to load.
  int64_t is_slab = u0 / nk;
  int64_t is_k = u0 - is_slab * nk;
  auto issue = [&](int j) {
    unsigned char* st = lds + (j % NS) * STAGE;
    const int64_t kk = is_k * kGuBK;
    const T* wbase = wg + is_slab * slab_stride + kk;
#pragma unroll
    for (int q = 0; q < WB; ++q) gu_load_lds16(wbase + wrow[q], st + (w * WB + q) * 1024);
#pragma unroll
    for (int jx = 0; jx < XBW; ++jx) gu_load_lds16(xsrc[jx] + kk, st + xdst[jx]);
    if (++is_k == nk) {
      is_k = 0;
      ++is_slab;
    }
  };

  f32x4 acc[MT][2];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt][0] = acc[mt][1] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Operand slots: lane (n, g) reads row n of a 16-row pair of blocks, unit 4h + g (k half h).
  auto slot = [&](int h) {
    const int r = n & 7;
    return (n >> 3) * 1024 + (8 * r + (((4 * h + g) ^ r) & 7)) * 16;
  };
  auto compute = [&](int j) {
    const unsigned char* st = lds + (j % NS) * STAGE;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int so = slot(h);
      const V8 wgate = *reinterpret_cast<const V8*>(st + (w * WB) * 1024 + so);
      const V8 wup = *reinterpret_cast<const V8*>(st + (w * WB + 2) * 1024 + so);
      V8 xv[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        xv[mt] = *reinterpret_cast<const V8*>(st + WBYTES + (PRIVX ? w * XB * 1024 : 0) + 2 * mt * 1024 + so);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        acc[mt][0] = M::run(wgate, xv[mt], acc[mt][0]);
        acc[mt][1] = M::run(wup, xv[mt], acc[mt][1]);
      }
    }
  };

  GuRun<T, MT> run(a, u0);

  // The ring: loads of unit j + NS - 1 are issued once every wave is past unit j - 1 (whose
  // buffer they overwrite). Each wave waits for its own loads of a unit, then the barrier
  // makes every wave's loads of it visible.
#pragma unroll
  for (int j = 0; j < NS - 1; ++j)
    if (j < nu) issue(j);
  for (int j = 0; j < nu; ++j) {
    const int ahead = min(NS - 2, nu - 1 - j);  // units issued past this one
    if (ahead >= 2) wait_vm<2 * LPS>();
    else if (ahead == 1) wait_vm<LPS>();
    else wait_vm<0>();
    if constexpr (PRIVX) {
      asm volatile("" ::: "memory");  // this wave's reads of the buffer it refills are done
    } else {
      gu_barrier();
    }
    if (j + NS - 1 < nu) issue(j + NS - 1);
    compute(j);
    run.end_unit(j, nu, acc);
  }
  run.merge(last_flags);
}

// The packed form: the weights pre-arranged once, for a grid of G workgroups
// (ember_gate_up_silu_pack_weight), so that every MFMA operand fragment a wave needs is one
// contiguous KiB. Unit u = (slab, 64-k step j) is 16 contiguous KiB,
//   unit[h][wave][part][lane][8]  (h: k32 half of the step; part 0 gate, 1 up; lane = 16 g + n
//   holds row 64 slab + 16 wave + n of the part, k = 64 j + 32 h + 8 g + [0, 8))
// and the units sit in the order of gu_packed_pos: the grid reads the array front to back,
// one G * 16 KiB window at a time, each load instruction moving 1 KiB with 64 consecutive
// 16-byte lanes, with no LDS. Measured on MI355X (Qwen3-8B, 201 MB): 35.0 us against 37.8
// for the same kernel with each workgroup's run stored as one contiguous range, and 40.5
// for k_gate_up_silu's direct-to-LDS stream of the unpacked rows. x comes from L2 in the
// B-operand layout. NS register stages per wave (the loop is unrolled by NS so every ring
// index is a compile-time constant).
template <typename T, int MT, int NS>
__global__ void __launch_bounds__(kGuWaves * kWave, 1)
k_gate_up_silu_packed(GuArgs a) {
  using M = GuMfma<T>;
  using V8 = typename M::v8;
  static_assert(NS >= 2 && NS <= 8, "stages");
  __shared__ int last_flags[kGuMaxFlush];
  const int64_t nk = a.H / kGuBK;
  const int64_t total = static_cast<int64_t>(a.I / kGuSlab) * nk;
  const int64_t u0 = gu_start(blockIdx.x, total, gridDim.x);
  const int nu = static_cast<int>(gu_start(blockIdx.x + 1, total, gridDim.x) - u0);  // >= 1
  GuRun<T, MT> run(a, u0);
  const int lane = run.lane, w = run.w, n = run.n, g = run.g;

  const T* wp = static_cast<const T*>(a.w) + (w * 2 * kWave + lane) * 8;
  const T* xg = static_cast<const T*>(a.x);
  const T* xrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
    xrow[mt] = xg + static_cast<int64_t>(min(16 * mt + n, a.T - 1)) * a.xs + 8 * g;  // padded tokens: the last real one

  struct Stage {
    V8 wgt[2], wup[2];
    V8 xv[MT][2];
  };
  Stage ring[NS];
  auto issue = [&](Stage& st, int j) {
    const int t = min(j, nu - 1);
    const int64_t kk = ((u0 + t) % nk) * kGuBK;
    // past the run: repeat its last unit (measured: as fast as reading x there instead)
    const T* up = wp + gu_packed_pos(blockIdx.x, t, total, gridDim.x) * (2 * kGuWaves * 2 * kWave * 8);
    constexpr int hs = kGuWaves * 2 * kWave * 8, ps = kWave * 8;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const T* f = up + h * hs;
      st.wgt[h] = __builtin_bit_cast(V8, load_stream<T, 8>(f));
      st.wup[h] = __builtin_bit_cast(V8, load_stream<T, 8>(f + ps));
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int h = 0; h < 2; ++h) st.xv[mt][h] = __builtin_bit_cast(V8, load_pack<T, 8>(xrow[mt] + kk + 32 * h));
  };
  f32x4 acc[MT][2];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt][0] = acc[mt][1] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int d = 0; d < NS; ++d) {
    issue(ring[d], d);
    __builtin_amdgcn_sched_barrier(0);  // stages issued in ring order, oldest consumed first
  }
  for (int j0 = 0; j0 < nu; j0 += NS) {
#pragma unroll
    for (int d = 0; d < NS; ++d) {
      const int j = j0 + d;
      if (j < nu) {  // uniform
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            acc[mt][0] = M::run(ring[d].wgt[h], ring[d].xv[mt][h], acc[mt][0]);
            acc[mt][1] = M::run(ring[d].wup[h], ring[d].xv[mt][h], acc[mt][1]);
          }
      }
      // Every unit issues the same loads on every path (past the run, again the run's last
      // unit, from L2), so the compiler can count how many are still in flight when a stage
      // is consumed: NS - 1 stages. With a skipped issue on one path it waits for all.
      issue(ring[d], j + NS);
      __builtin_amdgcn_sched_barrier(0);
      // Drain the slab's stores here (once per slab), for the same reason: with stores and
      // loads both pending, the loads cannot be counted apart.
      if (j < nu) run.template end_unit<true>(j, nu, acc);
    }
  }
  run.merge(last_flags);
}

// The packed kernel for 1-16 tokens with x resident in LDS. At 16 tokens x (16 x H) no
// longer fits a CU's L1, so k_gate_up_silu_packed re-reads it from L2 for every slab of its
// run, in every workgroup: next to the weight stream that is a large share of L2's
// bandwidth. Here each workgroup loads x once, at the start, in the B-operand fragment order
// (k32 fragment s at s KiB, lane (n, g): token n, k 32 s + 8 g + [0, 8)), and every unit
// reads its two fragments from LDS. The same weight ring, units, runs, epilogue and merge
// as k_gate_up_silu_packed: the same results bit for bit. H <= 32 * kGuXrFrags.
constexpr int kGuXrFrags = 148;  // 148 KiB of LDS: H <= 4736

template <typename T, int NS>
__global__ void __launch_bounds__(kGuWaves * kWave, 1)
k_gate_up_silu_packed_xr(GuArgs a) {
  using M = GuMfma<T>;
  using V8 = typename M::v8;
  constexpr int MT = 1;
  static_assert(NS >= 2 && NS <= 8, "stages");
  __shared__ __attribute__((aligned(16))) unsigned char xlds[kGuXrFrags * 1024];
  __shared__ int last_flags[kGuMaxFlush];
  const int64_t nk = a.H / kGuBK;
  const int64_t total = static_cast<int64_t>(a.I / kGuSlab) * nk;
  const int64_t u0 = gu_start(blockIdx.x, total, gridDim.x);
  const int nu = static_cast<int>(gu_start(blockIdx.x + 1, total, gridDim.x) - u0);  // >= 1
  GuRun<T, MT> run(a, u0);
  const int lane = run.lane, w = run.w, n = run.n, g = run.g;

  // x into LDS first: its loads are the oldest in flight
  {
    const T* xl = static_cast<const T*>(a.x) + static_cast<int64_t>(min(n, a.T - 1)) * a.xs + 8 * g;
    for (int f = w; f < a.H / 32; f += kGuWaves) gu_load_lds16(xl + 32 * f, xlds + f * 1024);
  }
  const T* wp = static_cast<const T*>(a.w) + (w * 2 * kWave + lane) * 8;
  struct Stage {
    V8 wgt[2], wup[2];
  };
  Stage ring[NS];
  auto issue = [&](Stage& st, int j) {
    const int t = min(j, nu - 1);  // past the run: repeat its last unit
    const T* up = wp + gu_packed_pos(blockIdx.x, t, total, gridDim.x) * (2 * kGuWaves * 2 * kWave * 8);
    constexpr int hs = kGuWaves * 2 * kWave * 8, ps = kWave * 8;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      st.wgt[h] = __builtin_bit_cast(V8, load_stream<T, 8>(up + h * hs));
      st.wup[h] = __builtin_bit_cast(V8, load_stream<T, 8>(up + h * hs + ps));
    }
  };
  f32x4 acc[MT][2];
  acc[0][0] = acc[0][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int d = 0; d < NS; ++d) {
    issue(ring[d], d);
    __builtin_amdgcn_sched_barrier(0);  // stages issued in ring order, oldest consumed first
  }
  // every wave's x loads are done (only the weight stages are left in flight), then visible
  wait_vm<NS * 4>();
  gu_barrier();
  int jk = static_cast<int>(u0 % nk);  // k step of the next unit to compute
  for (int j0 = 0; j0 < nu; j0 += NS) {
#pragma unroll
    for (int d = 0; d < NS; ++d) {
      const int j = j0 + d;
      if (j < nu) {  // uniform
        const unsigned char* xs = xlds + (2 * jk) * 1024 + lane * 16;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const V8 xv = *reinterpret_cast<const V8*>(xs + h * 1024);
          acc[0][0] = M::run(ring[d].wgt[h], xv, acc[0][0]);
          acc[0][1] = M::run(ring[d].wup[h], xv, acc[0][1]);
        }
        if (++jk == nk) jk = 0;
      }
      // the same loads on every path (see k_gate_up_silu_packed)
      issue(ring[d], j + NS);
      __builtin_amdgcn_sched_barrier(0);
      if (j < nu) run.template end_unit<true>(j, nu, acc);
    }
  }
  run.merge(last_flags);
}

// The packed kernel for 17-64 tokens. Per unit, every wave needs the x slice of all tokens
// (MT token tiles, 2 KiB each per 64-k step); loading it per lane from L2, as
// k_gate_up_silu_packed does, reads 4 copies per unit and stops scaling past 16 tokens
// (Qwen3-8B: 42 us at 32 tokens, 66 at 64). Here the four waves share one copy in an LDS
// ring, in the B-operand fragment order (fragment f = 2 mt + h of a unit at f KiB, lane
// (n, g) at 16 lane: token 16 mt + n, k 32 h + 8 g + [0, 8)), each wave direct-loading a
// quarter of the fragments. Per unit: wait for this wave's loads of it (a counted vmcnt:
// NS - 2 later stages stay in flight), a barrier (every wave's x of it has landed, and every
// wave is done with the stage the next issue overwrites), the next issue, the MFMAs. The
// weights stream through the register ring of k_gate_up_silu_packed, with the same units,
// runs, epilogue and merge, so each token's result is bit-identical to the other kernels'.
// Measured on MI355X (Qwen3-8B / Qwen2.5-7B): 37.1 / 52.0 us at 32 tokens, 44.5 / 65.0 at 64.
// 8 and 16 token tiles (up to 256 tokens) were built and measured slower than hipBLASLt +
// silu_and_mul (Qwen3-8B at 128 tokens 64.1 vs 54.7 us, at 256 tokens 128.1 vs 74.7): every
// wave reads every token's x from LDS and runs MFMAs for all of them, which grows with T
// past the weight stream.
template <typename T, int MT, int NS>
__global__ void __launch_bounds__(kGuWaves * kWave, 1)
k_gate_up_silu_packed_x(GuArgs a) {
  using M = GuMfma<T>;
  using V8 = typename M::v8;
  static_assert((MT == 1 || MT % 2 == 0) && MT <= 4, "token tiles");
  static_assert(NS >= 2 && NS <= 4, "stages");
  // x fragments each wave loads per unit; with one tile (2 fragments) waves 2 and 3 load
  // waves 0 and 1's again (identical bytes), so every wave issues the same count
  constexpr int XF = MT == 1 ? 1 : MT / 2;
  constexpr int LPS = 4 + XF;         // loads per wave per unit
  static_assert(LPS * (NS - 1) < 64, "vmcnt");
  constexpr int XSTAGE = MT * 2 * 1024;
  __shared__ __attribute__((aligned(16))) unsigned char lds[NS * XSTAGE];
  __shared__ int last_flags[kGuMaxFlush];
  const int64_t nk = a.H / kGuBK;
  const int64_t total = static_cast<int64_t>(a.I / kGuSlab) * nk;
  const int64_t u0 = gu_start(blockIdx.x, total, gridDim.x);
  const int nu = static_cast<int>(gu_start(blockIdx.x + 1, total, gridDim.x) - u0);  // >= 1
  GuRun<T, MT> run(a, u0);
  const int lane = run.lane, w = run.w, n = run.n, g = run.g;

  const T* wp = static_cast<const T*>(a.w) + (w * 2 * kWave + lane) * 8;
  const T* xsrc[XF];
  int xdst[XF];
#pragma unroll
  for (int i = 0; i < XF; ++i) {
    const int f = MT == 1 ? (w & 1) : w + kGuWaves * i;  // fragment 2 mt + h
    const int mt = f >> 1, h = f & 1;
    xsrc[i] = static_cast<const T*>(a.x) + static_cast<int64_t>(min(16 * mt + n, a.T - 1)) * a.xs + 32 * h + 8 * g;
    xdst[i] = f * 1024;
  }

  struct Stage {
    V8 wgt[2], wup[2];
  };
  Stage ring[NS];
  auto issue = [&](Stage& st, int d, int j) {
    const int t = min(j, nu - 1);  // past the run: repeat its last unit
    const int64_t kk = ((u0 + t) % nk) * kGuBK;
    const T* up = wp + gu_packed_pos(blockIdx.x, t, total, gridDim.x) * (2 * kGuWaves * 2 * kWave * 8);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const T* f = up + h * (kGuWaves * 2 * kWave * 8);
      st.wgt[h] = __builtin_bit_cast(V8, load_stream<T, 8>(f));
      st.wup[h] = __builtin_bit_cast(V8, load_stream<T, 8>(f + kWave * 8));
    }
    unsigned char* xs = lds + d * XSTAGE;
#pragma unroll
    for (int i = 0; i < XF; ++i) gu_load_lds16(xsrc[i] + kk, xs + xdst[i]);
  };
  f32x4 acc[MT][2];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt][0] = acc[mt][1] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int d = 0; d < NS - 1; ++d) {
    issue(ring[d], d, d);
    __builtin_amdgcn_sched_barrier(0);  // stages issued in ring order, oldest consumed first
  }
  for (int j0 = 0; j0 < nu; j0 += NS) {
#pragma unroll
    for (int d = 0; d < NS; ++d) {
      const int j = j0 + d;
      // this wave's loads of unit j are done (the NS - 2 units issued after it may not be),
      // then every wave's are, and every wave has read the stage the next issue overwrites
      wait_vm<(NS - 2) * LPS>();
      gu_barrier();
      const int dn = (d + NS - 1) % NS;  // a constant once the loop is unrolled
      issue(ring[dn], dn, j + NS - 1);
      __builtin_amdgcn_sched_barrier(0);
      if (j < nu) {  // uniform
        const unsigned char* xs = lds + d * XSTAGE + lane * 16;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const V8 xv = *reinterpret_cast<const V8*>(xs + (2 * mt + h) * 1024);
            acc[mt][0] = M::run(ring[d].wgt[h], xv, acc[mt][0]);
            acc[mt][1] = M::run(ring[d].wup[h], xv, acc[mt][1]);
          }
        }
        run.template end_unit<true>(j, nu, acc);
      }
    }
  }
  run.merge(last_flags);
}

// Packs W [2I, H] (row stride ws) into the layout of k_gate_up_silu_packed for a grid of G
// workgroups: thread t of the grid moves the 16-byte piece t of the unit-major order
// ((((slab * nk32 + step) * 4 + wave) * 2 + part) * 64 + lane) to its unit's packed place.
template <typename T>
__global__ void __launch_bounds__(256) k_gu_pack(const T* __restrict__ w, int64_t ws, T* __restrict__ dst, int H,
                                                 int I, int64_t G, int64_t pieces) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (t >= pieces) return;
  const int lane = static_cast<int>(t & 63);
  int64_t r = t >> 6;
  const int part = static_cast<int>(r & 1);
  r >>= 1;
  const int wave = static_cast<int>(r & 3);
  r >>= 2;
  const int nk32 = H / 32;
  const int step = static_cast<int>(r % nk32);
  const int64_t slab = r / nk32;
  const int64_t row = part * static_cast<int64_t>(I) + slab * kGuSlab + wave * kGuRows + (lane & 15);
  const int64_t k = static_cast<int64_t>(step) * 32 + 8 * (lane >> 4);
  const int64_t nk = H / kGuBK, total = static_cast<int64_t>(I / kGuSlab) * nk;
  const int64_t u = slab * nk + step / 2;
  const int64_t b = gu_owner(u, total, G);
  const int64_t pos = gu_packed_pos(b, u - gu_start(b, total, G), total, G);
  const int64_t in_unit = ((((step & 1) * kGuWaves + wave) * 2 + part) * kWave + lane);
  store_pack<T, 8>(dst + (pos * (2 * kGuWaves * 2 * kWave) + in_unit) * 8, load_pack<T, 8>(w + row * ws + k));
}

template <typename T, int MT>
int launch_gu(const GuArgs& a, int64_t programs, hipStream_t st) {
  hipLaunchKernelGGL((k_gate_up_silu<T, MT, EMBER_GU_STAGES, (MT <= EMBER_GU_PRIVX_MT)>),
                     dim3(static_cast<uint32_t>(programs)), dim3(kGuWaves * kWave), 0, st, a);
  return launch_status();
}

template <typename T, int MT>
int launch_gu_packed(const GuArgs& a, int64_t programs, hipStream_t st) {
  hipLaunchKernelGGL((k_gate_up_silu_packed<T, MT, EMBER_GU_PACKED_STAGES>), dim3(static_cast<uint32_t>(programs)),
                     dim3(kGuWaves * kWave), 0, st, a);
  return launch_status();
}

template <typename T, int MT>
int launch_gu_packed_x(const GuArgs& a, int64_t programs, hipStream_t st) {
  hipLaunchKernelGGL((k_gate_up_silu_packed_x<T, MT, EMBER_GU_PACKED_STAGES>), dim3(static_cast<uint32_t>(programs)),
                     dim3(kGuWaves * kWave), 0, st, a);
  return launch_status();
}

template <typename T>
int launch_gu_packed_xr(const GuArgs& a, int64_t programs, hipStream_t st) {
  hipLaunchKernelGGL((k_gate_up_silu_packed_xr<T, EMBER_GU_PACKED_STAGES>), dim3(static_cast<uint32_t>(programs)),
                     dim3(kGuWaves * kWave), 0, st, a);
  return launch_status();
}

// Up to 16 tokens x stays in LDS for the whole run (k_gate_up_silu_packed_xr; each wave
// loads its own from L2, k_gate_up_silu_packed, where H is too wide); above, the waves
// share each unit's x through an LDS ring (k_gate_up_silu_packed_x), with the token tiles
// padded to 2 or 4.
template <typename T>
int launch_gu_packed_typed(const GuArgs& a, int64_t programs, hipStream_t st) {
  const int tiles = (a.T + 15) / 16;
  // x resident where every run is whole slabs (no partials: measured 30.9 vs 30.5 us at one
  // token and 33.3 vs 34.7 at 16 for Qwen3-8B over 192 workgroups; 43.8 / 45.6 vs 44.3 / 53.3
  // for Qwen2.5-7B over 148); with runs that split slabs the per-wave loads measured faster
  // (Qwen3-8B over 256: 35.4 / 35.6 vs 36.2 / 38.0 us).
  const bool whole_slabs = (a.I / kGuSlab) % programs == 0;
  if (tiles <= 1 && EMBER_GU_PACKED_XR && whole_slabs && a.H <= 32 * kGuXrFrags)
    return launch_gu_packed_xr<T>(a, programs, st);
  if (tiles <= EMBER_GU_PACKED_PRIVX_MT) return launch_gu_packed<T, 1>(a, programs, st);
  if (tiles <= 1) return launch_gu_packed_x<T, 1>(a, programs, st);
  if (tiles <= 2) return launch_gu_packed_x<T, 2>(a, programs, st);
  if (tiles <= 4) return launch_gu_packed_x<T, 4>(a, programs, st);
  return EMBER_EINVAL;
}

template <typename T>
int launch_gu_typed(const GuArgs& a, int64_t programs, hipStream_t st) {
  switch ((a.T + 15) / 16) {
    case 1: return launch_gu<T, 1>(a, programs, st);
    case 2: return launch_gu<T, 2>(a, programs, st);
    case 3: return launch_gu<T, 3>(a, programs, st);
    case 4: return launch_gu<T, 4>(a, programs, st);
    default: return EMBER_EINVAL;
  }
}

// One slab partial: the token tiles rounded up to a power of two, the most any kernel pads
// them to (the row kernels use the exact count, the LDS-x packed kernel 2, 4, 8 or 16).
int64_t gu_partial_floats(int64_t tokens) {
  int64_t mt = 1;
  while (mt < (tokens + 15) / 16) mt *= 2;
  return kGuWaves * mt * 2 * kWave * 4;
}

// The plan of a launch: workgroups G (at most one per unit) and the most workgroups that
// share one slab (the partial slots per slab).
struct GuPlan {
  int64_t programs = 0, max_parts = 0;
};

GuPlan gu_plan(int64_t hidden, int64_t inter, int64_t programs) {
  GuPlan p;
  const int64_t nk = hidden / kGuBK, slabs = inter / kGuSlab, total = nk * slabs;
  p.programs = std::min(programs, total);
  for (int64_t s = 0; s < slabs; ++s) {
    const int64_t parts = gu_owner(s * nk + nk - 1, total, p.programs) - gu_owner(s * nk, total, p.programs) + 1;
    p.max_parts = std::max(p.max_parts, parts);
  }
  return p;
}


// ---------------------------------------------------------------- routed experts (MoE)
//
// The grouped form of the routed experts' gate_up projection + silu_and_mul
// (fused_moe_forward, emberserve/model/moe_triton.py:332-345: _grouped_gemm over the
// moe_align layout, then ops.silu_and_mul): for every assignment id = token * k + choice
// placed in a 16-row block of expert e = block_expert[b],
//   out[id, j] = round(round(silu(g)) * u),  g = round(x[id / k] . W[e, j]),
//   u = round(x[id / k] . W[e, I + j]).
// One workgroup per (block, 64-column slab, k split); blocks past the last expert
// (block_expert >= E) exit at once, padding rows (sorted_ids >= num_valid) are computed on
// row 0 and not stored. The per-step ring, operand layout and epilogue are
// k_gate_up_silu's with one 16-row token tile and private x copies. With several k splits
// (small batches, where blocks x slabs alone leave CUs idle) each split stores fp32
// partials at its rows' assignment ids, and the last split of a (block, slab) to arrive
// sums them in k order.
// Blocks per call: the grid's third dimension (1M assignments in 16-row blocks).
constexpr int64_t kMoeMaxBlocks = 65535;
constexpr int kMoeDirectChunks = 4;  // routing ids a direct-mode lane holds: at most 4 x 64 assignments

struct MoeGuArgs {
  const void* x;
  int64_t xs, ntok;
  const void* w;
  int64_t wes, ws;  // expert and row strides of the [E, 2I, H] weight (elements)
  void* out;
  int64_t os;
  const int32_t* sorted_ids;
  const int32_t* block_expert;
  const void* topk;   // direct mode (no alignment): assignment ids' experts; null otherwise
  int id_bytes;       // 4 or 8 (topk)
  int E, H, I, num_valid, a_div;
  int kc;             // k per split
  float* part;        // [splits][num_valid][2I] fp32 partials (splits > 1)
  uint32_t* counters; // [num_blocks][I / 64] arrival counters (splits > 1)
  uint32_t* err;
};

// The end of a routed-expert workgroup (block blk, slab): with k splits, leave this split's
// fp32 partials, and the last split of (blk, slab) to arrive sums them in k order; then the
// silu_and_mul epilogue at the block's assignment rows. Shared by both weight layouts.
// A routed-expert workgroup's (block, slab, k split). The grid is (slabs, splits, blocks):
// the workgroups of one block dispatch together, and the used blocks (the layout's first)
// before the empty ones, which exit at once. Measured on MI355X at one token (6 of 60
// blocks used): the packed kernel takes 24 us with the block index fastest (its working
// workgroups then land on few CUs) and 15 us this way; the row kernel 17 and 12.7 us.
struct MoeTile {
  int blk, slab, split, splits;
};
__device__ __forceinline__ MoeTile moe_tile() {
  return MoeTile{static_cast<int>(blockIdx.z), static_cast<int>(blockIdx.x), static_cast<int>(blockIdx.y),
                 static_cast<int>(gridDim.y)};
}

template <typename T>
__device__ __forceinline__ void moe_finish(const MoeGuArgs& a, f32x4 (&acc)[2], const MoeTile& tile, int w,
                                           int lane, int id) {
  const int blk = tile.blk, slab = tile.slab;
  const int g = lane >> 4;
  // lane (n, g): assignment id (slot n of the block), output columns slab * 64 + 16 w + 4g + [0, 4)
  const bool mine = id >= 0 && id < a.num_valid;
  const int64_t col = static_cast<int64_t>(slab) * kGuSlab + w * kGuRows + 4 * g;
  const int splits = tile.splits;
  if (splits > 1) {
    const int64_t row_floats = 2 * static_cast<int64_t>(a.I);
    const int part_floats = static_cast<int>(splits * a.num_valid * row_floats);
    const CoherentRsrc rs = coherent_rsrc(a.part, part_floats);
    const int off = static_cast<int>(((tile.split * static_cast<int64_t>(a.num_valid) + (mine ? id : 0)) * row_floats + col) * 4);
    if (mine) {
      store_coherent<4>(rs, off, acc[0]);
      store_coherent<4>(rs, off + a.I * 4, acc[1]);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __shared__ int is_last;
    __syncthreads();
    if (threadIdx.x == 0) {
      uint32_t* cnt = a.counters + static_cast<int64_t>(blk) * (a.I / kGuSlab) + slab;
      const uint32_t prev = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      is_last = prev == static_cast<uint32_t>(splits - 1);
      if (is_last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!is_last || !mine) return;
    // the splits in k order, all loads in flight together (at most 4 splits)
    f32x4 v[4][2];
    const int row0 = static_cast<int>((static_cast<int64_t>(id) * row_floats + col) * 4);
#pragma unroll
    for (int sp = 0; sp < 4; ++sp) {
      const int o = static_cast<int>(min(sp, splits - 1) * static_cast<int64_t>(a.num_valid) * row_floats * 4) + row0;
      v[sp][0] = load_coherent<4>(rs, o);
      v[sp][1] = load_coherent<4>(rs, o + a.I * 4);
    }
    acc[0] = acc[1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int sp = 0; sp < 4; ++sp)
      if (sp < splits) {
        acc[0] += v[sp][0];
        acc[1] += v[sp][1];
      }
  }
  if (mine) {
    Pack<T, 4> o;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float gf = round_to<T>(acc[0][i]);
      const float uf = round_to<T>(acc[1][i]);
      const float act = round_to<T>(gf / (1.0f + expf(-gf)));
      o.v[i] = half_product<T>(act, uf);
    }
    store_pack<T, 4>(static_cast<T*>(a.out) + static_cast<int64_t>(id) * a.os + col, o);
  }
}

template <typename T, int NS>
__global__ void __launch_bounds__(kGuWaves * kWave, 1)
k_moe_gate_up_silu(MoeGuArgs a) {
  using M = GuMfma<T>;
  using V8 = typename M::v8;
  constexpr int XB = 2;   // one 16-row token tile: two 8-row blocks, per wave
  constexpr int WB = 4;
  constexpr int WBYTES = kGuWaves * WB * 1024;
  constexpr int STAGE = WBYTES + kGuWaves * XB * 1024;
  constexpr int LPS = WB + XB;
  static_assert(NS >= 2 && NS <= 4, "stages");
  __shared__ __attribute__((aligned(16))) unsigned char lds[NS * STAGE];

  const MoeTile tile = moe_tile();
  const int blk = tile.blk;
  const int e = a.block_expert[blk];  // uniform (scalar load)
  if (e < 0 || e >= a.E) return;
  const int slab = tile.slab;
  const int lane = threadIdx.x & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15;
  const int g = lane >> 4;
  const int nk = a.kc / kGuBK;
  const int k0 = tile.split * a.kc;
  const int lr = lane >> 3;
  const int lc = (lane & 7) ^ lr;

  const T* xg = static_cast<const T*>(a.x) + k0;
  const T* wg = static_cast<const T*>(a.w) + static_cast<int64_t>(e) * a.wes + k0;
  const T* wsrc[WB];
#pragma unroll
  for (int q = 0; q < WB; ++q) {
    const int row = (q < 2 ? 0 : a.I) + slab * kGuSlab + w * kGuRows + 8 * (q & 1) + lr;
    wsrc[q] = wg + static_cast<int64_t>(row) * a.ws + 8 * lc;
  }
  const T* xsrc[XB];
#pragma unroll
  for (int q = 0; q < XB; ++q) {
    const int id = a.sorted_ids[blk * 16 + 8 * q + lr];
    int64_t row = id >= 0 && id < a.num_valid ? id / a.a_div : 0;
    if (row >= a.ntok) {
      atomicOr(a.err, EMBER_ERR_ROW_INDEX);
      row = 0;
    }
    xsrc[q] = xg + row * a.xs + 8 * lc;
  }
  auto issue = [&](int j) {
    unsigned char* st = lds + (j % NS) * STAGE;
    const int kk = j * kGuBK;
#pragma unroll
    for (int q = 0; q < WB; ++q) gu_load_lds16(wsrc[q] + kk, st + (w * WB + q) * 1024);
#pragma unroll
    for (int q = 0; q < XB; ++q) gu_load_lds16(xsrc[q] + kk, st + WBYTES + (w * XB + q) * 1024);
  };
  f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
  auto compute = [&](int j) {
    const unsigned char* st = lds + (j % NS) * STAGE;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int r = n & 7;
      const int so = (n >> 3) * 1024 + (8 * r + (((4 * h + g) ^ r) & 7)) * 16;
      const V8 wgate = *reinterpret_cast<const V8*>(st + (w * WB) * 1024 + so);
      const V8 wup = *reinterpret_cast<const V8*>(st + (w * WB + 2) * 1024 + so);
      const V8 xv = *reinterpret_cast<const V8*>(st + WBYTES + w * XB * 1024 + so);
      acc[0] = M::run(wgate, xv, acc[0]);
      acc[1] = M::run(wup, xv, acc[1]);
    }
  };
#pragma unroll
  for (int j = 0; j < NS - 1; ++j)
    if (j < nk) issue(j);
  for (int j = 0; j < nk; ++j) {
    const int ahead = min(NS - 2, nk - 1 - j);
    if (ahead >= 2) wait_vm<2 * LPS>();
    else if (ahead == 1) wait_vm<LPS>();
    else wait_vm<0>();
    asm volatile("" ::: "memory");  // this wave's reads of the buffer it refills are done
    if (j + NS - 1 < nk) issue(j + NS - 1);
    compute(j);
  }
  moe_finish<T>(a, acc, tile, w, lane, a.sorted_ids[tile.blk * 16 + (lane & 15)]);
}


// The packed form of the routed experts' kernel: each expert's weights pre-arranged once
// (ember_moe_gate_up_silu_pack_weight) in the dense packed kernel's 16 KiB units, ordered
// k-major: expert e, unit (j, slab) at e * 2 I H + (j * I / 64 + slab) * 8192 elements. The
// workgroups of one expert and k split then read one window of I / 64 adjacent units at a
// time, each load instruction moves 1 KiB of consecutive lanes, and the ring is in registers,
// so no LDS limits how many workgroups share a CU. Same grid, products, order and epilogue
// as k_moe_gate_up_silu: bit-identical results.
//
// WPB = 2 (one k split only): a workgroup of two waves covers half a slab (waves 2 hs and
// 2 hs + 1 of the slab's layout, hs = the grid's slab index % 2), so a small batch's
// (block, slab) pairs become twice as many workgroups without a k split to merge. Measured
// at Moonlight's geometry, one token (6 used blocks x 22 slabs): see moe_half_slabs.
template <typename T, int NS, int WPB>
__global__ void __launch_bounds__(WPB * kWave)
k_moe_gate_up_silu_packed(MoeGuArgs a) {
  using M = GuMfma<T>;
  using V8 = typename M::v8;
  static_assert(NS >= 2 && NS <= 8, "stages");
  static_assert(WPB == 4 || WPB == 2, "waves per workgroup");
  MoeTile tile = moe_tile();
  const int blk = tile.blk;
  const int lane = threadIdx.x & (kWave - 1);
  const int n = lane & 15;
  const int g = lane >> 4;
  // Direct mode: "block" blk is assignment blk; its expert is read from the routing ids
  // themselves. The assignments of one expert form groups of 16 in assignment order (the
  // order of the aligned layout's runs); the workgroup of each group's first assignment
  // computes the whole group, one assignment per row n, and the others exit. Each lane holds
  // up to kMoeDirectChunks x 64 routing ids in registers for the two scans.
  const bool direct = a.topk != nullptr;  // uniform
  int e, id;
  if (direct) {
    auto eid = [&](int i) -> int64_t {
      return a.id_bytes == 8 ? static_cast<const int64_t*>(a.topk)[i] : static_cast<const int32_t*>(a.topk)[i];
    };
    const int64_t e64 = eid(blk);
    e = static_cast<int>(e64);
    if (e64 < 0 || e64 >= a.E) {  // dropped, as moe_align drops it
      if (threadIdx.x == 0 && tile.slab == 0) atomicOr(a.err, EMBER_ERR_EXPERT_ID);
      return;
    }
    const int na = a.num_valid;
    bool match[kMoeDirectChunks];
#pragma unroll
    for (int c = 0; c < kMoeDirectChunks; ++c) {
      const int i = c * kWave + lane;
      match[c] = i < na && eid(min(i, na - 1)) == e64;
    }
    int before = 0;  // assignments of this expert before blk
#pragma unroll
    for (int c = 0; c < kMoeDirectChunks; ++c)
      before += static_cast<int>(__popcll(__ballot(match[c] && c * kWave + lane < blk)));
    if (before % 16 != 0) return;  // not the first of its group (uniform)
    // row n: the (before + n)-th assignment of this expert, padding past the last
    id = a.num_valid;
    int seen = 0;
#pragma unroll
    for (int c = 0; c < kMoeDirectChunks; ++c) {
      const uint64_t m = __ballot(match[c]);
      const int cnt = static_cast<int>(__popcll(m));
      int k = before + n - seen;
      if (k >= 0 && k < cnt) {  // the k-th set bit of m
        uint64_t mm = m;
        int pos = 0;
#pragma unroll
        for (int step = 32; step >= 1; step >>= 1) {
          const int low = static_cast<int>(__popcll(mm & ((uint64_t(1) << step) - 1)));
          if (low <= k) {
            k -= low;
            mm >>= step;
            pos += step;
          }
        }
        id = c * kWave + pos;
      }
      seen += cnt;
    }
  } else {
    e = a.block_expert[blk];  // uniform (scalar load)
    if (e < 0 || e >= a.E) return;
    id = a.sorted_ids[blk * 16 + n];
  }
  // the wave's place in its 64-column slab
  const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6) + (WPB == 2 ? 2 * (tile.slab & 1) : 0));
  if (WPB == 2) tile.slab >>= 1;
  const int slab = tile.slab;
  const int nk = a.kc / kGuBK;
  const int slabs = a.I / kGuSlab;
  constexpr int kUnit = 2 * kGuWaves * 2 * kWave * 8;  // elements
  const T* wp = static_cast<const T*>(a.w) + static_cast<int64_t>(e) * a.wes +
                (static_cast<int64_t>(tile.split) * nk * slabs + slab) * kUnit + (w * 2 * kWave + lane) * 8;
  const int64_t ustride = static_cast<int64_t>(slabs) * kUnit;
  int64_t row = id >= 0 && id < a.num_valid ? id / a.a_div : 0;
  if (row >= a.ntok) {
    atomicOr(a.err, EMBER_ERR_ROW_INDEX);
    row = 0;
  }
  const T* xrow = static_cast<const T*>(a.x) + row * a.xs + static_cast<int64_t>(tile.split) * a.kc + 8 * g;

  struct Stage {
    V8 wgt[2], wup[2], xv[2];
  };
  Stage ring[NS];
  auto issue = [&](Stage& st, int j) {
    const int jj = min(j, nk - 1);
    // past the range: the same instructions on this lane's x row (L2), not more weights.
    // Measured: 0.3-1 us faster than re-reading the range's last unit at 1-4 tokens.
    const bool real = j < nk;
    const T* f = real ? wp + jj * ustride : xrow;
    const int hs = real ? kGuWaves * 2 * kWave * 8 : 0, ps = real ? kWave * 8 : 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      st.wgt[h] = __builtin_bit_cast(V8, load_stream<T, 8>(f + h * hs));
      st.wup[h] = __builtin_bit_cast(V8, load_stream<T, 8>(f + h * hs + ps));
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) st.xv[h] = __builtin_bit_cast(V8, load_pack<T, 8>(xrow + jj * kGuBK + 32 * h));
  };
  f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
  for (int d = 0; d < NS; ++d) {
    issue(ring[d], d);
    __builtin_amdgcn_sched_barrier(0);  // stages issued in ring order, oldest consumed first
  }
  for (int j0 = 0; j0 < nk; j0 += NS) {
#pragma unroll
    for (int d = 0; d < NS; ++d) {
      if (j0 + d < nk) {  // uniform
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          acc[0] = M::run(ring[d].wgt[h], ring[d].xv[h], acc[0]);
          acc[1] = M::run(ring[d].wup[h], ring[d].xv[h], acc[1]);
        }
      }
      // the same loads on every path, so the compiler counts NS - 1 stages in flight
      issue(ring[d], j0 + d + NS);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  moe_finish<T>(a, acc, tile, w, lane, id);
}

// Packs the routed experts' W [E, 2I, H] (strides wes, ws) into k_moe_gate_up_silu_packed's
// layout: thread t of the grid moves the 16-byte piece t of the source order
// (((((e * I / 64 + slab) * H / 32 + step) * 4 + wave) * 2 + part) * 64 + lane).
template <typename T>
__global__ void __launch_bounds__(256) k_moe_gu_pack(const T* __restrict__ w, int64_t wes, int64_t ws,
                                                     T* __restrict__ dst, int H, int I, int64_t pieces) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (t >= pieces) return;
  const int lane = static_cast<int>(t & 63);
  int64_t r = t >> 6;
  const int part = static_cast<int>(r & 1);
  r >>= 1;
  const int wave = static_cast<int>(r & 3);
  r >>= 2;
  const int nk32 = H / 32, slabs = I / kGuSlab;
  const int step = static_cast<int>(r % nk32);
  r /= nk32;
  const int slab = static_cast<int>(r % slabs);
  const int64_t e = r / slabs;
  const int64_t row = part * static_cast<int64_t>(I) + slab * kGuSlab + wave * kGuRows + (lane & 15);
  const int64_t k = static_cast<int64_t>(step) * 32 + 8 * (lane >> 4);
  const int64_t in_unit = ((((step & 1) * kGuWaves + wave) * 2 + part) * kWave + lane);
  const int64_t unit = static_cast<int64_t>(step / 2) * slabs + slab;
  store_pack<T, 8>(dst + e * (2 * static_cast<int64_t>(I) * H) + (unit * (2 * kGuWaves * 2 * kWave) + in_unit) * 8,
                   load_pack<T, 8>(w + e * wes + row * ws + k));
}

}  // namespace
}  // namespace ember

using namespace ember;

extern "C" {

int64_t ember_gate_up_silu_workspace_bytes(int64_t tokens, int64_t hidden, int64_t inter, int64_t num_workgroups) {
  if (tokens < 1 || tokens > kGuMaxTokens || hidden < kGuBK || hidden % kGuBK != 0 || inter < kGuSlab ||
      inter % kGuSlab != 0 || num_workgroups < 1)
    return -1;
  const GuPlan p = gu_plan(hidden, inter, num_workgroups);
  if (p.programs == 0) return -1;
  const int64_t slabs = inter / kGuSlab;
  const int64_t partials = slabs * p.max_parts * gu_partial_floats(tokens) * int64_t(sizeof(float));
  return partials + (slabs * int64_t(sizeof(uint32_t)) + 255) / 256 * 256;
}

}  // extern "C"

namespace ember {
namespace {

// Validates a dense call and fills its arguments (w_row_stride is ignored for packed weights).
int gu_setup(GuArgs& a, GuPlan& p, const void* x, int64_t x_row_stride, const void* w, int64_t w_row_stride,
             bool packed, int dtype, int64_t tokens, int64_t hidden, int64_t inter, int64_t num_workgroups,
             void* workspace, int64_t workspace_bytes, void* out, int64_t out_row_stride) {
  if (tokens < 0 || tokens > kGuMaxTokens || hidden < kGuBK || hidden % kGuBK != 0 || inter < kGuSlab ||
      inter % kGuSlab != 0 || inter > (int64_t(1) << 29) || hidden > (int64_t(1) << 24) || num_workgroups < 1)
    return EMBER_EINVAL;
  if (dtype != EMBER_F16 && dtype != EMBER_BF16) return EMBER_EINVAL;
  if (x == nullptr || w == nullptr || out == nullptr || workspace == nullptr || !aligned16(x) || !aligned16(w) ||
      !aligned16(out) || !aligned16(workspace))
    return EMBER_EINVAL;
  // 16-byte rows and 8-byte output packs
  if (x_row_stride < hidden || out_row_stride < inter || x_row_stride % 8 != 0 || out_row_stride % 4 != 0)
    return EMBER_EINVAL;
  if (!packed && (w_row_stride < hidden || w_row_stride % 8 != 0)) return EMBER_EINVAL;
  const int64_t need = ember_gate_up_silu_workspace_bytes(tokens, hidden, inter, num_workgroups);
  if (need < 0 || workspace_bytes < need) return EMBER_EINVAL;
  p = gu_plan(hidden, inter, num_workgroups);
  a.x = x;
  a.xs = x_row_stride;
  a.w = w;
  a.ws = w_row_stride;
  a.out = out;
  a.os = out_row_stride;
  a.T = static_cast<int>(tokens);
  a.H = static_cast<int>(hidden);
  a.I = static_cast<int>(inter);
  a.max_parts = p.max_parts;
  const int64_t slabs = inter / kGuSlab;
  a.part = static_cast<float*>(workspace);
  a.counters = reinterpret_cast<uint32_t*>(static_cast<char*>(workspace) +
                                           slabs * p.max_parts * gu_partial_floats(tokens) * int64_t(sizeof(float)));
  return EMBER_OK;
}

}  // namespace
}  // namespace ember

extern "C" {

int ember_gate_up_silu(const void* x, int64_t x_row_stride, const void* w, int64_t w_row_stride, int dtype,
                       int64_t tokens, int64_t hidden, int64_t inter, int64_t num_workgroups, void* workspace,
                       int64_t workspace_bytes, void* out, int64_t out_row_stride, void* stream) {
  if (tokens == 0) return EMBER_OK;
  GuArgs a{};
  GuPlan p;
  const int rc = gu_setup(a, p, x, x_row_stride, w, w_row_stride, false, dtype, tokens, hidden, inter, num_workgroups,
                          workspace, workspace_bytes, out, out_row_stride);
  if (rc != EMBER_OK) return rc;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  return dtype == EMBER_F16 ? launch_gu_typed<_Float16>(a, p.programs, st)
                            : launch_gu_typed<__bf16>(a, p.programs, st);
}

int ember_gate_up_silu_pack_weight(const void* w, int64_t w_row_stride, int dtype, int64_t hidden, int64_t inter,
                                   int64_t num_workgroups, void* packed, void* stream) {
  if (dtype != EMBER_F16 && dtype != EMBER_BF16) return EMBER_EINVAL;
  if (num_workgroups < 1) return EMBER_EINVAL;
  if (hidden < kGuBK || hidden % kGuBK != 0 || inter < kGuSlab || inter % kGuSlab != 0 ||
      inter > (int64_t(1) << 29) || hidden > (int64_t(1) << 24) || w_row_stride < hidden || w_row_stride % 8 != 0)
    return EMBER_EINVAL;
  if (w == nullptr || packed == nullptr || !aligned16(w) || !aligned16(packed)) return EMBER_EINVAL;
  const int64_t G = gu_plan(hidden, inter, num_workgroups).programs;  // as the kernel's grid
  const int64_t pieces = 2 * inter * hidden / 8;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<uint32_t>(cdiv(pieces, 256)));
  if (dtype == EMBER_F16)
    hipLaunchKernelGGL(k_gu_pack<_Float16>, grid, dim3(256), 0, st, static_cast<const _Float16*>(w), w_row_stride,
                       static_cast<_Float16*>(packed), static_cast<int>(hidden), static_cast<int>(inter), G, pieces);
  else
    hipLaunchKernelGGL(k_gu_pack<__bf16>, grid, dim3(256), 0, st, static_cast<const __bf16*>(w), w_row_stride,
                       static_cast<__bf16*>(packed), static_cast<int>(hidden), static_cast<int>(inter), G, pieces);
  return launch_status();
}

int ember_gate_up_silu_packed(const void* x, int64_t x_row_stride, const void* packed_w, int dtype, int64_t tokens,
                              int64_t hidden, int64_t inter, int64_t num_workgroups, void* workspace,
                              int64_t workspace_bytes, void* out, int64_t out_row_stride, void* stream) {
  if (tokens == 0) return EMBER_OK;
  GuArgs a{};
  GuPlan p;
  const int rc = gu_setup(a, p, x, x_row_stride, packed_w, 0, true, dtype, tokens, hidden, inter, num_workgroups,
                          workspace, workspace_bytes, out, out_row_stride);
  if (rc != EMBER_OK) return rc;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  return dtype == EMBER_F16 ? launch_gu_packed_typed<_Float16>(a, p.programs, st)
                            : launch_gu_packed_typed<__bf16>(a, p.programs, st);
}

int64_t ember_moe_gate_up_silu_workspace_bytes(int64_t num_valid, int64_t inter, int64_t num_blocks,
                                               int64_t num_splits) {
  if (num_valid < 0 || inter < kGuSlab || inter % kGuSlab != 0 || num_blocks < 0 || num_splits < 1 ||
      num_splits > 4)
    return -1;
  if (num_splits == 1) return 0;
  const int64_t part = num_splits * num_valid * 2 * inter * int64_t(sizeof(float));
  if (part >= (int64_t(1) << 31)) return -1;  // one buffer resource addresses the partials
  return (part + 255) / 256 * 256 + (num_blocks * (inter / kGuSlab) * int64_t(sizeof(uint32_t)) + 255) / 256 * 256;
}

}  // extern "C"

namespace ember {
namespace {

dim3 moe_grid(int64_t num_blocks, int64_t inter, int64_t num_splits) {
  return dim3(static_cast<uint32_t>(inter / kGuSlab), static_cast<uint32_t>(num_splits),
              static_cast<uint32_t>(num_blocks));
}

// Validates a routed-expert call and fills its arguments (strides ignored for packed weights).
int moe_setup(MoeGuArgs& a, const void* x, int64_t x_row_stride, int64_t num_tokens, const void* w,
              int64_t w_expert_stride, int64_t w_row_stride, bool packed, int dtype, int64_t num_experts,
              int64_t hidden, int64_t inter, const int32_t* sorted_ids, const int32_t* block_expert, int64_t num_blocks,
              int64_t num_valid, int64_t top_k, int64_t num_splits, void* workspace, int64_t workspace_bytes, void* out,
              int64_t out_row_stride) {
  if (num_splits < 1 || num_splits > 4 || (hidden / kGuBK) % num_splits != 0 || hidden / kGuBK / num_splits < 2)
    return EMBER_EINVAL;
  if (num_blocks < 0 || num_blocks > kMoeMaxBlocks || num_valid < 0 || num_valid > 0x7fffffffLL || top_k < 1 ||
      num_tokens < 1 || num_experts < 1 || num_experts > 0x7fffffffLL || hidden < kGuBK || hidden % kGuBK != 0 ||
      hidden > (int64_t(1) << 24) || inter < kGuSlab || inter % kGuSlab != 0 || inter > (int64_t(1) << 29))
    return EMBER_EINVAL;
  if (dtype != EMBER_F16 && dtype != EMBER_BF16) return EMBER_EINVAL;
  if (x == nullptr || w == nullptr || out == nullptr || sorted_ids == nullptr || block_expert == nullptr ||
      !aligned16(x) || !aligned16(w) || !aligned16(out))
    return EMBER_EINVAL;
  if (x_row_stride < hidden || out_row_stride < inter || x_row_stride % 8 != 0 || out_row_stride % 4 != 0)
    return EMBER_EINVAL;
  if (packed) {
    w_row_stride = hidden;
    w_expert_stride = 2 * inter * hidden;
  } else if (w_row_stride < hidden || w_expert_stride < 2 * inter * w_row_stride || w_row_stride % 8 != 0 ||
             w_expert_stride % 8 != 0) {
    return EMBER_EINVAL;
  }
  a.x = x;
  a.xs = x_row_stride;
  a.ntok = num_tokens;
  a.w = w;
  a.wes = w_expert_stride;
  a.ws = w_row_stride;
  a.out = out;
  a.os = out_row_stride;
  a.sorted_ids = sorted_ids;
  a.block_expert = block_expert;
  a.E = static_cast<int>(num_experts);
  a.H = static_cast<int>(hidden);
  a.I = static_cast<int>(inter);
  a.num_valid = static_cast<int>(num_valid);
  a.a_div = static_cast<int>(top_k);
  a.kc = static_cast<int>(hidden / num_splits);
  if (num_splits > 1) {
    const int64_t need = ember_moe_gate_up_silu_workspace_bytes(num_valid, inter, num_blocks, num_splits);
    if (need < 0 || workspace == nullptr || workspace_bytes < need || !aligned16(workspace)) return EMBER_EINVAL;
    const int64_t part = num_splits * num_valid * 2 * inter * int64_t(sizeof(float));
    a.part = static_cast<float*>(workspace);
    a.counters = reinterpret_cast<uint32_t*>(static_cast<char*>(workspace) + (part + 255) / 256 * 256);
  }
  a.err = device_error_word();
  if (a.err == nullptr) return EMBER_ENODEV;
  return EMBER_OK;
}

}  // namespace
}  // namespace ember

extern "C" {

int ember_moe_gate_up_silu(const void* x, int64_t x_row_stride, int64_t num_tokens, const void* w,
                           int64_t w_expert_stride, int64_t w_row_stride, int dtype, int64_t num_experts,
                           int64_t hidden, int64_t inter, const int32_t* sorted_ids, const int32_t* block_expert,
                           int64_t num_blocks, int64_t num_valid, int64_t top_k, int64_t num_splits, void* workspace,
                           int64_t workspace_bytes, void* out, int64_t out_row_stride, void* stream) {
  if (num_blocks == 0 || num_valid == 0) return EMBER_OK;
  MoeGuArgs a{};
  const int rc = moe_setup(a, x, x_row_stride, num_tokens, w, w_expert_stride, w_row_stride, false, dtype, num_experts,
                           hidden, inter, sorted_ids, block_expert, num_blocks, num_valid, top_k, num_splits, workspace,
                           workspace_bytes, out, out_row_stride);
  if (rc != EMBER_OK) return rc;
  const dim3 grid = moe_grid(num_blocks, inter, num_splits);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == EMBER_F16) {
    hipLaunchKernelGGL((k_moe_gate_up_silu<_Float16, EMBER_MOE_STAGES>), grid, dim3(kGuWaves * kWave), 0, st, a);
  } else {
    hipLaunchKernelGGL((k_moe_gate_up_silu<__bf16, EMBER_MOE_STAGES>), grid, dim3(kGuWaves * kWave), 0, st, a);
  }
  return launch_status();
}

int ember_moe_gate_up_silu_pack_weight(const void* w, int64_t w_expert_stride, int64_t w_row_stride, int dtype,
                                       int64_t num_experts, int64_t hidden, int64_t inter, void* packed,
                                       void* stream) {
  if (dtype != EMBER_F16 && dtype != EMBER_BF16) return EMBER_EINVAL;
  if (num_experts < 1 || num_experts > 0x7fffffffLL || hidden < kGuBK || hidden % kGuBK != 0 ||
      hidden > (int64_t(1) << 24) || inter < kGuSlab || inter % kGuSlab != 0 || inter > (int64_t(1) << 29) ||
      w_row_stride < hidden || w_expert_stride < 2 * inter * w_row_stride || w_row_stride % 8 != 0 ||
      w_expert_stride % 8 != 0)
    return EMBER_EINVAL;
  if (w == nullptr || packed == nullptr || !aligned16(w) || !aligned16(packed)) return EMBER_EINVAL;
  const int64_t pieces = num_experts * 2 * inter * hidden / 8;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<uint32_t>(cdiv(pieces, 256)));
  if (dtype == EMBER_F16)
    hipLaunchKernelGGL(k_moe_gu_pack<_Float16>, grid, dim3(256), 0, st, static_cast<const _Float16*>(w),
                       w_expert_stride, w_row_stride, static_cast<_Float16*>(packed), static_cast<int>(hidden),
                       static_cast<int>(inter), pieces);
  else
    hipLaunchKernelGGL(k_moe_gu_pack<__bf16>, grid, dim3(256), 0, st, static_cast<const __bf16*>(w), w_expert_stride,
                       w_row_stride, static_cast<__bf16*>(packed), static_cast<int>(hidden), static_cast<int>(inter),
                       pieces);
  return launch_status();
}

int ember_moe_gate_up_silu_direct(const void* x, int64_t x_row_stride, int64_t num_tokens, const void* packed_w,
                                  int dtype, int64_t num_experts, int64_t hidden, int64_t inter, const void* topk_ids,
                                  int id_bytes, int64_t num_assignments, int64_t top_k, int64_t half_slabs, void* out,
                                  int64_t out_row_stride, void* stream) {
  if (num_assignments == 0) return EMBER_OK;
  if (topk_ids == nullptr || (id_bytes != 4 && id_bytes != 8) || (half_slabs != 0 && half_slabs != 1) ||
      num_assignments < 0 || num_assignments > kMoeDirectChunks * kWave || top_k < 1 || num_assignments % top_k != 0 ||
      num_assignments / top_k > num_tokens)
    return EMBER_EINVAL;
  MoeGuArgs a{};
  // moe_setup's index checks stand in for the routing ids here (never read as such)
  const int32_t* ids = static_cast<const int32_t*>(topk_ids);
  const int rc = moe_setup(a, x, x_row_stride, num_tokens, packed_w, 0, 0, true, dtype, num_experts, hidden, inter,
                           ids, ids, num_assignments, num_assignments, top_k, 1, nullptr, 0, out, out_row_stride);
  if (rc != EMBER_OK) return rc;
  a.sorted_ids = nullptr;
  a.block_expert = nullptr;
  a.topk = topk_ids;
  a.id_bytes = id_bytes;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const uint32_t slabs = static_cast<uint32_t>(inter / kGuSlab);
  const uint32_t na = static_cast<uint32_t>(num_assignments);
  if (half_slabs) {
    if (dtype == EMBER_F16)
      hipLaunchKernelGGL((k_moe_gate_up_silu_packed<_Float16, EMBER_MOE_PACKED_STAGES, 2>), dim3(2 * slabs, 1u, na),
                         dim3(2 * kWave), 0, st, a);
    else
      hipLaunchKernelGGL((k_moe_gate_up_silu_packed<__bf16, EMBER_MOE_PACKED_STAGES, 2>), dim3(2 * slabs, 1u, na),
                         dim3(2 * kWave), 0, st, a);
  } else {
    if (dtype == EMBER_F16)
      hipLaunchKernelGGL((k_moe_gate_up_silu_packed<_Float16, EMBER_MOE_PACKED_STAGES, 4>), dim3(slabs, 1u, na),
                         dim3(kGuWaves * kWave), 0, st, a);
    else
      hipLaunchKernelGGL((k_moe_gate_up_silu_packed<__bf16, EMBER_MOE_PACKED_STAGES, 4>), dim3(slabs, 1u, na),
                         dim3(kGuWaves * kWave), 0, st, a);
  }
  return launch_status();
}

int ember_moe_gate_up_silu_packed(const void* x, int64_t x_row_stride, int64_t num_tokens, const void* packed_w,
                                  int dtype, int64_t num_experts, int64_t hidden, int64_t inter,
                                  const int32_t* sorted_ids, const int32_t* block_expert, int64_t num_blocks,
                                  int64_t num_valid, int64_t top_k, int64_t num_splits, int64_t half_slabs,
                                  void* workspace, int64_t workspace_bytes, void* out, int64_t out_row_stride,
                                  void* stream) {
  if (num_blocks == 0 || num_valid == 0) return EMBER_OK;
  MoeGuArgs a{};
  const int rc = moe_setup(a, x, x_row_stride, num_tokens, packed_w, 0, 0, true, dtype, num_experts, hidden, inter,
                           sorted_ids, block_expert, num_blocks, num_valid, top_k, num_splits, workspace,
                           workspace_bytes, out, out_row_stride);
  if (rc != EMBER_OK) return rc;
  const dim3 grid = moe_grid(num_blocks, inter, num_splits);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (half_slabs != 0 && half_slabs != 1) return EMBER_EINVAL;
  if (half_slabs && num_splits != 1) return EMBER_EINVAL;
  if (half_slabs) {
    const dim3 hgrid(static_cast<uint32_t>(2 * (inter / kGuSlab)), 1u, static_cast<uint32_t>(num_blocks));
    if (dtype == EMBER_F16)
      hipLaunchKernelGGL((k_moe_gate_up_silu_packed<_Float16, EMBER_MOE_PACKED_STAGES, 2>), hgrid, dim3(2 * kWave), 0,
                         st, a);
    else
      hipLaunchKernelGGL((k_moe_gate_up_silu_packed<__bf16, EMBER_MOE_PACKED_STAGES, 2>), hgrid, dim3(2 * kWave), 0,
                         st, a);
    return launch_status();
  }
  if (dtype == EMBER_F16) {
    hipLaunchKernelGGL((k_moe_gate_up_silu_packed<_Float16, EMBER_MOE_PACKED_STAGES, 4>), grid,
                       dim3(kGuWaves * kWave), 0, st, a);
  } else {
    hipLaunchKernelGGL((k_moe_gate_up_silu_packed<__bf16, EMBER_MOE_PACKED_STAGES, 4>), grid, dim3(kGuWaves * kWave),
                       0, st, a);
  }
  return launch_status();
}

}  // extern "C"
