// Neox rotary embedding, Qwen3 QK-RMSNorm + rope, and the MLA latent norm + decoupled
// rope, for gfx950.
//
// Rope (emberserve/model/ops.py:66-81, ops_triton.py:37-70), for i < D/2:
//   o[i]       = round(x[i] * c[i] - x[i + D/2] * s[i])
//   o[i + D/2] = round(x[i + D/2] * c[i] + x[i] * s[i])
// c, s = cos/sin_table[pos][i] (fp32 tables whose halves are equal), each product and the
// sum rounded separately in fp32 (the library builds with -ffp-contract=off).
//
// QK-norm (qwen2.py:95-101): each head row is first RMS-normalised exactly as
// ember_rmsnorm does (y = round(round(x * inv) * w)) and the rope is applied to y; the
// fused kernel keeps y in registers instead of writing and re-reading it.
//
// Layout: q [T, Hq, D] and k [T, Hk, D] with unit stride inside a head, any token/head
// strides (views into the fused qkv projection output). Updates are in place.
//
// Work mapping (rope and qk-norm): J = D / (2 * VEC) lanes own one head row; lane j holds
// the 16-byte pack j of the first half and pack j of the second half, i.e. exactly the
// pairs it rotates, so no lane exchange is needed. A lane processes G heads of one token
// (loads of all G heads are issued before any arithmetic) and reads that token's c/s
// packs once for all of them. The qk-norm sum of squares is a J-lane DPP reduction.
#include "ember_common.h"

// Wave-uniform token index when a token's lanes fill whole waves. Measured on MI355X
// (interleaved A/B): qk-norm + rope [8192, 32q+8kv] 31.8 -> 29.1 us, rope [4096, 28q+4kv]
// 13.5 -> 13.0 us, T = 256 shapes 7% faster.
#ifndef EMBER_ROPE_WAVE_TOK
#define EMBER_ROPE_WAVE_TOK 1
#endif
#ifndef EMBER_ROPE_BLOCK
#define EMBER_ROPE_BLOCK 256
#endif
constexpr int kRopeBlock = EMBER_ROPE_BLOCK;  // lanes per workgroup of k_rope and k_mla

#ifndef EMBER_ROPE_G1_MAX_THREADS
#define EMBER_ROPE_G1_MAX_THREADS (int64_t(1) << 26)
#endif

namespace ember {
namespace {

// Sum of squares of one head row held by J lanes as two VEC-element halves per lane (lane j:
// elements j VEC.. and half + j VEC..). With 8-element packs and J in {4, 8, 16} (head_dim
// 64, 128, 256 in fp16/bf16) the sum follows PyTorch's CPU order exactly (the first half's
// packs are vectors 0..J-1, the second half's J..2J-1), so the normalised head matches the
// reference's rmsnorm bit for bit; otherwise a DPP tree.
template <int J, int VEC>
__device__ __forceinline__ float head_sumsq(const float (&f1)[VEC], const float (&f2)[VEC]) {
  if constexpr (VEC == 8 && (J == 4 || J == 8 || J == 16)) {
    float sq[2][8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      sq[0][e] = f1[e] * f1[e];
      sq[1][e] = f2[e] * f2[e];
    }
    return torch_order_sumsq<J, 2>(sq);
  } else {
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) ss += f1[e] * f1[e] + f2[e] * f2[e];
    return group_sum<J>(ss);
  }
}

template <typename T, typename WT, int VEC, int J, int G, bool NORM, bool WAVE_TOK>
__global__ void __launch_bounds__(kRopeBlock)
k_rope(T* __restrict__ q, int64_t qts, int64_t qhs, int hq, T* __restrict__ k, int64_t kts, int64_t khs,
       int hk, int half, const WT* __restrict__ qw, const WT* __restrict__ kw, float eps,
       const float* __restrict__ cos_t, const float* __restrict__ sin_t, int64_t trows, int64_t tstride,
       const int64_t* __restrict__ pos, uint32_t ntok, uint32_t ngroups, FastDiv gdiv,
       uint32_t* __restrict__ err) {
  const uint32_t gt = blockIdx.x * static_cast<uint32_t>(kRopeBlock) + threadIdx.x;
  const uint32_t j = gt % J;
  const uint32_t rowid = gt / J;
  uint32_t tok = gdiv.div(rowid);
  // WAVE_TOK: a token's lanes fill whole waves (ngroups * J % 64 == 0), so the token index
  // is wave-uniform; readfirstlane lets the position come through a scalar load.
  if constexpr (WAVE_TOK) tok = __builtin_amdgcn_readfirstlane(tok);
  if (tok >= ntok) return;  // whole J-lane groups leave together
  const uint32_t hg = rowid - tok * ngroups;
  const int nh = hq + hk;
  const int64_t off = static_cast<int64_t>(j) * VEC;

  // Load order matters: vector loads retire in issue order (vmcnt), so the position is
  // loaded first, then the head rows; the c/s table loads then wait only for the position
  // while the head rows are still in flight, and nothing branches on the position before
  // the head-row loads are issued.
  const int64_t p = pos[tok];
  Pack<T, VEC> x1[G];
  Pack<T, VEC> x2[G];
  T* ptr[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int h = min(static_cast<int>(hg) * G + g, nh - 1);
    ptr[g] = (h < hq ? q + tok * qts + h * qhs : k + tok * kts + (h - hq) * khs) + off;
    x1[g] = load_stream<T, VEC>(ptr[g]);
    x2[g] = load_stream<T, VEC>(ptr[g] + half);
  }
  const bool bad = p < 0 || p >= trows;
  const int64_t pc = bad ? 0 : p;
  float c[VEC];
  float s[VEC];
  load_vals<float, VEC>(cos_t + pc * tstride + off, c);
  load_vals<float, VEC>(sin_t + pc * tstride + off, s);
  // Norm weights (L2-resident), issued after the table loads. With one head per lane the
  // head is either a q or a k head, so one weight is loaded; with G > 1 a lane's heads may
  // straddle the q/k boundary and both are loaded.
  float wq1[VEC], wq2[VEC], wk1[VEC], wk2[VEC];
  Pack<WT, VEC> wp1, wp2;  // G == 1: kept packed, widened at use (no early wait)
  if constexpr (NORM) {
    if constexpr (G == 1) {
      const WT* w0 = static_cast<int>(hg) < hq ? qw : kw;
      wp1 = load_pack<WT, VEC>(w0 + off);
      wp2 = load_pack<WT, VEC>(w0 + half + off);
    } else {
      load_vals<WT, VEC>(qw + off, wq1);
      load_vals<WT, VEC>(qw + half + off, wq2);
      load_vals<WT, VEC>(kw + off, wk1);
      load_vals<WT, VEC>(kw + half + off, wk2);
    }
  }
  // Keep every load above this point: without it the scheduler computes the sum of squares
  // (which waits for the head rows) before issuing the table loads, serialising the two
  // latencies.
  __builtin_amdgcn_sched_barrier(0);

  // No branch depends on the position: a branch would let the compiler sink the head-row
  // loads below it (re-serialising them after the position load). An out-of-range
  // position instead stores the loaded rows back unchanged.
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int h = static_cast<int>(hg) * G + g;
    if (G == 1 || h < nh) {  // uniform across the J lanes; always true for G == 1
      float f1[VEC];
      float f2[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        f1[e] = to_f32(x1[g].v[e]);
        f2[e] = to_f32(x2[g].v[e]);
      }
      if constexpr (NORM) {
        const float tot = head_sumsq<J>(f1, f2);
        const float inv = 1.0f / sqrt_rn(tot / static_cast<float>(2 * half) + eps);
        const bool isq = h < hq;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const float w1 = G == 1 ? to_f32(wp1.v[e]) : (isq ? wq1[e] : wk1[e]);
          const float w2 = G == 1 ? to_f32(wp2.v[e]) : (isq ? wq2[e] : wk2[e]);
          f1[e] = round_to<T>(round_to<T>(f1[e] * inv) * w1);
          f2[e] = round_to<T>(round_to<T>(f2[e] * inv) * w2);
        }
      }
      Pack<T, VEC> o1;
      Pack<T, VEC> o2;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        o1.v[e] = bad ? x1[g].v[e] : from_f32<T>(f1[e] * c[e] - f2[e] * s[e]);
        o2.v[e] = bad ? x2[g].v[e] : from_f32<T>(f2[e] * c[e] + f1[e] * s[e]);
      }
      store_stream<T, VEC>(ptr[g], o1);
      store_stream<T, VEC>(ptr[g] + half, o2);
    }
  }
  if (bad && j == 0 && hg == 0) atomicOr(err, EMBER_ERR_ROPE_POS);
}

// Rope (optionally with the Qwen3 qk-norm) fused with the paged KV-cache write that
// consumes it (qwen2.py:95-101 then kv/cache.py:54-61): per token the Hq + 2 Hkv head rows
// are q heads (rotated in place), k heads (rotated in place and stored to k_cache[slot])
// and v heads (copied to v_cache[slot]). Same mapping and load discipline as k_rope with
// one head per lane; the k rows are not read back for the cache write.
template <typename T, typename WT, int VEC, int J, bool NORM, bool WAVE_TOK>
__global__ void __launch_bounds__(kRopeBlock)
k_rope_kv(T* __restrict__ q, int64_t qts, int64_t qhs, int hq, T* __restrict__ k, int64_t kts, int64_t khs,
          int hk, const T* __restrict__ v, int64_t vts, int64_t vhs, int half, const WT* __restrict__ qw,
          const WT* __restrict__ kw, float eps, const float* __restrict__ cos_t, const float* __restrict__ sin_t,
          int64_t trows, int64_t tstride, const int64_t* __restrict__ pos, const int64_t* __restrict__ slots,
          T* __restrict__ kc, T* __restrict__ vc, int64_t num_slots, int64_t css, int64_t chs, uint32_t ntok,
          FastDiv hdiv, uint32_t* __restrict__ err) {
  const uint32_t gt = blockIdx.x * static_cast<uint32_t>(kRopeBlock) + threadIdx.x;
  const uint32_t j = gt % J;
  const uint32_t rowid = gt / J;
  uint32_t tok = hdiv.div(rowid);  // head rows per token: hq + 2 hk
  if constexpr (WAVE_TOK) tok = __builtin_amdgcn_readfirstlane(tok);
  if (tok >= ntok) return;
  const int h = static_cast<int>(rowid - tok * hdiv.d);
  const int kind = h < hq ? 0 : (h < hq + hk ? 1 : 2);  // q, k, v: uniform across the J lanes
  const int hh = kind == 0 ? h : (kind == 1 ? h - hq : h - hq - hk);
  const int64_t off = static_cast<int64_t>(j) * VEC;

  const int64_t p = pos[tok];
  const int64_t slot = slots[tok];
  T* ptr = kind == 0 ? q + tok * qts + hh * qhs : k + tok * kts + hh * khs;
  const T* src = (kind == 2 ? v + tok * vts + hh * vhs : ptr) + off;
  const Pack<T, VEC> x1 = load_stream<T, VEC>(src);
  const Pack<T, VEC> x2 = load_stream<T, VEC>(src + half);
  const bool bad = p < 0 || p >= trows;
  const int64_t pc = bad ? 0 : p;
  float c[VEC];
  float s[VEC];
  load_vals<float, VEC>(cos_t + pc * tstride + off, c);
  load_vals<float, VEC>(sin_t + pc * tstride + off, s);
  Pack<WT, VEC> wp1, wp2;
  if constexpr (NORM) {
    const WT* w0 = kind == 0 ? qw : kw;
    wp1 = load_pack<WT, VEC>(w0 + off);
    wp2 = load_pack<WT, VEC>(w0 + half + off);
  }
  __builtin_amdgcn_sched_barrier(0);  // every load issued before any arithmetic

  Pack<T, VEC> o1 = x1;
  Pack<T, VEC> o2 = x2;
  if (kind != 2) {
    float f1[VEC];
    float f2[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      f1[e] = to_f32(x1.v[e]);
      f2[e] = to_f32(x2.v[e]);
    }
    if constexpr (NORM) {
      const float tot = head_sumsq<J>(f1, f2);
      const float inv = 1.0f / sqrt_rn(tot / static_cast<float>(2 * half) + eps);
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        f1[e] = round_to<T>(round_to<T>(f1[e] * inv) * to_f32(wp1.v[e]));
        f2[e] = round_to<T>(round_to<T>(f2[e] * inv) * to_f32(wp2.v[e]));
      }
    }
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      o1.v[e] = bad ? x1.v[e] : from_f32<T>(f1[e] * c[e] - f2[e] * s[e]);
      o2.v[e] = bad ? x2.v[e] : from_f32<T>(f2[e] * c[e] + f1[e] * s[e]);
    }
    store_stream<T, VEC>(ptr + off, o1);
    store_stream<T, VEC>(ptr + off + half, o2);
  }
  const bool slot_ok = slot >= 0 && slot < num_slots;
  if (kind != 0 && slot_ok) {
    T* dst = (kind == 1 ? kc : vc) + slot * css + hh * chs + off;
    store_stream<T, VEC>(dst, o1);
    store_stream<T, VEC>(dst + half, o2);
  }
  if (j == 0 && h == 0) {
    if (bad) atomicOr(err, EMBER_ERR_ROPE_POS);
    if (!slot_ok && slot != kPadSlot) atomicOr(err, EMBER_ERR_KV_SLOT);
  }
}

// Any head_dim, any alignment: one wave per (token, head), scalar accesses, loops over the
// half dimension (the norm variant reads the row twice, the second time from cache).
template <typename T, typename WT, bool NORM>
__global__ void __launch_bounds__(256)
k_rope_any(T* __restrict__ q, int64_t qts, int64_t qhs, int hq, T* __restrict__ k, int64_t kts, int64_t khs,
           int hk, int half, const WT* __restrict__ qw, const WT* __restrict__ kw, float eps,
           const float* __restrict__ cos_t, const float* __restrict__ sin_t, int64_t trows, int64_t tstride,
           const int64_t* __restrict__ pos, int64_t ntok, uint32_t* __restrict__ err) {
  const int64_t rowid = static_cast<int64_t>(blockIdx.x) * 4 + threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const int nh = hq + hk;
  const int64_t tok = rowid / nh;
  const int h = static_cast<int>(rowid - tok * nh);
  if (tok >= ntok) return;
  const int64_t p = pos[tok];
  if (p < 0 || p >= trows) {
    if (lane == 0 && h == 0) atomicOr(err, EMBER_ERR_ROPE_POS);
    return;
  }
  T* ptr = h < hq ? q + tok * qts + h * qhs : k + tok * kts + (h - hq) * khs;
  const WT* w = h < hq ? qw : kw;
  float inv = 1.f;
  if constexpr (NORM) {
    float ss = 0.f;
    for (int i = lane; i < 2 * half; i += kWave) {
      const float f = to_f32(ptr[i]);
      ss += f * f;
    }
    const float tot = group_sum<kWave>(ss);
    inv = 1.0f / sqrt_rn(tot / static_cast<float>(2 * half) + eps);
  }
  for (int i = lane; i < half; i += kWave) {
    float f1 = to_f32(ptr[i]);
    float f2 = to_f32(ptr[half + i]);
    if constexpr (NORM) {
      f1 = round_to<T>(round_to<T>(f1 * inv) * to_f32(w[i]));
      f2 = round_to<T>(round_to<T>(f2 * inv) * to_f32(w[half + i]));
    }
    const float c = cos_t[p * tstride + i];
    const float s = sin_t[p * tstride + i];
    ptr[i] = from_f32<T>(f1 * c - f2 * s);
    ptr[half + i] = from_f32<T>(f2 * c + f1 * s);
  }
}

struct RopeArgs {
  void* q;
  int64_t qts, qhs, hq;
  void* k;
  int64_t kts, khs, hk;
  int64_t head_dim;
  const void* qw;
  const void* kw;
  float eps;
  const float* cos_t;
  const float* sin_t;
  int64_t trows, tstride;
  const int64_t* pos;
  int64_t ntok;
  hipStream_t stream;
  uint32_t* err;
};

template <typename T, typename WT, int VEC, int J, int G, bool NORM, bool WAVE_TOK>
int launch_vec_tok(const RopeArgs& a) {
  const int64_t nh = a.hq + a.hk;
  const int64_t ngroups = cdiv(nh, G);
  const int64_t threads = a.ntok * ngroups * J;
  if (threads > 0x7fffffffLL) return EMBER_EINVAL;  // FastDiv needs indices < 2^31
  const int64_t grid = cdiv(threads, kRopeBlock);
  hipLaunchKernelGGL((k_rope<T, WT, VEC, J, G, NORM, WAVE_TOK>), dim3(static_cast<uint32_t>(grid)), dim3(kRopeBlock), 0, a.stream,
                     static_cast<T*>(a.q), a.qts, a.qhs, static_cast<int>(a.hq), static_cast<T*>(a.k), a.kts,
                     a.khs, static_cast<int>(a.hk), static_cast<int>(a.head_dim / 2),
                     static_cast<const WT*>(a.qw), static_cast<const WT*>(a.kw), a.eps, a.cos_t, a.sin_t,
                     a.trows, a.tstride, a.pos, static_cast<uint32_t>(a.ntok), static_cast<uint32_t>(ngroups),
                     FastDiv::make(static_cast<uint32_t>(ngroups)), a.err);
  return launch_status();
}

template <typename T, typename WT, int VEC, int J, int G, bool NORM>
int launch_vec(const RopeArgs& a) {
  if (EMBER_ROPE_WAVE_TOK && (cdiv(a.hq + a.hk, G) * J) % kWave == 0)
    return launch_vec_tok<T, WT, VEC, J, G, NORM, true>(a);
  return launch_vec_tok<T, WT, VEC, J, G, NORM, false>(a);
}

template <typename T, typename WT, int VEC, int J, bool NORM>
int launch_g(const RopeArgs& a) {
  // Heads per lane. Measured on MI355X (rope, T = 4096-16384): one head per lane beats
  // two or four (more waves in flight outweigh the extra c/s table reads), so G > 1 is
  // used only when a launch would exceed EMBER_ROPE_G1_MAX_THREADS lanes.
  const int64_t nh = a.hq + a.hk;
  if (a.ntok * nh * J <= EMBER_ROPE_G1_MAX_THREADS) return launch_vec<T, WT, VEC, J, 1, NORM>(a);
  if (a.ntok * cdiv(nh, 2) * J <= EMBER_ROPE_G1_MAX_THREADS) return launch_vec<T, WT, VEC, J, 2, NORM>(a);
  return launch_vec<T, WT, VEC, J, 4, NORM>(a);
}

template <typename T, typename WT, bool NORM>
int launch_typed(const RopeArgs& a) {
  constexpr int VEC = 16 / sizeof(T);
  const int64_t half = a.head_dim / 2;
  const int64_t j = half / VEC;
  const bool have_k = a.hk > 0;
  bool vec_ok = half % VEC == 0 && (j & (j - 1)) == 0 && j >= 1 && j <= 32 && aligned16(a.q) &&
                a.qts % VEC == 0 && a.qhs % VEC == 0 && aligned16(a.cos_t) && aligned16(a.sin_t) &&
                a.tstride % 4 == 0;
  if (have_k) vec_ok = vec_ok && aligned16(a.k) && a.kts % VEC == 0 && a.khs % VEC == 0;
  if (NORM) vec_ok = vec_ok && aligned16(a.qw) && (!have_k || aligned16(a.kw));
  if (vec_ok) {
    switch (j) {
      case 1: return launch_g<T, WT, VEC, 1, NORM>(a);
      case 2: return launch_g<T, WT, VEC, 2, NORM>(a);
      case 4: return launch_g<T, WT, VEC, 4, NORM>(a);
      case 8: return launch_g<T, WT, VEC, 8, NORM>(a);
      case 16: return launch_g<T, WT, VEC, 16, NORM>(a);
      case 32: return launch_g<T, WT, VEC, 32, NORM>(a);
      default: break;
    }
  }
  const int64_t rows = a.ntok * (a.hq + a.hk);
  const int64_t grid = cdiv(rows, 4);
  if (grid > 0x7fffffffLL) return EMBER_EINVAL;
  hipLaunchKernelGGL((k_rope_any<T, WT, NORM>), dim3(static_cast<uint32_t>(grid)), dim3(256), 0, a.stream,
                     static_cast<T*>(a.q), a.qts, a.qhs, static_cast<int>(a.hq), static_cast<T*>(a.k), a.kts,
                     a.khs, static_cast<int>(a.hk), static_cast<int>(half), static_cast<const WT*>(a.qw),
                     static_cast<const WT*>(a.kw), a.eps, a.cos_t, a.sin_t, a.trows, a.tstride, a.pos, a.ntok,
                     a.err);
  return launch_status();
}

int check_rope_args(const RopeArgs& a) {
  if (a.ntok < 0 || a.hq < 0 || a.hk < 0 || a.head_dim <= 0 || a.head_dim % 2 != 0) return EMBER_EINVAL;
  if (a.head_dim > 4096 || a.hq + a.hk > 0x7fffffff || a.trows < 0 || a.tstride < a.head_dim / 2)
    return EMBER_EINVAL;
  if (a.ntok == 0 || a.hq + a.hk == 0) return -1;  // nothing to do
  if (a.cos_t == nullptr || a.sin_t == nullptr || a.pos == nullptr) return EMBER_EINVAL;
  if (a.hq > 0 && a.q == nullptr) return EMBER_EINVAL;
  if (a.hk > 0 && a.k == nullptr) return EMBER_EINVAL;
  return EMBER_OK;
}

struct RopeKvArgs {
  RopeArgs r;
  const void* v;
  int64_t vts, vhs;
  const int64_t* slots;
  void* kc;
  void* vc;
  int64_t num_slots, css, chs;
};

template <typename T, typename WT, int VEC, int J, bool NORM>
int launch_rope_kv_vec(const RopeKvArgs& a) {
  const RopeArgs& r = a.r;
  const int64_t per_tok = r.hq + 2 * r.hk;
  const int64_t threads = r.ntok * per_tok * J;
  if (threads > 0x7fffffffLL) return EMBER_EINVAL;
  const int64_t grid = cdiv(threads, kRopeBlock);
  const FastDiv hdiv = FastDiv::make(static_cast<uint32_t>(per_tok));
#define EMBER_LAUNCH_ROPE_KV(WT_)                                                                             \
  hipLaunchKernelGGL((k_rope_kv<T, WT, VEC, J, NORM, WT_>), dim3(static_cast<uint32_t>(grid)), dim3(kRopeBlock), 0, \
                     r.stream, static_cast<T*>(r.q), r.qts, r.qhs, static_cast<int>(r.hq), static_cast<T*>(r.k),     \
                     r.kts, r.khs, static_cast<int>(r.hk), static_cast<const T*>(a.v), a.vts, a.vhs,                \
                     static_cast<int>(r.head_dim / 2), static_cast<const WT*>(r.qw), static_cast<const WT*>(r.kw),    \
                     r.eps, r.cos_t, r.sin_t, r.trows, r.tstride, r.pos, a.slots, static_cast<T*>(a.kc),           \
                     static_cast<T*>(a.vc), a.num_slots, a.css, a.chs, static_cast<uint32_t>(r.ntok), hdiv, r.err)
  if ((per_tok * J) % kWave == 0) {
    EMBER_LAUNCH_ROPE_KV(true);
  } else {
    EMBER_LAUNCH_ROPE_KV(false);
  }
#undef EMBER_LAUNCH_ROPE_KV
  return launch_status();
}

template <typename T, typename WT, bool NORM>
int launch_rope_kv_typed(const RopeKvArgs& a) {
  constexpr int VEC = 16 / sizeof(T);
  const RopeArgs& r = a.r;
  const int64_t half = r.head_dim / 2;
  const int64_t j = half / VEC;
  const bool vec_ok = half % VEC == 0 && (j & (j - 1)) == 0 && j >= 1 && j <= 32 && aligned16(r.q) &&
                      aligned16(r.k) && aligned16(a.v) && aligned16(a.kc) && aligned16(a.vc) &&
                      aligned16(r.cos_t) && aligned16(r.sin_t) && r.tstride % 4 == 0 && r.qts % VEC == 0 &&
                      r.qhs % VEC == 0 && r.kts % VEC == 0 && r.khs % VEC == 0 && a.vts % VEC == 0 &&
                      a.vhs % VEC == 0 && a.css % VEC == 0 && a.chs % VEC == 0 &&
                      (!NORM || (aligned16(r.qw) && aligned16(r.kw)));
  if (!vec_ok) return EMBER_EALIGN;  // the caller runs the two unfused ops instead
  switch (j) {
    case 1: return launch_rope_kv_vec<T, WT, VEC, 1, NORM>(a);
    case 2: return launch_rope_kv_vec<T, WT, VEC, 2, NORM>(a);
    case 4: return launch_rope_kv_vec<T, WT, VEC, 4, NORM>(a);
    case 8: return launch_rope_kv_vec<T, WT, VEC, 8, NORM>(a);
    case 16: return launch_rope_kv_vec<T, WT, VEC, 16, NORM>(a);
    case 32: return launch_rope_kv_vec<T, WT, VEC, 32, NORM>(a);
    default: return EMBER_EALIGN;
  }
}

// ---------------------------------------------------------------- MLA latent path
//
// deepseek.py:124-133 with the rope permutation folded into the weights: per token,
//   latent[:R] = rmsnorm(c, w), latent[R:R+Dr] = rope(k_pe), q_pe[h] = rope(q_pe[h]).
// Work is split into independent wave tasks over groups of TPW consecutive tokens: one
// "latent" wave (per token: the R-wide row as NVC packs per lane and a whole-wave DPP
// reduction, plus the key head's rope on the first J lanes) and ceil(H * J / 64) "query"
// waves (J lanes per query head). A wave issues the loads of all its TPW tokens before any
// arithmetic (the launcher uses TPW = 1; see launch_mla_vec).

template <typename T, typename WT, int VEC, int J, int NVC, int TPW, bool CACHE>
__global__ void __launch_bounds__(kRopeBlock)
k_mla(const T* __restrict__ c, int64_t cts, int R, const T* __restrict__ kpe, int64_t kts, T* __restrict__ qpe,
      int64_t qts, int64_t qhs, int H, int half, const WT* __restrict__ w, float eps,
      const float* __restrict__ cos_t, const float* __restrict__ sin_t, int64_t trows, int64_t tstride,
      const int64_t* __restrict__ pos, int64_t ntok, T* __restrict__ lat, int64_t lts, int tasks_per_group,
      const int64_t* __restrict__ slots, T* __restrict__ cache, int64_t num_slots, int64_t css,
      uint32_t* __restrict__ err) {
  // CACHE: the latent rows also go to cache[slots[t]] (PagedLatentCache.write fused in);
  // lat may then be null, and only the cache is written.
  // The task index is the same on every lane of a wave; readfirstlane makes that visible
  // to the compiler, so token indices live in SGPRs and the position is fetched with a
  // scalar load (its own counter, off the vector-load queue).
  const int task = __builtin_amdgcn_readfirstlane(
      static_cast<int>(blockIdx.x * (kRopeBlock / kWave) + threadIdx.x / kWave));
  const int lane = threadIdx.x % kWave;
  const int64_t group = task / tasks_per_group;
  const int sub = static_cast<int>(task - group * tasks_per_group);
  const int64_t tok0 = group * TPW;
  if (tok0 >= ntok) return;
  const int j = lane % J;
  const int64_t off = static_cast<int64_t>(j) * VEC;
  int64_t toks[TPW];
#pragma unroll
  for (int u = 0; u < TPW; ++u) toks[u] = min(tok0 + u, ntok - 1);  // loads stay in range

  if (sub == 0) {
    // Latent rows. Positions first (vector loads retire in issue order, so the table loads
    // then wait only for them), then c packs, weights, the key head, then the tables.
    const int ncv = R / VEC;
    int64_t p[TPW];
#pragma unroll
    for (int u = 0; u < TPW; ++u) p[u] = pos[toks[u]];
    Pack<T, VEC> cv[TPW][NVC];
    Pack<T, VEC> k1[TPW], k2[TPW];
#pragma unroll
    for (int u = 0; u < TPW; ++u) {
#pragma unroll
      for (int i = 0; i < NVC; ++i) {
        const int vi = min(lane + i * kWave, ncv - 1);
        cv[u][i] = load_stream<T, VEC>(c + toks[u] * cts + static_cast<int64_t>(vi) * VEC);
      }
      k1[u] = load_pack<T, VEC>(kpe + toks[u] * kts + off);
      k2[u] = load_pack<T, VEC>(kpe + toks[u] * kts + half + off);
    }
    Pack<WT, VEC> wv[NVC];
#pragma unroll
    for (int i = 0; i < NVC; ++i) wv[i] = load_pack<WT, VEC>(w + static_cast<int64_t>(min(lane + i * kWave, ncv - 1)) * VEC);
    bool bad[TPW];
    float cc[TPW][VEC], sn[TPW][VEC];
#pragma unroll
    for (int u = 0; u < TPW; ++u) {
      bad[u] = p[u] < 0 || p[u] >= trows;
      const int64_t pc = bad[u] ? 0 : p[u];
      load_vals<float, VEC>(cos_t + pc * tstride + off, cc[u]);
      load_vals<float, VEC>(sin_t + pc * tstride + off, sn[u]);
    }
    __builtin_amdgcn_sched_barrier(0);  // all loads issued before any arithmetic

#pragma unroll
    for (int u = 0; u < TPW; ++u) {
      const bool live = tok0 + u < ntok;  // uniform across the wave
      float v[NVC][VEC];
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < NVC; ++i) {
        const bool ok = lane + i * kWave < ncv;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const float f = ok ? to_f32(cv[u][i].v[e]) : 0.f;
          v[i][e] = f;
          ss += f * f;
        }
      }
      const float tot = group_sum<kWave>(ss);
      const float inv = 1.0f / sqrt_rn(tot / static_cast<float>(R) + eps);
      T* lrow = lat == nullptr ? nullptr : lat + toks[u] * lts;
      T* crow = nullptr;
      if constexpr (CACHE) {
        const int64_t slot = slots[toks[u]];
        if (slot >= 0 && slot < num_slots) {
          crow = cache + slot * css;
        } else if (live && lane == 0 && slot != kPadSlot) {
          atomicOr(err, EMBER_ERR_KV_SLOT);
        }
      }
#pragma unroll
      for (int i = 0; i < NVC; ++i) {
        const int vi = lane + i * kWave;
        if (live && vi < ncv) {
          Pack<T, VEC> o;
#pragma unroll
          for (int e = 0; e < VEC; ++e) o.v[e] = from_f32<T>(round_to<T>(v[i][e] * inv) * to_f32(wv[i].v[e]));
          if (lrow != nullptr) store_stream<T, VEC>(lrow + static_cast<int64_t>(vi) * VEC, o);
          if (CACHE && crow != nullptr) store_stream<T, VEC>(crow + static_cast<int64_t>(vi) * VEC, o);
        }
      }
      if (live && lane < J) {
        Pack<T, VEC> o1, o2;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const float f1 = to_f32(k1[u].v[e]);
          const float f2 = to_f32(k2[u].v[e]);
          // an out-of-range position zeroes the latent key slot (q_pe is left untouched)
          o1.v[e] = from_f32<T>(bad[u] ? 0.f : f1 * cc[u][e] - f2 * sn[u][e]);
          o2.v[e] = from_f32<T>(bad[u] ? 0.f : f2 * cc[u][e] + f1 * sn[u][e]);
        }
        if (lrow != nullptr) {
          store_stream<T, VEC>(lrow + R + off, o1);
          store_stream<T, VEC>(lrow + R + half + off, o2);
        }
        if (CACHE && crow != nullptr) {
          store_stream<T, VEC>(crow + R + off, o1);
          store_stream<T, VEC>(crow + R + half + off, o2);
        }
      }
      if (live && bad[u] && lane == 0) atomicOr(err, EMBER_ERR_ROPE_POS);
    }
    return;
  }

  // Query heads (64 / J per wave), TPW tokens.
  constexpr int kHeadsPerWave = kWave / J;
  const int head = (sub - 1) * kHeadsPerWave + lane / J;
  if (head >= H) return;  // whole J-lane groups
  int64_t p[TPW];
#pragma unroll
  for (int u = 0; u < TPW; ++u) p[u] = pos[toks[u]];
  T* ptr[TPW];
  Pack<T, VEC> a1[TPW], a2[TPW];
#pragma unroll
  for (int u = 0; u < TPW; ++u) {
    ptr[u] = qpe + toks[u] * qts + static_cast<int64_t>(head) * qhs + off;
    a1[u] = load_stream<T, VEC>(ptr[u]);
    a2[u] = load_stream<T, VEC>(ptr[u] + half);
  }
  bool bad[TPW];
  float cc[TPW][VEC], sn[TPW][VEC];
#pragma unroll
  for (int u = 0; u < TPW; ++u) {
    bad[u] = p[u] < 0 || p[u] >= trows;
    const int64_t pc = bad[u] ? 0 : p[u];
    load_vals<float, VEC>(cos_t + pc * tstride + off, cc[u]);
    load_vals<float, VEC>(sin_t + pc * tstride + off, sn[u]);
  }
  __builtin_amdgcn_sched_barrier(0);
  // Branch-free as in k_rope: a bad position stores q_pe back unchanged (the latent wave
  // reports the error).
#pragma unroll
  for (int u = 0; u < TPW; ++u) {
    Pack<T, VEC> o1, o2;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float f1 = to_f32(a1[u].v[e]);
      const float f2 = to_f32(a2[u].v[e]);
      o1.v[e] = bad[u] ? a1[u].v[e] : from_f32<T>(f1 * cc[u][e] - f2 * sn[u][e]);
      o2.v[e] = bad[u] ? a2[u].v[e] : from_f32<T>(f2 * cc[u][e] + f1 * sn[u][e]);
    }
    if (tok0 + u < ntok) {
      store_stream<T, VEC>(ptr[u], o1);
      store_stream<T, VEC>(ptr[u] + half, o2);
    }
  }
}

// One token per 64-lane workgroup (16-bit activations, the fast path of the MLA op).
//
// The whole token is one wave: NVC latent passes (pack lane + 64 i of the R-wide row, a
// whole-wave DPP reduction), NQ query passes and one key pass. In a head group of L = 2J
// lanes, lane r holds pack (r >> 1) + J (r & 1) of the head's Dr-wide slice: the L lanes of
// a group cover the slice's bytes in one instruction (full 128-byte lines at Dr = 64), and
// each lane's rotation partner (pack i <-> i + J) is lane r ^ 1, whose value arrives as a
// quad_perm DPP operand of the multiply. The partner product is formed with the sign folded
// into the sine (first-half lanes multiply by -s), so
//   first half:  x1 * c + x2 * (-s) == x1 * c - x2 * s
//   second half: x2 * c + x1 * s
// bit for bit the reference's separately rounded expression.
//
// Measured on MI355X (Moonlight shape, T = 8192, rotated inputs): 11.7 us against 13.9 us
// for k_mla. All loads are issued before any arithmetic, and every output is selected
// rather than branched on, so the compiler cannot sink a load under a branch (a sunk q load
// serialised position -> table -> q and cost 0.7 us).
template <typename T, typename WT, int VEC, int J, int NQ, int NVC, bool CACHE>
__global__ void __launch_bounds__(kWave)
k_mla_tok(const T* __restrict__ c, int64_t cts, int R, const T* __restrict__ kpe, int64_t kts, T* __restrict__ qpe,
          int64_t qts, int64_t qhs, int H, const WT* __restrict__ w, float eps, const float* __restrict__ cos_t,
          const float* __restrict__ sin_t, int64_t trows, int64_t tstride, const int64_t* __restrict__ pos,
          T* __restrict__ lat, int64_t lts, const int64_t* __restrict__ slots, T* __restrict__ cache,
          int64_t num_slots, int64_t css, uint32_t* __restrict__ err) {
  constexpr int L = 2 * J;          // lanes per head slice
  constexpr int kHeads = kWave / L;  // heads per query pass
  const int64_t tok = blockIdx.x;
  const int lane = threadIdx.x;
  const int r = lane % L;
  const int64_t pk = ((r >> 1) + J * (r & 1)) * VEC;  // element offset of this lane's pack
  const int64_t ci = (r >> 1) * VEC;                  // its cos/sin columns
  const int ncv = R / VEC;

  const int64_t p = pos[tok];  // scalar load (tok is uniform)
  int64_t slot = 0;
  if constexpr (CACHE) slot = slots[tok];
  Pack<T, VEC> cv[NVC];
#pragma unroll
  for (int i = 0; i < NVC; ++i) cv[i] = load_stream<T, VEC>(c + tok * cts + static_cast<int64_t>(min(lane + i * kWave, ncv - 1)) * VEC);
  Pack<T, VEC> qv[NQ];
  T* qp[NQ];
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    const int head = min(i * kHeads + lane / L, H - 1);
    qp[i] = qpe + tok * qts + static_cast<int64_t>(head) * qhs + pk;
    qv[i] = load_stream<T, VEC>(qp[i]);
  }
  const Pack<T, VEC> kv = load_stream<T, VEC>(kpe + tok * kts + pk);
  Pack<WT, VEC> wv[NVC];
#pragma unroll
  for (int i = 0; i < NVC; ++i) wv[i] = load_pack<WT, VEC>(w + static_cast<int64_t>(min(lane + i * kWave, ncv - 1)) * VEC);
  const bool bad = p < 0 || p >= trows;
  const int64_t pc = bad ? 0 : p;
  float cc[VEC], sn[VEC];
  load_vals<float, VEC>(cos_t + pc * tstride + ci, cc);
  load_vals<float, VEC>(sin_t + pc * tstride + ci, sn);
  // All loads are issued before any arithmetic: the asm memory clobber keeps the IR passes
  // from moving a load below this point (the weight load otherwise landed behind the query
  // stores), sched_barrier keeps the machine scheduler from doing so.
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);

  // Sine with the first-half sign folded in.
  const uint32_t sm = (r & 1) ? 0u : 0x80000000u;
  float sx[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) sx[e] = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, sn[e]) ^ sm);
  auto rotate = [&](const Pack<T, VEC>& x) {
    Pack<T, VEC> o;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float f = to_f32(x.v[e]);
      const float a = f * cc[e];
      const float b = dpp_f32<kDppQuadSwap1>(f) * sx[e];
      o.v[e] = from_f32<T>(a + b);
    }
    return o;
  };

  // Stores are unconditional: a lane past the last head (or latent pack) was clamped onto
  // the last one, loaded the same bytes and computes the same result, so it rewrites
  // identical bytes. A divergent store guard made the compiler sink the arithmetic under
  // it and wait for every load before the first store (13.5 us against 11.7 us).
  // Query heads: rotated in place; a bad position stores them back unchanged.
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    const Pack<T, VEC> o = rotate(qv[i]);
    store_stream<T, VEC>(qp[i], bad ? qv[i] : o);
  }

  // Latent row.
  float v[NVC][VEC];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NVC; ++i) {
    const bool ok = lane + i * kWave < ncv;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float f = ok ? to_f32(cv[i].v[e]) : 0.f;
      v[i][e] = f;
      ss += f * f;
    }
  }
  const float tot = group_sum<kWave>(ss);
  const float inv = 1.0f / sqrt_rn(tot / static_cast<float>(R) + eps);
  T* lrow = lat == nullptr ? nullptr : lat + tok * lts;
  T* crow = nullptr;
  if constexpr (CACHE) {
    if (slot >= 0 && slot < num_slots) {
      crow = cache + slot * css;
    } else if (lane == 0 && slot != kPadSlot) {
      atomicOr(err, EMBER_ERR_KV_SLOT);
    }
  }
#pragma unroll
  for (int i = 0; i < NVC; ++i) {
    const int64_t vi = min(lane + i * kWave, ncv - 1);
    Pack<T, VEC> o;
#pragma unroll
    for (int e = 0; e < VEC; ++e) o.v[e] = from_f32<T>(round_to<T>(to_f32(cv[i].v[e]) * inv) * to_f32(wv[i].v[e]));
    // Without the cache the latent tensor is always given; an unconditional store also
    // keeps the weight load from being sunk under a branch, behind the query stores.
    if (!CACHE || lrow != nullptr) store_stream<T, VEC>(lrow + vi * VEC, o);
    if (CACHE && crow != nullptr) store_stream<T, VEC>(crow + vi * VEC, o);
  }

  // The key head: rotated into the latent row's last Dr columns (zeros for a bad position).
  // Every L-lane group holds the same head, so all groups store it (identical bytes).
  Pack<T, VEC> ko = rotate(kv);
  if (bad) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) ko.v[e] = from_f32<T>(0.f);
  }
  if (!CACHE || lrow != nullptr) store_stream<T, VEC>(lrow + R + pk, ko);
  if (CACHE && crow != nullptr) store_stream<T, VEC>(crow + R + pk, ko);
  if (bad && lane == 0) atomicOr(err, EMBER_ERR_ROPE_POS);
}

// Any shape, any alignment: one wave per token, scalar accesses.
template <typename T, typename WT>
__global__ void __launch_bounds__(256)
k_mla_any(const T* __restrict__ c, int64_t cts, int R, const T* __restrict__ kpe, int64_t kts,
          T* __restrict__ qpe, int64_t qts, int64_t qhs, int H, int half, const WT* __restrict__ w, float eps,
          const float* __restrict__ cos_t, const float* __restrict__ sin_t, int64_t trows, int64_t tstride,
          const int64_t* __restrict__ pos, int64_t ntok, T* __restrict__ lat, int64_t lts,
          uint32_t* __restrict__ err) {
  const int64_t tok = static_cast<int64_t>(blockIdx.x) * 4 + threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  if (tok >= ntok) return;
  float ss = 0.f;
  for (int i = lane; i < R; i += kWave) {
    const float f = to_f32(c[tok * cts + i]);
    ss += f * f;
  }
  const float tot = group_sum<kWave>(ss);
  const float inv = 1.0f / sqrt_rn(tot / static_cast<float>(R) + eps);
  for (int i = lane; i < R; i += kWave)
    lat[tok * lts + i] = from_f32<T>(round_to<T>(to_f32(c[tok * cts + i]) * inv) * to_f32(w[i]));
  const int64_t p = pos[tok];
  if (p < 0 || p >= trows) {
    if (lane == 0) atomicOr(err, EMBER_ERR_ROPE_POS);
    for (int i = lane; i < 2 * half; i += kWave) lat[tok * lts + R + i] = from_f32<T>(0.f);
    return;
  }
  for (int it = lane; it < (H + 1) * half; it += kWave) {
    const int head = it / half;
    const int i = it - head * half;
    const T* src = head < H ? qpe + tok * qts + static_cast<int64_t>(head) * qhs : kpe + tok * kts;
    T* dst = head < H ? qpe + tok * qts + static_cast<int64_t>(head) * qhs : lat + tok * lts + R;
    const float f1 = to_f32(src[i]);
    const float f2 = to_f32(src[half + i]);
    const float cv = cos_t[p * tstride + i];
    const float sv = sin_t[p * tstride + i];
    dst[i] = from_f32<T>(f1 * cv - f2 * sv);
    dst[half + i] = from_f32<T>(f2 * cv + f1 * sv);
  }
}

struct MlaArgs {
  const void* c;
  int64_t cts, R;
  const void* kpe;
  int64_t kts;
  void* qpe;
  int64_t qts, qhs, H, rope_dim;
  const void* w;
  float eps;
  const float* cos_t;
  const float* sin_t;
  int64_t trows, tstride;
  const int64_t* pos;
  int64_t ntok;
  void* lat;
  int64_t lts;
  hipStream_t stream;
  uint32_t* err;
  const int64_t* slots = nullptr;  // the fused latent-cache write (null: none)
  void* cache = nullptr;
  int64_t num_slots = 0;
  int64_t css = 0;
};

template <typename T, typename WT, int VEC, int J, int NQ, int NVC>
int launch_mla_tok(const MlaArgs& a) {
#define EMBER_LAUNCH_MLA_TOK(CACHE_)                                                                             \
  hipLaunchKernelGGL((k_mla_tok<T, WT, VEC, J, NQ, NVC, CACHE_>), dim3(static_cast<uint32_t>(a.ntok)), dim3(kWave), \
                     0, a.stream, static_cast<const T*>(a.c), a.cts, static_cast<int>(a.R),                      \
                     static_cast<const T*>(a.kpe), a.kts, static_cast<T*>(a.qpe), a.qts, a.qhs,                  \
                     static_cast<int>(a.H), static_cast<const WT*>(a.w), a.eps, a.cos_t, a.sin_t, a.trows,        \
                     a.tstride, a.pos, static_cast<T*>(a.lat), a.lts, a.slots, static_cast<T*>(a.cache),         \
                     a.num_slots, a.css, a.err)
  if (a.cache != nullptr) {
    EMBER_LAUNCH_MLA_TOK(true);
  } else {
    EMBER_LAUNCH_MLA_TOK(false);
  }
#undef EMBER_LAUNCH_MLA_TOK
  return launch_status();
}

template <typename T, typename WT, int VEC, int J>
int launch_mla_tok_nq(const MlaArgs& a, int nq, int nvc) {
  if (nvc == 1) {
    switch (nq) {
      case 1: return launch_mla_tok<T, WT, VEC, J, 1, 1>(a);
      case 2: return launch_mla_tok<T, WT, VEC, J, 2, 1>(a);
      case 4: return launch_mla_tok<T, WT, VEC, J, 4, 1>(a);
      default: return EMBER_EINVAL;
    }
  }
  switch (nq) {
    case 1: return launch_mla_tok<T, WT, VEC, J, 1, 2>(a);
    case 2: return launch_mla_tok<T, WT, VEC, J, 2, 2>(a);
    case 4: return launch_mla_tok<T, WT, VEC, J, 4, 2>(a);
    default: return EMBER_EINVAL;
  }
}

template <typename T, typename WT, int VEC, int J, int NVC>
int launch_mla_vec(const MlaArgs& a) {
  // One token per wave task: measured on MI355X (Moonlight shape, T = 8192) TPW = 1, 2, 4
  // take 14.8, 15.5 and 18.2 us. More waves in flight beat more bytes per wave here.
  constexpr int TPW = 1;
  const int64_t tasks_per_group = 1 + cdiv(a.H * J, kWave);
  const int64_t grid = cdiv(cdiv(a.ntok, TPW) * tasks_per_group, kRopeBlock / kWave);
  if (grid * (kRopeBlock / kWave) > 0x7fffffffLL) return EMBER_EINVAL;  // task index is an int
#define EMBER_LAUNCH_MLA(CACHE_)                                                                              \
  hipLaunchKernelGGL((k_mla<T, WT, VEC, J, NVC, TPW, CACHE_>), dim3(static_cast<uint32_t>(grid)), dim3(kRopeBlock), 0, \
                     a.stream, static_cast<const T*>(a.c), a.cts, static_cast<int>(a.R),                          \
                     static_cast<const T*>(a.kpe), a.kts, static_cast<T*>(a.qpe), a.qts, a.qhs,                  \
                     static_cast<int>(a.H), static_cast<int>(a.rope_dim / 2), static_cast<const WT*>(a.w), a.eps,  \
                     a.cos_t, a.sin_t, a.trows, a.tstride, a.pos, a.ntok, static_cast<T*>(a.lat), a.lts,           \
                     static_cast<int>(tasks_per_group), a.slots, static_cast<T*>(a.cache), a.num_slots, a.css, a.err)
  if (a.cache != nullptr) {
    EMBER_LAUNCH_MLA(true);
  } else {
    EMBER_LAUNCH_MLA(false);
  }
#undef EMBER_LAUNCH_MLA
  return launch_status();
}

template <typename T, typename WT, int VEC, int J>
int launch_mla_nvc(const MlaArgs& a, int nvc) {
  switch (nvc) {
    case 1: return launch_mla_vec<T, WT, VEC, J, 1>(a);
    case 2: return launch_mla_vec<T, WT, VEC, J, 2>(a);
    case 4: return launch_mla_vec<T, WT, VEC, J, 4>(a);
    case 8: return launch_mla_vec<T, WT, VEC, J, 8>(a);
    default: return EMBER_EINVAL;
  }
}

template <typename T, typename WT>
int launch_mla_typed(const MlaArgs& a) {
  constexpr int VEC = 16 / sizeof(T);
  const int64_t half = a.rope_dim / 2;
  const int64_t j = half / VEC;
  const int64_t ncv = a.R / VEC;
  const bool vec_ok = a.R % VEC == 0 && ncv <= 8 * kWave && half % VEC == 0 && (j & (j - 1)) == 0 && j >= 1 &&
                      j <= 16 && aligned16(a.c) && aligned16(a.kpe) && aligned16(a.qpe) && aligned16(a.lat) &&
                      aligned16(a.w) && aligned16(a.cos_t) && aligned16(a.sin_t) && a.tstride % 4 == 0 &&
                      a.cts % VEC == 0 && a.kts % VEC == 0 && a.qts % VEC == 0 && a.qhs % VEC == 0 &&
                      a.lts % VEC == 0 && (a.cache == nullptr || (aligned16(a.cache) && a.css % VEC == 0));
  if constexpr (sizeof(T) == 2) {
    // one token per 64-lane workgroup: up to 4 query passes, up to 2 latent packs per lane
    const int64_t nq = pow2_ceil(cdiv(a.H * 2 * j, kWave));
    const int64_t nvc = cdiv(ncv, kWave);
    if (vec_ok && a.H >= 1 && a.ntok <= 0x7fffffffLL && nq <= 4 && nvc <= 2 && (j == 2 || j == 4 || j == 8)) {
      switch (j) {
        case 2: return launch_mla_tok_nq<T, WT, VEC, 2>(a, static_cast<int>(nq), static_cast<int>(nvc));
        case 4: return launch_mla_tok_nq<T, WT, VEC, 4>(a, static_cast<int>(nq), static_cast<int>(nvc));
        case 8: return launch_mla_tok_nq<T, WT, VEC, 8>(a, static_cast<int>(nq), static_cast<int>(nvc));
        default: break;
      }
    }
  }
  if (vec_ok) {
    const int nvc = pow2_ceil(cdiv(ncv, kWave));
    switch (j) {
      case 1: return launch_mla_nvc<T, WT, VEC, 1>(a, nvc);
      case 2: return launch_mla_nvc<T, WT, VEC, 2>(a, nvc);
      case 4: return launch_mla_nvc<T, WT, VEC, 4>(a, nvc);
      case 8: return launch_mla_nvc<T, WT, VEC, 8>(a, nvc);
      case 16: return launch_mla_nvc<T, WT, VEC, 16>(a, nvc);
      default: break;
    }
  }
  if (a.cache != nullptr) return EMBER_EALIGN;  // the caller runs the unfused pair
  const int64_t grid = cdiv(a.ntok, 4);
  hipLaunchKernelGGL((k_mla_any<T, WT>), dim3(static_cast<uint32_t>(grid)), dim3(256), 0, a.stream,
                     static_cast<const T*>(a.c), a.cts, static_cast<int>(a.R), static_cast<const T*>(a.kpe), a.kts,
                     static_cast<T*>(a.qpe), a.qts, a.qhs, static_cast<int>(a.H), static_cast<int>(half),
                     static_cast<const WT*>(a.w), a.eps, a.cos_t, a.sin_t, a.trows, a.tstride, a.pos, a.ntok,
                     static_cast<T*>(a.lat), a.lts, a.err);
  return launch_status();
}

}  // namespace
}  // namespace ember

extern "C" {

int ember_rope(void* q, int64_t q_token_stride, int64_t q_head_stride, int64_t num_q_heads, void* k,
               int64_t k_token_stride, int64_t k_head_stride, int64_t num_k_heads, int64_t head_dim,
               const float* cos_table, const float* sin_table, int64_t table_rows, int64_t table_row_stride,
               const int64_t* positions, int64_t num_tokens, int dtype, void* stream) {
  using namespace ember;
  RopeArgs a{q,        q_token_stride, q_head_stride, num_q_heads, k,        k_token_stride,
             k_head_stride, num_k_heads, head_dim, nullptr,     nullptr,  0.f,
             cos_table, sin_table, table_rows, table_row_stride, positions, num_tokens,
             static_cast<hipStream_t>(stream), nullptr};
  const int st = check_rope_args(a);
  if (st < 0) return EMBER_OK;
  if (st != EMBER_OK) return st;
  if (num_tokens > 0x7fffffffLL) return EMBER_EINVAL;
  a.err = device_error_word();
  if (a.err == nullptr) return EMBER_ENODEV;
  switch (dtype) {
    case EMBER_F32: return launch_typed<float, float, false>(a);
    case EMBER_F16: return launch_typed<_Float16, _Float16, false>(a);
    case EMBER_BF16: return launch_typed<__bf16, __bf16, false>(a);
    default: return EMBER_EINVAL;
  }
}

int ember_qk_norm_rope(void* q, int64_t q_token_stride, int64_t q_head_stride, int64_t num_q_heads, void* k,
                       int64_t k_token_stride, int64_t k_head_stride, int64_t num_k_heads, int64_t head_dim,
                       const void* q_weight, const void* k_weight, int weight_dtype, float eps,
                       const float* cos_table, const float* sin_table, int64_t table_rows,
                       int64_t table_row_stride, const int64_t* positions, int64_t num_tokens, int dtype,
                       void* stream) {
  using namespace ember;
  RopeArgs a{q,        q_token_stride, q_head_stride, num_q_heads, k,        k_token_stride,
             k_head_stride, num_k_heads, head_dim, q_weight,    k_weight, eps,
             cos_table, sin_table, table_rows, table_row_stride, positions, num_tokens,
             static_cast<hipStream_t>(stream), nullptr};
  const int st = check_rope_args(a);
  if (st < 0) return EMBER_OK;
  if (st != EMBER_OK) return st;
  if (num_tokens > 0x7fffffffLL) return EMBER_EINVAL;
  if ((num_q_heads > 0 && q_weight == nullptr) || (num_k_heads > 0 && k_weight == nullptr)) return EMBER_EINVAL;
  if (num_k_heads == 0) a.kw = q_weight;  // never read; keeps the pointer valid
  if (num_q_heads == 0) a.qw = k_weight;
  if (weight_dtype != dtype && weight_dtype != EMBER_F32) return EMBER_EINVAL;
  a.err = device_error_word();
  if (a.err == nullptr) return EMBER_ENODEV;
  const bool wf = weight_dtype == EMBER_F32;
  switch (dtype) {
    case EMBER_F32: return launch_typed<float, float, true>(a);
    case EMBER_F16: return wf ? launch_typed<_Float16, float, true>(a) : launch_typed<_Float16, _Float16, true>(a);
    case EMBER_BF16: return wf ? launch_typed<__bf16, float, true>(a) : launch_typed<__bf16, __bf16, true>(a);
    default: return EMBER_EINVAL;
  }
}

}  // extern "C"

namespace ember {
namespace {

int mla_entry(const void* c, int64_t c_token_stride, int64_t kv_lora_rank, const void* k_pe,
              int64_t k_pe_token_stride, void* q_pe, int64_t q_token_stride, int64_t q_head_stride,
              int64_t num_heads, int64_t rope_dim, const void* weight, int weight_dtype, float eps,
              const float* cos_table, const float* sin_table, int64_t table_rows, int64_t table_row_stride,
              const int64_t* positions, int64_t num_tokens, void* latent, int64_t latent_token_stride,
              const int64_t* slot_mapping, void* cache, int64_t num_slots, int64_t cache_slot_stride, int dtype,
              void* stream) {
  if (num_tokens < 0 || kv_lora_rank <= 0 || num_heads < 0 || rope_dim <= 0 || rope_dim % 2 != 0) return EMBER_EINVAL;
  if (kv_lora_rank > (1 << 20) || rope_dim > 4096 || num_heads > (1 << 20)) return EMBER_EINVAL;
  if (table_rows < 0 || table_row_stride < rope_dim / 2) return EMBER_EINVAL;
  if (weight_dtype != dtype && weight_dtype != EMBER_F32) return EMBER_EINVAL;
  if (num_tokens == 0) return EMBER_OK;
  if (num_tokens > 0x1ffffffffLL) return EMBER_EINVAL;
  if (c == nullptr || k_pe == nullptr || weight == nullptr || positions == nullptr || cos_table == nullptr ||
      sin_table == nullptr || (num_heads > 0 && q_pe == nullptr))
    return EMBER_EINVAL;
  if (latent == nullptr && cache == nullptr) return EMBER_EINVAL;
  if (latent != nullptr && latent_token_stride < kv_lora_rank + rope_dim) return EMBER_EINVAL;
  if (cache != nullptr && (slot_mapping == nullptr || num_slots < 0 || cache_slot_stride < kv_lora_rank + rope_dim))
    return EMBER_EINVAL;
  MlaArgs a{c,          c_token_stride, kv_lora_rank, k_pe,      k_pe_token_stride,
            q_pe == nullptr ? (latent != nullptr ? latent : cache) : q_pe,
            q_token_stride, q_head_stride, num_heads, rope_dim, weight,   eps,
            cos_table,  sin_table,      table_rows,   table_row_stride, positions, num_tokens,
            latent,     latent_token_stride, static_cast<hipStream_t>(stream), nullptr};
  a.slots = slot_mapping;
  a.cache = cache;
  a.num_slots = num_slots;
  a.css = cache_slot_stride;
  a.err = device_error_word();
  if (a.err == nullptr) return EMBER_ENODEV;
  const bool wf = weight_dtype == EMBER_F32 && dtype != EMBER_F32;
  switch (dtype) {
    case EMBER_F32: return launch_mla_typed<float, float>(a);
    case EMBER_F16: return wf ? launch_mla_typed<_Float16, float>(a) : launch_mla_typed<_Float16, _Float16>(a);
    case EMBER_BF16: return wf ? launch_mla_typed<__bf16, float>(a) : launch_mla_typed<__bf16, __bf16>(a);
    default: return EMBER_EINVAL;
  }
}

}  // namespace
}  // namespace ember

extern "C" {

int ember_mla_latent_rope(const void* c, int64_t c_token_stride, int64_t kv_lora_rank, const void* k_pe,
                          int64_t k_pe_token_stride, void* q_pe, int64_t q_token_stride, int64_t q_head_stride,
                          int64_t num_heads, int64_t rope_dim, const void* weight, int weight_dtype, float eps,
                          const float* cos_table, const float* sin_table, int64_t table_rows,
                          int64_t table_row_stride, const int64_t* positions, int64_t num_tokens, void* latent,
                          int64_t latent_token_stride, int dtype, void* stream) {
  if (latent == nullptr) return EMBER_EINVAL;
  return ember::mla_entry(c, c_token_stride, kv_lora_rank, k_pe, k_pe_token_stride, q_pe, q_token_stride,
                          q_head_stride, num_heads, rope_dim, weight, weight_dtype, eps, cos_table, sin_table,
                          table_rows, table_row_stride, positions, num_tokens, latent, latent_token_stride, nullptr,
                          nullptr, 0, 0, dtype, stream);
}

int ember_mla_latent_rope_cache(const void* c, int64_t c_token_stride, int64_t kv_lora_rank, const void* k_pe,
                                int64_t k_pe_token_stride, void* q_pe, int64_t q_token_stride, int64_t q_head_stride,
                                int64_t num_heads, int64_t rope_dim, const void* weight, int weight_dtype, float eps,
                                const float* cos_table, const float* sin_table, int64_t table_rows,
                                int64_t table_row_stride, const int64_t* positions, int64_t num_tokens,
                                void* latent, int64_t latent_token_stride, const int64_t* slot_mapping, void* cache,
                                int64_t num_slots, int64_t cache_slot_stride, int dtype, void* stream) {
  if (cache == nullptr) return EMBER_EINVAL;
  return ember::mla_entry(c, c_token_stride, kv_lora_rank, k_pe, k_pe_token_stride, q_pe, q_token_stride,
                          q_head_stride, num_heads, rope_dim, weight, weight_dtype, eps, cos_table, sin_table,
                          table_rows, table_row_stride, positions, num_tokens, latent, latent_token_stride,
                          slot_mapping, cache, num_slots, cache_slot_stride, dtype, stream);
}

int ember_rope_kv_cache(void* q, int64_t q_token_stride, int64_t q_head_stride, int64_t num_q_heads, void* k,
                        int64_t k_token_stride, int64_t k_head_stride, int64_t num_kv_heads, const void* v,
                        int64_t v_token_stride, int64_t v_head_stride, int64_t head_dim, const void* q_weight,
                        const void* k_weight, int weight_dtype, float eps, const float* cos_table,
                        const float* sin_table, int64_t table_rows, int64_t table_row_stride,
                        const int64_t* positions, const int64_t* slot_mapping, int64_t num_tokens, void* k_cache,
                        void* v_cache, int64_t num_slots, int64_t cache_slot_stride, int64_t cache_head_stride,
                        int dtype, void* stream) {
  using namespace ember;
  RopeKvArgs a{RopeArgs{q,        q_token_stride, q_head_stride, num_q_heads, k,        k_token_stride,
                        k_head_stride, num_kv_heads, head_dim, q_weight,    k_weight, eps,
                        cos_table, sin_table, table_rows, table_row_stride, positions, num_tokens,
                        static_cast<hipStream_t>(stream), nullptr},
               v, v_token_stride, v_head_stride, slot_mapping, k_cache, v_cache, num_slots, cache_slot_stride,
               cache_head_stride};
  const int st = check_rope_args(a.r);
  if (st < 0) return EMBER_OK;
  if (st != EMBER_OK) return st;
  if (num_kv_heads <= 0 || v == nullptr || k == nullptr || slot_mapping == nullptr || k_cache == nullptr ||
      v_cache == nullptr || num_slots < 0 || num_tokens > 0x7fffffffLL)
    return EMBER_EINVAL;
  const bool norm = q_weight != nullptr;
  if (norm && (k_weight == nullptr || (weight_dtype != dtype && weight_dtype != EMBER_F32))) return EMBER_EINVAL;
  a.r.err = device_error_word();
  if (a.r.err == nullptr) return EMBER_ENODEV;
  const bool wf = norm && weight_dtype == EMBER_F32 && dtype != EMBER_F32;
  switch (dtype) {
    case EMBER_F32:
      return norm ? launch_rope_kv_typed<float, float, true>(a) : launch_rope_kv_typed<float, float, false>(a);
    case EMBER_F16:
      if (!norm) return launch_rope_kv_typed<_Float16, _Float16, false>(a);
      return wf ? launch_rope_kv_typed<_Float16, float, true>(a) : launch_rope_kv_typed<_Float16, _Float16, true>(a);
    case EMBER_BF16:
      if (!norm) return launch_rope_kv_typed<__bf16, __bf16, false>(a);
      return wf ? launch_rope_kv_typed<__bf16, float, true>(a) : launch_rope_kv_typed<__bf16, __bf16, true>(a);
    default: return EMBER_EINVAL;
  }
}

}  // extern "C"
