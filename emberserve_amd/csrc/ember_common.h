// Device-side building blocks shared by the gfx950 kernels of libember_ops.so.
//
// Conventions of every kernel in this library:
//  * storage dtypes fp32 / fp16 / bf16, all arithmetic in fp32;
//  * "round_to<T>(v)" is the round-to-nearest-even cast to T and back, i.e. the rounding a
//    PyTorch eager op applies when it writes a half-precision tensor;
//  * the library is compiled with -ffp-contract=off, so a*b+c is two rounded operations,
//    as in the reference's separate element-wise tensor ops;
//  * 16-byte (dwordx4) accesses: a "Pack<T, VEC>" is VEC elements = 16 bytes for the
//    vector kernels (VEC = 8 for fp16/bf16, 4 for fp32);
//  * reductions stay inside a wavefront (DPP row ops, one ds_swizzle, v_readlane) and
//    touch LDS only to combine the waves of a multi-wave row team.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/ember_ops.h"

namespace ember {

constexpr int kWave = 64;

// The slot of a padding row in the paged-cache writes: skipped without an error.
constexpr int64_t kPadSlot = -1;

// ---------------------------------------------------------------- dtype conversion

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(_Float16 v) { return static_cast<float>(v); }
__device__ __forceinline__ float to_f32(__bf16 v) { return static_cast<float>(v); }

template <typename T>
__device__ __forceinline__ T from_f32(float v) { return static_cast<T>(v); }  // RNE

// The fp16 cast takes an fp32 value that is already rounded: without the empty asm, hipcc
// folds `(_Float16)(a * b)` into v_fma_mixlo_f16, which rounds the exact product to fp16
// once, where the reference rounds it to fp32 first and then to fp16 (the two differ when
// the fp32 rounding lands on an fp16 tie).
template <>
__device__ __forceinline__ _Float16 from_f32<_Float16>(float v) {
  asm("" : "+v"(v));
  return static_cast<_Float16>(v);
}

template <typename T>
__device__ __forceinline__ float round_to(float v) { return to_f32(from_f32<T>(v)); }

// The product of two fp16/bf16 values is exact in fp32 (at most 22 significant bits, far
// from fp32's range limits), so rounding the exact product to T once, as v_fma_mixlo_f16
// does, equals rounding its fp32 value: the plain cast, free to fold.
template <typename T>
__device__ __forceinline__ T half_product(float a_half, float b_half) {
  return static_cast<T>(a_half * b_half);
}

// Correctly rounded fp32 square root (the value of IEEE sqrt, as torch's CPU rsqrt path
// 1 / sqrt(x) uses). v_sqrt_f32 alone is accurate to 1 ulp, so its result s is corrected by
// the sign of the exact residuals x - s' s for the neighbours s' = s -/+ 1 ulp (one fma
// each): x <= s_dn s puts sqrt(x) at or below the s_dn / s midpoint, x > s_up s above the
// s / s_up midpoint. Inputs below 2^-96 are scaled by 2^32 first (and the root by 2^-16) so
// that the neighbours stay normal; zero, infinity, NaN and negative inputs take the
// hardware result.
__device__ __forceinline__ float sqrt_rn(float x) {
  const bool tiny = x < 0x1p-96f;
  const float xs = tiny ? x * 0x1p+32f : x;
  const float s0 = __builtin_amdgcn_sqrtf(xs);
  const int bits = __builtin_bit_cast(int, s0);
  const float s_dn = __builtin_bit_cast(float, bits - 1);
  const float s_up = __builtin_bit_cast(float, bits + 1);
  const float r_dn = __builtin_fmaf(-s_dn, s0, xs);
  const float r_up = __builtin_fmaf(-s_up, s0, xs);
  float s = r_dn <= 0.f ? s_dn : s0;
  s = r_up > 0.f ? s_up : s;
  s = (xs > 0.f && xs < __builtin_huge_valf()) ? s : s0;
  return tiny ? s * 0x1p-16f : s;
}

// ---------------------------------------------------------------- 16-byte packs

template <typename T, int N>
struct alignas(sizeof(T) * N) Pack {
  T v[N];
};

template <typename T, int N>
__device__ __forceinline__ Pack<T, N> load_pack(const T* p) {
  return *reinterpret_cast<const Pack<T, N>*>(p);
}

template <typename T, int N>
__device__ __forceinline__ void store_pack(T* p, const Pack<T, N>& v) {
  *reinterpret_cast<Pack<T, N>*>(p) = v;
}

// Streaming (non-temporal) 16-byte accesses for data touched exactly once per launch
// (activations read, rows written): the nt hint keeps these lines from displacing reused
// data (weights, cos/sin tables, positions) in L2 and the Infinity Cache. Measured on
// MI355X: +13-17% HBM throughput for the in-place rope and the copy-like kernels. Packs of
// other sizes (the scalar fallback kernels) use ordinary accesses.
template <typename T, int N>
__device__ __forceinline__ Pack<T, N> load_stream(const T* p) {
  if constexpr (sizeof(T) * N == 16) {
    using V = unsigned int __attribute__((ext_vector_type(4)));
    const V v = __builtin_nontemporal_load(reinterpret_cast<const V*>(p));
    return __builtin_bit_cast(Pack<T, N>, v);
  } else {
    return load_pack<T, N>(p);
  }
}

template <typename T, int N>
__device__ __forceinline__ void store_stream(T* p, const Pack<T, N>& v) {
  if constexpr (sizeof(T) * N == 16) {
    using V = unsigned int __attribute__((ext_vector_type(4)));
    __builtin_nontemporal_store(__builtin_bit_cast(V, v), reinterpret_cast<V*>(p));
  } else {
    store_pack<T, N>(p, v);
  }
}

// Loads N consecutive values of type T (16-byte aligned when N * sizeof(T) >= 16) as fp32.
template <typename T, int N>
__device__ __forceinline__ void load_vals(const T* p, float (&out)[N]) {
  constexpr int kPer = 16 / sizeof(T);
  if constexpr (N < kPer) {
#pragma unroll
    for (int e = 0; e < N; ++e) out[e] = to_f32(p[e]);
  } else {
#pragma unroll
    for (int h = 0; h < N; h += kPer) {
      Pack<T, kPer> q = load_pack<T, kPer>(p + h);
#pragma unroll
      for (int e = 0; e < kPer; ++e) out[h + e] = to_f32(q.v[e]);
    }
  }
}

// ---------------------------------------------------------------- wave reductions

// DPP controls (GCN/CDNA encoding).
constexpr int kDppQuadSwap1 = 0xB1;     // quad_perm [1,0,3,2]
constexpr int kDppQuadSwap2 = 0x4E;     // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

template <int Ctrl>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), Ctrl, 0xF, 0xF, false));
}

// ds_swizzle in bit-mask mode: lane i reads lane (i ^ 16) within its 32-lane half.
__device__ __forceinline__ float swizzle_xor16(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
}

// Sum over aligned groups of W lanes (W a power of two <= 64). Every lane of a group must
// be active; lanes only read lanes of their own group, so other groups may be inactive.
// All lanes of a group return the same bits (the pairing order is symmetric).
template <int W>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(W >= 1 && W <= 64 && (W & (W - 1)) == 0, "group width");
  if constexpr (W >= 2) v += dpp_f32<kDppQuadSwap1>(v);
  if constexpr (W >= 4) v += dpp_f32<kDppQuadSwap2>(v);
  if constexpr (W >= 8) v += dpp_f32<kDppRowHalfMirror>(v);
  if constexpr (W >= 16) v += dpp_f32<kDppRowMirror>(v);
  if constexpr (W >= 32) v += swizzle_xor16(v);
  if constexpr (W >= 64) {
    const float lo = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float hi = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    v = lo + hi;
  }
  return v;
}

// Lane i of a 16-lane DPP row reads lane i + N of the same row (N in 1..15). Lanes whose
// source lies past the row end read 0; callers only use lanes whose source is in-row.
template <int N>
__device__ __forceinline__ float dpp_shl(float v) {
  static_assert(N >= 1 && N <= 15, "row_shl distance");
  return dpp_f32<0x100 + N>(v);
}

// Sum of squares of one row in the order of PyTorch's CPU fp32 sum over a contiguous last
// dimension (aten/src/ATen/native/cpu/SumKernel.cpp: 8-wide vectors, four interleaved
// accumulators; for at most 64 vectors per row, i.e. at most 16 vectors per accumulator,
// every accumulator is a plain left-to-right chain). With that order the kernel's sum is
// bit-identical to `x.float().pow(2).mean(-1)` * cols on the CPU, so the normalised row
// rounds exactly as torch-eager's does.
//
// Row layout: an aligned group of TPR lanes (TPR in {4, 8, 16}: the group lies inside one
// DPP row) holds the row's 8-element vectors, vector v in lane v % TPR, register v / TPR,
// as `sq[v / TPR][e]` = element 8 v + e squared (already rounded to fp32). Accumulator k
// (k < 4) sums vectors k, k + 4, k + 8, ... element-wise; lane k of the group runs that
// chain. The four accumulators are then added in order (lane 0 reads lanes 1, 2, 3) and
// lane 0's eight elements summed left to right; a swizzle hands lane 0's total to the
// group. Every lane of the group must be active.
template <int TPR, int NV>
__device__ __forceinline__ float torch_order_sumsq(const float (&sq)[NV][8]) {
  constexpr int kVecs = TPR * NV;
  static_assert(TPR == 4 || TPR == 8 || TPR == 16, "group must fit one DPP row");
  static_assert(kVecs % 4 == 0 && kVecs <= 64, "sequential-accumulator regime only");
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = sq[0][e];
#pragma unroll
  for (int r = 1; r < kVecs / 4; ++r) {
    const int i = (4 * r) / TPR;  // compile-time after unrolling
    const int d = (4 * r) % TPR;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float x = sq[i][e];
      if (d == 4) x = dpp_shl<4>(x);
      else if (d == 8) x = dpp_shl<8>(x);
      else if (d == 12) x = dpp_shl<12>(x);
      acc[e] = acc[e] + x;
    }
  }
  float tot = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float p = acc[e] + dpp_shl<1>(acc[e]);
    p = p + dpp_shl<2>(acc[e]);
    p = p + dpp_shl<3>(acc[e]);
    tot = tot + p;
  }
  // ds_swizzle bit mode: lane i reads lane (i & ~(TPR - 1)) of its 32-lane half.
  constexpr int kAnd = 0x1F & ~(TPR - 1);
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, tot), kAnd));
}

// ---------------------------------------------------------------- packed gate_up layout
//
// The dense gate_up weight packed for a grid of G decode workgroups: total = (I / 64) (H / 64)
// units of 16 KiB, unit u = slab * (H / 64) + j holding the 64-row slab's gate and up rows
// over k in [64 j, 64 j + 64) as MFMA operand fragments. The decode kernel's workgroups own
// contiguous unit runs; the prefill GEMM reads the same array by unit.
// Workgroup b's units are [start(b), start(b + 1)), start(b) = floor(b total / G); the
// workgroup that holds unit u is floor(((u + 1) G - 1) / total).
__device__ __host__ __forceinline__ int64_t gu_start(int64_t b, int64_t total, int64_t G) { return b * total / G; }
__device__ __host__ __forceinline__ int64_t gu_owner(int64_t u, int64_t total, int64_t G) {
  return ((u + 1) * G - 1) / total;
}
// Where the packed weight layout keeps unit t of workgroup b's run, in units: runs hold q =
// total / G or q + 1 units, so the t-th units of all workgroups (t < q) are stored side by
// side in workgroup order, t-major, and the extra units of the longer runs follow, also in
// workgroup order. At any moment the grid then reads one narrow window of the array.
__device__ __host__ __forceinline__ int64_t gu_packed_pos(int64_t b, int64_t t, int64_t total, int64_t G) {
  const int64_t q = total / G;
  return t < q ? t * G + b : q * G + (gu_start(b, total, G) - b * q);
}


// ---------------------------------------------------------------- integer division

// Division of a uint32 n < 2^31 by a runtime-constant d >= 1 with one mul-hi
// (Granlund-Montgomery, round-up variant).
struct FastDiv {
  uint32_t d;
  uint32_t m;
  uint32_t s;

  __host__ static FastDiv make(uint32_t d) {
    FastDiv f;
    f.d = d;
    uint32_t s = 0;
    while ((uint64_t(1) << s) < d) ++s;
    f.s = s;
    f.m = static_cast<uint32_t>(((uint64_t(1) << 32) * ((uint64_t(1) << s) - d)) / d + 1);
    return f;
  }
  __device__ __forceinline__ uint32_t div(uint32_t n) const {
    return (__umulhi(n, m) + n) >> s;
  }
};

// ---------------------------------------------------------------- host helpers

// ---------------------------------------------------------------- split-K partials

// Agent-coherent vector accesses for split-K partials that one workgroup writes and another
// (possibly on another XCD, whose L2 is separate) reads in the same launch: buffer
// loads/stores with the sc1 cache policy, the bit that agent-scope atomic accesses carry,
// so stores are written through and loads are served from memory, not a stale L2 line.
typedef __amdgpu_buffer_rsrc_t CoherentRsrc;
constexpr int kBufferWord3 = 0x00020000;  // raw 32-bit buffer, gfx9 format
constexpr int kPolicySc1 = 16;

template <int V>
struct FloatVec;
template <>
struct FloatVec<2> {
  typedef float type __attribute__((ext_vector_type(2)));
};
template <>
struct FloatVec<4> {
  typedef float type __attribute__((ext_vector_type(4)));
};

// A resource over `floats` fp32 values from `base` (out-of-range accesses return zero and
// are dropped by the hardware).
__device__ __forceinline__ CoherentRsrc coherent_rsrc(const float* base, int floats) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, floats * int(sizeof(float)), kBufferWord3);
}

template <int V>
__device__ __forceinline__ void store_coherent(CoherentRsrc r, int byte_off, typename FloatVec<V>::type v) {
  if constexpr (V == 4) {
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, byte_off, 0, kPolicySc1);
  } else {
    typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, v), r, byte_off, 0, kPolicySc1);
  }
}

template <int V>
__device__ __forceinline__ typename FloatVec<V>::type load_coherent(CoherentRsrc r, int byte_off) {
  using F = typename FloatVec<V>::type;
  if constexpr (V == 4) return __builtin_bit_cast(F, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kPolicySc1));
  else return __builtin_bit_cast(F, __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, kPolicySc1));
}

// ---------------------------------------------------------------- host helpers
__host__ inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

__host__ inline int dtype_size(int dtype) {
  switch (dtype) {
    case EMBER_F32: return 4;
    case EMBER_F16: return 2;
    case EMBER_BF16: return 2;
    default: return 0;
  }
}

__host__ inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

__host__ inline int pow2_ceil(int64_t v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}

// Returns the device address of this library's error word on the current device.
__host__ uint32_t* device_error_word();

// Compute units of the current device (cached per device); 0 if the query fails.
__host__ int device_cu_count();

__host__ inline int launch_status() {
  return hipGetLastError() == hipSuccess ? EMBER_OK : EMBER_ELAUNCH;
}

}  // namespace ember
