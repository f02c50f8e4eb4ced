// RMSNorm and fused residual-add + RMSNorm for gfx950.
//
// Reference semantics (emberserve/model/ops.py:51-63, ops_triton.py:16-34):
//   r'  = round(x + r)                                   (fused variant only)
//   y   = round(v * (1 / sqrt(sum(v^2) / H + eps)))      v = r' or x, fp32 math
//   out = round(y * w)
//
// Layout in HBM: rows of H elements, unit stride inside a row, arbitrary row stride.
// Work mapping: a "row team" of TPR lanes owns one row; lane l holds the 16-byte packs
// l, l+TPR, ..., l+(NV-1)*TPR of the row in registers, so each input byte is read from HBM
// exactly once and the sum of squares and the scale pass both run out of registers. A
// team of <= 64 lanes reduces with DPP inside its wave; wider teams combine per-wave
// partials through LDS. TPR is chosen per launch so that small batches still spread over
// enough waves to fill the chip.
#include "ember_common.h"

#ifdef EMBER_NORM_DEBUG_TOTAL
__device__ float ember_norm_debug_total[4096];
#endif

namespace ember {
namespace {

template <typename T, typename WT, int VEC, int TPR, int NV, bool RESID>
__global__ void __launch_bounds__(TPR >= 256 ? TPR : 256)
k_rmsnorm(const T* __restrict__ x, int64_t xs, const T* __restrict__ r, int64_t rs,
          const WT* __restrict__ w, T* __restrict__ out, int64_t os,
          T* __restrict__ rout, int64_t ros, int64_t rows, int cols, float eps) {
  constexpr int kBlock = TPR >= 256 ? TPR : 256;
  constexpr int kRowsPerBlock = kBlock / TPR;
  constexpr int kWavesPerTeam = TPR > kWave ? TPR / kWave : 1;
  const int team = threadIdx.x / TPR;
  const int lane = threadIdx.x % TPR;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + team;
  const bool live = row < rows;
  const int nvec = cols / VEC;
  // Loads are unconditional, from clamped (always valid) addresses, so that every load of
  // the row is in flight before the first wait; masked lanes discard what they read.
  const int64_t lrow = live ? row : rows - 1;

  Pack<T, VEC> a[NV];
  Pack<T, VEC> b[NV];
  float wv[NV][VEC];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int vi = min(lane + i * TPR, nvec - 1);
    a[i] = load_stream<T, VEC>(x + lrow * xs + static_cast<int64_t>(vi) * VEC);
    if constexpr (RESID) b[i] = load_stream<T, VEC>(r + lrow * rs + static_cast<int64_t>(vi) * VEC);
  }
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int vi = min(lane + i * TPR, nvec - 1);
    load_vals<WT, VEC>(w + static_cast<int64_t>(vi) * VEC, wv[i]);
  }

  float v[NV][VEC];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int vi = lane + i * TPR;
    const bool ok = live && vi < nvec;
    Pack<T, VEC> s;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      float f = to_f32(a[i].v[e]);
      if constexpr (RESID) {
        const T sum = from_f32<T>(f + to_f32(b[i].v[e]));
        s.v[e] = sum;
        f = to_f32(sum);
      }
      f = ok ? f : 0.f;  // packs past the row end (clamped loads) contribute nothing
      v[i][e] = f;
      ss += f * f;
    }
    if constexpr (RESID) {
      if (ok) store_stream<T, VEC>(rout + row * ros + static_cast<int64_t>(vi) * VEC, s);
    }
  }

  float total;
  if constexpr (VEC == 8 && TPR <= 16 && TPR * NV <= 64) {
    // Rows of at most 64 packs whose pack count is a multiple of 4 (the launcher caps the
    // team at 16 lanes for them): PyTorch's CPU summation order, zero packs past the row
    // end extending the accumulator chains without changing them.
    (void)ss;
    float sq[NV][8];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
#pragma unroll
      for (int e = 0; e < 8; ++e) sq[i][e] = v[i][e] * v[i][e];
    }
    total = nvec % 4 == 0 ? torch_order_sumsq<TPR, NV>(sq) : group_sum<TPR>(ss);
  } else if constexpr (TPR <= kWave) {
    total = group_sum<TPR>(ss);
  } else {
    __shared__ float partial[kRowsPerBlock][kWavesPerTeam];
    const float wsum = group_sum<kWave>(ss);
    const int wave_in_team = lane / kWave;
    if ((lane % kWave) == 0) partial[team][wave_in_team] = wsum;
    __syncthreads();
    total = 0.f;
#pragma unroll
    for (int k = 0; k < kWavesPerTeam; ++k) total += partial[team][k];
  }
#ifdef EMBER_NORM_DEBUG_TOTAL
  if (lane == 0 && live) ember_norm_debug_total[row] = total;
#endif
  const float var = total / static_cast<float>(cols);
  const float inv = 1.0f / sqrt_rn(var + eps);

#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int vi = lane + i * TPR;
    if (live && vi < nvec) {
      Pack<T, VEC> o;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float y = round_to<T>(v[i][e] * inv);
        o.v[e] = from_f32<T>(y * wv[i][e]);
      }
      store_stream<T, VEC>(out + row * os + static_cast<int64_t>(vi) * VEC, o);
    }
  }
}

// Any shape, any alignment: one 256-lane block per row, scalar accesses, two passes (the
// second re-reads the row, normally from L2). Used only when the vector path's
// alignment or size conditions fail.
template <typename T, bool RESID>
__global__ void __launch_bounds__(256)
k_rmsnorm_any(const T* __restrict__ x, int64_t xs, const T* __restrict__ r, int64_t rs,
              const void* __restrict__ w, int w_f32, T* __restrict__ out, int64_t os,
              T* __restrict__ rout, int64_t ros, int cols, float eps) {
  const int64_t row = blockIdx.x;
  float ss = 0.f;
  for (int c = threadIdx.x; c < cols; c += 256) {
    float f = to_f32(x[row * xs + c]);
    if constexpr (RESID) {
      const T sum = from_f32<T>(f + to_f32(r[row * rs + c]));
      rout[row * ros + c] = sum;
      f = to_f32(sum);
    }
    ss += f * f;
  }
  __shared__ float partial[256 / kWave];
  const float wsum = group_sum<kWave>(ss);
  if ((threadIdx.x % kWave) == 0) partial[threadIdx.x / kWave] = wsum;
  __syncthreads();
  float total = 0.f;
#pragma unroll
  for (int k = 0; k < 256 / kWave; ++k) total += partial[k];
  const float inv = 1.0f / sqrt_rn(total / static_cast<float>(cols) + eps);
  for (int c = threadIdx.x; c < cols; c += 256) {
    float f = to_f32(x[row * xs + c]);
    if constexpr (RESID) f = round_to<T>(f + to_f32(r[row * rs + c]));
    const float wf = w_f32 ? static_cast<const float*>(w)[c] : to_f32(static_cast<const T*>(w)[c]);
    out[row * os + c] = from_f32<T>(round_to<T>(f * inv) * wf);
  }
}

struct NormArgs {
  const void* x;
  int64_t xs;
  const void* r;
  int64_t rs;
  const void* w;
  bool w_f32;  // fp32 weights with half-precision activations
  void* out;
  int64_t os;
  void* rout;
  int64_t ros;
  int64_t rows;
  int64_t cols;
  float eps;
  hipStream_t stream;
};

template <typename T, typename WT, int VEC, int TPR, int NV, bool RESID>
int launch_vec(const NormArgs& a) {
  constexpr int kBlock = TPR >= 256 ? TPR : 256;
  constexpr int kRowsPerBlock = kBlock / TPR;
  const int64_t grid = cdiv(a.rows, kRowsPerBlock);
  hipLaunchKernelGGL((k_rmsnorm<T, WT, VEC, TPR, NV, RESID>), dim3(static_cast<uint32_t>(grid)),
                     dim3(kBlock), 0, a.stream, static_cast<const T*>(a.x), a.xs, static_cast<const T*>(a.r),
                     a.rs, static_cast<const WT*>(a.w), static_cast<T*>(a.out), a.os, static_cast<T*>(a.rout),
                     a.ros, a.rows, static_cast<int>(a.cols), a.eps);
  return launch_status();
}

template <typename T, typename WT, int VEC, int TPR, bool RESID>
int launch_nv(const NormArgs& a, int nv) {
  switch (nv) {
    case 1: return launch_vec<T, WT, VEC, TPR, 1, RESID>(a);
    case 2: return launch_vec<T, WT, VEC, TPR, 2, RESID>(a);
    case 4: return launch_vec<T, WT, VEC, TPR, 4, RESID>(a);
    case 8: return launch_vec<T, WT, VEC, TPR, 8, RESID>(a);
    default: return EMBER_EINVAL;
  }
}

template <typename T, typename WT, int VEC, bool RESID>
int launch_tpr(const NormArgs& a, int tpr, int nv) {
  switch (tpr) {
    case 8: return launch_nv<T, WT, VEC, 8, RESID>(a, nv);
    case 16: return launch_nv<T, WT, VEC, 16, RESID>(a, nv);
    case 32: return launch_nv<T, WT, VEC, 32, RESID>(a, nv);
    case 64: return launch_nv<T, WT, VEC, 64, RESID>(a, nv);
    case 128: return launch_nv<T, WT, VEC, 128, RESID>(a, nv);
    case 256: return launch_nv<T, WT, VEC, 256, RESID>(a, nv);
    case 512: return launch_nv<T, WT, VEC, 512, RESID>(a, nv);
    case 1024: return launch_nv<T, WT, VEC, 1024, RESID>(a, nv);
    default: return EMBER_EINVAL;
  }
}

// Row teams are widened (fewer packs per lane) until a launch has this many lanes or the
// team reaches one pack per lane. Measured on MI355X ([8192, 4096] bf16 fused add): 64
// lanes x 8 packs 69%, 256 x 2 74%, 512 x 1 76% of HBM peak.
#ifndef EMBER_NORM_TARGET_THREADS
#define EMBER_NORM_TARGET_THREADS 4194304
#endif
constexpr int64_t kTargetThreads = EMBER_NORM_TARGET_THREADS;

// Picks the row-team width: the narrowest team that holds the row in <= 8 packs per lane,
// widened (fewer packs per lane) while the launch would have too few threads in flight.
// Rows of <= 64 packs of 8 elements (a multiple of 4 packs) stay on teams of <= 16 lanes,
// where the kernel sums the squares in PyTorch's CPU order.
__host__ inline void pick_team(int64_t nvec, int64_t rows, bool torch_order, int* tpr_out, int* nv_out) {
  int tpr = pow2_ceil(cdiv(nvec, 8));
  if (tpr < 8) tpr = 8;
  if (tpr > 1024) {
    *tpr_out = 0;
    return;
  }
  const int64_t p2 = pow2_ceil(nvec);
  const int cap = torch_order && nvec <= 64 && nvec % 4 == 0 ? 16 : 1024;
  while (tpr < cap && tpr * 2 <= p2 && rows * tpr < kTargetThreads) tpr *= 2;
  *tpr_out = tpr;
  *nv_out = pow2_ceil(cdiv(nvec, tpr));
}

template <typename T, typename WT, bool RESID>
int launch_typed(const NormArgs& a) {
  constexpr int VEC = 16 / sizeof(T);
  bool vec_ok = a.cols % VEC == 0 && a.xs % VEC == 0 && a.os % VEC == 0 && aligned16(a.x) &&
                aligned16(a.out) && aligned16(a.w);
  if (RESID) vec_ok = vec_ok && a.rs % VEC == 0 && a.ros % VEC == 0 && aligned16(a.r) && aligned16(a.rout);
  if (vec_ok) {
    int tpr = 0, nv = 0;
    pick_team(a.cols / VEC, a.rows, VEC == 8, &tpr, &nv);
    if (tpr != 0) return launch_tpr<T, WT, VEC, RESID>(a, tpr, nv);
  }
  hipLaunchKernelGGL((k_rmsnorm_any<T, RESID>), dim3(static_cast<uint32_t>(a.rows)), dim3(256), 0, a.stream,
                     static_cast<const T*>(a.x), a.xs, static_cast<const T*>(a.r), a.rs, a.w,
                     a.w_f32 ? 1 : 0, static_cast<T*>(a.out), a.os, static_cast<T*>(a.rout), a.ros,
                     static_cast<int>(a.cols), a.eps);
  return launch_status();
}

template <bool RESID>
int launch(NormArgs a, int dtype, int weight_dtype) {
  if (a.rows < 0 || a.cols <= 0 || a.cols > (int64_t(1) << 30)) return EMBER_EINVAL;
  if (a.rows > 0x7fffffffLL) return EMBER_EINVAL;
  if (weight_dtype != dtype && weight_dtype != EMBER_F32) return EMBER_EINVAL;
  if (a.rows == 0) return EMBER_OK;
  if (a.x == nullptr || a.w == nullptr || a.out == nullptr) return EMBER_EINVAL;
  if (RESID && (a.r == nullptr || a.rout == nullptr)) return EMBER_EINVAL;
  a.w_f32 = weight_dtype == EMBER_F32 && dtype != EMBER_F32;
  switch (dtype) {
    case EMBER_F32: return launch_typed<float, float, RESID>(a);
    case EMBER_F16:
      return a.w_f32 ? launch_typed<_Float16, float, RESID>(a) : launch_typed<_Float16, _Float16, RESID>(a);
    case EMBER_BF16:
      return a.w_f32 ? launch_typed<__bf16, float, RESID>(a) : launch_typed<__bf16, __bf16, RESID>(a);
    default: return EMBER_EINVAL;
  }
}

}  // namespace
}  // namespace ember

extern "C" {

int ember_rmsnorm(const void* x, int64_t x_row_stride, const void* weight, int weight_dtype, void* out,
                  int64_t out_row_stride, int64_t rows, int64_t cols, float eps, int dtype, void* stream) {
  const ember::NormArgs a{x,   x_row_stride,   nullptr, 0,    weight, false, out,
                          out_row_stride, nullptr, 0,    rows, cols,   eps,   static_cast<hipStream_t>(stream)};
  return ember::launch<false>(a, dtype, weight_dtype);
}

int ember_fused_add_rmsnorm(const void* x, int64_t x_row_stride, const void* residual,
                            int64_t residual_row_stride, const void* weight, int weight_dtype, void* out,
                            int64_t out_row_stride, void* residual_out, int64_t residual_out_row_stride,
                            int64_t rows, int64_t cols, float eps, int dtype, void* stream) {
  const ember::NormArgs a{x,    x_row_stride, residual, residual_row_stride, weight, false,
                          out,  out_row_stride, residual_out, residual_out_row_stride,
                          rows, cols,         eps,      static_cast<hipStream_t>(stream)};
  return ember::launch<true>(a, dtype, weight_dtype);
}

}  // extern "C"
