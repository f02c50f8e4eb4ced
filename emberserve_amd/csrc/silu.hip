// SiLU-and-mul (SwiGLU activation) for gfx950.
//
// Reference semantics (emberserve/model/ops.py:84-87, ops_triton.py:73-83):
//   out[r, j] = round(round(g / (1 + exp(-g))) * u),  g = x[r, j], u = x[r, I + j]
// with fp32 math and rounding to the storage dtype at the two marked points.
//
// Layout: x is [rows, 2I] (gate half then up half of each row), out is [rows, I]; unit
// stride inside rows. Work mapping: a 256-lane block owns U * 256 consecutive 16-byte packs
// of one row's gate half and the matching packs of its up half; every load of the block
// is issued before the first use. Traffic is the minimum, 3 * I * elem bytes per row.
#include "ember_common.h"

#ifndef EMBER_SILU_U
#define EMBER_SILU_U 2
#endif
#ifndef EMBER_SILU_MIN_THREADS
#define EMBER_SILU_MIN_THREADS 131072
#endif

namespace ember {
namespace {

template <typename T, int VEC, int U>
__global__ void __launch_bounds__(256)
k_silu_mul(const T* __restrict__ x, int64_t xs, T* __restrict__ out, int64_t os, int nvec,
           int col_blocks) {
  const uint32_t row = blockIdx.x / static_cast<uint32_t>(col_blocks);
  const int cblk = static_cast<int>(blockIdx.x - row * static_cast<uint32_t>(col_blocks));
  const int base = cblk * (256 * U) + static_cast<int>(threadIdx.x);
  const int64_t inter = static_cast<int64_t>(nvec) * VEC;
  const T* xr = x + static_cast<int64_t>(row) * xs;
  T* orow = out + static_cast<int64_t>(row) * os;

  Pack<T, VEC> g[U];
  Pack<T, VEC> u[U];
#pragma unroll
  for (int k = 0; k < U; ++k) {
    const int64_t vi = min(base + k * 256, nvec - 1);
    g[k] = load_stream<T, VEC>(xr + vi * VEC);
    u[k] = load_stream<T, VEC>(xr + inter + vi * VEC);
  }
#pragma unroll
  for (int k = 0; k < U; ++k) {
    const int vi = base + k * 256;
    if (vi < nvec) {
      Pack<T, VEC> o;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float gf = to_f32(g[k].v[e]);
        const float act = round_to<T>(gf / (1.0f + expf(-gf)));
        o.v[e] = half_product<T>(act, to_f32(u[k].v[e]));
      }
      store_stream<T, VEC>(orow + static_cast<int64_t>(vi) * VEC, o);
    }
  }
}

template <typename T, int VEC, int U>
int launch_vec(const T* x, int64_t xs, T* out, int64_t os, int64_t rows, int64_t nvec, hipStream_t stream) {
  const int64_t cb = cdiv(nvec, 256 * U);
  const int64_t grid = rows * cb;
  if (grid > 0x7fffffffLL) return EMBER_EINVAL;
  hipLaunchKernelGGL((k_silu_mul<T, VEC, U>), dim3(static_cast<uint32_t>(grid)), dim3(256), 0, stream, x, xs,
                     out, os, static_cast<int>(nvec), static_cast<int>(cb));
  return launch_status();
}

template <typename T>
int launch_typed(const void* xv, int64_t xs, void* outv, int64_t os, int64_t rows, int64_t inter,
                 hipStream_t stream) {
  constexpr int VEC = 16 / sizeof(T);
  const T* x = static_cast<const T*>(xv);
  T* out = static_cast<T*>(outv);
  const bool vec_ok = inter % VEC == 0 && xs % VEC == 0 && os % VEC == 0 && aligned16(x) && aligned16(out);
  if (vec_ok) {
    const int64_t nvec = inter / VEC;
    // More packs per lane only when the launch is big enough to fill the chip anyway.
    if (EMBER_SILU_U >= 4 && rows * nvec >= 4 * EMBER_SILU_MIN_THREADS)
      return launch_vec<T, VEC, 4>(x, xs, out, os, rows, nvec, stream);
    if (EMBER_SILU_U >= 2 && rows * nvec >= 2 * EMBER_SILU_MIN_THREADS)
      return launch_vec<T, VEC, 2>(x, xs, out, os, rows, nvec, stream);
    return launch_vec<T, VEC, 1>(x, xs, out, os, rows, nvec, stream);
  }
  return launch_vec<T, 1, 1>(x, xs, out, os, rows, inter, stream);
}

}  // namespace
}  // namespace ember

extern "C" int ember_silu_and_mul(const void* x, int64_t x_row_stride, void* out, int64_t out_row_stride,
                                  int64_t rows, int64_t inter, int dtype, void* stream) {
  if (rows < 0 || inter <= 0 || inter > 0x3fffffffLL) return EMBER_EINVAL;
  if (rows == 0) return EMBER_OK;
  if (x == nullptr || out == nullptr || x_row_stride < 2 * inter) return EMBER_EINVAL;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case EMBER_F32: return ember::launch_typed<float>(x, x_row_stride, out, out_row_stride, rows, inter, s);
    case EMBER_F16: return ember::launch_typed<_Float16>(x, x_row_stride, out, out_row_stride, rows, inter, s);
    case EMBER_BF16: return ember::launch_typed<__bf16>(x, x_row_stride, out, out_row_stride, rows, inter, s);
    default: return EMBER_EINVAL;
  }
}
