// Embedding gather for gfx950: out[t, :] = weight[ids[t], :], a bit-exact row copy.
//
// Reference: torch.nn.Embedding.forward as called by emberserve/model/qwen2.py:182 and
// deepseek.py:205 (F.embedding without max_norm / padding_idx effects on the forward).
//
// Work mapping: a team of TPR lanes per token. The row is copied in 16-byte units when row
// bytes, strides and base pointers allow it (else 8/4/2/1-byte units); each lane keeps U
// units in flight, so with TPR = 128 and U = 4 a 8 KiB row (hidden 4096, bf16) is one
// round of 4 dwordx4 loads per lane (measured best of TPR 64/128/256 x U 2/4/8).
// An id outside [0, vocab) writes a zero row and sets EMBER_ERR_EMBED_ID; it never reads
// outside the table.
#include "ember_common.h"

#ifndef EMBER_EMB_U
#define EMBER_EMB_U 4
#endif
#ifndef EMBER_EMB_TPR
#define EMBER_EMB_TPR 128
#endif

namespace ember {
namespace {

template <int VB>
struct Unit;
template <>
struct Unit<16> {
  using type = Pack<uint32_t, 4>;
};
template <>
struct Unit<8> {
  using type = Pack<uint32_t, 2>;
};
template <>
struct Unit<4> {
  using type = uint32_t;
};
template <>
struct Unit<2> {
  using type = uint16_t;
};
template <>
struct Unit<1> {
  using type = uint8_t;
};

// Table rows are read with ordinary (cached) loads and the output rows written with
// non-temporal stores. Measured on MI355X ([151936, 4096] bf16, T = 8192, rotated ids):
// non-temporal table loads 25.1 us, cached loads 23.6 us (the copy of the same bytes
// takes 23.3 us).
template <typename V>
__device__ __forceinline__ V load_unit(const V* p) {
  return *p;
}

template <typename V>
__device__ __forceinline__ void store_unit(V* p, const V& v) {
  if constexpr (sizeof(V) == 16) {
    store_stream<uint32_t, 4>(reinterpret_cast<uint32_t*>(p), __builtin_bit_cast(Pack<uint32_t, 4>, v));
  } else {
    *p = v;
  }
}

// PAD (the mixed-step query pack): a negative id is a padding row, written as zeros with no
// error; only ids >= vocab are errors (EMBER_ERR_ROW_INDEX).
template <int VB, int U, int TPR, bool PAD = false>
__global__ void __launch_bounds__(256)
k_embedding(const int64_t* __restrict__ ids, int64_t ntok, const uint8_t* __restrict__ w, int64_t vocab,
            int64_t w_stride_bytes, uint8_t* __restrict__ out, int64_t out_stride_bytes, int nunits,
            uint32_t* __restrict__ err) {
  using V = typename Unit<VB>::type;
  static_assert(TPR % kWave == 0, "a wave must not straddle two tokens");
  // Wave-uniform token index (readfirstlane): the id is then a scalar load, and the row
  // address an SGPR base.
  const int64_t tok = __builtin_amdgcn_readfirstlane(
      static_cast<int>(blockIdx.x * (256 / TPR) + threadIdx.x / TPR));
  const int lane = threadIdx.x % TPR;
  if (tok >= ntok) return;
  const int64_t id = ids[tok];
  V* dst = reinterpret_cast<V*>(out + tok * out_stride_bytes);
  if (id < 0 || id >= vocab) {
    if (lane == 0 && (!PAD || id >= 0)) atomicOr(err, PAD ? EMBER_ERR_ROW_INDEX : EMBER_ERR_EMBED_ID);
    V zero{};
    for (int i = lane; i < nunits; i += TPR) dst[i] = zero;
    return;
  }
  const V* src = reinterpret_cast<const V*>(w + id * w_stride_bytes);
  for (int base = 0; base < nunits; base += TPR * U) {
    V buf[U];
#pragma unroll
    for (int k = 0; k < U; ++k) buf[k] = load_unit(src + min(base + lane + k * TPR, nunits - 1));
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int i = base + lane + k * TPR;
      if (i < nunits) store_unit(dst + i, buf[k]);
    }
  }
}

// Two-source row scatter (the mixed-step output unpack): packed row t < n0 is src0[t], row
// t >= n0 is src1[t - n0]; it goes to dst[rows[t]]. A negative rows[t] is a padding row and
// is dropped; rows[t] >= dst_rows is dropped with EMBER_ERR_ROW_INDEX. The row is loaded
// before its destination is known to be valid, so the loads never wait for the index.
template <int VB, int U, int TPR>
__global__ void __launch_bounds__(256)
k_scatter_rows2(const uint8_t* __restrict__ src0, int64_t s0_stride_bytes, int64_t n0,
                const uint8_t* __restrict__ src1, int64_t s1_stride_bytes, int64_t n1,
                const int64_t* __restrict__ rows, uint8_t* __restrict__ dst, int64_t dst_rows,
                int64_t dst_stride_bytes, int nunits, uint32_t* __restrict__ err) {
  using V = typename Unit<VB>::type;
  static_assert(TPR % kWave == 0, "a wave must not straddle two rows");
  const int64_t t = __builtin_amdgcn_readfirstlane(static_cast<int>(blockIdx.x * (256 / TPR) + threadIdx.x / TPR));
  const int lane = threadIdx.x % TPR;
  if (t >= n0 + n1) return;
  const int64_t d = rows[t];
  const V* src = reinterpret_cast<const V*>(t < n0 ? src0 + t * s0_stride_bytes : src1 + (t - n0) * s1_stride_bytes);
  V* out = reinterpret_cast<V*>(dst + (d < 0 || d >= dst_rows ? 0 : d) * dst_stride_bytes);
  for (int base = 0; base < nunits; base += TPR * U) {
    V buf[U];
#pragma unroll
    for (int k = 0; k < U; ++k) buf[k] = load_unit(src + min(base + lane + k * TPR, nunits - 1));
    if (d < 0 || d >= dst_rows) continue;
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int i = base + lane + k * TPR;
      if (i < nunits) store_unit(out + i, buf[k]);
    }
  }
  if (d >= dst_rows && lane == 0) atomicOr(err, EMBER_ERR_ROW_INDEX);
}

template <int VB, bool PAD = false>
int launch_vb(const int64_t* ids, int64_t ntok, const void* w, int64_t vocab, int64_t wsb, void* out,
              int64_t osb, int64_t row_bytes, uint32_t* err, hipStream_t stream) {
  const int64_t nunits = row_bytes / VB;
  constexpr int kTpr = EMBER_EMB_TPR;
  const int64_t grid = cdiv(ntok, 256 / kTpr);
  if (grid * 256 > 0x7fffffffLL || nunits > 0x7fffffffLL) return EMBER_EINVAL;
  hipLaunchKernelGGL((k_embedding<VB, EMBER_EMB_U, kTpr, PAD>), dim3(static_cast<uint32_t>(grid)), dim3(256), 0, stream, ids, ntok,
                     static_cast<const uint8_t*>(w), vocab, wsb, static_cast<uint8_t*>(out), osb,
                     static_cast<int>(nunits), err);
  return launch_status();
}

template <int VB>
int launch_scatter2(const void* s0, int64_t s0b, int64_t n0, const void* s1, int64_t s1b, int64_t n1,
                    const int64_t* rows, void* dst, int64_t dst_rows, int64_t db, int64_t row_bytes, uint32_t* err,
                    hipStream_t stream) {
  const int64_t nunits = row_bytes / VB;
  constexpr int kTpr = EMBER_EMB_TPR;
  const int64_t grid = cdiv(n0 + n1, 256 / kTpr);
  if (grid * 256 > 0x7fffffffLL || nunits > 0x7fffffffLL) return EMBER_EINVAL;
  hipLaunchKernelGGL((k_scatter_rows2<VB, EMBER_EMB_U, kTpr>), dim3(static_cast<uint32_t>(grid)), dim3(256), 0,
                     stream, static_cast<const uint8_t*>(s0), s0b, n0, static_cast<const uint8_t*>(s1), s1b, n1, rows,
                     static_cast<uint8_t*>(dst), dst_rows, db, static_cast<int>(nunits), err);
  return launch_status();
}

// Widest unit (16/8/4/2/1 bytes) that divides every base pointer, stride and the row size.
inline int unit_bytes(uintptr_t bits) {
  if ((bits & 15u) == 0) return 16;
  if ((bits & 7u) == 0) return 8;
  if ((bits & 3u) == 0) return 4;
  if ((bits & 1u) == 0) return 2;
  return 1;
}

// A streaming copy of n16 16-byte units: one unit per lane, non-temporal loads and stores.
// The bandwidth reference of the benchmark's copy-ceiling rows. Measured on MI355X against
// 2-8 units per lane, grid-stride forms and hipMemcpyAsync, at 24-256 MB: the fastest or
// within 1% at every size (32 MB: 12.8 us; 64 MB: 22.8 us; hipMemcpyAsync 14.4 / 26.6 us).
__global__ void __launch_bounds__(256) k_stream_copy(const uint32_t* __restrict__ src, uint32_t* __restrict__ dst,
                                                     int64_t n16) {
  using V = unsigned int __attribute__((ext_vector_type(4)));
  const int64_t k = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (k < n16)
    __builtin_nontemporal_store(__builtin_nontemporal_load(reinterpret_cast<const V*>(src) + k),
                                reinterpret_cast<V*>(dst) + k);
}

}  // namespace
}  // namespace ember

extern "C" int ember_stream_copy(const void* src, void* dst, int64_t bytes, void* stream) {
  using namespace ember;
  if (bytes == 0) return EMBER_OK;
  if (bytes < 0 || bytes % 16 != 0 || src == nullptr || dst == nullptr ||
      (reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) % 16 != 0 || bytes / 16 > (int64_t(1) << 38))
    return EMBER_EINVAL;
  const int64_t n16 = bytes / 16;
  hipLaunchKernelGGL(k_stream_copy, dim3(static_cast<uint32_t>(cdiv(n16, int64_t(256)))), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint32_t*>(src), static_cast<uint32_t*>(dst), n16);
  return launch_status();
}

extern "C" int ember_gather_rows(const void* src, int64_t src_rows, int64_t src_row_stride, const int64_t* rows,
                                 int64_t num_rows, void* dst, int64_t dst_row_stride, int64_t row_elems,
                                 int64_t elem_bytes, void* stream) {
  using namespace ember;
  if (num_rows < 0 || row_elems <= 0 || src_rows < 0) return EMBER_EINVAL;
  if (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4 && elem_bytes != 8) return EMBER_EINVAL;
  if (num_rows == 0) return EMBER_OK;
  if (src == nullptr || rows == nullptr || dst == nullptr) return EMBER_EINVAL;
  uint32_t* err = device_error_word();
  if (err == nullptr) return EMBER_ENODEV;
  const int64_t rb = row_elems * elem_bytes, ssb = src_row_stride * elem_bytes, dsb = dst_row_stride * elem_bytes;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  switch (unit_bytes(reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst) |
                     static_cast<uintptr_t>(rb) | static_cast<uintptr_t>(ssb) | static_cast<uintptr_t>(dsb))) {
    case 16: return launch_vb<16, true>(rows, num_rows, src, src_rows, ssb, dst, dsb, rb, err, s);
    case 8: return launch_vb<8, true>(rows, num_rows, src, src_rows, ssb, dst, dsb, rb, err, s);
    case 4: return launch_vb<4, true>(rows, num_rows, src, src_rows, ssb, dst, dsb, rb, err, s);
    case 2: return launch_vb<2, true>(rows, num_rows, src, src_rows, ssb, dst, dsb, rb, err, s);
    default: return launch_vb<1, true>(rows, num_rows, src, src_rows, ssb, dst, dsb, rb, err, s);
  }
}

extern "C" int ember_scatter_rows2(const void* src0, int64_t src0_rows, int64_t src0_row_stride, const void* src1,
                                   int64_t src1_rows, int64_t src1_row_stride, const int64_t* rows, void* dst,
                                   int64_t dst_rows, int64_t dst_row_stride, int64_t row_elems, int64_t elem_bytes,
                                   void* stream) {
  using namespace ember;
  if (src0_rows < 0 || src1_rows < 0 || dst_rows < 0 || row_elems <= 0) return EMBER_EINVAL;
  if (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4 && elem_bytes != 8) return EMBER_EINVAL;
  if (src0_rows + src1_rows == 0) return EMBER_OK;
  if ((src0_rows > 0 && src0 == nullptr) || (src1_rows > 0 && src1 == nullptr) || rows == nullptr || dst == nullptr)
    return EMBER_EINVAL;
  if (src0 == nullptr) src0 = src1;  // never read: keeps the pointer arithmetic defined
  if (src1 == nullptr) src1 = src0;
  uint32_t* err = device_error_word();
  if (err == nullptr) return EMBER_ENODEV;
  const int64_t rb = row_elems * elem_bytes, s0b = src0_row_stride * elem_bytes, s1b = src1_row_stride * elem_bytes,
                db = dst_row_stride * elem_bytes;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const uintptr_t bits = reinterpret_cast<uintptr_t>(src0) | reinterpret_cast<uintptr_t>(src1) |
                         reinterpret_cast<uintptr_t>(dst) | static_cast<uintptr_t>(rb) | static_cast<uintptr_t>(s0b) |
                         static_cast<uintptr_t>(s1b) | static_cast<uintptr_t>(db);
  switch (unit_bytes(bits)) {
    case 16: return launch_scatter2<16>(src0, s0b, src0_rows, src1, s1b, src1_rows, rows, dst, dst_rows, db, rb, err, s);
    case 8: return launch_scatter2<8>(src0, s0b, src0_rows, src1, s1b, src1_rows, rows, dst, dst_rows, db, rb, err, s);
    case 4: return launch_scatter2<4>(src0, s0b, src0_rows, src1, s1b, src1_rows, rows, dst, dst_rows, db, rb, err, s);
    case 2: return launch_scatter2<2>(src0, s0b, src0_rows, src1, s1b, src1_rows, rows, dst, dst_rows, db, rb, err, s);
    default: return launch_scatter2<1>(src0, s0b, src0_rows, src1, s1b, src1_rows, rows, dst, dst_rows, db, rb, err, s);
  }
}

extern "C" int ember_embedding(const int64_t* ids, int64_t num_tokens, const void* weight, int64_t vocab,
                               int64_t hidden, int64_t weight_row_stride, void* out, int64_t out_row_stride,
                               int64_t elem_bytes, void* stream) {
  using namespace ember;
  if (num_tokens < 0 || hidden <= 0 || vocab < 0) return EMBER_EINVAL;
  if (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4 && elem_bytes != 8) return EMBER_EINVAL;
  if (num_tokens == 0) return EMBER_OK;
  if (ids == nullptr || weight == nullptr || out == nullptr) return EMBER_EINVAL;
  uint32_t* err = device_error_word();
  if (err == nullptr) return EMBER_ENODEV;
  const int64_t row_bytes = hidden * elem_bytes;
  const int64_t wsb = weight_row_stride * elem_bytes;
  const int64_t osb = out_row_stride * elem_bytes;
  const uintptr_t bits = reinterpret_cast<uintptr_t>(weight) | reinterpret_cast<uintptr_t>(out) |
                         static_cast<uintptr_t>(row_bytes) | static_cast<uintptr_t>(wsb) |
                         static_cast<uintptr_t>(osb);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if ((bits & 15u) == 0) return launch_vb<16>(ids, num_tokens, weight, vocab, wsb, out, osb, row_bytes, err, s);
  if ((bits & 7u) == 0) return launch_vb<8>(ids, num_tokens, weight, vocab, wsb, out, osb, row_bytes, err, s);
  if ((bits & 3u) == 0) return launch_vb<4>(ids, num_tokens, weight, vocab, wsb, out, osb, row_bytes, err, s);
  if ((bits & 1u) == 0) return launch_vb<2>(ids, num_tokens, weight, vocab, wsb, out, osb, row_bytes, err, s);
  return launch_vb<1>(ids, num_tokens, weight, vocab, wsb, out, osb, row_bytes, err, s);
}
