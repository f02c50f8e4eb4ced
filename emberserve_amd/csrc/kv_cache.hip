// Paged KV-cache writes for gfx950: the scatter that consumes the rope output.
//
// Reference semantics:
//   PagedKVCache.write     (emberserve/kv/cache.py:54-61):
//     k_cache.view(num_slots, Hkv, D).index_copy_(0, slots, k); same for v
//   PagedLatentCache.write (emberserve/kv/cache.py:152-157):
//     latent_cache.view(num_slots, latent_dim).index_copy_(0, slots, latent)
// Bit-exact copies. Slot -1 marks a padding row (a graph replayed at a token bucket larger
// than the real row count) and is skipped silently. Any other slot outside [0, num_slots) is
// skipped and sets EMBER_ERR_KV_SLOT
// (torch's index_copy_ raises there); duplicate slots leave one of the writers, as
// index_copy_ does.
//
// Work mapping (k/v): the k heads and v heads of a token are 2*Hkv "rows" of D elements;
// J = D*e/16 lanes own one row, one 16-byte pack each. When a token's 2*Hkv*J lanes fill
// whole waves the token index is wave-uniform and its slot comes through a scalar load.
// Latent rows: a team of 64 lanes per token, U packs per lane (the embedding kernel's
// gather turned into a scatter).
#include "ember_common.h"

namespace ember {
namespace {

using Unit16 = Pack<uint32_t, 4>;

template <int J, bool WAVE_TOK>
__global__ void __launch_bounds__(256)
k_kv_write(const uint8_t* __restrict__ k, int64_t kts, int64_t khs, const uint8_t* __restrict__ v, int64_t vts,
           int64_t vhs, int hk, const int64_t* __restrict__ slots, uint32_t ntok, uint8_t* __restrict__ kc,
           uint8_t* __restrict__ vc, int64_t num_slots, int64_t css, int64_t chs, FastDiv rdiv,
           uint32_t* __restrict__ err) {
  // strides in bytes
  const uint32_t gt = blockIdx.x * 256u + threadIdx.x;
  const uint32_t j = gt % J;
  const uint32_t rowid = gt / J;
  uint32_t tok = rdiv.div(rowid);  // rows per token = 2 * hk
  if constexpr (WAVE_TOK) tok = __builtin_amdgcn_readfirstlane(tok);
  if (tok >= ntok) return;
  const int r = static_cast<int>(rowid - tok * static_cast<uint32_t>(2 * hk));
  const int64_t slot = slots[tok];
  const bool isk = r < hk;
  const int h = isk ? r : r - hk;
  const uint8_t* src = (isk ? k + tok * kts + h * khs : v + tok * vts + h * vhs) + j * 16;
  const Unit16 x = load_stream<uint32_t, 4>(reinterpret_cast<const uint32_t*>(src));
  if (slot < 0 || slot >= num_slots) {
    if (j == 0 && r == 0 && slot != kPadSlot) atomicOr(err, EMBER_ERR_KV_SLOT);
    return;
  }
  uint8_t* dst = (isk ? kc : vc) + slot * css + h * chs + j * 16;
  store_stream<uint32_t, 4>(reinterpret_cast<uint32_t*>(dst), x);
}

// Any geometry (row bytes not a multiple of 16, odd strides): one wave per (token, k|v,
// head) row, byte-granular 4/2/1 units chosen by the caller through EB.
template <typename E>
__global__ void __launch_bounds__(256)
k_kv_write_any(const E* __restrict__ k, int64_t kts, int64_t khs, const E* __restrict__ v, int64_t vts,
               int64_t vhs, int hk, int d, const int64_t* __restrict__ slots, int64_t ntok, E* __restrict__ kc,
               E* __restrict__ vc, int64_t num_slots, int64_t css, int64_t chs, uint32_t* __restrict__ err) {
  // strides in elements
  const int64_t rowid = static_cast<int64_t>(blockIdx.x) * 4 + threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const int64_t tok = rowid / (2 * hk);
  const int r = static_cast<int>(rowid - tok * 2 * hk);
  if (tok >= ntok) return;
  const int64_t slot = slots[tok];
  if (slot < 0 || slot >= num_slots) {
    if (lane == 0 && r == 0 && slot != kPadSlot) atomicOr(err, EMBER_ERR_KV_SLOT);
    return;
  }
  const bool isk = r < hk;
  const int h = isk ? r : r - hk;
  const E* src = isk ? k + tok * kts + h * khs : v + tok * vts + h * vhs;
  E* dst = (isk ? kc : vc) + slot * css + h * chs;
  for (int i = lane; i < d; i += kWave) dst[i] = src[i];
}

template <int U>
__global__ void __launch_bounds__(256)
k_row_scatter(const uint8_t* __restrict__ src, int64_t src_stride, const int64_t* __restrict__ slots, int64_t ntok,
              uint8_t* __restrict__ dst, int64_t num_slots, int64_t dst_stride, int nunits,
              uint32_t* __restrict__ err) {
  const int64_t tok = __builtin_amdgcn_readfirstlane(static_cast<int>(blockIdx.x * 4 + threadIdx.x / kWave));
  const int lane = threadIdx.x % kWave;
  if (tok >= ntok) return;
  const int64_t slot = slots[tok];
  const Unit16* s = reinterpret_cast<const Unit16*>(src + tok * src_stride);
  if (slot < 0 || slot >= num_slots) {
    if (lane == 0 && slot != kPadSlot) atomicOr(err, EMBER_ERR_KV_SLOT);
    return;
  }
  Unit16* d = reinterpret_cast<Unit16*>(dst + slot * dst_stride);
  for (int base = 0; base < nunits; base += kWave * U) {
    Unit16 buf[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      buf[u] = load_stream<uint32_t, 4>(reinterpret_cast<const uint32_t*>(s + min(base + lane + u * kWave, nunits - 1)));
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = base + lane + u * kWave;
      if (i < nunits) store_stream<uint32_t, 4>(reinterpret_cast<uint32_t*>(d + i), buf[u]);
    }
  }
}

template <typename E>
__global__ void __launch_bounds__(256)
k_row_scatter_any(const E* __restrict__ src, int64_t src_stride, const int64_t* __restrict__ slots, int64_t ntok,
                  E* __restrict__ dst, int64_t num_slots, int64_t dst_stride, int n, uint32_t* __restrict__ err) {
  const int64_t tok = static_cast<int64_t>(blockIdx.x) * 4 + threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  if (tok >= ntok) return;
  const int64_t slot = slots[tok];
  if (slot < 0 || slot >= num_slots) {
    if (lane == 0 && slot != kPadSlot) atomicOr(err, EMBER_ERR_KV_SLOT);
    return;
  }
  for (int i = lane; i < n; i += kWave) dst[slot * dst_stride + i] = src[tok * src_stride + i];
}

template <typename E>
int launch_kv_any(const void* k, int64_t kts, int64_t khs, const void* v, int64_t vts, int64_t vhs, int64_t hk,
                  int64_t d, const int64_t* slots, int64_t ntok, void* kc, void* vc, int64_t num_slots, int64_t css,
                  int64_t chs, uint32_t* err, hipStream_t s) {
  const int64_t grid = cdiv(ntok * 2 * hk, 4);
  if (grid > 0x7fffffffLL) return EMBER_EINVAL;
  hipLaunchKernelGGL((k_kv_write_any<E>), dim3(static_cast<uint32_t>(grid)), dim3(256), 0, s,
                     static_cast<const E*>(k), kts, khs, static_cast<const E*>(v), vts, vhs, static_cast<int>(hk),
                     static_cast<int>(d), slots, ntok, static_cast<E*>(kc), static_cast<E*>(vc), num_slots, css, chs,
                     err);
  return launch_status();
}

template <int J>
int launch_kv_vec(const void* k, int64_t kts, int64_t khs, const void* v, int64_t vts, int64_t vhs, int64_t hk,
                  const int64_t* slots, int64_t ntok, void* kc, void* vc, int64_t num_slots, int64_t css, int64_t chs,
                  uint32_t* err, hipStream_t s) {
  const int64_t threads = ntok * 2 * hk * J;
  if (threads > 0x7fffffffLL) return EMBER_EINVAL;
  const int64_t grid = cdiv(threads, 256);
  const FastDiv rdiv = FastDiv::make(static_cast<uint32_t>(2 * hk));
  auto* kp = static_cast<const uint8_t*>(k);
  auto* vp = static_cast<const uint8_t*>(v);
  auto* kcp = static_cast<uint8_t*>(kc);
  auto* vcp = static_cast<uint8_t*>(vc);
  if ((2 * hk * J) % kWave == 0) {
    hipLaunchKernelGGL((k_kv_write<J, true>), dim3(static_cast<uint32_t>(grid)), dim3(256), 0, s, kp, kts, khs, vp,
                       vts, vhs, static_cast<int>(hk), slots, static_cast<uint32_t>(ntok), kcp, vcp, num_slots, css,
                       chs, rdiv, err);
  } else {
    hipLaunchKernelGGL((k_kv_write<J, false>), dim3(static_cast<uint32_t>(grid)), dim3(256), 0, s, kp, kts, khs, vp,
                       vts, vhs, static_cast<int>(hk), slots, static_cast<uint32_t>(ntok), kcp, vcp, num_slots, css,
                       chs, rdiv, err);
  }
  return launch_status();
}

}  // namespace
}  // namespace ember

extern "C" {

int ember_kv_cache_write(const void* k, int64_t k_token_stride, int64_t k_head_stride, const void* v,
                         int64_t v_token_stride, int64_t v_head_stride, int64_t num_kv_heads, int64_t head_dim,
                         const int64_t* slot_mapping, int64_t num_tokens, void* k_cache, void* v_cache,
                         int64_t num_slots, int64_t cache_slot_stride, int64_t cache_head_stride, int64_t elem_bytes,
                         void* stream) {
  using namespace ember;
  if (num_tokens < 0 || num_kv_heads < 0 || head_dim <= 0 || num_slots < 0) return EMBER_EINVAL;
  if (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4 && elem_bytes != 8) return EMBER_EINVAL;
  if (num_tokens == 0 || num_kv_heads == 0) return EMBER_OK;
  if (num_kv_heads > 0x7fff || head_dim > (1 << 20)) return EMBER_EINVAL;
  if (k == nullptr || v == nullptr || slot_mapping == nullptr || k_cache == nullptr || v_cache == nullptr)
    return EMBER_EINVAL;
  uint32_t* err = device_error_word();
  if (err == nullptr) return EMBER_ENODEV;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t eb = elem_bytes;
  const int64_t row_bytes = head_dim * eb;
  const uintptr_t bits = reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v) |
                         reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache) |
                         static_cast<uintptr_t>(row_bytes) | static_cast<uintptr_t>(k_token_stride * eb) |
                         static_cast<uintptr_t>(k_head_stride * eb) | static_cast<uintptr_t>(v_token_stride * eb) |
                         static_cast<uintptr_t>(v_head_stride * eb) | static_cast<uintptr_t>(cache_slot_stride * eb) |
                         static_cast<uintptr_t>(cache_head_stride * eb);
  const int64_t j = row_bytes / 16;
  if ((bits & 15u) == 0 && (j & (j - 1)) == 0 && j >= 1 && j <= 64) {
    const int64_t kts = k_token_stride * eb, khs = k_head_stride * eb, vts = v_token_stride * eb,
                  vhs = v_head_stride * eb, css = cache_slot_stride * eb, chs = cache_head_stride * eb;
    switch (j) {
      case 1: return launch_kv_vec<1>(k, kts, khs, v, vts, vhs, num_kv_heads, slot_mapping, num_tokens, k_cache, v_cache, num_slots, css, chs, err, s);
      case 2: return launch_kv_vec<2>(k, kts, khs, v, vts, vhs, num_kv_heads, slot_mapping, num_tokens, k_cache, v_cache, num_slots, css, chs, err, s);
      case 4: return launch_kv_vec<4>(k, kts, khs, v, vts, vhs, num_kv_heads, slot_mapping, num_tokens, k_cache, v_cache, num_slots, css, chs, err, s);
      case 8: return launch_kv_vec<8>(k, kts, khs, v, vts, vhs, num_kv_heads, slot_mapping, num_tokens, k_cache, v_cache, num_slots, css, chs, err, s);
      case 16: return launch_kv_vec<16>(k, kts, khs, v, vts, vhs, num_kv_heads, slot_mapping, num_tokens, k_cache, v_cache, num_slots, css, chs, err, s);
      case 32: return launch_kv_vec<32>(k, kts, khs, v, vts, vhs, num_kv_heads, slot_mapping, num_tokens, k_cache, v_cache, num_slots, css, chs, err, s);
      case 64: return launch_kv_vec<64>(k, kts, khs, v, vts, vhs, num_kv_heads, slot_mapping, num_tokens, k_cache, v_cache, num_slots, css, chs, err, s);
      default: break;
    }
  }
  switch (elem_bytes) {
    case 1: return launch_kv_any<uint8_t>(k, k_token_stride, k_head_stride, v, v_token_stride, v_head_stride, num_kv_heads, head_dim, slot_mapping, num_tokens, k_cache, v_cache, num_slots, cache_slot_stride, cache_head_stride, err, s);
    case 2: return launch_kv_any<uint16_t>(k, k_token_stride, k_head_stride, v, v_token_stride, v_head_stride, num_kv_heads, head_dim, slot_mapping, num_tokens, k_cache, v_cache, num_slots, cache_slot_stride, cache_head_stride, err, s);
    case 4: return launch_kv_any<uint32_t>(k, k_token_stride, k_head_stride, v, v_token_stride, v_head_stride, num_kv_heads, head_dim, slot_mapping, num_tokens, k_cache, v_cache, num_slots, cache_slot_stride, cache_head_stride, err, s);
    default: return launch_kv_any<uint64_t>(k, k_token_stride, k_head_stride, v, v_token_stride, v_head_stride, num_kv_heads, head_dim, slot_mapping, num_tokens, k_cache, v_cache, num_slots, cache_slot_stride, cache_head_stride, err, s);
  }
}

int ember_latent_cache_write(const void* latent, int64_t latent_token_stride, int64_t latent_dim,
                             const int64_t* slot_mapping, int64_t num_tokens, void* cache, int64_t num_slots,
                             int64_t cache_slot_stride, int64_t elem_bytes, void* stream) {
  using namespace ember;
  if (num_tokens < 0 || latent_dim <= 0 || num_slots < 0) return EMBER_EINVAL;
  if (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4 && elem_bytes != 8) return EMBER_EINVAL;
  if (num_tokens == 0) return EMBER_OK;
  if (latent == nullptr || slot_mapping == nullptr || cache == nullptr) return EMBER_EINVAL;
  if (num_tokens > 0x1fffffffLL || latent_dim > (1 << 24)) return EMBER_EINVAL;
  uint32_t* err = device_error_word();
  if (err == nullptr) return EMBER_ENODEV;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t eb = elem_bytes;
  const int64_t row_bytes = latent_dim * eb;
  const uintptr_t bits = reinterpret_cast<uintptr_t>(latent) | reinterpret_cast<uintptr_t>(cache) |
                         static_cast<uintptr_t>(row_bytes) | static_cast<uintptr_t>(latent_token_stride * eb) |
                         static_cast<uintptr_t>(cache_slot_stride * eb);
  const int64_t grid = cdiv(num_tokens, 4);
  if ((bits & 15u) == 0) {
    hipLaunchKernelGGL((k_row_scatter<4>), dim3(static_cast<uint32_t>(grid)), dim3(256), 0, s,
                       static_cast<const uint8_t*>(latent), latent_token_stride * eb, slot_mapping, num_tokens,
                       static_cast<uint8_t*>(cache), num_slots, cache_slot_stride * eb,
                       static_cast<int>(row_bytes / 16), err);
    return launch_status();
  }
#define EMBER_SCATTER_ANY(E)                                                                                  \
  hipLaunchKernelGGL((k_row_scatter_any<E>), dim3(static_cast<uint32_t>(grid)), dim3(256), 0, s,             \
                     static_cast<const E*>(latent), latent_token_stride, slot_mapping, num_tokens,            \
                     static_cast<E*>(cache), num_slots, cache_slot_stride, static_cast<int>(latent_dim), err); \
  return launch_status()
  switch (elem_bytes) {
    case 1: EMBER_SCATTER_ANY(uint8_t);
    case 2: EMBER_SCATTER_ANY(uint16_t);
    case 4: EMBER_SCATTER_ANY(uint32_t);
    default: EMBER_SCATTER_ANY(uint64_t);
  }
#undef EMBER_SCATTER_ANY
}

}  // extern "C"
