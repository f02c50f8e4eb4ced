// The routed experts' block-aligned layout (the `moe_align` contract of
// emberserve/model/moe_triton.py:215-254, whose decode-time form is the single launch
// `_moe_align_kernel`, :97-160) as one gfx950 workgroup.
//
// Given assignment ids i = token * k + choice with expert ids e_i, the layout is
//   * sorted_ids [max_padded]: expert 0's assignments in ascending i, padded with num_valid
//     to a multiple of block_m, then expert 1's, ...; num_valid past the last run;
//   * block_expert [max_blocks]: the expert of each block_m-slot block, num_experts past the
//     last used block;
// with max_padded = round_up(num_valid + E (block_m - 1), block_m).
//
// One workgroup of 16 waves, in five LDS phases (no global scratch, no second launch):
//   1. wave s counts the experts of its contiguous segment of assignments (LDS atomics into
//      its own row of a [16][E] histogram);
//   2. per expert, the rows become exclusive prefixes over the segments, and the expert's
//      total and padded run length fall out;
//   3. a workgroup scan of the padded lengths gives each expert's run start; the prefixes
//      become per-(segment, expert) write cursors;
//   4. wave s walks its segment in 64-assignment chunks, in order: one ballot per distinct
//      expert of a chunk gives each lane its rank among the chunk's lanes of that expert,
//      so every run keeps ascending assignment order (the stable layout) with no sort;
//   5. every slot that phase 4 did not fill (run padding, the tail) and every block_expert
//      entry is written by a binary search over the run ends.
// Phases 4 and 5 write disjoint slots. An expert id outside [0, E) drops that assignment
// from the layout and sets EMBER_ERR_EXPERT_ID.
#include "ember_common.h"

namespace ember {
namespace {

constexpr int kAlignWaves = 16;
constexpr int kAlignThreads = kAlignWaves * kWave;
constexpr int kAlignMaxExperts = 1024;

template <typename I>
__global__ void __launch_bounds__(kAlignThreads)
k_moe_align(const I* __restrict__ ids, int nv, int E, int bm, int32_t* __restrict__ sorted_ids, int max_padded,
            int32_t* __restrict__ block_expert, int max_blocks, uint32_t* err) {
  __shared__ int hist[kAlignWaves * kAlignMaxExperts];  // counts, then prefixes, then cursors
  __shared__ int run_start[kAlignMaxExperts];
  __shared__ int run_total[kAlignMaxExperts];
  __shared__ int run_end_block[kAlignMaxExperts];      // inclusive prefix of padded blocks
  __shared__ int wave_sum[kAlignWaves];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int w = tid >> 6;
  for (int j = tid; j < kAlignWaves * E; j += kAlignThreads) hist[j] = 0;
  __syncthreads();

  // 1. per-segment histograms
  const int seg = (nv + kAlignWaves - 1) / kAlignWaves;
  const int s0 = min(nv, w * seg);
  const int s1 = min(nv, s0 + seg);
  bool bad = false;
  for (int i = s0 + lane; i < s1; i += kWave) {
    const int64_t e = static_cast<int64_t>(ids[i]);
    if (e >= 0 && e < E) atomicAdd(&hist[w * E + static_cast<int>(e)], 1);
    else bad = true;
  }
  if (bad) atomicOr(err, EMBER_ERR_EXPERT_ID);
  __syncthreads();

  // 2. prefixes over segments, totals, padded lengths (E <= the thread count: one expert
  // per thread)
  int padded = 0;
  if (tid < E) {
    int run = 0;
#pragma unroll
    for (int s = 0; s < kAlignWaves; ++s) {
      const int c = hist[s * E + tid];
      hist[s * E + tid] = run;
      run += c;
    }
    run_total[tid] = run;
    padded = (run + bm - 1) / bm * bm;
  }

  // 3. exclusive scan of the padded lengths across the workgroup
  int incl = padded;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int v = __shfl_up(incl, d, kWave);
    if (lane >= d) incl += v;
  }
  if (lane == kWave - 1) wave_sum[w] = incl;
  __syncthreads();
  int before = 0;
  for (int v = 0; v < w; ++v) before += wave_sum[v];
  incl += before;
  if (tid < E) {
    const int start = incl - padded;
    run_start[tid] = start;
    run_end_block[tid] = incl / bm;
#pragma unroll
    for (int s = 0; s < kAlignWaves; ++s) hist[s * E + tid] += start;
  }
  __syncthreads();

  // 4. stable placement, one chunk of 64 assignments of this wave's segment at a time
  const uint64_t below = (uint64_t(1) << lane) - 1;
  for (int base = s0; base < s1; base += kWave) {
    const int i = base + lane;
    int e = -1;
    if (i < s1) {
      const int64_t v = static_cast<int64_t>(ids[i]);
      if (v >= 0 && v < E) e = static_cast<int>(v);
    }
    uint64_t todo = __ballot(e >= 0);
    while (todo != 0) {
      const int leader = __builtin_ctzll(todo);
      const int v = __builtin_amdgcn_readlane(e, leader);
      const uint64_t mask = __ballot(e == v);
      const int cur = hist[w * E + v];
      if (e == v) sorted_ids[cur + __popcll(mask & below)] = i;
      if (lane == 0) hist[w * E + v] = cur + static_cast<int>(__popcll(mask));
      todo &= ~mask;
    }
  }

  // 5. padding and tail slots, block experts: the expert of block b is the first one whose
  // run ends past b (E when none does)
  auto expert_of_block = [&](int b) {
    int lo = 0, hi = E;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (run_end_block[mid] <= b) lo = mid + 1;
      else hi = mid;
    }
    return lo;
  };
  for (int p = tid; p < max_padded; p += kAlignThreads) {
    const int e = expert_of_block(p / bm);
    if (e >= E || p - run_start[e] >= run_total[e]) sorted_ids[p] = nv;
  }
  for (int b = tid; b < max_blocks; b += kAlignThreads) block_expert[b] = expert_of_block(b);
}

}  // namespace
}  // namespace ember

extern "C" {

int64_t ember_moe_align_padded_size(int64_t num_valid, int64_t num_experts, int64_t block_m) {
  if (num_valid < 0 || num_experts < 1 || block_m < 1) return -1;
  return (num_valid + num_experts * (block_m - 1) + block_m - 1) / block_m * block_m;
}

int ember_moe_align(const void* topk_ids, int id_bytes, int64_t num_valid, int64_t num_experts, int64_t block_m,
                    int32_t* sorted_ids, int64_t max_padded, int32_t* block_expert, int64_t max_blocks,
                    void* stream) {
  using namespace ember;
  if (id_bytes != 4 && id_bytes != 8) return EMBER_EINVAL;
  if (num_valid < 0 || num_experts < 1 || num_experts > kAlignMaxExperts || block_m < 1 || block_m > 4096)
    return EMBER_EINVAL;
  const int64_t need = ember_moe_align_padded_size(num_valid, num_experts, block_m);
  if (need > 0x7fffffffLL || max_padded != need || max_blocks != need / block_m) return EMBER_EINVAL;
  if (sorted_ids == nullptr || block_expert == nullptr || (num_valid > 0 && topk_ids == nullptr))
    return EMBER_EINVAL;
  uint32_t* err = device_error_word();
  if (err == nullptr) return EMBER_ENODEV;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (id_bytes == 8)
    hipLaunchKernelGGL((k_moe_align<int64_t>), dim3(1), dim3(kAlignThreads), 0, s,
                       static_cast<const int64_t*>(topk_ids), static_cast<int>(num_valid),
                       static_cast<int>(num_experts), static_cast<int>(block_m), sorted_ids,
                       static_cast<int>(max_padded), block_expert, static_cast<int>(max_blocks), err);
  else
    hipLaunchKernelGGL((k_moe_align<int32_t>), dim3(1), dim3(kAlignThreads), 0, s,
                       static_cast<const int32_t*>(topk_ids), static_cast<int>(num_valid),
                       static_cast<int>(num_experts), static_cast<int>(block_m), sorted_ids,
                       static_cast<int>(max_padded), block_expert, static_cast<int>(max_blocks), err);
  return launch_status();
}

}  // extern "C"
