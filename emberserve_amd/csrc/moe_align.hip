// The routed experts' block-aligned layout (the `moe_align` contract of
// emberserve/model/moe_triton.py:215-254, whose decode-time form is the single launch
// `_moe_align_kernel`, :97-160).
//
// Given assignment ids i = token * k + choice with expert ids e_i, the layout is
//   * sorted_ids [max_padded]: expert 0's assignments in ascending i, padded with num_valid
//     to a multiple of block_m, then expert 1's, ...; num_valid past the last run;
//   * block_expert [max_blocks]: the expert of each block_m-slot block, num_experts past the
//     last used block;
// with max_padded = round_up(num_valid + E (block_m - 1), block_m).
//
// The assignments are cut into contiguous segments, one per workgroup, and each segment into
// one contiguous run of 64-assignment chunks per wave. The stable rank of an assignment
// among the earlier ones of its expert is then
//   run_start[e] + (earlier segments' count of e) + (earlier waves' count of e in this
//   segment) + (earlier chunks' count in this wave) + (earlier lanes' count in this chunk).
// The last term comes from a peer mask: log2(E) ballots over the bits of the expert id give
// each lane the set of lanes holding its expert, so a chunk costs a fixed handful of
// instructions whatever its experts are; the lowest lane of each peer set carries the
// set's count into the wave's per-expert LDS cursor.
//
// Two forms, one kernel body (k_align_place):
//   * one workgroup (no workspace): counts its whole input per wave, then places;
//   * a grid of up to kAlignMaxSegments workgroups: k_align_count writes each segment's
//     per-expert counts to the caller's workspace [segments][E]; k_align_place reads that
//     table, forms the prefix over earlier segments and the totals itself, then places
//     its own segment and writes its share of the padding slots and block experts.
// Every slot the placement does not fill (run padding, the tail) and every block_expert
// entry is written by a binary search over the run ends, so no memset is needed and the
// launches can be captured in a HIP graph. An expert id outside [0, E) drops that
// assignment from the layout and sets EMBER_ERR_EXPERT_ID.
#include "ember_common.h"

namespace ember {
namespace {

constexpr int kAlignWaves = 16;
constexpr int kAlignThreads = kAlignWaves * kWave;
constexpr int kAlignMaxExperts = 1024;   // one expert per thread in the scan
constexpr int kAlignMaxSegments = 64;    // workgroups of the grid form
constexpr int kAlignSegment = 2048;      // assignments per workgroup the grid form aims for
#ifndef EMBER_ALIGN_GRID_FROM
#define EMBER_ALIGN_GRID_FROM 3072
#endif
constexpr int kAlignGridFrom = EMBER_ALIGN_GRID_FROM;  // num_valid past which the grid form is used

// Segment [s0, s1) of workgroup seg out of nseg, and this wave's part [w0, w1) of it (whole
// chunks of 64).
struct AlignSpan {
  int w0, w1;
};

__device__ inline AlignSpan align_span(int nv, int nseg, int seg, int w) {
  const int per_seg = ((nv + nseg - 1) / nseg + kWave - 1) / kWave * kWave;
  const int s0 = min(nv, seg * per_seg);
  const int s1 = min(nv, s0 + per_seg);
  const int per_wave = ((s1 - s0 + kAlignWaves - 1) / kAlignWaves + kWave - 1) / kWave * kWave;
  const int w0 = min(s1, s0 + w * per_wave);
  return {w0, min(s1, w0 + per_wave)};
}

// The expert of assignment i: -1 when i is past the span or the id is out of range (bad).
template <typename I>
__device__ inline int align_expert(const I* __restrict__ ids, int i, int end, int E, bool& bad) {
  if (i >= end) return -1;
  const int64_t v = static_cast<int64_t>(ids[i]);
  if (v >= 0 && v < E) return static_cast<int>(v);
  bad = true;
  return -1;
}

// The lanes of this chunk that hold this lane's expert (0 for a lane without one).
__device__ inline uint64_t align_peers(int e, int ebits) {
  uint64_t peers = __ballot(e >= 0);
  for (int k = 0; k < ebits; ++k) {
    const bool bit = (e >> k) & 1;
    const uint64_t b = __ballot(bit);
    peers &= bit ? b : ~b;
  }
  return e >= 0 ? peers : 0;
}

constexpr int kAlignChunkGroup = 4;  // chunks whose ids are loaded before any is used

// Calls f(e, i) for the chunks of this wave's span in order (e: this lane's expert or -1, i:
// its assignment id), loading the ids of kAlignChunkGroup chunks at a time so that their
// memory latencies overlap.
template <typename I, typename F>
__device__ inline bool align_walk(const I* __restrict__ ids, AlignSpan sp, int E, int lane, F&& f) {
  bool bad = false;
  for (int base = sp.w0; base < sp.w1; base += kAlignChunkGroup * kWave) {
    int e[kAlignChunkGroup];
#pragma unroll
    for (int u = 0; u < kAlignChunkGroup; ++u) e[u] = align_expert(ids, base + u * kWave + lane, sp.w1, E, bad);
#pragma unroll
    for (int u = 0; u < kAlignChunkGroup; ++u)
      if (base + u * kWave < sp.w1) f(e[u], base + u * kWave + lane);
  }
  return bad;
}

// Adds each peer set's size to cnt_w[e] (LDS) through its lowest lane.
struct AlignCounter {
  int* cnt_w;
  int ebits;
  uint64_t below;
  __device__ void operator()(int e, int) const {
    const uint64_t peers = align_peers(e, ebits);
    if (peers != 0 && (peers & below) == 0) atomicAdd(&cnt_w[e], static_cast<int>(__popcll(peers)));
  }
};

template <typename I>
__global__ void __launch_bounds__(kAlignThreads)
k_align_count(const I* __restrict__ ids, int nv, int E, int ebits, int nseg, int32_t* __restrict__ seg_counts,
              uint32_t* err) {
  __shared__ int cnt[kAlignWaves * kAlignMaxExperts];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid >> 6;
  for (int j = tid; j < kAlignWaves * E; j += kAlignThreads) cnt[j] = 0;
  __syncthreads();
  const AlignCounter count{cnt + w * E, ebits, (uint64_t(1) << lane) - 1};
  if (align_walk(ids, align_span(nv, nseg, blockIdx.x, w), E, lane, count)) atomicOr(err, EMBER_ERR_EXPERT_ID);
  __syncthreads();
  for (int e = tid; e < E; e += kAlignThreads) {
    int c = 0;
#pragma unroll
    for (int v = 0; v < kAlignWaves; ++v) c += cnt[v * E + e];
    seg_counts[static_cast<int64_t>(blockIdx.x) * E + e] = c;
  }
}

// nseg == 1: the whole input in this one workgroup, seg_counts unused. nseg > 1: the grid
// form, seg_counts [nseg][E] from k_align_count.
template <typename I>
__global__ void __launch_bounds__(kAlignThreads)
k_align_place(const I* __restrict__ ids, int nv, int E, int ebits, int bm, int nseg,
              const int32_t* __restrict__ seg_counts, int32_t* __restrict__ sorted_ids, int max_padded,
              int32_t* __restrict__ block_expert, int max_blocks, uint32_t* err) {
  __shared__ int cnt[kAlignWaves * kAlignMaxExperts];  // counts, then cursors
  __shared__ int run_start[kAlignMaxExperts];
  __shared__ int run_total[kAlignMaxExperts];
  __shared__ int run_end_block[kAlignMaxExperts];      // inclusive prefix of padded blocks
  __shared__ int seg_total[kAlignMaxExperts];         // grid form: counts over all segments
  __shared__ int seg_before[kAlignMaxExperts];        // ... and over the segments before this one
  __shared__ int wave_sum[kAlignWaves];

  const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid >> 6;
  const int seg = blockIdx.x;
  const AlignSpan sp = align_span(nv, nseg, seg, w);
  // A span of at most kAlignChunkGroup chunks (every one below 4096 assignments in one
  // workgroup or 64 x 4096 in the grid form) is loaded once, before anything else, and
  // held in registers for both passes.
  const bool resident = sp.w1 - sp.w0 <= kAlignChunkGroup * kWave;
  int held[kAlignChunkGroup];
  bool bad = false;
  if (resident) {
#pragma unroll
    for (int u = 0; u < kAlignChunkGroup; ++u) held[u] = align_expert(ids, sp.w0 + u * kWave + lane, sp.w1, E, bad);
  }
  auto each = [&](const auto& f) {
    if (resident) {
#pragma unroll
      for (int u = 0; u < kAlignChunkGroup; ++u)
        if (sp.w0 + u * kWave < sp.w1) f(held[u], sp.w0 + u * kWave + lane);
    } else {
      bad |= align_walk(ids, sp, E, lane, f);
    }
  };
  for (int j = tid; j < kAlignWaves * E; j += kAlignThreads) cnt[j] = 0;
  for (int j = tid; j < E; j += kAlignThreads) seg_total[j] = seg_before[j] = 0;
  __syncthreads();
  if (nseg > 1) {
    // The count table [nseg][E], spread over all threads with eight loads in flight each
    // (its rows were written by workgroups on other XCDs: every load misses this L2).
    const int n = nseg * E;
    for (int j0 = tid; j0 < n; j0 += 8 * kAlignThreads) {
      int c[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) c[u] = j0 + u * kAlignThreads < n ? seg_counts[j0 + u * kAlignThreads] : 0;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int j = j0 + u * kAlignThreads;
        if (c[u] != 0) {
          const int e = j % E;
          atomicAdd(&seg_total[e], c[u]);
          if (j / E < seg) atomicAdd(&seg_before[e], c[u]);
        }
      }
    }
  }
  const uint64_t below = (uint64_t(1) << lane) - 1;
  each(AlignCounter{cnt + w * E, ebits, below});
  if (bad && nseg == 1) atomicOr(err, EMBER_ERR_EXPERT_ID);  // the grid form flags in k_align_count
  __syncthreads();

  // Per expert (one per thread): this segment's offset and the expert's total, its padded
  // run, the workgroup scan of the padded runs, then per-wave cursors.
  int total = 0, before = 0, padded = 0;
  if (tid < E) {
    if (nseg == 1) {
#pragma unroll
      for (int v = 0; v < kAlignWaves; ++v) total += cnt[v * E + tid];
    } else {
      total = seg_total[tid];
      before = seg_before[tid];
    }
    padded = (total + bm - 1) / bm * bm;
  }
  int incl = padded;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int v = __shfl_up(incl, d, kWave);
    if (lane >= d) incl += v;
  }
  if (lane == kWave - 1) wave_sum[w] = incl;
  __syncthreads();
  for (int v = 0; v < w; ++v) incl += wave_sum[v];
  if (tid < E) {
    const int start = incl - padded;
    run_start[tid] = start;
    run_total[tid] = total;
    run_end_block[tid] = incl / bm;
    int cur = start + before;
#pragma unroll
    for (int v = 0; v < kAlignWaves; ++v) {
      const int c = cnt[v * E + tid];
      cnt[v * E + tid] = cur;
      cur += c;
    }
  }
  __syncthreads();

  // Stable placement: chunks of this wave's span in order, lanes in order within a chunk.
  int* cur_w = cnt + w * E;
  each([&](int e, int i) {
    const uint64_t peers = align_peers(e, ebits);
    const int leader = peers != 0 ? __builtin_ctzll(peers) : lane;
    int at = 0;
    if (peers != 0 && leader == lane) at = atomicAdd(&cur_w[e], static_cast<int>(__popcll(peers)));
    at = __shfl(at, leader, kWave);
    if (peers != 0) sorted_ids[at + __popcll(peers & below)] = i;
  });

  // This workgroup's share of the padding and tail slots and of the block experts: the
  // expert of block b is the first one whose run ends past b (E when none does).
  auto expert_of_block = [&](int b) {
    int lo = 0, hi = E;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (run_end_block[mid] <= b) lo = mid + 1;
      else hi = mid;
    }
    return lo;
  };
  const int pblk = (max_blocks + nseg - 1) / nseg;
  const int b0 = min(max_blocks, seg * pblk), b1 = min(max_blocks, b0 + pblk);
  for (int p = b0 * bm + tid; p < b1 * bm; p += kAlignThreads) {
    const int e = expert_of_block(p / bm);
    if (e >= E || p - run_start[e] >= run_total[e]) sorted_ids[p] = nv;
  }
  for (int b = b0 + tid; b < b1; b += kAlignThreads) block_expert[b] = expert_of_block(b);
}

// Workgroups of the grid form for num_valid assignments (1: the one-workgroup form).
inline int align_segments(int64_t nv) {
  if (nv <= kAlignGridFrom) return 1;
  const int64_t n = (nv + kAlignSegment - 1) / kAlignSegment;
  return n < kAlignMaxSegments ? static_cast<int>(n) : kAlignMaxSegments;
}

template <typename I>
void launch_align(const void* ids, int nv, int E, int bm, int32_t* sorted_ids, int max_padded,
                  int32_t* block_expert, int max_blocks, int nseg, int32_t* seg_counts, uint32_t* err,
                  hipStream_t s) {
  const I* p = static_cast<const I*>(ids);
  int ebits = 0;
  while ((1 << ebits) < E) ++ebits;
  if (nseg > 1)
    hipLaunchKernelGGL((k_align_count<I>), dim3(nseg), dim3(kAlignThreads), 0, s, p, nv, E, ebits, nseg,
                       seg_counts, err);
  hipLaunchKernelGGL((k_align_place<I>), dim3(nseg), dim3(kAlignThreads), 0, s, p, nv, E, ebits, bm, nseg,
                     seg_counts, sorted_ids, max_padded, block_expert, max_blocks, err);
}

}  // namespace
}  // namespace ember

extern "C" {

int64_t ember_moe_align_padded_size(int64_t num_valid, int64_t num_experts, int64_t block_m) {
  if (num_valid < 0 || num_experts < 1 || block_m < 1) return -1;
  return (num_valid + num_experts * (block_m - 1) + block_m - 1) / block_m * block_m;
}

int64_t ember_moe_align_workspace_bytes(int64_t num_valid, int64_t num_experts) {
  if (num_valid < 0 || num_experts < 1 || num_experts > ember::kAlignMaxExperts) return -1;
  const int nseg = ember::align_segments(num_valid);
  return nseg > 1 ? static_cast<int64_t>(nseg) * num_experts * 4 : 0;
}

int ember_moe_align(const void* topk_ids, int id_bytes, int64_t num_valid, int64_t num_experts, int64_t block_m,
                    int32_t* sorted_ids, int64_t max_padded, int32_t* block_expert, int64_t max_blocks,
                    void* workspace, int64_t workspace_bytes, void* stream) {
  using namespace ember;
  if (id_bytes != 4 && id_bytes != 8) return EMBER_EINVAL;
  // num_valid <= INT32_MAX / 2 keeps the kernels' int span arithmetic (nv + nseg - 1, ...) in range
  if (num_valid < 0 || num_valid > INT32_MAX / 2 || num_experts < 1 || num_experts > kAlignMaxExperts ||
      block_m < 1 || block_m > 4096)
    return EMBER_EINVAL;
  const int64_t need = ember_moe_align_padded_size(num_valid, num_experts, block_m);
  if (need > 0x7fffffffLL || max_padded != need || max_blocks != need / block_m) return EMBER_EINVAL;
  if (sorted_ids == nullptr || block_expert == nullptr || (num_valid > 0 && topk_ids == nullptr))
    return EMBER_EINVAL;
  if (workspace_bytes < 0 || (workspace_bytes > 0 && workspace == nullptr)) return EMBER_EINVAL;
  uint32_t* err = device_error_word();
  if (err == nullptr) return EMBER_ENODEV;
  // The grid form when the workspace holds its count table, else the one-workgroup form.
  int nseg = align_segments(num_valid);
  if (nseg > 1 && workspace_bytes < ember_moe_align_workspace_bytes(num_valid, num_experts)) nseg = 1;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  auto* counts = static_cast<int32_t*>(workspace);
  if (id_bytes == 8)
    launch_align<int64_t>(topk_ids, static_cast<int>(num_valid), static_cast<int>(num_experts),
                          static_cast<int>(block_m), sorted_ids, static_cast<int>(max_padded), block_expert,
                          static_cast<int>(max_blocks), nseg, counts, err, s);
  else
    launch_align<int32_t>(topk_ids, static_cast<int>(num_valid), static_cast<int>(num_experts),
                          static_cast<int>(block_m), sorted_ids, static_cast<int>(max_padded), block_expert,
                          static_cast<int>(max_blocks), nseg, counts, err, s);
  return launch_status();
}

}  // extern "C"
