// Token -> expert align: stable counting sort of (token, slot) pairs by expert, each expert's run padded to
// a multiple of block_m rows (fused_moe.py:154-173). One workgroup of 16 waves; bit-exact and deterministic:
// every pair's destination is fixed by its expert's padded start plus its rank among earlier pairs of that
// expert, with no atomics that decide order.
#include "mm_common.h"

namespace {

using namespace mmd;

constexpr int kWaves = 16;
constexpr int kThreads = kWaves * kWave;
constexpr int kMaxSlots = 256;
constexpr int kIdBatch = 8;            // id loads in flight per lane
constexpr int kMaxStaged = 48 * 1024;  // pairs whose expert ids stay in LDS (2 bytes each) between the passes
constexpr uint16_t kNoExpert = 0xffff;

// STAGED: the counting pass keeps each pair's expert id in LDS (dynamic, P x 2 bytes), so the scatter pass
// reads ids from LDS instead of a second, latency-bound pass over global memory.
// Id i of the flat ids (int64 or int32 by the template flag: a branch on a run-time dtype put each of a batch's
// loads behind it, and the wave waited for each in turn).
template <bool I64>
__device__ __forceinline__ int64_t flat_id(const void* flat, int64_t i) {
  if constexpr (I64) return static_cast<const int64_t*>(flat)[i];
  else return static_cast<int64_t>(static_cast<const int32_t*>(flat)[i]);
}

template <bool STAGED, bool I64>
__global__ __launch_bounds__(kThreads) void align_kernel(const void* __restrict__ flat, int P, int E1,
                                                         int BM, int32_t* __restrict__ sorted_ids,
                                                         int32_t* __restrict__ bexp, int nb,
                                                         int32_t* __restrict__ expert_offsets) {
  __shared__ int cnt[kWaves][kMaxSlots];                 // per-wave counts, then per-wave write cursors
  __shared__ unsigned long long lanes[kWaves][kMaxSlots]; // per-wave lane masks of one 64-pair chunk
  __shared__ int pend[kMaxSlots];                         // padded end row of each expert
  extern __shared__ uint16_t staged[];                    // STAGED: expert id of pair p (kNoExpert: dropped)
  const int tid = threadIdx.x;
  const int wave = tid / kWave, lane = lane_id();

  for (int i = tid; i < kWaves * kMaxSlots; i += kThreads) {
    (&cnt[0][0])[i] = 0;
    (&lanes[0][0])[i] = 0ull;
  }
  const int total_rows = nb * BM;
  for (int i = tid; i < total_rows; i += kThreads) sorted_ids[i] = P;
  __syncthreads();

  // each wave owns a contiguous, 64-aligned segment of pairs
  const int seg = ((P + kWaves - 1) / kWaves + kWave - 1) / kWave * kWave;
  const int beg = min(P, wave * seg), end = min(P, beg + seg);
  // ids in batches of kIdBatch loads per lane, all issued before the first is used (a lane past the end
  // re-reads the segment's last id and discards it)
  for (int c0 = beg; c0 < end; c0 += kWave * kIdBatch) {
    int64_t ev[kIdBatch];
#pragma unroll
    for (int u = 0; u < kIdBatch; ++u) ev[u] = flat_id<I64>(flat, min(c0 + u * kWave + lane, end - 1));
#pragma unroll
    for (int u = 0; u < kIdBatch; ++u) {
      const int p = c0 + u * kWave + lane;
      if (p >= end) continue;
      const bool valid = ev[u] >= 0 && ev[u] < E1;
      if (STAGED) staged[p] = valid ? static_cast<uint16_t>(ev[u]) : kNoExpert;
      if (valid) atomicAdd(&cnt[wave][ev[u]], 1);
    }
  }
  __syncthreads();

  // padded sizes, their inclusive scan (Hillis-Steele over <= 256 experts), per-wave write cursors
  int padded = 0;
  if (tid < kMaxSlots && tid < E1) {
    int tot = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) tot += cnt[w][tid];
    padded = (tot + BM - 1) / BM * BM;
  }
  if (tid < kMaxSlots) pend[tid] = padded;
  __syncthreads();
  for (int off = 1; off < kMaxSlots; off <<= 1) {
    int v = 0;
    if (tid < kMaxSlots && tid >= off) v = pend[tid - off];
    __syncthreads();
    if (tid < kMaxSlots) pend[tid] += v;
    __syncthreads();
  }
  if (tid < E1) {
    int run = pend[tid] - padded;  // padded start of expert tid
    if (expert_offsets) expert_offsets[tid] = run;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const int c = cnt[w][tid];
      cnt[w][tid] = run;
      run += c;
    }
  }
  if (tid == 0 && expert_offsets) expert_offsets[E1] = pend[E1 - 1];
  __syncthreads();

  // scatter: chunks of 64 pairs in order; rank inside a chunk = earlier lanes with the same expert
  for (int c0 = beg; c0 < end; c0 += kWave) {
    const int p = c0 + lane;
    int64_t e = -1;
    if (STAGED) {
      if (p < end && staged[p] != kNoExpert) e = staged[p];
    } else if (p < end) {
      e = flat_id<I64>(flat, p);
    }
    const bool valid = e >= 0 && e < E1;
    if (valid) atomicOr(&lanes[wave][e], 1ull << lane);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    unsigned long long m = 0;
    int cur = 0;
    if (valid) {
      m = lanes[wave][e];
      cur = cnt[wave][e];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (valid) {
      const unsigned long long below = (lane == 0) ? 0ull : (m & ((1ull << lane) - 1ull));
      const int rank = __popcll(below);
      sorted_ids[cur + rank] = p;
      if (rank == 0) {
        cnt[wave][e] = cur + __popcll(m);
        lanes[wave][e] = 0ull;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }

  // block -> expert: first expert whose padded end lies beyond the block start (searchsorted right)
  for (int b = tid; b < nb; b += kThreads) {
    const int pos = b * BM;
    int lo = 0, hi = E1;  // first index in [0, E1) with pend > pos, E1 if none
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (pend[mid] > pos) hi = mid;
      else lo = mid + 1;
    }
    bexp[b] = lo < E1 ? lo : -1;
  }
}

}  // namespace

extern "C" int mm_align_blocks(const void* flat, int flat_dtype, int64_t P, int32_t n_slots, int32_t block_m,
                               int32_t* sorted_ids, int32_t* bexp, int64_t nb, int32_t* expert_offsets, void* stream) {
  MM_REQUIRE(flat_dtype == MM_INT32 || flat_dtype == MM_INT64, "align_blocks: ids must be int32 or int64");
  MM_REQUIRE(P >= 0 && P <= (1LL << 30), "align_blocks: P=%lld out of range", (long long)P);
  MM_REQUIRE(n_slots >= 1 && n_slots <= kMaxSlots, "align_blocks: n_slots=%d must be in [1, %d]", n_slots, kMaxSlots);
  MM_REQUIRE(block_m >= 1 && block_m <= 4096, "align_blocks: block_m=%d out of range", block_m);
  const int64_t want = (P + static_cast<int64_t>(n_slots) * (block_m - 1) + block_m - 1) / block_m;
  MM_REQUIRE(nb == want, "align_blocks: nb=%lld, expected ceil((P + n_slots*(block_m-1))/block_m)=%lld", (long long)nb,
             (long long)want);
  MM_REQUIRE(nb * block_m <= (1LL << 31) - 1, "align_blocks: too many rows");
  MM_REQUIRE(sorted_ids && bexp && (P == 0 || flat), "align_blocks: null pointer");
  const bool i64 = flat_dtype == MM_INT64;
  auto kernel = P <= kMaxStaged ? (i64 ? align_kernel<true, true> : align_kernel<true, false>)
                                : (i64 ? align_kernel<false, true> : align_kernel<false, false>);
  size_t lds = 0;
  if (P <= kMaxStaged) {
    lds = (static_cast<size_t>(P) * 2 + 15) / 16 * 16;
    int rc = mm::allow_lds(kernel, static_cast<size_t>(kMaxStaged) * 2, "align_blocks");
    if (rc) return rc;
  }
  hipLaunchKernelGGL(kernel, dim3(1), dim3(kThreads), lds, MM_STREAM(stream), flat, static_cast<int>(P),
                     static_cast<int>(n_slots), static_cast<int>(block_m), sorted_ids, bexp, static_cast<int>(nb),
                     expert_offsets);
  return mm::check_launch("align_blocks");
}
