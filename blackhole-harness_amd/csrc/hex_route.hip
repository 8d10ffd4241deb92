// Slot planning for the HEX MoE kernels (the routing itself is in hex_router.hip).
//
//   bh_hex_align       stable counting sort of slots by expert, padded to block_m
//                      (runtime/blackhole_runtime/hex_moe.py:201-222)
//   bh_hex_direct      one block per slot (hex_moe.py:228-237)
//
// align runs in one workgroup of 1024 threads. Counts come from LDS atomics; the order of slots
// inside an expert's run is the slot order (the reference's stable argsort). Each wave finds,
// for each of its 64 slots, the lanes holding the same expert by intersecting one ballot per bit
// of the expert id (log2(E) ballots, independent of how many experts the wave holds); the
// slot's rank inside its run is then the run's offset so far + the counts of earlier waves of
// the chunk + the same-expert lanes below it.
#include <string>

#include "hex_common.h"

namespace bh {

// ----------------------------------------------------------------------------------- align

constexpr int kAlignThreads = 1024;
constexpr int kAlignWaves = kAlignThreads / kWave;
constexpr int kAlignMaxExperts = 1024;
constexpr int64_t kAlignSplit = 4096;     // slots above which the placement runs on many workgroups

template <int IDT>
__device__ __forceinline__ int64_t load_id(const void* p, int64_t i) {
  if constexpr (IDT == BH_HEX_I64) return reinterpret_cast<const int64_t*>(p)[i];
  else return reinterpret_cast<const int32_t*>(p)[i];
}

// The expert slot i is placed under, or -1: ids outside [0, n) are not placed, nor, for a tier's
// plan (TIER), experts the tier does not hold (lookup < 0). (A template flag, not a null test:
// the plain plan's batched id loads then compile without the dependent lookup load.)
template <int IDT, bool TIER>
__device__ __forceinline__ int64_t placed_id(const void* p, int64_t i, int32_t n, const int32_t* lookup) {
  const int64_t e = load_id<IDT>(p, i);
  if constexpr (TIER) return (e >= 0 && e < n && lookup[e] >= 0) ? e : -1;
  else return (e >= 0 && e < n) ? e : -1;
}

// Stable counting sort of the slots by expert, each expert's run padded to bm. Wave w owns the
// contiguous slot range [w P, (w + 1) P): it counts its slots per expert (lanes with the same
// key found by ballots over the key bits, so each key is counted once per 64-slot chunk), one
// pass over the waves turns the counts into each wave's offset inside every expert's run, and
// each wave then places its own range in order with no further workgroup barrier.
// Without SCATTER the workgroup only counts (LDS atomics) and writes the block plan; the slots
// are then placed by align_scatter_kernel, one workgroup per 1024 slots.
template <int IDT, bool SCATTER, bool TIER>
__global__ __launch_bounds__(kAlignThreads) void align_kernel(const void* __restrict__ ids, int64_t S, int32_t n,
                                                              const int32_t* __restrict__ lookup, int32_t bm,
                                                              int64_t max_blocks,
                                                              int32_t* __restrict__ sorted_ids,
                                                              int32_t* __restrict__ expert_ids,
                                                              int32_t* __restrict__ npp, int32_t* __restrict__ ws) {
  __shared__ int cnt[kAlignMaxExperts];      // slots per expert
  __shared__ int start[kAlignMaxExperts];    // first padded row of the expert's run
  __shared__ int wcnt[kAlignWaves][kAlignMaxExperts];   // per wave: count, then offset in the run
  __shared__ int wsum[kAlignWaves];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  int nbits = 1;
  while ((1 << nbits) <= n) ++nbits;          // keys in [0, n] (n marks "not placed")
  const uint64_t below = (lane ? (~0ull >> (64 - lane)) : 0ull);
  // whole 64-slot chunks per wave (a small batch leaves the later waves empty)
  const int64_t per = ((S + kAlignWaves - 1) / kAlignWaves + kWave - 1) / kWave * kWave;
  const int64_t r0 = min(S, (int64_t)w * per), r1 = min(S, r0 + per);
  constexpr int kBatch = 16;                 // id loads issued together by the counting loop
  auto match = [&](int key) { return match_key(key, nbits); };

  // With SCATTER (at most kAlignSplit slots) a wave's range is at most kSC chunks of 64, so its
  // keys and their lane matches are kept in registers from the count to the placement (one
  // round trip to the ids), and only the waves that hold slots (nw) enter the offset pass.
  constexpr int kSC = (int)(kAlignSplit / kAlignThreads);
  int skey[kSC];
  uint64_t ssame[kSC];
  const int nw = per ? (int)((S + per - 1) / per) : 0;
  if constexpr (SCATTER) {
    if (r0 < r1) {
      for (int e = lane; e < n; e += kWave) wcnt[w][e] = 0;
#pragma unroll
      for (int k = 0; k < kSC; ++k) {
        const int64_t i = r0 + k * kWave + lane;
        const int64_t e = i < r1 ? placed_id<IDT, TIER>(ids, i, n, lookup) : -1;
        skey[k] = (e >= 0 && e < n) ? (int)e : n;
      }
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int k = 0; k < kSC; ++k) {
        if (r0 + k * kWave >= r1) break;                 // (uniform: the wave's range ends)
        ssame[k] = match(skey[k]);
        if (skey[k] < n && __popcll(ssame[k] & below) == 0) wcnt[w][skey[k]] += __popcll(ssame[k]);
        __builtin_amdgcn_wave_barrier();
      }
    }
    __syncthreads();
    for (int e = tid; e < n; e += kAlignThreads) {        // counts -> offsets over the waves
      int acc = 0;
      for (int v = 0; v < nw; ++v) {
        const int c = wcnt[v][e];
        wcnt[v][e] = acc;
        acc += c;
      }
      cnt[e] = acc;
    }
  } else if (ws) {
    // align_count_kernel's counts per 1024-slot chunk -> each chunk's exclusive prefix per
    // expert (in place, read by align_scatter_kernel) and the totals. When they fit, the counts
    // pass through the (here unused) per-wave counter array in LDS: one round trip to the
    // workspace each way, with every thread loading, instead of one per 8 chunks per expert.
    const int nch = (int)((S + kAlignThreads - 1) / kAlignThreads);
    const int nv = nch * n;
    int* const lc = &wcnt[0][0];
    if (nv <= kAlignWaves * kAlignMaxExperts) {
      for (int v = tid; v < nv; v += kAlignThreads) lc[v] = ws[v];
      __syncthreads();
      for (int e = tid; e < n; e += kAlignThreads) {
        int acc = 0;
        for (int c = 0; c < nch; ++c) {
          const int v = lc[c * n + e];
          lc[c * n + e] = acc;
          acc += v;
        }
        cnt[e] = acc;
      }
      __syncthreads();
      for (int v = tid; v < nv; v += kAlignThreads) ws[v] = lc[v];
    } else {
      for (int e = tid; e < n; e += kAlignThreads) {
        int acc = 0;
        for (int c0 = 0; c0 < nch; c0 += 8) {
          int v[8];
#pragma unroll
          for (int d = 0; d < 8; ++d) v[d] = c0 + d < nch ? ws[(int64_t)(c0 + d) * n + e] : 0;
#pragma unroll
          for (int d = 0; d < 8; ++d)
            if (c0 + d < nch) {
              ws[(int64_t)(c0 + d) * n + e] = acc;
              acc += v[d];
            }
        }
        cnt[e] = acc;
      }
    }
  } else {
    for (int e = tid; e < n; e += kAlignThreads) cnt[e] = 0;
    __syncthreads();
    for (int64_t b0 = 0; b0 < S; b0 += kBatch * kAlignThreads) {
      int64_t e[kBatch];
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const int64_t i = b0 + k * kAlignThreads + tid;
        e[k] = i < S ? placed_id<IDT, TIER>(ids, i, n, lookup) : -1;
      }
#pragma unroll
      for (int k = 0; k < kBatch; ++k)
        if (e[k] >= 0 && e[k] < n) atomicAdd(&cnt[e[k]], 1);
    }
  }
  __syncthreads();

  // blocks per expert -> block ends (inclusive scan over experts, each thread a run of them)
  const int pe = (n + kAlignThreads - 1) / kAlignThreads;
  const int e0 = tid * pe, e1 = min(n, e0 + pe);
  int local = 0;
  for (int e = e0; e < e1; ++e) local += (cnt[e] + bm - 1) / bm;
  const int incl = block_incl_scan(local, wsum);
  int run = incl - local;                      // blocks before this thread's experts
  for (int e = e0; e < e1; ++e) {
    const int nb = (cnt[e] + bm - 1) / bm;
    start[e] = run * bm;
    for (int b = run; b < run + nb; ++b) expert_ids[b] = e;
    // rows of the run that no slot fills
    for (int64_t r = (int64_t)run * bm + cnt[e]; r < (int64_t)(run + nb) * bm; ++r) sorted_ids[r] = (int32_t)S;
    run += nb;
  }
  __shared__ int total_blocks;
  if (tid == kAlignThreads - 1) total_blocks = incl;
  __syncthreads();
  const int used = total_blocks;
  for (int64_t b = used + tid; b < max_blocks; b += kAlignThreads) expert_ids[b] = -1;
  for (int64_t r = (int64_t)used * bm + tid; r < max_blocks * bm; r += kAlignThreads) sorted_ids[r] = (int32_t)S;
  if (tid == 0) npp[0] = used * bm;
  if constexpr (!SCATTER) return;

  // each wave places its range, chunk by chunk in slot order: a lane's row is its expert's
  // run start + the wave's offset in that run + its rank among the chunk's lanes of the expert;
  // the key's lowest lane then moves the wave's offset on (after every lane has read it)
#pragma unroll
  for (int k = 0; k < kSC; ++k) {
    if (r0 + k * kWave >= r1) break;                     // (uniform: the wave's range ends)
    const int64_t i = r0 + k * kWave + lane;
    const int rank = __popcll(ssame[k] & below);
    if (skey[k] < n) {
      const int64_t pos = (int64_t)start[skey[k]] + wcnt[w][skey[k]] + rank;
      if (pos < max_blocks * bm) sorted_ids[pos] = (int32_t)i;
    }
    __builtin_amdgcn_wave_barrier();
    if (skey[k] < n && rank == 0) wcnt[w][skey[k]] += __popcll(ssame[k]);
    __builtin_amdgcn_wave_barrier();
  }
}

// Counts the placed slots of chunk blockIdx.x (1024 slots) per expert into ws[chunk * n + e]
// (every entry of the chunk's row is written, so the workspace needs no clearing).
template <int IDT, bool TIER>
__global__ __launch_bounds__(kAlignThreads) void align_count_kernel(const void* __restrict__ ids, int64_t S,
                                                                    int32_t n, const int32_t* __restrict__ lookup,
                                                                    int32_t* __restrict__ ws) {
  __shared__ int cnt[kAlignMaxExperts];
  __shared__ int lk[TIER ? kAlignMaxExperts : 1];   // the tier lookup
  const int tid = threadIdx.x;
  // the slot's id and the lookup together (one round trip; the lookup of the id then from LDS)
  const int64_t i = (int64_t)blockIdx.x * kAlignThreads + tid;
  const int64_t id = i < S ? load_id<IDT>(ids, i) : -1;
  for (int e = tid; e < n; e += kAlignThreads) {
    cnt[e] = 0;
    if constexpr (TIER) lk[e] = lookup[e];
  }
  __syncthreads();
  if (id >= 0 && id < n && (!TIER || lk[TIER ? id : 0] >= 0)) atomicAdd(&cnt[id], 1);
  __syncthreads();
  for (int e = tid; e < n; e += kAlignThreads) ws[(int64_t)blockIdx.x * n + e] = cnt[e];
}

// Places the slots of chunk blockIdx.x (1024 slots) after align_kernel<IDT, false> wrote the
// block plan: the chunk's slots of each expert go after the expert's slots in earlier chunks
// (read from the workspace's prefix when there is one, else counted again here), in slot order
// (per wave by ballot rank, then over the waves).
template <int IDT, bool TIER>
__global__ __launch_bounds__(kAlignThreads) void align_scatter_kernel(const void* __restrict__ ids, int64_t S,
                                                                      int32_t n, const int32_t* __restrict__ lookup,
                                                                      int32_t bm, int64_t max_blocks,
                                                                      int32_t* __restrict__ sorted_ids,
                                                                      const int32_t* __restrict__ expert_ids,
                                                                      const int32_t* __restrict__ npp,
                                                                      const int32_t* __restrict__ ws) {
  __shared__ int pre[kAlignMaxExperts];      // the expert's slots in earlier chunks
  __shared__ int start[kAlignMaxExperts];    // first padded row of the expert's run
  __shared__ int wcnt[kAlignWaves][kAlignMaxExperts];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  int nbits = 1;
  while ((1 << nbits) <= n) ++nbits;
  const uint64_t below = (lane ? (~0ull >> (64 - lane)) : 0ull);
  const int64_t c0 = (int64_t)blockIdx.x * kAlignThreads;
  for (int e = tid; e < n; e += kAlignThreads) pre[e] = ws ? ws[(int64_t)blockIdx.x * n + e] : 0;
  for (int e = lane; e < n; e += kWave) wcnt[w][e] = 0;
  __syncthreads();
  constexpr int kBatch = 16;
  const int64_t pre_end = ws ? 0 : c0;        // without a workspace: count the slots before the chunk
  for (int64_t b0 = 0; b0 < pre_end; b0 += kBatch * kAlignThreads) {
    int64_t e[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int64_t i = b0 + k * kAlignThreads + tid;
      e[k] = i < pre_end ? placed_id<IDT, TIER>(ids, i, n, lookup) : -1;
    }
#pragma unroll
    for (int k = 0; k < kBatch; ++k)
      if (e[k] >= 0 && e[k] < n) atomicAdd(&pre[e[k]], 1);
  }
  const int used = npp[0] / bm;
  for (int b = tid; b < used; b += kAlignThreads) {
    const int e = expert_ids[b];
    if (e >= 0 && e < n && (b == 0 || expert_ids[b - 1] != e)) start[e] = b * bm;
  }
  const int64_t i = c0 + tid;
  int key = n;
  if (i < S) {
    const int64_t e = placed_id<IDT, TIER>(ids, i, n, lookup);
    if (e >= 0) key = (int)e;
  }
  const uint64_t same = match_key(key, nbits);
  const int rank = __popcll(same & below);
  if (key < n && rank == 0) wcnt[w][key] = __popcll(same);
  __syncthreads();
  for (int e = tid; e < n; e += kAlignThreads) {        // offsets: earlier chunks, then earlier waves
    int acc = pre[e];
    for (int v = 0; v < kAlignWaves; ++v) {
      const int c = wcnt[v][e];
      wcnt[v][e] = acc;
      acc += c;
    }
  }
  __syncthreads();
  if (key < n) {
    const int64_t pos = (int64_t)start[key] + wcnt[w][key] + rank;
    if (pos < max_blocks * bm) sorted_ids[pos] = (int32_t)i;
  }
}

// The block plan and the placement in one launch after align_count_kernel, one workgroup per
// 1024-slot chunk, when every chunk's counts fit in LDS (chunks x experts <= kPlaceMaxCounts).
// Each workgroup reads all chunks' counts, forms each expert's total and its slots in earlier
// chunks, scans the experts' block counts for their runs' first rows, and places its own slots
// as align_scatter_kernel does. The block plan's other rows are spread over the workgroups:
// expert e's blocks and unfilled rows by workgroup e % chunks, the rows and blocks past the used
// ones in turn. Same result as align_kernel<IDT, false> followed by align_scatter_kernel.
constexpr int kPlaceMaxCounts = kAlignWaves * kAlignMaxExperts;

template <int IDT, bool TIER>
__global__ __launch_bounds__(kAlignThreads) void align_place_kernel(const void* __restrict__ ids, int64_t S,
                                                                    int32_t n, const int32_t* __restrict__ lookup,
                                                                    int32_t bm, int64_t max_blocks,
                                                                    int32_t* __restrict__ sorted_ids,
                                                                    int32_t* __restrict__ expert_ids,
                                                                    int32_t* __restrict__ npp,
                                                                    const int32_t* __restrict__ ws) {
  __shared__ int lc[kPlaceMaxCounts];        // every chunk's counts, [chunk][expert]
  __shared__ int wcnt[kAlignWaves][kAlignMaxExperts];   // per wave: count, then offset in the run
  __shared__ int pre[kAlignMaxExperts];      // the expert's slots in earlier chunks
  __shared__ int start[kAlignMaxExperts];    // first padded row of the expert's run
  __shared__ int wsum[kAlignWaves];
  __shared__ int total_blocks;
  __shared__ int lk[TIER ? kAlignMaxExperts : 1];   // the tier lookup
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int nch = (int)gridDim.x, c = (int)blockIdx.x;
  int nbits = 1;
  while ((1 << nbits) <= n) ++nbits;
  const uint64_t below = (lane ? (~0ull >> (64 - lane)) : 0ull);
  // every chunk's counts (all loads before any store: indices past the last repeat it, so no
  // branch and no wait between them), then this thread's slot
  const int nv = nch * n;
  constexpr int kPT = kPlaceMaxCounts / kAlignThreads;
  int cv[kPT];
#pragma unroll
  for (int q = 0; q < kPT; ++q) cv[q] = ws[min(tid + q * kAlignThreads, nv - 1)];
  const int64_t i = (int64_t)c * kAlignThreads + tid;
  const int64_t id = i < S ? load_id<IDT>(ids, i) : -1;
  if constexpr (TIER)
    for (int e = tid; e < n; e += kAlignThreads) lk[e] = lookup[e];
  for (int e = lane; e < n; e += kWave) wcnt[w][e] = 0;
#pragma unroll
  for (int q = 0; q < kPT; ++q)
    if (tid + q * kAlignThreads < nv) lc[tid + q * kAlignThreads] = cv[q];
  __syncthreads();
  const int key = (id >= 0 && id < n && (!TIER || lk[TIER ? id : 0] >= 0)) ? (int)id : n;
  // thread e: expert e's slots in earlier chunks and in all (n <= kAlignThreads)
  // (no store inside the loop, so its reads are issued together)
  int tot = 0, mine = 0;
  if (tid < n) {
#pragma unroll 8
    for (int cc = 0; cc < nch; ++cc) {
      const int v = lc[cc * n + tid];
      mine += cc < c ? v : 0;
      tot += v;
    }
    pre[tid] = mine;
  }
  const int nb = (tot + bm - 1) / bm;
  const int incl = block_incl_scan(nb, wsum);  // (its barriers order the LDS accesses around it)
  const int run = incl - nb;                   // blocks before expert tid's run
  if (tid < n) start[tid] = run * bm;
  if (tid == kAlignThreads - 1) total_blocks = incl;
  const uint64_t same = match_key(key, nbits);
  const int rank = __popcll(same & below);
  if (key < n && rank == 0) wcnt[w][key] = __popcll(same);
  __syncthreads();
  const int used = total_blocks;
  if (tid < n && tid % nch == c) {
    for (int b = run; b < run + nb; ++b) expert_ids[b] = tid;
    for (int64_t r = (int64_t)run * bm + tot; r < (int64_t)(run + nb) * bm; ++r) sorted_ids[r] = (int32_t)S;
  }
  const int64_t step = (int64_t)nch * kAlignThreads;
  for (int64_t b = used + (int64_t)c * kAlignThreads + tid; b < max_blocks; b += step) expert_ids[b] = -1;
  for (int64_t r = (int64_t)used * bm + (int64_t)c * kAlignThreads + tid; r < max_blocks * bm; r += step)
    sorted_ids[r] = (int32_t)S;
  if (c == 0 && tid == 0) npp[0] = used * bm;
  for (int e = tid; e < n; e += kAlignThreads) {        // offsets: earlier chunks, then earlier waves
    int cw[kAlignWaves];
#pragma unroll
    for (int v = 0; v < kAlignWaves; ++v) cw[v] = wcnt[v][e];   // (all reads before the writes)
    int acc = pre[e];
#pragma unroll
    for (int v = 0; v < kAlignWaves; ++v) {
      wcnt[v][e] = acc;
      acc += cw[v];
    }
  }
  __syncthreads();
  if (key < n) {
    const int64_t pos = (int64_t)start[key] + wcnt[w][key] + rank;
    if (pos < max_blocks * bm) sorted_ids[pos] = (int32_t)i;
  }
}

template <int IDT>
__global__ __launch_bounds__(256) void direct_kernel(const void* __restrict__ ids, int64_t S, int32_t bm,
                                                     int32_t* __restrict__ sorted_ids, int32_t* __restrict__ expert_ids,
                                                     int32_t* __restrict__ npp) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r < S * bm) {
    const int64_t s = r / bm;
    sorted_ids[r] = (r - s * bm) == 0 ? (int32_t)s : (int32_t)S;
  }
  if (r < S) expert_ids[r] = (int32_t)load_id<IDT>(ids, r);
  if (r == 0) npp[0] = (int32_t)(S * bm);
}

}  // namespace bh

using namespace bh;

extern "C" int64_t bh_hex_align_max_blocks(int64_t S, int32_t n_experts, int32_t block_m) {
  if (block_m <= 0 || S < 0 || n_experts < 0) return -1;
  return cdiv(S, block_m) + (S < n_experts ? S : (int64_t)n_experts);
}

extern "C" int64_t bh_hex_align_workspace(int64_t S, int32_t n_experts) {
  if (S < 0 || n_experts <= 0) return -1;
  return S > kAlignSplit ? cdiv(S, kAlignThreads) * n_experts : 0;
}

// ws: null (the slots before each chunk are counted again by its placing workgroup), or
// bh_hex_align_workspace(S, n) int32 values for the per-chunk counts.
static int align_run(const char* who, const void* ids, int32_t ids_dtype, int64_t S, int32_t n_experts,
                     const int32_t* lookup, int32_t block_m, int32_t* ws, int64_t ws_len, int32_t* sorted_ids,
                     int32_t* expert_ids, int32_t* npp, void* stream) {
  const std::string w(who);
  if (block_m <= 0) return fail(BH_HEX_ERR_VALUE, w + ": block_m must be positive");
  if (n_experts <= 0 || n_experts > kAlignMaxExperts)
    return fail(BH_HEX_ERR_UNSUPPORTED, w + ": experts must be in 1.." + std::to_string(kAlignMaxExperts));
  if (S < 0 || S > (int64_t)INT32_MAX / 2) return fail(BH_HEX_ERR_VALUE, w + ": slot count out of range");
  if (ids_dtype != BH_HEX_I32 && ids_dtype != BH_HEX_I64)
    return fail(BH_HEX_ERR_UNSUPPORTED, w + ": ids dtype must be I32 or I64");
  if (!npp || (S > 0 && (!ids || !sorted_ids || !expert_ids))) return fail(BH_HEX_ERR_VALUE, w + ": null pointer");
  const int64_t max_blocks = bh_hex_align_max_blocks(S, n_experts, block_m);
  if (max_blocks * block_m > (int64_t)INT32_MAX) return fail(BH_HEX_ERR_VALUE, w + ": plan too large");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  // up to kAlignSplit slots one workgroup does everything; above, with a workspace, one workgroup
  // per 1024 slots first counts them, and then (when every chunk's counts fit in LDS) one
  // workgroup per chunk forms the block plan and places its slots; otherwise one workgroup writes
  // the block plan and one per chunk places the slots
  const bool split = S > kAlignSplit;
  if (!split) ws = nullptr;
  if (ws && ws_len < bh_hex_align_workspace(S, n_experts)) return fail(BH_HEX_ERR_VALUE, w + ": workspace too small");
  const dim3 chunks((unsigned)cdiv(S, kAlignThreads));
  const dim3 one(1), threads(kAlignThreads);
  const bool place = ws && cdiv(S, kAlignThreads) * n_experts <= kPlaceMaxCounts;
#define BH_ALIGN(IDT, TIER)                                                                                       \
  do {                                                                                                            \
    if (split) {                                                                                                  \
      if (ws)                                                                                                     \
        hipLaunchKernelGGL((align_count_kernel<IDT, TIER>), chunks, threads, 0, st, ids, S, n_experts, lookup, ws); \
      if (place) {                                                                                                \
        hipLaunchKernelGGL((align_place_kernel<IDT, TIER>), chunks, threads, 0, st, ids, S, n_experts, lookup,    \
                           block_m, max_blocks, sorted_ids, expert_ids, npp, ws);                                 \
        break;                                                                                                    \
      }                                                                                                           \
      hipLaunchKernelGGL((align_kernel<IDT, false, TIER>), one, threads, 0, st, ids, S, n_experts, lookup,        \
                         block_m, max_blocks, sorted_ids, expert_ids, npp, ws);                                   \
      hipLaunchKernelGGL((align_scatter_kernel<IDT, TIER>), chunks, threads, 0, st, ids, S, n_experts, lookup,    \
                         block_m, max_blocks, sorted_ids, expert_ids, npp, ws);                                   \
    } else {                                                                                                      \
      hipLaunchKernelGGL((align_kernel<IDT, true, TIER>), one, threads, 0, st, ids, S, n_experts, lookup, block_m, \
                         max_blocks, sorted_ids, expert_ids, npp, nullptr);                                       \
    }                                                                                                             \
  } while (0)
  if (lookup) {
    if (ids_dtype == BH_HEX_I64) BH_ALIGN(BH_HEX_I64, true);
    else BH_ALIGN(BH_HEX_I32, true);
  } else {
    if (ids_dtype == BH_HEX_I64) BH_ALIGN(BH_HEX_I64, false);
    else BH_ALIGN(BH_HEX_I32, false);
  }
#undef BH_ALIGN
  return check_launch(who);
}

extern "C" int bh_hex_align(const void* ids, int32_t ids_dtype, int64_t S, int32_t n_experts, int32_t block_m,
                            int32_t* sorted_ids, int32_t* expert_ids, int32_t* npp, void* stream) {
  return align_run("bh_hex_align", ids, ids_dtype, S, n_experts, nullptr, block_m, nullptr, 0, sorted_ids, expert_ids,
                   npp, stream);
}

extern "C" int bh_hex_align_tier(const void* ids, int32_t ids_dtype, int64_t S, int32_t n_experts,
                                 const int32_t* lookup, int32_t block_m, int32_t* sorted_ids, int32_t* expert_ids,
                                 int32_t* npp, void* stream) {
  if (!lookup) return fail(BH_HEX_ERR_VALUE, "bh_hex_align_tier: null lookup");
  return align_run("bh_hex_align_tier", ids, ids_dtype, S, n_experts, lookup, block_m, nullptr, 0, sorted_ids,
                   expert_ids, npp, stream);
}

extern "C" int bh_hex_align_ws(const void* ids, int32_t ids_dtype, int64_t S, int32_t n_experts, const int32_t* lookup,
                               int32_t block_m, int32_t* workspace, int64_t workspace_len, int32_t* sorted_ids,
                               int32_t* expert_ids, int32_t* npp, void* stream) {
  const int64_t need = bh_hex_align_workspace(S, n_experts);
  if (need > 0 && !workspace) return fail(BH_HEX_ERR_VALUE, "bh_hex_align_ws: null workspace");
  return align_run("bh_hex_align_ws", ids, ids_dtype, S, n_experts, lookup, block_m, workspace, workspace_len,
                   sorted_ids, expert_ids, npp, stream);
}

extern "C" int bh_hex_direct(const void* ids, int32_t ids_dtype, int64_t S, int32_t block_m, int32_t* sorted_ids,
                             int32_t* expert_ids, int32_t* npp, void* stream) {
  if (block_m <= 0) return fail(BH_HEX_ERR_VALUE, "bh_hex_direct: block_m must be positive");
  if (S < 0 || S * block_m > (int64_t)INT32_MAX) return fail(BH_HEX_ERR_VALUE, "bh_hex_direct: slot count out of range");
  if (ids_dtype != BH_HEX_I32 && ids_dtype != BH_HEX_I64)
    return fail(BH_HEX_ERR_UNSUPPORTED, "bh_hex_direct: ids dtype must be I32 or I64");
  if (!npp || (S > 0 && (!ids || !sorted_ids || !expert_ids))) return fail(BH_HEX_ERR_VALUE, "bh_hex_direct: null pointer");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int64_t work = S * block_m > 0 ? S * block_m : 1;
  const dim3 grid((unsigned)cdiv(work, 256));
  if (ids_dtype == BH_HEX_I64)
    hipLaunchKernelGGL((direct_kernel<BH_HEX_I64>), grid, dim3(256), 0, st, ids, S, block_m, sorted_ids, expert_ids, npp);
  else
    hipLaunchKernelGGL((direct_kernel<BH_HEX_I32>), grid, dim3(256), 0, st, ids, S, block_m, sorted_ids, expert_ids, npp);
  return check_launch("bh_hex_direct");
}
