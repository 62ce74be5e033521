// Device-side slot cache over an out-of-core table (the MoE expert cache): LRU admission and
// the bookkeeping kernels around it. Only the maps and the copy plan are touched here; the
// rows themselves move with the index-copy kernels of expert_copy.hip.
//
// Maps (all device memory, owned by the caller):
//   slot_of_id [num_total]  int32  id -> slot, -1 when not resident
//   id_of_slot [num_cached] int32  slot -> id, -1 when empty
//   usage      [num_cached] int64  step at which each slot was last touched
//   step       []           int64  monotonic clock, +1 per admission call
// Ids are flat: a caller whose table is split (one partition per MoE layer) passes
// partition-local ids with id_base = partition * partition_size.
//
// lru_ensure_kernel is one 1024-thread workgroup: admission is a small sequential decision
// (a few hundred ids against a few thousand slots), so the whole state of a call lives in LDS
// and every phase is a barrier-separated parallel pass:
//   1. dedup the query, split hits and misses, rank the distinct misses by id, bump hits
//      (match counts over the query read four ids at a time);
//   2. victims in ascending (usage, slot) order among the slots not touched by this call:
//      rounds that take every remaining slot holding the smallest usage, in slot order (each
//      thread owns consecutive slots: a block min, an exclusive scan); an LRU cache fed by
//      calls that each touch many slots needs two or three rounds. After 8 rounds the call
//      falls back to a bitonic sort of packed (usage << bits | slot) keys in LDS;
//   3. the i-th smallest missing id takes the i-th victim: maps, usage and the copy plan.
#include <algorithm>

#include "pia_internal.h"

namespace pia {
namespace {

constexpr int LRU_THREADS = 1024;
constexpr int LRU_MAX_QUERY = 2048;
constexpr int LRU_MAX_CACHED = 16384;
constexpr unsigned long long kKeyNone = ~0ull;  // sorts after every evictable slot

__device__ __forceinline__ int block_sum(int v, int* red) {
  // wave sums, then one wave over the 16 partials
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  int t = (threadIdx.x < LRU_THREADS / 64) ? red[threadIdx.x] : 0;
  if (wave == 0) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) t += __shfl_xor(t, o, 64);
    if (lane == 0) red[LRU_THREADS / 64] = t;
  }
  __syncthreads();
  return red[LRU_THREADS / 64];
}

__device__ __forceinline__ long long block_min64(long long v, long long* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o, 64));
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  long long t = red[0];
#pragma unroll
  for (int w = 1; w < LRU_THREADS / 64; ++w) t = min(t, red[w]);
  return t;
}

// exclusive prefix of v over threads in index order; *total gets the sum
__device__ __forceinline__ int block_excl_scan(int v, int* red, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(incl, o, 64);
    if (lane >= o) incl += t;
  }
  __syncthreads();
  if (lane == 63) red[wave] = incl;
  __syncthreads();
  int before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < LRU_THREADS / 64; ++w) {
    const int t = red[w];
    before += w < wave ? t : 0;
    all += t;
  }
  *total = all;
  return before + incl - v;
}

// number of j < n with q[j] == v (q 16-byte aligned)
__device__ __forceinline__ int count_equal(const int32_t* q, int n, int v) {
  const int4* q4 = reinterpret_cast<const int4*>(q);
  int c = 0;
  const int full = n >> 2;
#pragma unroll 4
  for (int j = 0; j < full; ++j) {
    const int4 x = q4[j];
    c += (x.x == v) + (x.y == v) + (x.z == v) + (x.w == v);
  }
  for (int j = full * 4; j < n; ++j) c += q[j] == v;
  return c;
}

// number of j < n with q[j] < v (q 16-byte aligned)
__device__ __forceinline__ int count_below(const int32_t* q, int n, int v) {
  const int4* q4 = reinterpret_cast<const int4*>(q);
  int c = 0;
  const int full = n >> 2;
#pragma unroll 4
  for (int j = 0; j < full; ++j) {
    const int4 x = q4[j];
    c += (x.x < v) + (x.y < v) + (x.z < v) + (x.w < v);
  }
  for (int j = full * 4; j < n; ++j) c += q[j] < v;
  return c;
}

constexpr int LRU_SPT = LRU_MAX_CACHED / LRU_THREADS;  // slots per thread in the victim rounds
constexpr int LRU_MAX_ROUNDS = 8;
constexpr long long kUsageNone = 0x7fffffffffffffffll;

constexpr int LRU_QPT = LRU_MAX_QUERY / LRU_THREADS;  // queries per thread
constexpr int kIdNone = 0x7fffffff;

// Phase 1 of an admission call, shared by both kernels: advance the clock; load the query
// (out-of-range ids are inert: never resident, never admitted, out = -1); find the first
// occurrences and the first misses among them; bump every hit slot to the new step; rank every
// missing position by the number of distinct missing ids below it (a duplicate shares its first
// occurrence's rank) and list the distinct missing ids in ascending order in miss_ids.
// Ends with a barrier, which also orders the hit bumps before any later read of usage.
__device__ __forceinline__ void lru_phase1(
    const int32_t* __restrict__ query, int K, const int32_t* __restrict__ slot_of_id,
    int64_t num_total, int64_t* __restrict__ usage, int C, int64_t* __restrict__ step_ptr,
    int64_t id_base, int32_t* q_lds, int32_t* fm_ids, int32_t* miss_ids, int* red,
    int64_t* step_lds, int32_t (&qi)[LRU_QPT], int32_t (&si)[LRU_QPT], int (&rank)[LRU_QPT],
    int* distinct_out, int* M_out, int64_t* step_out) {
  const int tid = threadIdx.x;
  constexpr int QPT = LRU_QPT;
  if (tid == 0) {
    const int64_t s = *step_ptr + 1;
    *step_ptr = s;
    *step_lds = s;
  }
#pragma unroll
  for (int r = 0; r < QPT; ++r) {
    const int i = tid + r * LRU_THREADS;
    qi[r] = -1;
    si[r] = -1;
    if (i < K) {
      const int64_t g = int64_t(query[i]) + id_base;
      if (g >= 0 && g < num_total) {
        qi[r] = int32_t(g);
        si[r] = slot_of_id[g];
        if (si[r] >= C) si[r] = -1;  // a map entry past the cache is not a hit
      }
    }
    if (i < LRU_MAX_QUERY) q_lds[i] = i < K ? qi[r] : -1;
  }
  __syncthreads();
  const int64_t step = *step_lds;
  int nfirst = 0, nfm = 0;
#pragma unroll
  for (int r = 0; r < QPT; ++r) {
    const int i = tid + r * LRU_THREADS;
    if (i >= K) continue;
    const bool first = qi[r] >= 0 && count_equal(q_lds, i, qi[r]) == 0;
    const bool fm = first && si[r] < 0;
    fm_ids[i] = fm ? qi[r] : kIdNone;
    nfirst += first ? 1 : 0;
    nfm += fm ? 1 : 0;
    if (si[r] >= 0) usage[si[r]] = step;  // duplicated hits store the same value
  }
  *distinct_out = block_sum(nfirst, red);
  *M_out = block_sum(nfm, red);  // barriers inside also publish fm_ids[]
#pragma unroll
  for (int r = 0; r < QPT; ++r) {
    const int i = tid + r * LRU_THREADS;
    rank[r] = -1;
    if (i >= K || qi[r] < 0 || si[r] >= 0) continue;
    const int rk = count_below(fm_ids, K, qi[r]);
    rank[r] = rk;
    if (fm_ids[i] != kIdNone) miss_ids[rk] = qi[r];
  }
  __syncthreads();
  *step_out = step;
}

__global__ __launch_bounds__(LRU_THREADS) void lru_ensure_kernel(
    const int32_t* __restrict__ query, int K, int32_t* __restrict__ slot_of_id,
    int64_t num_total, int32_t* __restrict__ id_of_slot, int64_t* __restrict__ usage,
    int C, int c_pad, int slot_bits, int64_t* __restrict__ step_ptr,
    int32_t* __restrict__ out, int32_t* __restrict__ src_plan, int32_t* __restrict__ dst_plan,
    int64_t* __restrict__ num_copy, int64_t* __restrict__ stats, int64_t id_base) {
  // keys: the fallback sort; its first 8 KiB hold the round victims otherwise
  __shared__ __attribute__((aligned(16))) unsigned long long keys[LRU_MAX_CACHED];
  __shared__ __attribute__((aligned(16))) int32_t q_lds[LRU_MAX_QUERY];
  __shared__ __attribute__((aligned(16))) int32_t fm_ids[LRU_MAX_QUERY];  // first misses' ids
  __shared__ int32_t miss_ids[LRU_MAX_QUERY];
  __shared__ int red[LRU_THREADS / 64 + 1];
  __shared__ long long red64[LRU_THREADS / 64];
  __shared__ int64_t step_lds;
  int32_t* victims = reinterpret_cast<int32_t*>(keys);
  const int tid = threadIdx.x;

  int32_t qi[LRU_QPT], si[LRU_QPT];
  int rank[LRU_QPT];
  int distinct, M;
  int64_t step;
  lru_phase1(query, K, slot_of_id, num_total, usage, C, step_ptr, id_base, q_lds, fm_ids,
             miss_ids, red, &step_lds, qi, si, rank, &distinct, &M, &step);
  int admitted = 0;
  bool sorted_path = false;
  const unsigned long long slot_mask = (1ull << slot_bits) - 1;
  if (M > 0) {
    // Phase 2: victims. This thread's slots are c0 .. c0 + LRU_SPT - 1.
    const int c0 = tid * LRU_SPT;
    long long u[LRU_SPT];
#pragma unroll
    for (int s = 0; s < LRU_SPT; ++s) {
      const int c = c0 + s;
      u[s] = kUsageNone;
      if (c < C) {
        const int64_t v = usage[c];
        if (v != step) u[s] = v;
      }
    }
    int taken = 0, rounds = 0;
    while (taken < M) {
      long long lmin = kUsageNone;
#pragma unroll
      for (int s = 0; s < LRU_SPT; ++s) lmin = min(lmin, u[s]);
      const long long umin = block_min64(lmin, red64);
      if (umin == kUsageNone) break;  // no evictable slot left
      if (++rounds > LRU_MAX_ROUNDS) {
        sorted_path = true;
        break;
      }
      int cnt = 0;
#pragma unroll
      for (int s = 0; s < LRU_SPT; ++s) cnt += u[s] == umin ? 1 : 0;
      int total;
      int pos = taken + block_excl_scan(cnt, red, &total);
#pragma unroll
      for (int s = 0; s < LRU_SPT; ++s)
        if (u[s] == umin) {
          if (pos < M) victims[pos] = c0 + s;
          ++pos;
          u[s] = kUsageNone;
        }
      taken += min(total, M - taken);
    }
    if (sorted_path) {
      __syncthreads();  // victims (aliasing keys) are no longer read
      // packed (usage, slot) keys of evictable slots, ascending
      for (int c = tid; c < c_pad; c += LRU_THREADS) {
        unsigned long long k = kKeyNone;
        if (c < C) {
          const int64_t v = usage[c];
          if (v != step) k = (static_cast<unsigned long long>(v) << slot_bits) | unsigned(c);
        }
        keys[c] = k;
      }
      __syncthreads();
      for (int size = 2; size <= c_pad; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
          for (int t = tid; t < c_pad / 2; t += LRU_THREADS) {
            const int lo = 2 * t - (t & (stride - 1));
            const int hi = lo + stride;
            const bool up = (lo & size) == 0;
            const unsigned long long a = keys[lo], b = keys[hi];
            if ((a > b) == up) {
              keys[lo] = b;
              keys[hi] = a;
            }
          }
          __syncthreads();
        }
      }
      int nev = 0;
      for (int c = tid; c < C; c += LRU_THREADS) nev += keys[c] != kKeyNone ? 1 : 0;
      taken = min(M, block_sum(nev, red));
    } else {
      __syncthreads();  // victims[] complete
    }
    // Misses beyond the evictable slots (a caller breaking |distinct(query)| <= cache size)
    // are left unadmitted: out = -1 and no plan entry.
    admitted = taken;

    // Phase 3: install. Victims are distinct slots and the evicted ids (resident) never
    // equal the admitted ones (not resident), so the map writes of different i never meet.
    for (int i = tid; i < admitted; i += LRU_THREADS) {
      const int victim = sorted_path ? int(keys[i] & slot_mask) : victims[i];
      const int32_t e = miss_ids[i];
      const int32_t old = id_of_slot[victim];
      if (old >= 0 && old < num_total) slot_of_id[old] = -1;
      id_of_slot[victim] = e;
      slot_of_id[e] = victim;
      usage[victim] = step;
      dst_plan[i] = victim;
      src_plan[i] = int32_t(int64_t(e) - id_base);
    }
  }
  // out may alias query: every query read happened before the barriers above.
#pragma unroll
  for (int r = 0; r < LRU_QPT; ++r) {
    const int i = tid + r * LRU_THREADS;
    if (i >= K) continue;
    int32_t o = si[r];
    if (rank[r] >= 0)
      o = rank[r] < admitted ? (sorted_path ? int32_t(keys[rank[r]] & slot_mask)
                                            : victims[rank[r]])
                             : -1;
    out[i] = o;
  }
  if (tid == 0) {
    *num_copy = admitted;
    if (stats) {
      stats[0] += distinct;
      stats[1] += admitted;
      stats[2] += 1;
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Admission of queries longer than LRU_MAX_QUERY ids (caches of up to LRU_MAX_CACHED slots), with
// the same decisions and no scratch memory: the query is not held in LDS. Hits take the new step
// and every missing id is marked in slot_of_id itself (kMark, a value no slot takes); a scan of
// the queried id range in ascending order then lists the marked ids in batches of up to
// LRU_MAX_QUERY, and each batch takes, in order, the least-recently-used slots not touched by
// this call (victims of earlier batches carry this call's step, so they are touched), exactly
// the slots the ascending misses take one by one in the sequential rule. Ids left without a slot
// are unmarked (-1). Finally every query position reads its slot back from the maps.
// (Assumes consistent maps: id_of_slot[slot_of_id[g]] == g for every resident id g.)
// ---------------------------------------------------------------------------------------------
constexpr int32_t kMark = -2;
constexpr int LRU_WIDE_MAX_QUERY = 1 << 24;

// One batch: the n ids in miss_ids[0, n) (ascending) take the n smallest (usage, slot) of the
// slots whose usage is not `step`, as far as such slots exist; maps, usage and the plan (at
// plan_at) are written. Returns the number admitted. Starts and ends with the workgroup in step.
__device__ int lru_wide_admit(int n, const int32_t* miss_ids, int32_t* victims,
                              int32_t* __restrict__ slot_of_id, int64_t num_total,
                              int32_t* __restrict__ id_of_slot, int64_t* __restrict__ usage,
                              int C, int64_t step, int32_t* __restrict__ src_plan,
                              int32_t* __restrict__ dst_plan, int plan_at, int64_t id_base,
                              int* red, long long* red64) {
  const int tid = threadIdx.x;
  const int c0 = tid * LRU_SPT;
  long long u[LRU_SPT];
#pragma unroll
  for (int s = 0; s < LRU_SPT; ++s) {
    const int c = c0 + s;
    u[s] = kUsageNone;
    if (c < C) {
      const int64_t v = usage[c];
      if (v != step) u[s] = v;
    }
  }
  int taken = 0;
  while (taken < n) {
    long long lmin = kUsageNone;
#pragma unroll
    for (int s = 0; s < LRU_SPT; ++s) lmin = min(lmin, u[s]);
    const long long umin = block_min64(lmin, red64);
    if (umin == kUsageNone) break;  // no evictable slot left
    int cnt = 0;
#pragma unroll
    for (int s = 0; s < LRU_SPT; ++s) cnt += u[s] == umin ? 1 : 0;
    int total;
    int pos = taken + block_excl_scan(cnt, red, &total);
#pragma unroll
    for (int s = 0; s < LRU_SPT; ++s)
      if (u[s] == umin) {
        if (pos < n) victims[pos] = c0 + s;
        ++pos;
        u[s] = kUsageNone;
      }
    taken += min(total, n - taken);
  }
  __syncthreads();  // victims[] complete
  for (int i = tid; i < n; i += LRU_THREADS) {
    const int32_t e = miss_ids[i];
    if (i >= taken) {  // no slot left for it
      slot_of_id[e] = -1;
      continue;
    }
    const int victim = victims[i];
    const int32_t old = id_of_slot[victim];
    if (old >= 0 && old < num_total) slot_of_id[old] = -1;
    id_of_slot[victim] = e;
    slot_of_id[e] = victim;
    usage[victim] = step;
    dst_plan[plan_at + i] = victim;
    src_plan[plan_at + i] = int32_t(int64_t(e) - id_base);
  }
  __syncthreads();  // maps written; miss_ids / victims may be reused
  return taken;
}

__global__ __launch_bounds__(LRU_THREADS) void lru_ensure_wide_kernel(
    const int32_t* __restrict__ query, int K, int32_t* __restrict__ slot_of_id,
    int64_t num_total, int32_t* __restrict__ id_of_slot, int64_t* __restrict__ usage, int C,
    int64_t* __restrict__ step_ptr, int32_t* __restrict__ out, int32_t* __restrict__ src_plan,
    int32_t* __restrict__ dst_plan, int64_t* __restrict__ num_copy, int64_t* __restrict__ stats,
    int64_t id_base) {
  __shared__ int32_t miss_ids[LRU_MAX_QUERY];
  __shared__ int32_t victims[LRU_MAX_QUERY];
  __shared__ int red[LRU_THREADS / 64 + 1];
  __shared__ long long red64[LRU_THREADS / 64];
  __shared__ int64_t step_lds;
  const int tid = threadIdx.x;
  if (tid == 0) {
    const int64_t s = *step_ptr + 1;
    *step_ptr = s;
    step_lds = s;
  }
  __syncthreads();
  const int64_t step = step_lds;
  // hits take the step, missing ids are marked; the range of the valid ids
  long long lo = kUsageNone, neg_hi = kUsageNone;
  for (int i = tid; i < K; i += LRU_THREADS) {
    const int64_t g = int64_t(query[i]) + id_base;
    if (g < 0 || g >= num_total) continue;  // inert: never resident, never admitted
    const int32_t s = slot_of_id[g];
    if (s >= 0 && s < C) usage[s] = step;   // duplicated hits store the same value
    else slot_of_id[g] = kMark;             // a map entry past the cache is not a hit
    lo = min(lo, (long long)g);
    neg_hi = min(neg_hi, -(long long)g);
  }
  lo = block_min64(lo, red64);
  const long long hi = -block_min64(neg_hi, red64);
  __syncthreads();  // marks and hit bumps are visible to the whole workgroup
  // distinct hits: the slots that carry the new step
  int nhit = 0;
  for (int c = tid; c < C; c += LRU_THREADS) nhit += usage[c] == step ? 1 : 0;
  const int hits = block_sum(nhit, red);
  // the marked ids in ascending order, admitted a batch at a time
  int admitted = 0, misses = 0, nb = 0;
  for (long long base = lo; base <= hi; base += LRU_THREADS) {
    const long long g = base + tid;
    const int mk = (g <= hi && slot_of_id[g] == kMark) ? 1 : 0;
    int total;
    const int pos = block_excl_scan(mk, red, &total);
    if (nb + total > LRU_MAX_QUERY) {  // uniform: the batch is full
      admitted += lru_wide_admit(nb, miss_ids, victims, slot_of_id, num_total, id_of_slot,
                                 usage, C, step, src_plan, dst_plan, admitted, id_base, red,
                                 red64);
      nb = 0;
    }
    if (mk) miss_ids[nb + pos] = int32_t(g);
    nb += total;
    misses += total;
    __syncthreads();  // miss_ids of this chunk written
  }
  if (nb > 0)
    admitted += lru_wide_admit(nb, miss_ids, victims, slot_of_id, num_total, id_of_slot, usage,
                               C, step, src_plan, dst_plan, admitted, id_base, red, red64);
  // out may alias query: each position is read and then written by the same thread
  for (int i = tid; i < K; i += LRU_THREADS) {
    const int64_t g = int64_t(query[i]) + id_base;
    out[i] = (g >= 0 && g < num_total) ? slot_of_id[g] : -1;
  }
  if (tid == 0) {
    *num_copy = admitted;
    if (stats) {
      stats[0] += hits + misses;
      stats[1] += admitted;
      stats[2] += 1;
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Admission over caches larger than the LDS-resident kernel holds (16384 < C <= 2^24 slots):
// the same decisions, with the slot state streamed from global memory. Phase 1 is shared.
// Victims: the `take` = min(M, evictable) smallest (usage, slot) keys among the untouched
// slots, found without sorting the cache:
//   a. one pass: smallest and largest usage of an evictable slot, and their count;
//   b. a byte-wise radix select of the take-th smallest usage U over rel = usage - min (only
//      the bytes in which rel can differ: an LRU cache's usages span few of them); per-byte
//      256-bin histograms in LDS, updated once per distinct bin of a wave (the usages of an
//      LRU cache cluster, so lanes mostly share bins); afterwards `need` is how many slots of
//      usage U are victims, the lowest slots first;
//   c. one pass in slot order collecting every evictable slot with usage < U and the first
//      `need` with usage == U (exactly `take` slots);
//   d. a bitonic sort of those by (usage, slot) in LDS.
// Phase 3 is the install of the LDS kernel.
// ---------------------------------------------------------------------------------------------
constexpr int LRU_STREAM_MAX_CACHED = 1 << 24;
constexpr int LRU_SORT_MAX = LRU_MAX_QUERY;  // victims per call (<= distinct misses)

__device__ __forceinline__ unsigned long long block_max_u64(unsigned long long v,
                                                            unsigned long long* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const unsigned long long t = __shfl_xor(v, o, 64);
    v = t > v ? t : v;
  }
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  unsigned long long t = red[0];
#pragma unroll
  for (int w = 1; w < LRU_THREADS / 64; ++w) t = red[w] > t ? red[w] : t;
  return t;
}

// hist[bin] += number of lanes of this wave with that bin (lanes with bin < 0 add nothing):
// one LDS atomic per distinct bin of the wave.
__device__ __forceinline__ void wave_bin_add(int* hist, int bin) {
  uint64_t pending = __ballot(bin >= 0);
  while (pending) {
    const int leader = __builtin_ctzll(pending);
    const int b = __builtin_amdgcn_readlane(bin, leader);
    const uint64_t same = __ballot(bin == b) & pending;
    if ((threadIdx.x & 63) == leader) atomicAdd(&hist[b], int(__popcll(same)));
    pending &= ~same;
  }
}

__global__ __launch_bounds__(LRU_THREADS) void lru_ensure_stream_kernel(
    const int32_t* __restrict__ query, int K, int32_t* __restrict__ slot_of_id,
    int64_t num_total, int32_t* __restrict__ id_of_slot, int64_t* __restrict__ usage, int C,
    int64_t* __restrict__ step_ptr, int32_t* __restrict__ out, int32_t* __restrict__ src_plan,
    int32_t* __restrict__ dst_plan, int64_t* __restrict__ num_copy, int64_t* __restrict__ stats,
    int64_t id_base) {
  __shared__ __attribute__((aligned(16))) int32_t q_lds[LRU_MAX_QUERY];
  __shared__ __attribute__((aligned(16))) int32_t fm_ids[LRU_MAX_QUERY];
  __shared__ int32_t miss_ids[LRU_MAX_QUERY];
  __shared__ unsigned long long cand_u[LRU_SORT_MAX];  // victims' rel usage, then sorted keys
  __shared__ int32_t cand_s[LRU_SORT_MAX];
  __shared__ int hist[256];
  __shared__ int red[LRU_THREADS / 64 + 1];
  __shared__ unsigned long long red64[LRU_THREADS / 64];
  __shared__ int64_t step_lds;
  __shared__ int sel_lds[2];
  const int tid = threadIdx.x;

  int32_t qi[LRU_QPT], si[LRU_QPT];
  int rank[LRU_QPT];
  int distinct, M;
  int64_t step;
  lru_phase1(query, K, slot_of_id, num_total, usage, C, step_ptr, id_base, q_lds, fm_ids,
             miss_ids, red, &step_lds, qi, si, rank, &distinct, &M, &step);
  int admitted = 0;
  if (M > 0) {
    // a. range and count of the evictable usages
    unsigned long long lmin = ~0ull, lmax = 0ull;
    int nev = 0;
    for (int c = tid; c < C; c += LRU_THREADS) {
      const int64_t v = usage[c];
      if (v != step) {
        const unsigned long long k = static_cast<unsigned long long>(v) ^ (1ull << 63);
        lmin = k < lmin ? k : lmin;
        lmax = k > lmax ? k : lmax;
        ++nev;
      }
    }
    const unsigned long long kmin = ~block_max_u64(~lmin, red64);
    const unsigned long long kmax = block_max_u64(lmax, red64);
    const int take = min(M, block_sum(nev, red));
    if (take > 0) {
      // b. radix select of the take-th smallest rel = key - kmin
      const unsigned long long range = kmax - kmin;
      int nbytes = 0;
      while (nbytes < 8 && (range >> (8 * nbytes)) != 0) ++nbytes;
      unsigned long long prefix = 0;  // selected bytes above the current one
      int left = take;                // rank (1-based) still to find inside the prefix
      for (int byte = nbytes - 1; byte >= 0; --byte) {
        for (int i = tid; i < 256; i += LRU_THREADS) hist[i] = 0;
        __syncthreads();
        const int sh = 8 * byte;
        for (int c0 = 0; c0 < C; c0 += LRU_THREADS) {
          const int c = c0 + tid;
          int bin = -1;
          if (c < C) {
            const int64_t v = usage[c];
            if (v != step) {
              const unsigned long long rel =
                  (static_cast<unsigned long long>(v) ^ (1ull << 63)) - kmin;
              const unsigned long long above = sh + 8 < 64 ? (rel >> (sh + 8)) : 0ull;
              if (above == (sh + 8 < 64 ? (prefix >> (sh + 8)) : 0ull))
                bin = int((rel >> sh) & 255u);
            }
          }
          wave_bin_add(hist, bin);
        }
        __syncthreads();
        if (tid < 64) {  // one wave picks the bin holding the left-th key
          int cnt[4], run = 0;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            cnt[j] = hist[4 * tid + j];
            run += cnt[j];
          }
          int incl = run;
#pragma unroll
          for (int o = 1; o < 64; o <<= 1) {
            const int t = __shfl_up(incl, o, 64);
            if (tid >= o) incl += t;
          }
          int before = incl - run;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            if (before < left && left <= before + cnt[j]) {
              sel_lds[0] = 4 * tid + j;
              sel_lds[1] = left - before;
            }
            before += cnt[j];
          }
        }
        __syncthreads();
        prefix |= static_cast<unsigned long long>(sel_lds[0]) << sh;
        left = sel_lds[1];
        __syncthreads();
      }
      const unsigned long long ustar = prefix;  // rel usage of the take-th smallest key
      const int need = left;                    // slots of usage ustar to take, lowest first
      // c. collect in slot order: rel < ustar, and the first `need` with rel == ustar
      int n_lt = 0, n_eq = 0;
      for (int c0 = 0; c0 < C; c0 += LRU_THREADS) {
        const int c = c0 + tid;
        unsigned long long rel = ~0ull;
        if (c < C) {
          const int64_t v = usage[c];
          if (v != step) rel = (static_cast<unsigned long long>(v) ^ (1ull << 63)) - kmin;
        }
        const int lt = rel < ustar ? 1 : 0, eq = rel == ustar ? 1 : 0;
        int tot_lt, tot_eq;
        const int p_lt = block_excl_scan(lt, red, &tot_lt);
        const int p_eq = block_excl_scan(eq, red, &tot_eq);
        if (lt) {
          cand_u[n_lt + p_lt] = rel;
          cand_s[n_lt + p_lt] = c;
        }
        if (eq && n_eq + p_eq < need) {
          const int at = (take - need) + n_eq + p_eq;
          cand_u[at] = rel;
          cand_s[at] = c;
        }
        n_lt += tot_lt;
        n_eq += tot_eq;
      }
      __syncthreads();
      // d. sort the take victims by (rel usage, slot): packed keys when the slot fits 24 bits
      //    under a rel usage of at most 40 bits, else pairs compared field by field
      int n_pad = 1;
      while (n_pad < take) n_pad <<= 1;
      for (int i = take + tid; i < n_pad; i += LRU_THREADS) {
        cand_u[i] = ~0ull;
        cand_s[i] = 0x7fffffff;
      }
      __syncthreads();
      for (int size = 2; size <= n_pad; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
          for (int t = tid; t < n_pad / 2; t += LRU_THREADS) {
            const int lo = 2 * t - (t & (stride - 1));
            const int hi = lo + stride;
            const bool up = (lo & size) == 0;
            const unsigned long long ua = cand_u[lo], ub = cand_u[hi];
            const int sa = cand_s[lo], sb = cand_s[hi];
            const bool a_gt_b = ua > ub || (ua == ub && sa > sb);
            if (a_gt_b == up) {
              cand_u[lo] = ub;
              cand_u[hi] = ua;
              cand_s[lo] = sb;
              cand_s[hi] = sa;
            }
          }
          __syncthreads();
        }
      }
      admitted = take;
      // Phase 3: install (as in the LDS kernel)
      for (int i = tid; i < admitted; i += LRU_THREADS) {
        const int victim = cand_s[i];
        const int32_t e = miss_ids[i];
        const int32_t old = id_of_slot[victim];
        if (old >= 0 && old < num_total) slot_of_id[old] = -1;
        id_of_slot[victim] = e;
        slot_of_id[e] = victim;
        usage[victim] = step;
        dst_plan[i] = victim;
        src_plan[i] = int32_t(int64_t(e) - id_base);
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < LRU_QPT; ++r) {
    const int i = tid + r * LRU_THREADS;
    if (i >= K) continue;
    int32_t o = si[r];
    if (rank[r] >= 0) o = rank[r] < admitted ? cand_s[rank[r]] : -1;
    out[i] = o;
  }
  if (tid == 0) {
    *num_copy = admitted;
    if (stats) {
      stats[0] += distinct;
      stats[1] += admitted;
      stats[2] += 1;
    }
  }
}

__global__ void slot_cache_reset_kernel(int32_t* __restrict__ slot_of_id, int64_t num_total,
                                        int32_t* __restrict__ id_of_slot,
                                        int64_t* __restrict__ usage, int64_t num_cached,
                                        int64_t* __restrict__ step,
                                        int32_t* __restrict__ active_mask, int num_experts,
                                        int64_t* __restrict__ num_indices) {
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
       i < std::max(num_total, num_cached); i += stride) {
    if (i < num_total) slot_of_id[i] = -1;
    if (i < num_cached) {
      id_of_slot[i] = -1;
      usage[i] = 0;
    }
    if (active_mask && i < num_experts) active_mask[i] = 0;
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    *step = 0;
    if (num_indices) *num_indices = 0;
  }
}

// Place partition `layer` whole into slots [0, E): evict the other partitions' owners of
// those slots, drop this partition's copies elsewhere, and plan the full-layer copy.
__global__ __launch_bounds__(LRU_THREADS) void slot_cache_materialize_kernel(
    int32_t* __restrict__ slot_of_id, int64_t num_total, int32_t* __restrict__ id_of_slot,
    int64_t* __restrict__ usage, int64_t num_cached, int64_t* __restrict__ step_ptr,
    int32_t* __restrict__ evict_slots, int32_t* __restrict__ src_indices,
    int64_t* __restrict__ num_indices, int64_t base, int E) {
  __shared__ int64_t step_lds;
  if (threadIdx.x == 0) {
    const int64_t s = *step_ptr + 1;
    *step_ptr = s;
    step_lds = s;
  }
  // every owner is read before any map entry changes
  for (int64_t s = threadIdx.x; s < num_cached; s += blockDim.x) {
    const int32_t old = id_of_slot[s];
    const bool same = old >= base && old < base + E;
    if (same) {
      id_of_slot[s] = -1;
      usage[s] = 0;
    } else if (s < E && old >= 0 && old < num_total) {
      slot_of_id[old] = -1;
    }
  }
  __syncthreads();
  const int64_t step = step_lds;
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    id_of_slot[e] = int32_t(base + e);
    slot_of_id[base + e] = e;
    usage[e] = step;
    evict_slots[e] = e;
    src_indices[e] = e;
  }
  if (threadIdx.x == 0) *num_indices = E;
}

// Empty slots [begin, end): their owners become non-resident and the slots the oldest.
__global__ void slot_cache_invalidate_kernel(int32_t* __restrict__ slot_of_id, int64_t num_total,
                                             int32_t* __restrict__ id_of_slot,
                                             int64_t* __restrict__ usage, int64_t begin,
                                             int64_t end) {
  const int64_t s = begin + int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (s >= end) return;
  const int32_t old = id_of_slot[s];
  if (old >= 0 && old < num_total) slot_of_id[old] = -1;
  id_of_slot[s] = -1;
  usage[s] = 0;
}

// Experts of one partition resident at or above `threshold`, compacted in expert order:
// dst = buffer row (buffer_base + e), src = their slot; num = count.
__global__ __launch_bounds__(LRU_THREADS) void prefill_hit_compact_kernel(
    const int32_t* __restrict__ slot_row, int32_t* __restrict__ dst, int32_t* __restrict__ src,
    int64_t* __restrict__ num, int64_t buffer_base, int64_t threshold, int E) {
  __shared__ int red[LRU_THREADS / 64 + 1];
  __shared__ int carry_lds;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (tid == 0) carry_lds = 0;
  __syncthreads();
  for (int e0 = 0; e0 < E; e0 += LRU_THREADS) {
    const int e = e0 + tid;
    const int32_t s = e < E ? slot_row[e] : -1;
    const int hit = (e < E && s >= threshold) ? 1 : 0;
    // inclusive scan within the wave, then across the 16 wave totals
    int v = hit;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int t = __shfl_up(v, o, 64);
      if (lane >= o) v += t;
    }
    if (lane == 63) red[wave] = v;
    __syncthreads();
    int before = carry_lds;
    for (int w = 0; w < wave; ++w) before += red[w];
    if (hit) {
      const int pos = before + v - 1;
      dst[pos] = int32_t(buffer_base + e);
      src[pos] = s;
    }
    __syncthreads();
    if (tid == 0) {
      int tot = 0;
      for (int w = 0; w < LRU_THREADS / 64; ++w) tot += red[w];
      carry_lds += tot;
    }
    __syncthreads();
  }
  if (tid == 0) *num = carry_lds;
}

}  // namespace
}  // namespace pia

using namespace pia;

extern "C" int pia_lru_ensure(const int32_t* query, int64_t num_queries, int32_t* slot_of_id,
                              int64_t num_total, int32_t* id_of_slot, int64_t* lru_usage,
                              int64_t num_cached, int64_t* lru_step, int32_t* out_indices,
                              int32_t* src_indices, int32_t* dst_indices, int64_t* num_copy,
                              int64_t* stats, int64_t id_base, void* stream) {
  if (num_queries < 0 || num_total < 0 || num_cached < 0)
    return fail(PIA_EINVAL, "lru_ensure: negative size");
  if (num_cached < 1 || num_cached > LRU_STREAM_MAX_CACHED)
    return fail(PIA_EUNSUPPORTED, "lru_ensure: cache of 1..2^24 slots supported");
  if (num_queries > LRU_MAX_QUERY &&
      (num_queries > LRU_WIDE_MAX_QUERY || num_cached > LRU_MAX_CACHED))
    return fail(PIA_EUNSUPPORTED, "lru_ensure: more than 2048 queries per call need a cache of "
                                  "at most 16384 slots, and at most 2^24 queries");
  if (num_total > 0x7fffffff) return fail(PIA_EINVAL, "lru_ensure: id space beyond int32");
  if (!slot_of_id || !id_of_slot || !lru_usage || !lru_step || !num_copy ||
      (num_queries > 0 && (!query || !out_indices)) || !src_indices || !dst_indices)
    return fail(PIA_EINVAL, "lru_ensure: null pointer");
  if (num_queries > LRU_MAX_QUERY) {
    hipLaunchKernelGGL(lru_ensure_wide_kernel, dim3(1), dim3(LRU_THREADS), 0, as_stream(stream),
                       query, int(num_queries), slot_of_id, num_total, id_of_slot, lru_usage,
                       int(num_cached), lru_step, out_indices, src_indices, dst_indices,
                       num_copy, stats, id_base);
    return check_launch("lru_ensure_wide");
  }
  if (num_cached > LRU_MAX_CACHED) {
    hipLaunchKernelGGL(lru_ensure_stream_kernel, dim3(1), dim3(LRU_THREADS), 0, as_stream(stream),
                       query, int(num_queries), slot_of_id, num_total, id_of_slot, lru_usage,
                       int(num_cached), lru_step, out_indices, src_indices, dst_indices,
                       num_copy, stats, id_base);
    return check_launch("lru_ensure_stream");
  }
  int c_pad = 2, slot_bits = 1;
  while (c_pad < num_cached) {
    c_pad <<= 1;
    ++slot_bits;
  }
  hipLaunchKernelGGL(lru_ensure_kernel, dim3(1), dim3(LRU_THREADS), 0, as_stream(stream), query,
                     int(num_queries), slot_of_id, num_total, id_of_slot, lru_usage,
                     int(num_cached), c_pad, slot_bits, lru_step, out_indices, src_indices,
                     dst_indices, num_copy, stats, id_base);
  return check_launch("lru_ensure");
}

extern "C" int pia_slot_cache_reset(int32_t* slot_of_id, int64_t num_total, int32_t* id_of_slot,
                                    int64_t* usage, int64_t num_cached, int64_t* step,
                                    int32_t* active_mask, int num_experts,
                                    int64_t* num_indices, void* stream) {
  if (num_total < 0 || num_cached < 0 || num_experts < 0)
    return fail(PIA_EINVAL, "slot_cache_reset: negative size");
  if (!slot_of_id || !id_of_slot || !usage || !step)
    return fail(PIA_EINVAL, "slot_cache_reset: null pointer");
  const int64_t n = std::max<int64_t>({num_total, num_cached, int64_t(num_experts), 1});
  const unsigned blocks = unsigned(std::min<int64_t>(ceil_div(n, 256), 1024));
  hipLaunchKernelGGL(slot_cache_reset_kernel, dim3(blocks), dim3(256), 0, as_stream(stream),
                     slot_of_id, num_total, id_of_slot, usage, num_cached, step, active_mask,
                     num_experts, num_indices);
  return check_launch("slot_cache_reset");
}

extern "C" int pia_slot_cache_materialize(int32_t* slot_of_id, int64_t num_total,
                                          int32_t* id_of_slot, int64_t* usage,
                                          int64_t num_cached, int64_t* step,
                                          int32_t* evict_slots, int32_t* src_indices,
                                          int64_t* num_indices, int layer_id, int num_experts,
                                          void* stream) {
  if (layer_id < 0 || num_experts <= 0 || num_cached < num_experts)
    return fail(PIA_EINVAL, "slot_cache_materialize: need 0 <= layer and E <= cache size");
  const int64_t base = int64_t(layer_id) * num_experts;
  if (base + num_experts > num_total)
    return fail(PIA_EINVAL, "slot_cache_materialize: layer outside the id space");
  if (!slot_of_id || !id_of_slot || !usage || !step || !evict_slots || !src_indices ||
      !num_indices)
    return fail(PIA_EINVAL, "slot_cache_materialize: null pointer");
  hipLaunchKernelGGL(slot_cache_materialize_kernel, dim3(1), dim3(LRU_THREADS), 0,
                     as_stream(stream), slot_of_id, num_total, id_of_slot, usage, num_cached,
                     step, evict_slots, src_indices, num_indices, base, num_experts);
  return check_launch("slot_cache_materialize");
}

extern "C" int pia_slot_cache_invalidate(int32_t* slot_of_id, int64_t num_total,
                                         int32_t* id_of_slot, int64_t* usage,
                                         int64_t num_cached, int64_t slot_begin,
                                         int64_t slot_end, void* stream) {
  if (slot_begin < 0 || slot_end < slot_begin || slot_end > num_cached)
    return fail(PIA_EINVAL, "slot_cache_invalidate: slot range outside the cache");
  if (slot_end == slot_begin) return 0;
  if (!slot_of_id || !id_of_slot || !usage)
    return fail(PIA_EINVAL, "slot_cache_invalidate: null pointer");
  hipLaunchKernelGGL(slot_cache_invalidate_kernel, dim3(unsigned(ceil_div(slot_end - slot_begin, 256))),
                     dim3(256), 0, as_stream(stream), slot_of_id, num_total, id_of_slot, usage,
                     slot_begin, slot_end);
  return check_launch("slot_cache_invalidate");
}

extern "C" int pia_prefill_hit_compact(const int32_t* slot_row, int32_t* dst, int32_t* src,
                                       int64_t* num, int64_t buffer_base, int64_t threshold,
                                       int num_experts, void* stream) {
  if (num_experts < 0) return fail(PIA_EINVAL, "prefill_hit_compact: negative size");
  if (!num || (num_experts > 0 && (!slot_row || !dst || !src)))
    return fail(PIA_EINVAL, "prefill_hit_compact: null pointer");
  hipLaunchKernelGGL(prefill_hit_compact_kernel, dim3(1), dim3(LRU_THREADS), 0,
                     as_stream(stream), slot_row, dst, src, num, buffer_base, threshold,
                     num_experts);
  return check_launch("prefill_hit_compact");
}
