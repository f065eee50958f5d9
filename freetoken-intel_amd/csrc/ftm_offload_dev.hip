// ftm_offload_dev.hip -- the slot pool's decode LRU and its copy engine on the GPU.
//
// The host LRU (ftm_offload.cpp) needs the routed expert ids on the host: a
// device -> host copy and a synchronisation per layer per step, then one
// hipMemcpyAsync per bank row.  Here both halves run on the device from the
// routing the top-k kernel left in device memory, so an offload decode step
// is enqueued without waiting for the GPU:
//   * k_lru_ensure (one workgroup): the policy of OffloadMoeCache.ensure_experts
//     (python/freetoken/moe/offload_cache.py:560-647) on device-resident state --
//     step += 1; resident routed experts stamp usage = step; the misses, in
//     ascending expert id, take the global LRU victims argmin (usage, slot) one
//     after another; slot_for_id is rebuilt from id_of_slot (:401-435).
//   * k_copy_slots: every staged (slot, host row) pair of every bank, read from
//     pinned host memory over PCIe by the kernel itself (the plan never leaves
//     the device), in 64 KiB pieces (replaces copy_missing, :651-674).
//
// Sequential argmin without a loop over the misses: a miss stamps its victim
// with the current step, the largest usage, so the misses take the slots not
// stamped in this call (usage < step) in ascending (usage, slot) order; once
// none is left every key is (step, slot) and each further miss takes slot 0.
// The k-th smallest key among the unstamped slots is found by an 8-pass radix
// select over the packed key (usage << 21 | slot) when there are more of them
// than misses, and the selected keys are ranked in LDS.
#include <hip/hip_runtime.h>

#include <stdint.h>

#include "ftmoe.h"
#include "ftm_internal.h"

namespace ftm {

constexpr int kLruThreads = 1024;
constexpr int kLruWaves = kLruThreads / 64;
constexpr int kLruSlotBits = 21;
constexpr int kLruMaxSlots = 1 << kLruSlotBits;  // slot index packed below the usage
static_assert(kMaxExperts <= kLruThreads, "one expert per thread");

struct LruArgs {
  int layer_id, L, E, S;
  const int32_t* ids;
  int n;
  int chunk, cap;
  int32_t* slot_for_id;
  int32_t* id_of_slot;
  int64_t* usage;
  int64_t* step;
  int32_t* evict;
  int32_t* src;
  int32_t* num;
  int32_t* ids_chunk;
  int64_t* stats;
  int32_t* status;
};

__device__ __forceinline__ uint64_t lru_key(int64_t u, int s) {
  return ((uint64_t)u << kLruSlotBits) | (uint64_t)s;
}

// Exclusive prefix of a 0/1 flag over the block in thread order, and the total.
__device__ int flag_scan(bool f, int* s_w, int& total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint64_t m = __ballot(f);
  const int pre = __popcll(m & ((1ull << lane) - 1ull));
  __syncthreads();  // s_w is reused
  if (lane == 0) s_w[wave] = __popcll(m);
  __syncthreads();
  int off = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < kLruWaves; ++w) {
    const int c = s_w[w];
    off += w < wave ? c : 0;
    tot += c;
  }
  total = tot;
  return off + pre;
}

__device__ int block_sum(int v, int* s_w) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) s_w[threadIdx.x >> 6] = v;
  __syncthreads();
  int tot = 0;
#pragma unroll
  for (int w = 0; w < kLruWaves; ++w) tot += s_w[w];
  return tot;
}

// The need-th smallest (1-based) of the packed keys of the slots with usage <
// st (need <= their count; keys are distinct).
__device__ uint64_t radix_select(const int64_t* usage, int S, int64_t st, int need, uint32_t* s_hist,
                                 uint64_t* s_pick, int* s_need) {
  const int tid = threadIdx.x, lane = tid & 63;
  uint64_t prefix = 0, mask = 0;
  for (int shift = 56; shift >= 0; shift -= 8) {
    for (int i = tid; i < 256; i += kLruThreads) s_hist[i] = 0u;
    __syncthreads();
    for (int s = tid; s < S; s += kLruThreads) {
      const int64_t u = usage[s];
      if (u < st) {
        const uint64_t k = lru_key(u, s);
        if ((k & mask) == prefix) atomicAdd(&s_hist[(k >> shift) & 255u], 1u);
      }
    }
    __syncthreads();
    if (tid < 64) {  // wave 0: lane l holds bins 4l .. 4l + 3
      uint32_t c[4];
      uint32_t sum = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        c[j] = s_hist[4 * lane + j];
        sum += c[j];
      }
      uint32_t incl = sum;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t t = __shfl_up(incl, o);
        if (lane >= o) incl += t;
      }
      const uint32_t before = incl - sum;
      const bool here = before < (uint32_t)need && (uint32_t)need <= incl;
      if (here) {
        uint32_t acc = before;
        int d = 4 * lane;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (acc + c[j] >= (uint32_t)need) {
            d = 4 * lane + j;
            break;
          }
          acc += c[j];
        }
        s_pick[0] = prefix | ((uint64_t)d << shift);
        s_need[0] = need - (int)acc;
      }
    }
    __syncthreads();
    prefix = s_pick[0];
    need = s_need[0];
    mask |= 0xffull << shift;
  }
  return prefix;
}

__global__ __launch_bounds__(kLruThreads) void k_lru_ensure(const LruArgs g) {
  __shared__ int32_t s_flag[kMaxExperts];
  __shared__ int32_t s_miss[kMaxExperts];
  __shared__ uint64_t s_key[kMaxExperts];
  __shared__ int32_t s_vict[kMaxExperts];
  __shared__ uint32_t s_hist[256];
  __shared__ int s_w[kLruWaves];
  __shared__ int s_int[4];
  __shared__ uint64_t s_pick[1];
  const int tid = threadIdx.x, E = g.E, S = g.S, base = g.layer_id * E;
  for (int e = tid; e < E; e += kLruThreads) s_flag[e] = 0;
  if (tid == 0) s_int[0] = 0;
  __syncthreads();
  // routed experts (ids < 0: a pair without an expert; >= E: an error)
  for (int i = tid; i < g.n; i += kLruThreads) {
    const int id = g.ids[i];
    if (id >= E) s_int[0] = 1;
    else if (id >= 0) s_flag[id] = 1;
  }
  __syncthreads();
  // this call's experts: ranks [chunk * cap, (chunk + 1) * cap) of the routed ones in ascending id
  const bool routed = tid < E && s_flag[tid] != 0;
  int nuniq;
  const int rank = flag_scan(routed, s_w, nuniq);
  const int r0 = g.chunk * g.cap;
  const bool mine = routed && rank >= r0 && rank - r0 < g.cap;
  __syncthreads();
  if (tid < E) s_flag[tid] = mine ? 1 : 0;
  if (tid == 0 && s_int[0] != 0 && g.status != nullptr) atomicOr(g.status, 1);
  __syncthreads();
  if (g.ids_chunk != nullptr)
    for (int i = tid; i < g.n; i += kLruThreads) {
      const int id = g.ids[i];
      g.ids_chunk[i] = (id >= 0 && id < E && s_flag[id] != 0) ? id : -1;
    }
  if (g.chunk > 0 && nuniq <= r0) {  // a chunk past the last routed expert: no LRU step
    if (tid == 0) *g.num = 0;
    return;
  }
  const int64_t st = g.step[0] + 1;
  // hits stamp their slots; the misses, in ascending expert id
  bool miss = false;
  if (tid < E && s_flag[tid] != 0) {
    const int s = g.slot_for_id[base + tid];
    if (s >= 0 && s < S) {
      g.usage[s] = st;
    } else {
      miss = true;
      if (s != -1 && g.status != nullptr) atomicOr(g.status, 2);  // corrupt map: reloaded as a miss
    }
  }
  int m;
  const int mi = flag_scan(miss, s_w, m);  // its barriers order the stamps before the reads below
  if (miss) s_miss[mi] = tid;
  if (tid == 0) g.step[0] = st;
  int u_loc = 0;
  for (int s = tid; s < S; s += kLruThreads) u_loc += g.usage[s] < st ? 1 : 0;
  const int U = block_sum(u_loc, s_w);
  const int mm = m < U ? m : U;  // misses that take an unstamped slot
  if (mm > 0) {
    const uint64_t tau = U > mm ? radix_select(g.usage, S, st, mm, s_hist, s_pick, &s_int[2]) : ~0ull;
    if (tid == 0) s_int[1] = 0;
    __syncthreads();
    for (int s = tid; s < S; s += kLruThreads) {
      const int64_t u = g.usage[s];
      if (u < st) {
        const uint64_t k = lru_key(u, s);
        if (k <= tau) s_key[atomicAdd(&s_int[1], 1)] = k;
      }
    }
    __syncthreads();
    for (int j = tid; j < mm; j += kLruThreads) {
      const uint64_t k = s_key[j];
      int r = 0;
      for (int q = 0; q < mm; ++q) r += s_key[q] < k ? 1 : 0;
      s_vict[r] = (int)(k & (uint64_t)(kLruMaxSlots - 1));
    }
    __syncthreads();
  }
  // the plan, and the new owners (distinct victims in parallel)
  for (int i = tid; i < m; i += kLruThreads) {
    const int v = i < mm ? s_vict[i] : 0;
    g.evict[i] = v;
    g.src[i] = s_miss[i];
    if (i < mm) {
      g.id_of_slot[v] = base + s_miss[i];
      g.usage[v] = st;
    }
  }
  __syncthreads();
  if (tid == 0) {
    if (m > mm) {  // every slot stamped: the remaining misses pass through slot 0, the last one stays
      g.id_of_slot[0] = base + s_miss[m - 1];
      g.usage[0] = st;
    }
    *g.num = m;
    if (g.stats != nullptr) {
      g.stats[0] += m;
      g.stats[1] += 1;
    }
  }
  __syncthreads();
  // slot_for_id rebuilt from id_of_slot (another layer's entry may have been evicted)
  const int nid = g.L * E;
  for (int i = tid; i < nid; i += kLruThreads) g.slot_for_id[i] = -1;
  __syncthreads();
  for (int s = tid; s < S; s += kLruThreads) {
    const int id = g.id_of_slot[s];
    if (id >= 0 && id < nid) g.slot_for_id[id] = s;
  }
}

constexpr int kCopyMaxBanks = 8;
constexpr int64_t kCopyPiece = 64 * 1024;  // bytes per workgroup
constexpr int kCopyThreads = 256;

struct CopyBank {
  const char* host;
  char* dev;
  int64_t row_bytes;
  int32_t pieces;
};
struct CopyArgs {
  CopyBank b[kCopyMaxBanks];
  int nb, per_row, max_rows, host_rows, pool_slots;
  const int32_t* evict;
  const int32_t* src;
  const int32_t* num;
};

// Workgroup (row i, piece c): piece c of row i's banks in bank order.  The
// plan is applied as copy_missing applies it, in order: a row whose slot a
// later row of the plan also takes is skipped, so the last one lands (when
// every slot is stamped, ensure_experts passes the remaining misses through
// slot 0 and only the last stays).
__global__ __launch_bounds__(kCopyThreads) void k_copy_slots(const CopyArgs g) {
  const int i = (int)blockIdx.x / g.per_row;
  int c = (int)blockIdx.x % g.per_row;
  const int n = min(g.num[0], g.max_rows);
  if (i >= n) return;
  const int row = g.src[i], slot = g.evict[i];
  if (row < 0 || row >= g.host_rows || slot < 0 || slot >= g.pool_slots) return;  // never outside the banks
  bool later = false;
  for (int j = i + 1 + (int)threadIdx.x; j < n; j += kCopyThreads) later = later || g.evict[j] == slot;
  if (__syncthreads_or(later)) return;
  int b = 0;
  while (b + 1 < g.nb && c >= g.b[b].pieces) c -= g.b[b++].pieces;
  const CopyBank B = g.b[b];
  const int64_t off = (int64_t)c * kCopyPiece;
  const int64_t rem = B.row_bytes - off;
  const int64_t len = rem < kCopyPiece ? rem : kCopyPiece;
  const char* src = B.host + (int64_t)row * B.row_bytes + off;
  char* dst = B.dev + (int64_t)slot * B.row_bytes + off;
  if ((((uintptr_t)src | (uintptr_t)dst | (uintptr_t)len) & 15u) == 0) {
    const int64_t nv = len / 16;
    const uint4* s4 = (const uint4*)src;
    uint4* d4 = (uint4*)dst;
    int64_t j = threadIdx.x;
    // four 16-byte reads in flight per lane before the writes
    for (; j + 3 * kCopyThreads < nv; j += 4 * kCopyThreads) {
      const uint4 a0 = s4[j], a1 = s4[j + kCopyThreads], a2 = s4[j + 2 * kCopyThreads], a3 = s4[j + 3 * kCopyThreads];
      d4[j] = a0;
      d4[j + kCopyThreads] = a1;
      d4[j + 2 * kCopyThreads] = a2;
      d4[j + 3 * kCopyThreads] = a3;
    }
    for (; j < nv; j += kCopyThreads) d4[j] = s4[j];
  } else {
    for (int64_t j = threadIdx.x; j < len; j += kCopyThreads) dst[j] = src[j];
  }
}

}  // namespace ftm

using namespace ftm;

extern "C" {

int ftm_lru_ensure_dev(int32_t layer_id, int32_t num_layers, int32_t num_experts, int32_t cache_size,
                       const int32_t* expert_ids, int32_t n, int32_t chunk, int32_t chunk_cap,
                       int32_t* slot_for_id, int32_t* id_of_slot, int64_t* usage, int64_t* step,
                       int32_t* evict_slots, int32_t* src_rows, int32_t* num_staged, int32_t* ids_chunk,
                       int64_t* stats, int32_t* status, void* stream) {
  if (num_layers <= 0 || num_experts <= 0 || num_experts > kMaxExperts || cache_size < 1 ||
      cache_size > kLruMaxSlots || layer_id < 0 || layer_id >= num_layers || n < 0 || chunk < 0 ||
      chunk_cap < 1)
    return FTM_ERR_DIM;
  if ((int64_t)num_layers * num_experts > INT32_MAX) return FTM_ERR_DIM;
  if (slot_for_id == nullptr || id_of_slot == nullptr || usage == nullptr || step == nullptr ||
      evict_slots == nullptr || src_rows == nullptr || num_staged == nullptr || (n > 0 && expert_ids == nullptr))
    return FTM_ERR_NULL;
  LruArgs g;
  g.layer_id = layer_id;
  g.L = num_layers;
  g.E = num_experts;
  g.S = cache_size;
  g.ids = expert_ids;
  g.n = n;
  g.chunk = chunk;
  g.cap = chunk_cap;
  g.slot_for_id = slot_for_id;
  g.id_of_slot = id_of_slot;
  g.usage = usage;
  g.step = step;
  g.evict = evict_slots;
  g.src = src_rows;
  g.num = num_staged;
  g.ids_chunk = ids_chunk;
  g.stats = stats;
  g.status = status;
  hipLaunchKernelGGL(k_lru_ensure, dim3(1), dim3(kLruThreads), 0, (hipStream_t)stream, g);
  return hipGetLastError() == hipSuccess ? FTM_OK : FTM_ERR_HIP;
}

int ftm_copy_slots_dev(const ftm_bank_copy* banks, int32_t num_banks, int32_t host_rows, int32_t pool_slots,
                       const int32_t* evict_slots, const int32_t* src_rows, const int32_t* num_staged,
                       int32_t max_rows, void* stream) {
  if (num_banks < 1 || num_banks > kCopyMaxBanks || max_rows < 0 || host_rows < 1 || pool_slots < 1)
    return FTM_ERR_DIM;
  if (banks == nullptr || evict_slots == nullptr || src_rows == nullptr || num_staged == nullptr)
    return FTM_ERR_NULL;
  CopyArgs g;
  int64_t per_row = 0;
  for (int b = 0; b < num_banks; ++b) {
    const ftm_bank_copy& B = banks[b];
    if (B.row_bytes <= 0) return FTM_ERR_DIM;
    if (B.host_bank == nullptr || B.dev_pool == nullptr) return FTM_ERR_NULL;
    g.b[b].pieces = (int32_t)((B.row_bytes + kCopyPiece - 1) / kCopyPiece);
    g.b[b].row_bytes = B.row_bytes;
    g.b[b].dev = (char*)B.dev_pool;
    per_row += g.b[b].pieces;
  }
  if (per_row * (int64_t)max_rows > INT32_MAX) return FTM_ERR_DIM;
  if (max_rows == 0) return FTM_OK;
  // the kernel reads the host banks itself: they must be pinned host memory
  // (page-locked, mapped for the device); anything else -- pageable or device
  // memory -- is refused here, not faulted on.  (hipHostGetDevicePointer is no
  // such check: it accepts a device pointer.)
  for (int b = 0; b < num_banks; ++b) {
    const char* h = (const char*)banks[b].host_bank;
    hipPointerAttribute_t at;
    if (hipPointerGetAttributes(&at, h) != hipSuccess || at.type != hipMemoryTypeHost ||
        at.devicePointer == nullptr || at.hostPointer == nullptr || h < (const char*)at.hostPointer) {
      (void)hipGetLastError();
      return FTM_ERR_HIP;
    }
    g.b[b].host = (const char*)at.devicePointer + (h - (const char*)at.hostPointer);  // this row of the allocation
  }
  g.nb = num_banks;
  g.per_row = (int)per_row;
  g.max_rows = max_rows;
  g.host_rows = host_rows;
  g.pool_slots = pool_slots;
  g.evict = evict_slots;
  g.src = src_rows;
  g.num = num_staged;
  hipLaunchKernelGGL(k_copy_slots, dim3((unsigned)(per_row * max_rows)), dim3(kCopyThreads), 0, (hipStream_t)stream,
                     g);
  return hipGetLastError() == hipSuccess ? FTM_OK : FTM_ERR_HIP;
}

}  // extern "C"
