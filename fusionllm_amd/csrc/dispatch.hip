// dispatch.hip — expert histogram, exclusive scan, stable counting-sort
// scatter and row gather.
//
// Replaces the permutation half of DeepSeekMoE._dispatch_scatter_gather,
// FusionLLM models/moe.py:55-64 (flatten, argsort, unique_consecutive,
// cumsum) and the per-expert gathers x[token_ids] (moe.py:73,75).  The
// reference sorts with torch.argsort (moe.py:58); this is a counting sort
// whose order is expert-major and slot-ascending inside each expert, the
// order of a stable argsort.  Nothing is copied to the host: the counts and
// offsets stay in device memory for the grouped GEMMs.
//
// Slots are processed in blocks of kSlotsPerBlock.  Stage 1 counts each
// block's slots per expert; stage 2 (one workgroup) turns the block counts
// into each block's first row per expert; stage 3 ranks each slot among the
// earlier slots of its block with the same expert (wave ballots, then an
// exclusive prefix over the waves of the block) and writes perm /
// pos_of_slot.  Stage 4 copies rows of x into the expert-contiguous buffer
// with 16-byte loads and stores, many rows per workgroup.
#include <atomic>
#include <mutex>

#include "fmoe_common.h"

namespace fmoe {

constexpr int kDispThreads = 256;
constexpr int kDispWaves = kDispThreads / 64;
constexpr int kSlotsPerThread = 1;  // small blocks: 128 of them at T*k = 32768
constexpr int kSlotsPerBlock = kDispThreads * kSlotsPerThread;

__global__ __launch_bounds__(kDispThreads) void dispatch_hist_kernel(
    const int32_t* __restrict__ idx, int n_slots, int E, int32_t* __restrict__ block_hist) {
  __shared__ int cnt[FMOE_MAX_EXPERTS];
  for (int e = threadIdx.x; e < E; e += blockDim.x) cnt[e] = 0;
  __syncthreads();
  const int base = blockIdx.x * kSlotsPerBlock;
#pragma unroll
  for (int i = 0; i < kSlotsPerThread; ++i) {
    const int s = base + i * kDispThreads + threadIdx.x;
    if (s < n_slots) {
      const int e = idx[s];
      if (static_cast<unsigned>(e) < static_cast<unsigned>(E)) atomicAdd(&cnt[e], 1);
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += blockDim.x)
    block_hist[static_cast<int64_t>(blockIdx.x) * E + e] = cnt[e];
}

// One workgroup of 16 waves.  block_base[b][e] = offsets[e] + sum_{b' < b}
// block_hist[b'][e].  Wave-row path (E divides 64): lane l takes expert
// l % E of the block rows l / E, l / E + 64 / E, ... of a contiguous range of
// blocks per wave, consecutive lanes reading consecutive counts, kScanBatch
// loads in flight at a time; the waves' per-expert sums meet in LDS, wave 0
// forms the totals and offsets (one 64-lane scan), and each wave then reads
// its blocks again (from L2) and walks them in order with shuffles across the
// lanes of an expert.  Otherwise: pass 1 adds each expert's block counts
// (wave reduction), pass 2 writes the per-block bases with a 64-lane
// inclusive scan (shfl_up) per chunk of 64 blocks, carried across chunks.
// Integer sums, so the order does not change the result.
constexpr int kScanThreads = 1024;
constexpr int kScanWaves = kScanThreads / 64;
constexpr int kScanBatch = 16;  // loads per lane in flight on the wave-row path

// The expert counts also go to counts_host (nullable): host memory that the
// caller reads once the stream has passed this kernel, written with
// system-scope stores (through to memory, visible to the host).
__device__ __forceinline__ void store_host(int32_t* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

__global__ __launch_bounds__(kScanThreads) void dispatch_scan_kernel(
    const int32_t* __restrict__ block_hist, int nblocks, int E, int32_t* __restrict__ block_base,
    int32_t* __restrict__ counts, int32_t* __restrict__ offsets, int32_t* __restrict__ counts_host) {
  __shared__ int total[FMOE_MAX_EXPERTS];
  __shared__ int start[FMOE_MAX_EXPERTS + 1];
  __shared__ int wsum[kScanWaves][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int per = (E > 0 && 64 % E == 0) ? 64 / E : 0;  // block rows per load instruction
  if (per) {  // uniform over the workgroup
    const int bw = ((nblocks + kScanWaves - 1) / kScanWaves + per - 1) / per * per;  // blocks per wave
    const int its = bw / per;
    const int e = lane % E, sub = lane / E;
    const int b0 = wave * bw;
    int loc = 0;
    for (int i0 = 0; i0 < its; i0 += kScanBatch) {
      int hv[kScanBatch];
#pragma unroll
      for (int u = 0; u < kScanBatch; ++u) {
        const int b = b0 + (i0 + u) * per + sub;
        hv[u] = (i0 + u < its && b < nblocks) ? block_hist[static_cast<int64_t>(b) * E + e] : 0;
      }
#pragma unroll
      for (int u = 0; u < kScanBatch; ++u) loc += hv[u];
    }
    int tot = loc;  // over the lanes of expert e: xor offsets E, 2E, ..., 32
    for (int off = E; off < 64; off <<= 1) tot += __shfl_xor(tot, off, 64);
    if (sub == 0) wsum[wave][e] = tot;
    __syncthreads();
    if (wave == 0) {
      int t = 0;
      if (lane < E)
        for (int w = 0; w < kScanWaves; ++w) t += wsum[w][lane];
      const int incl = wave_incl_scan(t, lane);
      if (lane < E) {
        total[lane] = t;
        start[lane] = incl - t;
        counts[lane] = t;
        offsets[lane] = incl - t;
        if (counts_host) store_host(counts_host + lane, t);
      }
      if (lane == 63) {
        start[E] = incl;
        offsets[E] = incl;
      }
    }
    __syncthreads();
    int base = start[e];
    for (int w = 0; w < wave; ++w) base += wsum[w][e];
    for (int i0 = 0; i0 < its; i0 += kScanBatch) {
      int hv[kScanBatch];
#pragma unroll
      for (int u = 0; u < kScanBatch; ++u) {
        const int b = b0 + (i0 + u) * per + sub;
        hv[u] = (i0 + u < its && b < nblocks) ? block_hist[static_cast<int64_t>(b) * E + e] : 0;
      }
#pragma unroll
      for (int u = 0; u < kScanBatch; ++u) {
        if (i0 + u < its) {  // uniform
          int incl = hv[u];  // inclusive over sub (lanes e, e + E, ...)
          for (int off = 1; off < per; off <<= 1) {
            const int v = __shfl_up(incl, off * E, 64);
            if (sub >= off) incl += v;
          }
          const int b = b0 + (i0 + u) * per + sub;
          if (b < nblocks) block_base[static_cast<int64_t>(b) * E + e] = base + incl - hv[u];
          base += __shfl(incl, (per - 1) * E + e, 64);  // the row's count for expert e
        }
      }
    }
    return;
  }
  constexpr int nwaves = kScanWaves;
  for (int e = wave; e < E; e += nwaves) {
    int sum = 0;
    for (int b = lane; b < nblocks; b += 64) sum += block_hist[static_cast<int64_t>(b) * E + e];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off, 64);
    if (lane == 0) total[e] = sum;
  }
  __syncthreads();
  if (threadIdx.x < 64) {
    const int lane0 = threadIdx.x;
    const int t = lane0 < E ? total[lane0] : 0;
    const int incl = wave_incl_scan(t, lane0);
    if (lane0 < E) start[lane0] = incl - t;
    if (lane0 == 63) start[E] = incl;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += kScanThreads) {
    counts[e] = total[e];
    offsets[e] = start[e];
    if (counts_host) store_host(counts_host + e, total[e]);
  }
  if (threadIdx.x == 0) offsets[E] = start[E];
  for (int e = wave; e < E; e += nwaves) {
    int carry = start[e];
    for (int b0 = 0; b0 < nblocks; b0 += 64) {
      const int b = b0 + lane;
      const int64_t o = static_cast<int64_t>(b) * E + e;
      const int h = b < nblocks ? block_hist[o] : 0;
      const int incl = wave_incl_scan(h, lane);
      if (b < nblocks) block_base[o] = carry + incl - h;
      carry += __shfl(incl, 63, 64);
    }
  }
}

__global__ __launch_bounds__(kDispThreads) void dispatch_scatter_kernel(
    const int32_t* __restrict__ idx, int n_slots, int E, const int32_t* __restrict__ block_base,
    int32_t* __restrict__ perm, int32_t* __restrict__ pos_of_slot) {
  __shared__ int running[FMOE_MAX_EXPERTS];
  __shared__ int wcount[kDispWaves][FMOE_MAX_EXPERTS];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  for (int e = threadIdx.x; e < E; e += blockDim.x)
    running[e] = block_base[static_cast<int64_t>(blockIdx.x) * E + e];
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int round = 0; round < kSlotsPerThread; ++round) {
    for (int i = threadIdx.x; i < kDispWaves * E; i += blockDim.x) wcount[i / E][i % E] = 0;
    __syncthreads();
    const int s = blockIdx.x * kSlotsPerBlock + round * kDispThreads + threadIdx.x;
    const int e_raw = s < n_slots ? idx[s] : -1;
    const bool valid = static_cast<unsigned>(e_raw) < static_cast<unsigned>(E);
    const int e = valid ? e_raw : -1;
    // Rank among lanes of this wave with the same expert (lower lanes first).
    uint64_t pending = __ballot(valid);
    int rank = 0;
    while (pending) {
      const int leader = __ffsll(static_cast<unsigned long long>(pending)) - 1;
      const int le = __shfl(e, leader);
      const uint64_t m = __ballot(e == le);
      if (e == le) rank = __popcll(m & lt_mask);
      if (lane == leader) wcount[wave][le] = __popcll(m);
      pending &= ~m;
    }
    __syncthreads();
    if (valid) {
      int pos = running[e] + rank;
      for (int w = 0; w < wave; ++w) pos += wcount[w][e];
      if (pos >= 0 && pos < n_slots) {  // always true for expert ids in range
        perm[pos] = s;
        pos_of_slot[s] = pos;
      }
    }
    __syncthreads();
    for (int q = threadIdx.x; q < E; q += blockDim.x) {
      int add = 0;
      for (int w = 0; w < kDispWaves; ++w) add += wcount[w][q];
      running[q] += add;
    }
    __syncthreads();
  }
}

// fmoe_route_and_dispatch's scatter: workgroup (b, y) takes the slots of the
// router's workgroup b (kRouteBlockTokens tokens, spb = kRouteBlockTokens * k
// <= 256 slots, one per thread) and ranks them exactly as
// dispatch_scatter_kernel does (ballots within a wave, then the counts of the
// earlier waves); y == 0 writes perm and pos_of_slot.  Every y then copies its
// share of the block's token rows: the block's tokens * chunks 16-byte chunks
// cut into ranges of kCopyPerWG, range y for workgroup y, one chunk per
// thread, each chunk of x read once and stored to the k rows of x_perm its
// token's slots go to.  Re-ranking in every y costs a few ballots; it buys
// enough workgroups to keep the copy's loads in flight.
constexpr int kCopyPerWG = kDispThreads;

__global__ __launch_bounds__(kDispThreads) void dispatch_scatter_copy_kernel(
    const int32_t* __restrict__ idx, int n_slots, int spb, int E, int k, const int32_t* __restrict__ block_base,
    const uint4* __restrict__ x, int chunks, int32_t* __restrict__ perm, int32_t* __restrict__ pos_of_slot,
    uint4* __restrict__ x_perm) {
  __shared__ int wcount[kDispWaves][FMOE_MAX_EXPERTS];
  __shared__ int base_sh[FMOE_MAX_EXPERTS];
  __shared__ int pos_sh[kDispThreads];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int s0 = blockIdx.x * spb;
  const int s = s0 + threadIdx.x;
  const bool mine = threadIdx.x < spb && s < n_slots;
  // the slot's expert and the block's bases are loaded side by side
  const int e_raw = mine ? idx[s] : -1;
  const int bb = threadIdx.x < E ? block_base[static_cast<int64_t>(blockIdx.x) * E + threadIdx.x] : 0;
  for (int i = threadIdx.x; i < kDispWaves * E; i += blockDim.x) wcount[i / E][i % E] = 0;
  if (threadIdx.x < E) base_sh[threadIdx.x] = bb;
  __syncthreads();
  const bool valid = static_cast<unsigned>(e_raw) < static_cast<unsigned>(E);
  const int e = valid ? e_raw : -1;
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  uint64_t pending = __ballot(valid);
  int rank = 0;
  while (pending) {
    const int leader = __ffsll(static_cast<unsigned long long>(pending)) - 1;
    const int le = __shfl(e, leader);
    const uint64_t m = __ballot(e == le);
    if (e == le) rank = __popcll(m & lt_mask);
    if (lane == leader) wcount[wave][le] = __popcll(m);
    pending &= ~m;
  }
  __syncthreads();
  int pos = -1;
  if (valid) {
    pos = base_sh[e] + rank;
    for (int w = 0; w < wave; ++w) pos += wcount[w][e];
    if (pos < 0 || pos >= n_slots) pos = -1;  // never, for expert ids in range
    if (pos >= 0 && blockIdx.y == 0) {
      perm[pos] = s;
      pos_of_slot[s] = pos;
    }
  }
  if (x_perm == nullptr) return;
  if (threadIdx.x < spb) pos_sh[threadIdx.x] = pos;
  __syncthreads();
  const int t0 = s0 / k;                       // the block's first token (spb is a multiple of k)
  const int ntok = min(spb, n_slots - s0) / k;  // n_slots = T * k: whole tokens
  const int g = blockIdx.y * kCopyPerWG + threadIdx.x;
  if (g < ntok * chunks) {
    const int i = g / chunks, c = g - i * chunks;
    const uint4 v = x[static_cast<int64_t>(t0 + i) * chunks + c];
    for (int j = 0; j < k; ++j) {
      const int p = pos_sh[i * k + j];
      if (p >= 0) x_perm[static_cast<int64_t>(p) * chunks + c] = v;
    }
  }
}

// x_perm[r] = x[perm[r] / k]: one 16-byte chunk per thread.
__global__ __launch_bounds__(256) void dispatch_gather_kernel(
    const int32_t* __restrict__ perm, const uint4* __restrict__ x, int64_t n_rows, int chunks,
    int k, uint4* __restrict__ x_perm) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (g >= n_rows * chunks) return;
  const int64_t r = g / chunks;
  const int c = static_cast<int>(g - r * chunks);
  const int64_t slot = perm[r];
  if (slot < 0 || slot >= n_rows) return;  // perm holds slots 0 .. n_rows-1
  x_perm[g] = x[(slot / k) * chunks + c];
}

// Decode-sized batches (n_slots <= kSmallSlots, dim <= 2048): the four stages
// in one launch.  Every workgroup ranks all the slots (one per thread, the
// ballot ranking of dispatch_scatter_kernel over the block's waves) and so
// knows the whole permutation; workgroup 0 writes counts, offsets, perm and
// pos_of_slot, and workgroup b copies rows kSmallRowsPerBlock * b .. + that
// many of x_perm.  Same counting sort, same output.
constexpr int kSmallSlots = kDispThreads;
constexpr int kSmallRowsPerBlock = 8;
constexpr int kSmallCopies = 8;  // 16-byte copies per thread, all loads issued first (dim <= 2048)

__global__ __launch_bounds__(kDispThreads) void dispatch_small_kernel(
    const int32_t* __restrict__ idx, int n_slots, int E, int k, const uint4* __restrict__ x, int chunks,
    int32_t* __restrict__ counts, int32_t* __restrict__ offsets, int32_t* __restrict__ perm,
    int32_t* __restrict__ pos_of_slot, uint4* __restrict__ x_perm) {
  __shared__ int wcount[kDispWaves][FMOE_MAX_EXPERTS];
  __shared__ int start[FMOE_MAX_EXPERTS + 1];
  __shared__ int perm_sh[kSmallSlots];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const bool first = blockIdx.x == 0;
  for (int i = threadIdx.x; i < kDispWaves * E; i += blockDim.x) wcount[i / E][i % E] = 0;
  __syncthreads();
  const int s = threadIdx.x;
  const int e_raw = s < n_slots ? idx[s] : -1;
  const bool valid = static_cast<unsigned>(e_raw) < static_cast<unsigned>(E);
  const int e = valid ? e_raw : -1;
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  uint64_t pending = __ballot(valid);
  int rank = 0;
  while (pending) {
    const int leader = __ffsll(static_cast<unsigned long long>(pending)) - 1;
    const int le = __shfl(e, leader);
    const uint64_t m = __ballot(e == le);
    if (e == le) rank = __popcll(m & lt_mask);
    if (lane == leader) wcount[wave][le] = __popcll(m);
    pending &= ~m;
  }
  __syncthreads();
  scan_wave_counts<kDispWaves>(wcount, E, start);
  __syncthreads();
  if (valid) {
    int pos = start[e] + rank;
    for (int w = 0; w < wave; ++w) pos += wcount[w][e];
    perm_sh[pos] = s;
    if (first) {
      perm[pos] = s;
      pos_of_slot[s] = pos;
    }
  }
  if (first) {
    for (int q = threadIdx.x; q < E; q += blockDim.x) {
      counts[q] = start[q + 1] - start[q];
      offsets[q] = start[q];
    }
    if (threadIdx.x == 0) offsets[E] = start[E];
  }
  if (x_perm == nullptr) return;
  __syncthreads();
  const int r0 = blockIdx.x * kSmallRowsPerBlock;
  const int r1 = min(r0 + kSmallRowsPerBlock, start[E]);  // rows that hold a slot
  const int g0 = r0 * chunks + threadIdx.x, g1 = r1 * chunks;
  uint4 v[kSmallCopies];
#pragma unroll
  for (int u = 0; u < kSmallCopies; ++u) {
    const int g = g0 + u * kDispThreads;
    if (g < g1) {
      const int r = g / chunks, c = g - r * chunks;
      v[u] = x[static_cast<int64_t>(perm_sh[r] / k) * chunks + c];
    }
  }
#pragma unroll
  for (int u = 0; u < kSmallCopies; ++u) {
    const int g = g0 + u * kDispThreads;
    if (g < g1) x_perm[g] = v[u];
  }
}

}  // namespace fmoe

using namespace fmoe;

extern "C" size_t fmoe_dispatch_workspace_bytes(int64_t T, int n_experts, int k) {
  if (T <= 0 || n_experts <= 0 || k <= 0) return 0;
  const int64_t nblocks = ceil_div(T * k, kSlotsPerBlock);
  return static_cast<size_t>(2 * nblocks * n_experts) * sizeof(int32_t);
}

namespace {

// ---- allocation-free variant -----------------------------------------------
// The scratch of fmoe_dispatch_noalloc (per-block expert counts and bases)
// lives in this file-scope device array, one copy per GPU for the life of the
// process.  Host code never passes `scratch` itself to a kernel: on the host
// it names a stand-in, not the device address.  Each device's address comes
// from hipGetSymbolAddress, called once per device with that device current,
// and is kept in scratch_dev[].
constexpr size_t kNoAllocScratchBytes = size_t(1) << 20;
static __device__ __align__(256) int32_t scratch[kNoAllocScratchBytes / sizeof(int32_t)];
constexpr int kMaxDevices = 64;
std::atomic<int32_t*> scratch_dev[kMaxDevices];
std::mutex scratch_mu;

// This device's copy of `scratch` (resolved on the first call on the device).
int device_scratch(int32_t** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return FMOE_ERR_LAUNCH;
  int32_t* p = scratch_dev[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(scratch_mu);
    p = scratch_dev[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      void* addr = nullptr;
      if (hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch)) != hipSuccess || addr == nullptr)
        return FMOE_ERR_LAUNCH;
      p = static_cast<int32_t*>(addr);
      scratch_dev[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return FMOE_OK;
}

}  // namespace

extern "C" int fmoe_dispatch(const int32_t* idx, const void* x, int64_t T, int64_t dim,
                             int n_experts, int k, int32_t* counts, int32_t* offsets,
                             int32_t* perm, int32_t* pos_of_slot, void* x_perm, void* workspace,
                             size_t workspace_bytes, void* stream) {
  if (T < 0 || dim <= 0) return FMOE_ERR_INVALID_ARG;
  if (n_experts <= 0 || n_experts > FMOE_MAX_EXPERTS) return FMOE_ERR_TOO_MANY_EXPERTS;
  if (k <= 0 || k > FMOE_MAX_TOPK || k > n_experts || dim % 64 != 0) return FMOE_ERR_SHAPE;
  if (!counts || !offsets) return FMOE_ERR_INVALID_ARG;
  const int64_t n_slots = T * k;
  if (n_slots > INT32_MAX / 2) return FMOE_ERR_SHAPE;
  hipStream_t s = as_stream(stream);
  const int64_t nblocks = ceil_div(n_slots, kSlotsPerBlock);
  if (T == 0) {
    // Empty batch: every count and offset is zero (scan over zero blocks).
    dispatch_scan_kernel<<<1, kScanThreads, 0, s>>>(nullptr, 0, n_experts, nullptr, counts, offsets, nullptr);
    return launch_status();
  }
  if (!idx || !x || !perm || !pos_of_slot || !workspace) return FMOE_ERR_INVALID_ARG;
  if (workspace_bytes < fmoe_dispatch_workspace_bytes(T, n_experts, k)) return FMOE_ERR_WORKSPACE;
  if (!aligned16(x) || (x_perm && !aligned16(x_perm))) return FMOE_ERR_ALIGN;
  if (n_slots <= kSmallSlots && kSmallRowsPerBlock * (dim / 8) <= kSmallCopies * kDispThreads) {
    const int chunks = static_cast<int>(dim / 8);
    const int64_t blocks = x_perm ? ceil_div(n_slots, kSmallRowsPerBlock) : 1;
    dispatch_small_kernel<<<dim3(blocks), dim3(kDispThreads), 0, s>>>(
        idx, (int)n_slots, n_experts, k, static_cast<const uint4*>(x), chunks, counts, offsets, perm,
        pos_of_slot, static_cast<uint4*>(x_perm));
    return launch_status();
  }
  int32_t* block_hist = static_cast<int32_t*>(workspace);
  int32_t* block_base = block_hist + nblocks * n_experts;
  dispatch_hist_kernel<<<dim3(nblocks), dim3(kDispThreads), 0, s>>>(idx, (int)n_slots, n_experts,
                                                                   block_hist);
  dispatch_scan_kernel<<<1, kScanThreads, 0, s>>>(block_hist, (int)nblocks, n_experts, block_base,
                                                  counts, offsets, nullptr);
  dispatch_scatter_kernel<<<dim3(nblocks), dim3(kDispThreads), 0, s>>>(
      idx, (int)n_slots, n_experts, block_base, perm, pos_of_slot);
  if (x_perm) {
    const int chunks = static_cast<int>(dim / 8);
    const int64_t total = n_slots * chunks;
    dispatch_gather_kernel<<<dim3(ceil_div(total, 256)), dim3(256), 0, s>>>(
        perm, static_cast<const uint4*>(x), n_slots, chunks, k, static_cast<uint4*>(x_perm));
  }
  return launch_status();
}

extern "C" int fmoe_dispatch_noalloc(const int32_t* idx, const void* x, int64_t T, int64_t dim,
                                     int n_experts, int k, int32_t* counts, int32_t* offsets,
                                     int32_t* perm, int32_t* pos_of_slot, void* x_perm, void* stream) {
  if (T < 0 || dim <= 0) return FMOE_ERR_INVALID_ARG;
  if (n_experts <= 0 || n_experts > FMOE_MAX_EXPERTS) return FMOE_ERR_TOO_MANY_EXPERTS;
  if (k <= 0 || k > FMOE_MAX_TOPK || k > n_experts || dim % 64 != 0) return FMOE_ERR_SHAPE;
  if (T * k > INT32_MAX / 2) return FMOE_ERR_SHAPE;
  const size_t need = fmoe_dispatch_workspace_bytes(T, n_experts, k);
  if (need > kNoAllocScratchBytes) return FMOE_ERR_SCRATCH;
  int32_t* ws = nullptr;
  const int rc = device_scratch(&ws);
  if (rc != FMOE_OK) return rc;
  return fmoe_dispatch(idx, x, T, dim, n_experts, k, counts, offsets, perm, pos_of_slot, x_perm, ws,
                       kNoAllocScratchBytes, stream);
}

extern "C" size_t fmoe_route_and_dispatch_workspace_bytes(int64_t T, int n_experts, int k) {
  if (T <= 0 || n_experts <= 0 || k <= 0) return 0;
  const int64_t nblocks = ceil_div(T, kRouteBlockTokens);
  return static_cast<size_t>(2 * nblocks * n_experts) * sizeof(int32_t);  // block counts, block bases
}

extern "C" int fmoe_route_and_dispatch(const void* x, const void* gate_w, const void* gate_b, int64_t T,
                                       int64_t dim, int n_experts, int k, float route_scale, int32_t* idx,
                                       int64_t* idx64, float* weights, float* topv, int32_t* counts,
                                       int32_t* offsets, int32_t* perm, int32_t* pos_of_slot, void* x_perm,
                                       int32_t* counts_host, void* workspace, size_t workspace_bytes,
                                       void* stream) {
  if (T < 0 || dim <= 0) return FMOE_ERR_INVALID_ARG;
  if (n_experts <= 0 || n_experts > FMOE_MAX_EXPERTS) return FMOE_ERR_TOO_MANY_EXPERTS;
  if (k <= 0 || k > FMOE_MAX_TOPK || k > n_experts || dim % 64 != 0 || dim > 2048) return FMOE_ERR_SHAPE;
  if (T * k > INT32_MAX / 2) return FMOE_ERR_SHAPE;
  if (!counts || !offsets) return FMOE_ERR_INVALID_ARG;
  hipStream_t s = as_stream(stream);
  if (T == 0) {
    // no tokens: empty experts (the scan over zero blocks writes counts 0, offsets 0)
    dispatch_scan_kernel<<<1, kScanThreads, 0, s>>>(nullptr, 0, n_experts, nullptr, counts, offsets, counts_host);
    return launch_status();
  }
  if (!x || !gate_w || !gate_b || !idx || !weights || !topv || !perm || !pos_of_slot) return FMOE_ERR_INVALID_ARG;
  if (!aligned16(x) || !aligned16(gate_w) || (x_perm && !aligned16(x_perm))) return FMOE_ERR_ALIGN;
  if (workspace_bytes < fmoe_route_and_dispatch_workspace_bytes(T, n_experts, k)) return FMOE_ERR_WORKSPACE;
  if (!workspace) return FMOE_ERR_INVALID_ARG;
  const int64_t nblocks = ceil_div(T, kRouteBlockTokens);
  int32_t* block_hist = static_cast<int32_t*>(workspace);
  int32_t* block_base = block_hist + nblocks * n_experts;
  int st = launch_router_hist(static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(gate_w),
                              static_cast<const uint16_t*>(gate_b), T, dim, n_experts, k, route_scale, idx, idx64,
                              weights, topv, block_hist, s);
  if (st) return st;
  const int64_t nsplit = x_perm ? ceil_div(static_cast<int64_t>(kRouteBlockTokens) * (dim / 8), kCopyPerWG) : 1;
  const dim3 grid(static_cast<unsigned>(nblocks), static_cast<unsigned>(nsplit));
  const int n_slots = static_cast<int>(T * k), spb = kRouteBlockTokens * k, chunks = static_cast<int>(dim / 8);
  const uint4* xs = static_cast<const uint4*>(x);
  uint4* xp = static_cast<uint4*>(x_perm);
  dispatch_scan_kernel<<<1, kScanThreads, 0, s>>>(block_hist, static_cast<int>(nblocks), n_experts, block_base,
                                                   counts, offsets, counts_host);
  dispatch_scatter_copy_kernel<<<grid, dim3(kDispThreads), 0, s>>>(idx, n_slots, spb, n_experts, k, block_base, xs,
                                                                 chunks, perm, pos_of_slot, xp);
  return launch_status();
}
