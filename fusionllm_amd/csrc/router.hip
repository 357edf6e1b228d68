// router.hip — biased-sigmoid top-k routing (forward) and its backward.
//
// Forward replaces DeepSeekMoE._route, FusionLLM models/moe.py:44-50.
// Backward replaces the autograd of the same lines plus the gate Linear
// weight/bias gradient.
//
// Logit summation order (reproduced exactly by oracle/router_ref.c):
//   (dim <= 2048: the forward keeps a token's x chunks in registers)
//   16 lanes cooperate on one token.  dim is cut into 8-element chunks;
//   lane j owns chunks j, j+16, j+32, ... and accumulates, chunk by chunk and
//   element by element in ascending order, acc = fmaf(x, w, acc) from 0.
//   The 16 partials are then combined by an xor butterfly with offsets
//   8, 4, 2, 1 (each stage: p[j] = p[j] + p[j^off]); finally logit = p + bias.
//   Products of two bf16 values are exact in fp32, so fmaf and mul+add agree.
#include "fmoe_common.h"

namespace fmoe {

constexpr int kRouterLanes = 16;
constexpr int kRouterTok = kRouteBlockTokens;  // tokens per workgroup
constexpr int kRouterPerGroup = 1;             // tokens per 16-lane group
constexpr int kRouterThreads = kRouterTok / kRouterPerGroup * kRouterLanes;
constexpr int kRouterEBlk = 8;       // experts whose gate rows sit in LDS at a time (fp32: 64 KB at dim 2048)
constexpr int kRouterMaxDim = 2048;  // a lane keeps its <= 16 x chunks per token in registers

// One workgroup routes 32 tokens.  The gate rows are staged in LDS as fp32,
// 8 experts at a time, so the gate matrix is read from memory once per 32
// tokens instead of once per token; each lane keeps its x chunks in
// registers across the expert blocks.  (The kernel can give each 16-lane
// group R tokens, every gate chunk read from LDS feeding all R; R = 2 was
// measured slower than R = 1: 13.7 against 11.0 us at dim 768 with 8
// experts, 708 against 427 us at dim 2048 with 64 experts — half the waves,
// each with twice the FMA chains.)  The logits (without bias) go to LDS; the
// scores are computed once per (token, expert), spread over the group's
// lanes, and every lane of a token's group then takes the top-k.
// Lane l gets v from lane l ^ off (off < 16): ds_swizzle in xor mode, within
// groups of 32 lanes.
__device__ __forceinline__ float xor_lane(float v, int off) {
  int r;
  switch (off) {
    case 8: r = __builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x001F | (8 << 10)); break;
    case 4: r = __builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x001F | (4 << 10)); break;
    case 2: r = __builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x001F | (2 << 10)); break;
    default: r = __builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x001F | (1 << 10)); break;
  }
  return __int_as_float(r);
}

// Gate bias of expert e: bf16 in memory, or already converted to fp32 (LDS).
__device__ __forceinline__ float bias_at(const uint16_t* __restrict__ b, int e) { return bf2f(b[e]); }
__device__ __forceinline__ float bias_at(const float* b, int e) { return b[e]; }

// Top-k of one token from its scores s[0 .. E), computed redundantly by the
// 16 lanes of the token's group; lane j < k writes the j-th choice.
template <int EB>
__device__ __forceinline__ void pick_topk(const float (&s)[EB], int E, int k, float route_scale, int lane16,
                                          bool active, int t, int32_t* __restrict__ idx,
                                          int64_t* __restrict__ idx64, float* __restrict__ wout,
                                          float* __restrict__ vout, int* idx_lds, int* hist_lds) {
  // k selection rounds (a runtime loop over the token's k); lane j keeps the
  // j-th choice, and the chosen scores are summed in choice order.
  uint64_t taken = 0;
  int e_sel = 0;
  float v_sel = 0.0f, sum = 0.0f;
  for (int j = 0; j < k; ++j) {
    int best = -1;
    float bv = 0.0f;
#pragma unroll
    for (int e = 0; e < EB; ++e) {
      if (e < E && !((taken >> e) & 1ull)) {
        if (best < 0 || score_beats(s[e], bv)) { best = e; bv = s[e]; }
      }
    }
    taken |= 1ull << best;
    sum = (j == 0) ? bv : sum + bv;
    if (j == lane16) { e_sel = best; v_sel = bv; }
  }
  const float denom = sum + 1e-10f;
  if (active && lane16 < k) {
    const int64_t o = static_cast<int64_t>(t) * k + lane16;
    idx[o] = e_sel;
    if (idx_lds) idx_lds[o] = e_sel;
    if (idx64) idx64[o] = e_sel;
    wout[o] = (v_sel / denom) * route_scale;
    vout[o] = v_sel;
    if (hist_lds) atomicAdd(&hist_lds[e_sel], 1);  // integer count: exact in any order
  }
}

// Scores and top-k of one token from its logits lg[0 .. E) in LDS (bias not
// yet added; overwritten with the scores).  Lane l of the token's 16-lane
// group forms the scores of experts l, l + 16, ... (one exp and one divide
// each: every lane forming all E of them in turn took 2.7 us at E = 8), then
// each lane reads all E scores back for the top-k.  The group's lanes are in
// one wave, whose LDS accesses complete in program order.
template <int EB, typename BiasT>
__device__ __forceinline__ void route_token(float* lg, const BiasT* bg, int E, int k,
                                            float route_scale, int lane16, bool active, int t,
                                            int32_t* __restrict__ idx, int64_t* __restrict__ idx64,
                                            float* __restrict__ wout, float* __restrict__ vout,
                                            int* idx_lds = nullptr, int* hist_lds = nullptr) {
  for (int e = lane16; e < E; e += kRouterLanes) lg[e] = fm_sigmoid(lg[e] + bias_at(bg, e));
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float s[EB];
#pragma unroll
  for (int e = 0; e < EB; ++e) s[e] = (e < E) ? lg[e] : 0.0f;
  pick_topk<EB>(s, E, k, route_scale, lane16, active, t, idx, idx64, wout, vout, idx_lds, hist_lds);
}

template <int EB, int NQ, int R>  // NQ: x chunks per lane, NQ * 16 * 8 >= dim; R tokens per group
// block_hist (nullable): the workgroup's choices counted per expert,
// block_hist[blockIdx.x * E + e] — the histogram stage of the dispatch for
// blocks of kRouterTok tokens (used by fmoe_route_and_dispatch).
// Group g (16 lanes) takes tokens g, g + 32 / R, ... of the workgroup's 32.
// The first expert block's gate loads are issued before the x loads, so that
// staging them (which waits for its loads, and memory loads return in issue
// order) does not wait for x.
__global__ __launch_bounds__(kRouterTok / R * kRouterLanes) void router_fwd_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ wg,
    const uint16_t* __restrict__ bg, int T, int dim, int E, int k, float route_scale,
    int32_t* __restrict__ idx, int64_t* __restrict__ idx64, float* __restrict__ wout,
    float* __restrict__ vout, int32_t* __restrict__ block_hist) {
  constexpr int EBLK = EB < kRouterEBlk ? EB : kRouterEBlk;  // experts per LDS block
  constexpr int NG = kRouterTok / R;                          // groups per workgroup
  constexpr int NT = NG * kRouterLanes;                       // threads
  constexpr int GMAX = (EBLK * NQ * kRouterLanes + NT - 1) / NT;  // gate chunks per thread and block
  // Gate rows converted to fp32 once per workgroup, each 8-element chunk as
  // two float4 planes (elements 0-3, 4-7): consecutive lanes read consecutive
  // 16-byte words, and no lane unpacks bf16 per token.
  __shared__ float4 wlo[EBLK * NQ * kRouterLanes];
  __shared__ float4 whi[EBLK * NQ * kRouterLanes];
  __shared__ float lsh[kRouterTok * EB];
  __shared__ float bsh[EB];
  __shared__ int hcnt[EB];
  if (block_hist != nullptr && threadIdx.x < EB) hcnt[threadIdx.x] = 0;  // ordered by the first barrier below
  const int lane16 = threadIdx.x % kRouterLanes;
  const int grp = threadIdx.x / kRouterLanes;
  const int nchunk = dim / 8;

  uint4 gr[GMAX];
  auto load_gate = [&](int e0, int ne) {
    const uint4* src = reinterpret_cast<const uint4*>(wg + static_cast<int64_t>(e0) * dim);
#pragma unroll
    for (int u = 0; u < GMAX; ++u) {
      const int i = threadIdx.x + u * NT;
      gr[u] = i < ne * nchunk ? src[i] : make_uint4(0, 0, 0, 0);
    }
  };
  auto store_gate = [&](int ne) {
#pragma unroll
    for (int u = 0; u < GMAX; ++u) {
      const int i = threadIdx.x + u * NT;
      if (i < ne * nchunk) {
        float f[8];
        unpack8(gr[u], f);
        wlo[i] = make_float4(f[0], f[1], f[2], f[3]);
        whi[i] = make_float4(f[4], f[5], f[6], f[7]);
      }
    }
  };
  load_gate(0, min(EBLK, E));
  const float bias = threadIdx.x < E ? bf2f(bg[threadIdx.x]) : 0.0f;

  uint4 xr[R][NQ];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int t = blockIdx.x * kRouterTok + grp + r * NG;
    const int tc = t < T ? t : T - 1;  // idle lanes route a copy of the last token
    const uint4* xrow = reinterpret_cast<const uint4*>(x + static_cast<int64_t>(tc) * dim);
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int c = lane16 + kRouterLanes * q;
      xr[r][q] = c < nchunk ? xrow[c] : make_uint4(0, 0, 0, 0);
    }
  }
  if (threadIdx.x < E) bsh[threadIdx.x] = bias;  // ordered by the first barrier below

  for (int e0 = 0; e0 < E; e0 += EBLK) {
    const int ne = min(EBLK, E - e0);
    if (e0 > 0) {
      __syncthreads();  // the previous block's gate rows are no longer read
      load_gate(e0, ne);
    }
    store_gate(ne);
    __syncthreads();
    float acc[R][EBLK];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int e = 0; e < EBLK; ++e) acc[r][e] = 0.0f;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int c = lane16 + kRouterLanes * q;
      if (c < nchunk) {
        float xf[R][8];
#pragma unroll
        for (int r = 0; r < R; ++r) unpack8(xr[r][q], xf[r]);
#pragma unroll
        for (int e = 0; e < EBLK; ++e) {
          if (e < ne) {
            const float4 a = wlo[e * nchunk + c], b = whi[e * nchunk + c];
            const float wf[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
              for (int i = 0; i < 8; ++i) acc[r][e] = fmaf(xf[r][i], wf[i], acc[r][e]);
          }
        }
      }
    }
#pragma unroll
    for (int off = kRouterLanes / 2; off >= 1; off >>= 1) {
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int e = 0; e < EBLK; ++e) acc[r][e] = acc[r][e] + xor_lane(acc[r][e], off);
    }
    // every lane now holds the block's logits; lane e writes expert e0 + e
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int e = 0; e < EBLK; ++e)
        if (e == lane16 && e < ne) lsh[(grp + r * NG) * EB + e0 + e] = acc[r][e];
  }
  __syncthreads();

  // scores: lane j of a group computes experts j, j + 16, ... of its tokens
  // (in place over the logits), then every lane reads all E of its token
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float* lg = lsh + (grp + r * NG) * EB;
    for (int e = lane16; e < E; e += kRouterLanes) lg[e] = fm_sigmoid(lg[e] + bsh[e]);
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int tl = grp + r * NG;
    const int t = blockIdx.x * kRouterTok + tl;
    float sc[EB];
#pragma unroll
    for (int e = 0; e < EB; ++e) sc[e] = (e < E) ? lsh[tl * EB + e] : 0.0f;
    pick_topk<EB>(sc, E, k, route_scale, lane16, t < T, t, idx, idx64, wout, vout, nullptr,
                  block_hist != nullptr ? hcnt : nullptr);
  }
  if (block_hist != nullptr) {
    __syncthreads();
    if (threadIdx.x < E) block_hist[static_cast<int64_t>(blockIdx.x) * E + threadIdx.x] = hcnt[threadIdx.x];
  }
}

// Many experts (E > 16, e.g. 64 at dim 2048): router_fwd_kernel reads every
// gate value from LDS once per token (32 bytes of fp32 per 8 FMAs), and its
// LDS reads bound it (C5: 426 us).  Here each 16-lane group sums a 4-token x
// S-expert block of logits (S = EB / 8): for every chunk it reads the 4
// tokens' x chunks and the S experts' gate chunks from LDS once and does
// 4 x S x 8 FMAs with them (1.5 bytes of LDS per FMA at S = 8).  The 32
// tokens of the workgroup (the router's blocks, as the dispatch histogram
// expects) are 8 token blocks, the experts 8 expert blocks: 64 groups, 1024
// threads, so that a lane holds 4 S sums and four waves share each SIMD.
// dim is walked in slices of 128 elements (one 8-element chunk per lane),
// staged in LDS as fp32 (x and gate, each chunk as two float4 planes),
// double buffered, the next slice's loads in flight while the current one is
// summed.  Each (token, expert) sum keeps the order at the top of this file:
// lane j takes chunks j, j + 16, ... in ascending order, elements in order,
// fmaf from 0, then the butterfly; so it gives the bits of
// router_fwd_kernel.  Scores and top-k as there.
constexpr int kWideTB = 4;         // tokens per group block
constexpr int kWideThreads = 1024;

template <int EB>
__global__ __launch_bounds__(kWideThreads) void router_wide_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ wg,
    const uint16_t* __restrict__ bg, int T, int dim, int E, int k, float route_scale,
    int32_t* __restrict__ idx, int64_t* __restrict__ idx64, float* __restrict__ wout,
    float* __restrict__ vout, int32_t* __restrict__ block_hist) {
  constexpr int S = EB / 8;  // experts per group block
  constexpr int NT = kWideThreads;
  constexpr int NTB = kRouterTok / kWideTB;  // token blocks
  static_assert(NTB * 8 * kRouterLanes == NT, "8 token blocks x 8 expert blocks of 16 lanes");
  // slice planes: [buffer][row][lane] of float4 (elements 0-3 / 4-7 of the row's chunk)
  __shared__ float4 xlo[2][kRouterTok][kRouterLanes], xhi[2][kRouterTok][kRouterLanes];
  __shared__ float4 glo[2][EB][kRouterLanes], ghi[2][EB][kRouterLanes];
  __shared__ float lsh[kRouterTok * EB];
  __shared__ float bsh[EB];
  __shared__ int hcnt[EB];
  const int tid = threadIdx.x;
  const int lane16 = tid % kRouterLanes, grp = tid / kRouterLanes;
  const int tb = grp % NTB, eb = grp / NTB;  // token block, expert block
  const int nchunk = dim / 8, nslice = (nchunk + kRouterLanes - 1) / kRouterLanes;
  if (block_hist != nullptr && tid < EB) hcnt[tid] = 0;  // ordered by the first barrier below
  if (tid < E) bsh[tid] = bf2f(bg[tid]);
  const int t0 = blockIdx.x * kRouterTok;

  // staging of slice q: x rows (32 tokens x 16 chunks: threads 0 .. 511, one
  // chunk each) and gate rows (EB x 16 chunks: one chunk per thread up to EB * 16)
  constexpr int XCH = kRouterTok * kRouterLanes, GCH = EB * kRouterLanes;
  static_assert(XCH <= NT && GCH <= NT, "one chunk per thread");
  // two register sets of staged chunks (slices two apart), so that two
  // slices' loads are in flight while one is summed
  uint4 xv[2] = {make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0)};
  uint4 gv[2] = {make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0)};
  const int s_row = tid / kRouterLanes, s_ch = tid % kRouterLanes;
  const uint16_t* xrow = x + static_cast<int64_t>(min(t0 + min(s_row, kRouterTok - 1), T - 1)) * dim;
  const uint16_t* grow = wg + static_cast<int64_t>(min(s_row, E - 1)) * dim;
  auto load_slice = [&](int q, uint4& xr, uint4& gr) {
    const int c = q * kRouterLanes + s_ch;
    if (tid < XCH) xr = c < nchunk ? reinterpret_cast<const uint4*>(xrow)[c] : make_uint4(0, 0, 0, 0);
    if (tid < GCH)
      gr = (s_row < E && c < nchunk) ? reinterpret_cast<const uint4*>(grow)[c] : make_uint4(0, 0, 0, 0);
  };
  auto store_slice = [&](int buf, const uint4& xr, const uint4& gr) {
    float f[8];
    if (tid < XCH) {
      unpack8(xr, f);
      xlo[buf][s_row][s_ch] = make_float4(f[0], f[1], f[2], f[3]);
      xhi[buf][s_row][s_ch] = make_float4(f[4], f[5], f[6], f[7]);
    }
    if (tid < GCH) {
      unpack8(gr, f);
      glo[buf][s_row][s_ch] = make_float4(f[0], f[1], f[2], f[3]);
      ghi[buf][s_row][s_ch] = make_float4(f[4], f[5], f[6], f[7]);
    }
  };

  float acc[kWideTB][S];
#pragma unroll
  for (int t = 0; t < kWideTB; ++t)
#pragma unroll
    for (int e = 0; e < S; ++e) acc[t][e] = 0.0f;
  auto sum_slice = [&](int q) {
    const int buf = q & 1;
    if (q * kRouterLanes + lane16 < nchunk) {
      float xf[kWideTB][8];
#pragma unroll
      for (int t = 0; t < kWideTB; ++t) {
        const float4 a = xlo[buf][tb * kWideTB + t][lane16], b = xhi[buf][tb * kWideTB + t][lane16];
        xf[t][0] = a.x; xf[t][1] = a.y; xf[t][2] = a.z; xf[t][3] = a.w;
        xf[t][4] = b.x; xf[t][5] = b.y; xf[t][6] = b.z; xf[t][7] = b.w;
      }
#pragma unroll
      for (int e = 0; e < S; ++e) {
        const float4 a = glo[buf][eb * S + e][lane16], b = ghi[buf][eb * S + e][lane16];
        const float wf[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int t = 0; t < kWideTB; ++t)
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[t][e] = fmaf(xf[t][i], wf[i], acc[t][e]);
      }
    }
  };
  // slice q: summed from LDS buffer q % 2; its chunks were loaded into
  // register set q % 2 two slices earlier.  After summing slice q: slice
  // q + 1 goes from its register set to the other buffer (last read while
  // summing q - 1, before the barrier that ended it), and that set loads
  // slice q + 3.
  load_slice(0, xv[0], gv[0]);
  if (nslice > 1) load_slice(1, xv[1], gv[1]);
  store_slice(0, xv[0], gv[0]);
  if (nslice > 2) load_slice(2, xv[0], gv[0]);
  __syncthreads();
  for (int q = 0; q < nslice; q += 2) {
    sum_slice(q);
    if (q + 1 < nslice) {
      store_slice(1, xv[1], gv[1]);
      if (q + 3 < nslice) load_slice(q + 3, xv[1], gv[1]);
      __syncthreads();
      sum_slice(q + 1);
      if (q + 2 < nslice) {
        store_slice(0, xv[0], gv[0]);
        if (q + 4 < nslice) load_slice(q + 4, xv[0], gv[0]);
        __syncthreads();
      }
    }
  }
#pragma unroll
  for (int off = kRouterLanes / 2; off >= 1; off >>= 1)
#pragma unroll
    for (int t = 0; t < kWideTB; ++t)
#pragma unroll
      for (int e = 0; e < S; ++e) acc[t][e] = acc[t][e] + xor_lane(acc[t][e], off);
  // every lane of the group holds the block's logits; lane j writes those of
  // its (t, e) with (t * S + e) % 16 == j
#pragma unroll
  for (int t = 0; t < kWideTB; ++t)
#pragma unroll
    for (int e = 0; e < S; ++e)
      if ((t * S + e) % kRouterLanes == lane16 && eb * S + e < E) lsh[(tb * kWideTB + t) * EB + eb * S + e] = acc[t][e];
  __syncthreads();

  // scores and top-k: group g < 32 takes token g of the workgroup (as router_fwd_kernel)
  if (grp < kRouterTok) {
    float* lg = lsh + grp * EB;
    for (int e = lane16; e < E; e += kRouterLanes) lg[e] = fm_sigmoid(lg[e] + bsh[e]);
  }
  __syncthreads();
  if (grp < kRouterTok) {
    const int t = t0 + grp;
    float sc[EB];
#pragma unroll
    for (int e = 0; e < EB; ++e) sc[e] = (e < E) ? lsh[grp * EB + e] : 0.0f;
    pick_topk<EB>(sc, E, k, route_scale, lane16, t < T, t, idx, idx64, wout, vout, nullptr,
                  block_hist != nullptr ? hcnt : nullptr);
  }
  if (block_hist != nullptr) {
    __syncthreads();
    if (tid < E) block_hist[static_cast<int64_t>(blockIdx.x) * E + tid] = hcnt[tid];
  }
}

// Decode-sized batches (T <= kRouterSmallT): one workgroup per token and one
// 16-lane group per expert (group g takes experts g, g + G, ...), so that the
// logits of a token are formed side by side instead of one expert after
// another.  Each logit is summed in exactly the order described at the top
// (the lanes of a group own the same chunks), so both kernels give the same
// bits.  The gate rows are read from memory (L2) by every token's workgroup.
constexpr int kRouterSmallT = 128;

template <int EB, int NQ>
__global__ __launch_bounds__(512) void router_small_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ wg,
    const uint16_t* __restrict__ bg, int dim, int E, int k, float route_scale,
    int32_t* __restrict__ idx, int64_t* __restrict__ idx64, float* __restrict__ wout,
    float* __restrict__ vout) {
  __shared__ float lsh[EB];
  __shared__ float bsh[EB];
  const int lane16 = threadIdx.x % kRouterLanes;
  const int grp = threadIdx.x / kRouterLanes, ngrp = blockDim.x / kRouterLanes;
  const int t = blockIdx.x;
  // the bias, loaded beside the logits' operands rather than after them
  if (threadIdx.x < E) bsh[threadIdx.x] = bf2f(bg[threadIdx.x]);
  const int nchunk = dim / 8;
  const uint4* xrow = reinterpret_cast<const uint4*>(x + static_cast<int64_t>(t) * dim);
  uint4 xr[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int c = lane16 + kRouterLanes * q;
    xr[q] = c < nchunk ? xrow[c] : make_uint4(0, 0, 0, 0);
  }
  for (int e = grp; e < E; e += ngrp) {
    const uint4* wrow = reinterpret_cast<const uint4*>(wg + static_cast<int64_t>(e) * dim);
    uint4 wr[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int c = lane16 + kRouterLanes * q;
      wr[q] = c < nchunk ? wrow[c] : make_uint4(0, 0, 0, 0);
    }
    float acc = 0.0f;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      if (lane16 + kRouterLanes * q < nchunk) {
        float xf[8], wf[8];
        unpack8(xr[q], xf);
        unpack8(wr[q], wf);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc = fmaf(xf[i], wf[i], acc);
      }
    }
#pragma unroll
    for (int off = kRouterLanes / 2; off >= 1; off >>= 1) acc = acc + xor_lane(acc, off);
    if (lane16 == 0) lsh[e] = acc;
  }
  __syncthreads();
  if (grp == 0)
    route_token<EB>(lsh, static_cast<const float*>(bsh), E, k, route_scale, lane16, true, t, idx, idx64, wout,
                    vout);
}

// ---- routing and dispatch of a tiny batch in one launch ---------------------
// T <= kTinyT tokens: one 512-thread workgroup forms all T * E logits (16-lane
// group g takes the (token, expert) pairs g, g + 32, ..., each summed in the
// order described at the top), routes every token (route_token, group t for
// token t), then does the dispatch of fmoe_dispatch on the T * k slots it
// holds in LDS: the same stable counting sort (ranks by wave ballots, wave
// counts added in wave order), the counts and offsets, and the row gather
// (from the token rows kept in LDS while the logits were formed).  Outputs are
// those of fmoe_router_fwd followed by fmoe_dispatch, bit for bit.  Meant for
// T * E <= 64 (one or two logits per 16-lane group); correct for any T <= 16.
constexpr int kTinyT = 16;
constexpr int kTinyThreads = 512;  // 256 VGPRs per lane: a token row and a gate row in registers
constexpr int kTinyWaves = kTinyThreads / 64;

template <int EB, int NQ>
__global__ __launch_bounds__(kTinyThreads) void route_dispatch_tiny_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ wg, const uint16_t* __restrict__ bg, int T,
    int dim, int E, int k, float route_scale, int32_t* __restrict__ idx, int64_t* __restrict__ idx64,
    float* __restrict__ wout, float* __restrict__ vout, int32_t* __restrict__ counts,
    int32_t* __restrict__ offsets, int32_t* __restrict__ perm, int32_t* __restrict__ pos_of_slot,
    uint4* __restrict__ x_perm) {
  __shared__ float lsh[kTinyT * EB];
  __shared__ int idx_sh[kTinyT * FMOE_MAX_TOPK];
  __shared__ int perm_sh[kTinyT * FMOE_MAX_TOPK];
  __shared__ int wcount[kTinyWaves][FMOE_MAX_EXPERTS];
  __shared__ int start[FMOE_MAX_EXPERTS + 1];
  __shared__ uint4 x_sh[kTinyT * (kRouterMaxDim / 8)];  // the token rows, for the gather
  __shared__ float bsh[FMOE_MAX_EXPERTS];
  const int tid = threadIdx.x, lane16 = tid % kRouterLanes, grp = tid / kRouterLanes;
  const int lane = tid & 63, wave = tid >> 6;
  const int nchunk = dim / 8, n_slots = T * k;
  for (int i = tid; i < kTinyWaves * E; i += kTinyThreads) wcount[i / E][i % E] = 0;
  // the bias, loaded beside the logits' operands rather than after them
  if (tid < E) bsh[tid] = bf2f(bg[tid]);

  // 1. logits
  for (int p = grp; p < T * E; p += kTinyThreads / kRouterLanes) {
    const int t = p / E, e = p - t * E;
    const uint4* xrow = reinterpret_cast<const uint4*>(x + static_cast<int64_t>(t) * dim);
    const uint4* wrow = reinterpret_cast<const uint4*>(wg + static_cast<int64_t>(e) * dim);
    uint4 xr[NQ], wr[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int c = lane16 + kRouterLanes * q;
      xr[q] = c < nchunk ? xrow[c] : make_uint4(0, 0, 0, 0);
      wr[q] = c < nchunk ? wrow[c] : make_uint4(0, 0, 0, 0);
    }
    if (e == 0) {  // one group per token keeps its row for the gather
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        const int c = lane16 + kRouterLanes * q;
        if (c < nchunk) x_sh[t * nchunk + c] = xr[q];
      }
    }
    float acc = 0.0f;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      if (lane16 + kRouterLanes * q < nchunk) {
        float xf[8], wf[8];
        unpack8(xr[q], xf);
        unpack8(wr[q], wf);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc = fmaf(xf[i], wf[i], acc);
      }
    }
#pragma unroll
    for (int off = kRouterLanes / 2; off >= 1; off >>= 1) acc = acc + xor_lane(acc, off);
    if (lane16 == 0) lsh[t * EB + e] = acc;
  }
  __syncthreads();

  // 2. routing: group t routes token t
  if (grp < T)
    route_token<EB>(lsh + grp * EB, static_cast<const float*>(bsh), E, k, route_scale, lane16, true, grp, idx,
                    idx64, wout, vout, idx_sh);
  __syncthreads();

  // 3. dispatch: rank slot s among the earlier slots with the same expert
  const int s = tid;
  const bool valid = s < n_slots;
  const int e = valid ? idx_sh[s] : -1;
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
  scan_wave_counts<kTinyWaves>(wcount, E, start);
  __syncthreads();
  if (valid) {
    int pos = start[e] + rank;
    for (int w = 0; w < wave; ++w) pos += wcount[w][e];
    perm_sh[pos] = s;
    perm[pos] = s;
    pos_of_slot[s] = pos;
  }
  for (int q = tid; q < E; q += kTinyThreads) {
    counts[q] = start[q + 1] - start[q];
    offsets[q] = start[q];
  }
  if (tid == 0) offsets[E] = start[E];
  if (x_perm == nullptr) return;
  __syncthreads();

  // 4. row gather from the rows kept in LDS, 16-byte stores
  const int total = n_slots * nchunk;
  for (int g = tid; g < total; g += kTinyThreads) {
    const int r = g / nchunk, c = g - r * nchunk;
    x_perm[g] = x_sh[(perm_sh[r] / k) * nchunk + c];
  }
}

// ---- backward ----------------------------------------------------------------
// Per token: w_j = (v_j / D) * rs with D = sum(v) + 1e-10.  Autograd of that:
//   dq_j = dw_j * rs;  dv_j = dq_j / D + dS,  dS = -sum_j dq_j * v_j / D^2;
// top-k backward routes dv_j to the selected score; sigmoid backward gives
//   dlogit_j = dv_j * (1 - v_j) * v_j.
// The normalisation and sigmoid backward of slot t*k + jr, the token's sums
// taken over j in ascending order.
__device__ __forceinline__ float slot_dlogit(const float* __restrict__ dwt, const float* __restrict__ vt, int k,
                                             int jr, float rs) {
  float sum = vt[0];
  for (int j = 1; j < k; ++j) sum = sum + vt[j];
  const float D = sum + 1e-10f;
  float dS = 0.0f;
  for (int j = 0; j < k; ++j) {
    const float dq = dwt[j] * rs;
    dS = dS - (dq * vt[j]) / (D * D);
  }
  const float dq = dwt[jr] * rs;
  const float dv = dq / D + dS;
  return (dv * (1.0f - vt[jr])) * vt[jr];
}

// Gate weight/bias gradient as a segmented column reduction over the
// expert-contiguous rows:  dWg[e] = sum_{r in e} dl_row[r] * x[perm[r] / k],
// dbg[e] = sum_{r in e} dl_row[r], where dl_row[r] is the logit gradient of
// slot perm[r] (row r's token rows are read from x through perm).  Expert e's rows are cut into ceil(M_e / kChunkRows) chunks,
// numbered consecutively over the experts (chunk_base(e) = sum of the chunk
// counts of experts < e).  Stage 1: one block per chunk reads the E + 1
// offsets once (into LDS), issues its first kPartialBatch row loads, forms
// the logit gradients of its rows (one thread per row, also
// written to d_logits by slot), then reduces its rows into
// partial[chunk][dim+1], row by row in order (loads issued kPartialBatch rows
// at a time).  Stage 2 adds the chunks of each
// expert in chunk order.  Both orders are fixed.
constexpr int kChunkRows = 32;
constexpr int kPartialBatch = 16;

constexpr int kPartialThreads = 128;

__global__ __launch_bounds__(kPartialThreads) void router_wgrad_partial_kernel(
    const float* __restrict__ dw, const float* __restrict__ v, const int32_t* __restrict__ perm, int k,
    float rs, float* __restrict__ dl, const int32_t* __restrict__ offsets, int E,
    const uint16_t* __restrict__ x, int dim, float* __restrict__ partial) {
  __shared__ int off_sh[FMOE_MAX_EXPERTS + 1];
  __shared__ float gsh[kChunkRows];
  __shared__ int tok_sh[kChunkRows];  // token of each row of the chunk (perm[r] / k)
  if (threadIdx.x <= E) off_sh[threadIdx.x] = offsets[threadIdx.x];  // one load for all E + 1
  __syncthreads();
  int c = blockIdx.x, e = 0;
  for (; e < E; ++e) {
    const int n = (off_sh[e + 1] - off_sh[e] + kChunkRows - 1) / kChunkRows;
    if (c < n) break;
    c -= n;
  }
  if (e >= E) return;  // grid is an upper bound on the chunk count
  const int r0 = off_sh[e] + c * kChunkRows;
  const int r1 = min(off_sh[e + 1], r0 + kChunkRows);
  float* out = partial + static_cast<int64_t>(blockIdx.x) * (dim + 1);
  const int nchunk8 = dim / 8;
  const int64_t ld = dim / 8;
  // The chunk's rows are token rows of x: row r is token perm[r] / k (rows
  // past r1 repeat row r1 - 1).
  int my_slot = 0;
  if (threadIdx.x < kChunkRows) {
    my_slot = perm[min(r0 + static_cast<int>(threadIdx.x), r1 - 1)];
    tok_sh[threadIdx.x] = my_slot / k;
  }
  __syncthreads();
  // Column passes of kPartialThreads columns (the same count for every
  // thread, so the barrier in the first pass is reached by all).
  for (int cb = 0; cb <= nchunk8; cb += kPartialThreads) {
    const int col8 = cb + threadIdx.x;
    const bool is_col = col8 < nchunk8;
    const uint4* xc = reinterpret_cast<const uint4*>(x) + (is_col ? col8 : 0);
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    // Batches of kPartialBatch rows: every load first (rows past r1 read row
    // r1 - 1, in bounds), then the rows below r1 added in order through a
    // select, so that no load waits on another.  The first batch's loads go
    // out before the logit gradients are formed.
    uint4 xv[kPartialBatch];
    auto load_batch = [&](int rb) {
#pragma unroll
      for (int u = 0; u < kPartialBatch; ++u) xv[u] = xc[static_cast<int64_t>(tok_sh[min(rb + u, r1 - 1) - r0]) * ld];
    };
    if (is_col) load_batch(r0);
    if (cb == 0) {
      if (threadIdx.x < r1 - r0) {
        const int slot = my_slot;
        const int t = slot / k, jr = slot - t * k;
        const float g = slot_dlogit(dw + static_cast<int64_t>(t) * k, v + static_cast<int64_t>(t) * k, k, jr, rs);
        dl[slot] = g;
        gsh[threadIdx.x] = g;
      }
      __syncthreads();
    }
    if (col8 == nchunk8) {  // bias column
      float bacc = 0.0f;
      for (int r = r0; r < r1; ++r) bacc = bacc + gsh[r - r0];
      out[dim] = bacc;
      continue;
    }
    if (!is_col) continue;
    for (int rb = r0; rb < r1; rb += kPartialBatch) {
      if (rb != r0) load_batch(rb);
#pragma unroll
      for (int u = 0; u < kPartialBatch; ++u) {
        const bool in = rb + u < r1;
        const float g = gsh[in ? rb + u - r0 : 0];
        float xf[8];
        unpack8(xv[u], xf);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float f = fmaf(g, xf[i], acc[i]);
          acc[i] = in ? f : acc[i];
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) out[col8 * 8 + i] = acc[i];
  }
}

// One block per (16 columns, expert): 16 chunk lanes per column each add the
// chunks c = lane, lane + 16, ... in order; the 16 lane sums are then added
// in lane order.  Fixed order, so deterministic.
__global__ __launch_bounds__(256) void router_wgrad_final_kernel(
    const float* __restrict__ partial, const int32_t* __restrict__ offsets, int E, int dim,
    int grad_dtype, void* __restrict__ dwg, void* __restrict__ dbg) {
  __shared__ float lsum[16][17];
  const int e = blockIdx.y;
  const int cl = threadIdx.x & 15, lanec = threadIdx.x >> 4;
  const int col = blockIdx.x * 16 + cl;
  int base = 0;  // uniform: scalar loads of the offsets
  for (int q = 0; q < e; ++q) base += (offsets[q + 1] - offsets[q] + kChunkRows - 1) / kChunkRows;
  const int nch = (offsets[e + 1] - offsets[e] + kChunkRows - 1) / kChunkRows;
  float acc = 0.0f;
  if (col <= dim) {
    const float* pc = partial + static_cast<int64_t>(base) * (dim + 1) + col;
    int c = lanec;
    const int last = max(nch - 1, 0);
    for (; c < nch; c += 16 * 16) {  // sixteen loads in flight (clamped in bounds), added in chunk order
      float p[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) p[u] = pc[static_cast<int64_t>(min(c + 16 * u, last)) * (dim + 1)];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const float sum = acc + p[u];
        acc = c + 16 * u < nch ? sum : acc;
      }
    }
  }
  lsum[lanec][cl] = acc;
  __syncthreads();
  if (lanec != 0 || col > dim) return;
  float tot = lsum[0][cl];
  for (int l = 1; l < 16; ++l) tot = tot + lsum[l][cl];
  if (col < dim) {
    const int64_t o = static_cast<int64_t>(e) * dim + col;
    if (grad_dtype == FMOE_BF16) static_cast<uint16_t*>(dwg)[o] = f2bf(tot);
    else static_cast<float*>(dwg)[o] = tot;
  } else {
    if (grad_dtype == FMOE_BF16) static_cast<uint16_t*>(dbg)[e] = f2bf(tot);
    else static_cast<float*>(dbg)[e] = tot;
  }
}

__global__ void zero_grad_kernel(void* dwg, void* dbg, int E, int dim, int grad_dtype) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= E * (dim + 1)) return;
  const bool is_w = i < E * dim;
  void* p = is_w ? dwg : dbg;
  const int o = is_w ? i : i - E * dim;
  if (grad_dtype == FMOE_BF16) static_cast<uint16_t*>(p)[o] = 0;
  else static_cast<float*>(p)[o] = 0.0f;
}

}  // namespace fmoe

using namespace fmoe;

extern "C" int fmoe_router_fwd(const void* x, const void* gate_w, const void* gate_b, int64_t T,
                               int64_t dim, int n_experts, int k, float route_scale, int32_t* idx,
                               int64_t* idx64, float* weights, float* topv, void* stream) {
  if (T < 0 || dim <= 0) return FMOE_ERR_INVALID_ARG;
  if (n_experts <= 0 || n_experts > FMOE_MAX_EXPERTS) return FMOE_ERR_TOO_MANY_EXPERTS;
  if (k <= 0 || k > FMOE_MAX_TOPK || k > n_experts || dim % 64 != 0 || dim > kRouterMaxDim)
    return FMOE_ERR_SHAPE;
  if (T == 0) return FMOE_OK;
  if (!x || !gate_w || !gate_b || !idx || !weights || !topv) return FMOE_ERR_INVALID_ARG;
  if (!aligned16(x) || !aligned16(gate_w)) return FMOE_ERR_ALIGN;
  const bool small = T <= kRouterSmallT;
  const int threads = small ? kRouterLanes * (n_experts < 32 ? n_experts : 32) : kRouterThreads;
  const int64_t blocks = small ? T : ceil_div(T, kRouterTok);
  hipStream_t s = as_stream(stream);
  auto xs = static_cast<const uint16_t*>(x);
  auto ws = static_cast<const uint16_t*>(gate_w);
  auto bs = static_cast<const uint16_t*>(gate_b);
#define FMOE_ROUTER_LAUNCH(EB, NQ)                                                                    \
  do {                                                                                                \
    if (small)                                                                                        \
      router_small_kernel<EB, NQ><<<dim3(blocks), dim3(threads), 0, s>>>(xs, ws, bs, (int)dim,         \
                                                                         n_experts, k, route_scale,  \
                                                                         idx, idx64, weights, topv); \
    else if (EB >= 32)                                                                                \
      router_wide_kernel<(EB >= 32 ? EB : 32)><<<dim3(blocks), dim3(kWideThreads), 0, s>>>(xs, ws, bs, (int)T, \
                                                                    (int)dim, n_experts, k, route_scale, \
                                                                    idx, idx64, weights, topv, nullptr); \
    else                                                                                              \
      router_fwd_kernel<EB, NQ, kRouterPerGroup><<<dim3(blocks), dim3(threads), 0, s>>>(xs, ws, bs, (int)T, (int)dim,  \
                                                                       n_experts, k, route_scale,    \
                                                                       idx, idx64, weights, topv,    \
                                                                       nullptr);                     \
  } while (0)
#define FMOE_ROUTER_LAUNCH_E(NQ)                 \
  do {                                           \
    if (n_experts <= 8) FMOE_ROUTER_LAUNCH(8, NQ);       \
    else if (n_experts <= 16) FMOE_ROUTER_LAUNCH(16, NQ); \
    else if (n_experts <= 32) FMOE_ROUTER_LAUNCH(32, NQ); \
    else FMOE_ROUTER_LAUNCH(64, NQ);                      \
  } while (0)
  if (dim <= 512) FMOE_ROUTER_LAUNCH_E(4);
  else if (dim <= 1024) FMOE_ROUTER_LAUNCH_E(8);
  else FMOE_ROUTER_LAUNCH_E(16);
#undef FMOE_ROUTER_LAUNCH_E
#undef FMOE_ROUTER_LAUNCH
  return launch_status();
}

namespace fmoe {
// The routing half of fmoe_route_and_dispatch: router_fwd_kernel for any T
// (for T <= kRouterSmallT it gives the bits of router_small_kernel, which
// sums each logit in the same order), with each workgroup's per-expert
// counts written to block_hist[ceil(T / kRouterTok)][E].  Arguments are
// checked by the caller.
int launch_router_hist(const uint16_t* xs, const uint16_t* ws, const uint16_t* bs, int64_t T, int64_t dim,
                       int n_experts, int k, float route_scale, int32_t* idx, int64_t* idx64, float* weights,
                       float* topv, int32_t* block_hist, hipStream_t s) {
  const int threads = kRouterThreads;
  const int64_t blocks = ceil_div(T, kRouterTok);
#define FMOE_ROUTER_H(EB, NQ)                                                                          \
  do {                                                                                                 \
    if (EB >= 32)                                                                                      \
      router_wide_kernel<(EB >= 32 ? EB : 32)><<<dim3(blocks), dim3(kWideThreads), 0, s>>>(xs, ws, bs, (int)T, \
                                                                    (int)dim, n_experts, k, route_scale, \
                                                                    idx, idx64, weights, topv, block_hist); \
    else                                                                                               \
      router_fwd_kernel<EB, NQ, kRouterPerGroup><<<dim3(blocks), dim3(threads), 0, s>>>(xs, ws, bs, (int)T, (int)dim, n_experts, \
                                                                   k, route_scale, idx, idx64, weights,   \
                                                                   topv, block_hist);                     \
  } while (0)
#define FMOE_ROUTER_H_E(NQ)                              \
  do {                                                   \
    if (n_experts <= 8) FMOE_ROUTER_H(8, NQ);            \
    else if (n_experts <= 16) FMOE_ROUTER_H(16, NQ);     \
    else if (n_experts <= 32) FMOE_ROUTER_H(32, NQ);     \
    else FMOE_ROUTER_H(64, NQ);                          \
  } while (0)
  if (dim <= 512) FMOE_ROUTER_H_E(4);
  else if (dim <= 1024) FMOE_ROUTER_H_E(8);
  else FMOE_ROUTER_H_E(16);
#undef FMOE_ROUTER_H_E
#undef FMOE_ROUTER_H
  return launch_status();
}
}  // namespace fmoe

extern "C" int fmoe_route_dispatch(const void* x, const void* gate_w, const void* gate_b, int64_t T,
                                   int64_t dim, int n_experts, int k, float route_scale, int32_t* idx,
                                   int64_t* idx64, float* weights, float* topv, int32_t* counts,
                                   int32_t* offsets, int32_t* perm, int32_t* pos_of_slot, void* x_perm,
                                   void* stream) {
  if (T < 0 || dim <= 0) return FMOE_ERR_INVALID_ARG;
  if (n_experts <= 0 || n_experts > FMOE_MAX_EXPERTS) return FMOE_ERR_TOO_MANY_EXPERTS;
  if (k <= 0 || k > FMOE_MAX_TOPK || k > n_experts || dim % 64 != 0 || dim > kRouterMaxDim || T > kTinyT)
    return FMOE_ERR_SHAPE;
  if (!counts || !offsets) return FMOE_ERR_INVALID_ARG;
  if (T > 0 && (!x || !gate_w || !gate_b || !idx || !weights || !topv || !perm || !pos_of_slot))
    return FMOE_ERR_INVALID_ARG;
  if (!aligned16(x) || !aligned16(gate_w) || (x_perm && !aligned16(x_perm))) return FMOE_ERR_ALIGN;
  hipStream_t s = as_stream(stream);
  auto xs = static_cast<const uint16_t*>(x);
  auto ws = static_cast<const uint16_t*>(gate_w);
  auto bs = static_cast<const uint16_t*>(gate_b);
  auto xp = static_cast<uint4*>(x_perm);
#define FMOE_TINY(EB, NQ)                                                                                 \
  route_dispatch_tiny_kernel<EB, NQ><<<1, kTinyThreads, 0, s>>>(xs, ws, bs, (int)T, (int)dim, n_experts, k, \
                                                                route_scale, idx, idx64, weights, topv,     \
                                                                counts, offsets, perm, pos_of_slot, xp)
#define FMOE_TINY_E(NQ)                                  \
  do {                                                   \
    if (n_experts <= 8) FMOE_TINY(8, NQ);                \
    else if (n_experts <= 16) FMOE_TINY(16, NQ);         \
    else if (n_experts <= 32) FMOE_TINY(32, NQ);         \
    else FMOE_TINY(64, NQ);                              \
  } while (0)
  if (dim <= 512) FMOE_TINY_E(4);
  else if (dim <= 1024) FMOE_TINY_E(8);
  else FMOE_TINY_E(16);
#undef FMOE_TINY_E
#undef FMOE_TINY
  return launch_status();
}

namespace fmoe {
// Upper bound of sum over experts of ceil(M_e / kChunkRows) with sum M_e = T*k.
inline int64_t router_max_chunks(int64_t T, int n_experts, int k) {
  return (T * k) / kChunkRows + n_experts;
}
}  // namespace fmoe

extern "C" size_t fmoe_router_bwd_workspace_bytes(int64_t T, int64_t dim, int n_experts, int k) {
  if (T <= 0 || dim <= 0 || n_experts <= 0 || k <= 0) return 0;
  // chunk partials
  return static_cast<size_t>(router_max_chunks(T, n_experts, k) * (dim + 1)) * sizeof(float);
}

extern "C" int fmoe_router_bwd(const float* d_weights, const float* topv, const int32_t* perm,
                               const int32_t* offsets, const void* x, int64_t T, int64_t dim,
                               int n_experts, int k, float route_scale, float* d_logits,
                               void* d_gate_w, void* d_gate_b, int grad_dtype, void* workspace,
                               size_t workspace_bytes, void* stream) {
  if (T < 0 || dim <= 0) return FMOE_ERR_INVALID_ARG;
  if (n_experts <= 0 || n_experts > FMOE_MAX_EXPERTS) return FMOE_ERR_TOO_MANY_EXPERTS;
  if (k <= 0 || k > FMOE_MAX_TOPK || k > n_experts || dim % 64 != 0) return FMOE_ERR_SHAPE;
  if (grad_dtype != FMOE_BF16 && grad_dtype != FMOE_F32) return FMOE_ERR_DTYPE;
  hipStream_t s = as_stream(stream);
  if (T == 0) {
    // No tokens: the gate gradients are zero.
    if (!d_gate_w || !d_gate_b) return FMOE_ERR_INVALID_ARG;
    const int64_t n = static_cast<int64_t>(n_experts) * (dim + 1);
    zero_grad_kernel<<<dim3(ceil_div(n, 256)), dim3(256), 0, s>>>(d_gate_w, d_gate_b,
                                                                  n_experts, (int)dim, grad_dtype);
    return launch_status();
  }
  if (!d_weights || !topv || !perm || !offsets || !x || !d_logits || !d_gate_w || !d_gate_b ||
      !workspace)
    return FMOE_ERR_INVALID_ARG;
  if (workspace_bytes < fmoe_router_bwd_workspace_bytes(T, dim, n_experts, k))
    return FMOE_ERR_WORKSPACE;
  if (!aligned16(x)) return FMOE_ERR_ALIGN;
  const int64_t max_chunks = router_max_chunks(T, n_experts, k);
  float* partial = static_cast<float*>(workspace);
  router_wgrad_partial_kernel<<<dim3(max_chunks), dim3(128), 0, s>>>(
      d_weights, topv, perm, k, route_scale, d_logits, offsets, n_experts,
      static_cast<const uint16_t*>(x), (int)dim, partial);
  router_wgrad_final_kernel<<<dim3(ceil_div(dim + 1, 16), n_experts), dim3(256), 0, s>>>(
      partial, offsets, n_experts, (int)dim, grad_dtype, d_gate_w, d_gate_b);
  return launch_status();
}
