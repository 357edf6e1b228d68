// norm.hip — the RMSNorm in front of the MoE block and its backward, fused
// with the per-token reduction of the block's input gradient.
//
// FusionLLMBlock's FFN half is x + ffn(norm2(x)) with
// norm2 = nn.RMSNorm(dim, eps=1e-6) (FusionLLM models/fusionllm.py:48,52).
// Forward: one wave per token computes r = 1/sqrt(mean(x^2) + eps) and writes
// the bf16 MoE input xn = (x*r)*w and r (the residual add is fused into the
// combine, combine.hip).  Backward: one wave per token sums the token's
// input-gradient rows of the MoE (as fmoe_dx_reduce) into d_xn, applies the
// RMSNorm backward
//   g = d_xn * w,  xh = x * r,  dx = r * (g - xh * sum(g*xh)/dim) + d_out
// and accumulates sum_t d_xn * xh (the norm weight's gradient) per column in
// registers; every workgroup writes one partial row, and two small kernels
// add the partial rows in a fixed tree order (deterministic, no atomics).
//
// Rows are split into 8-element chunks (16-byte bf16 loads); lane l of the
// wave owns chunks l, l+64, ... so a row lives in registers (dim <= 4096).
#include <algorithm>

#include "fmoe_common.h"
#include "choices.h"

namespace fmoe {

constexpr int kNormThreads = 256;
constexpr int kNormWaves = kNormThreads / 64;
constexpr int kNormMaxDim = 4096;
// Partial rows of the norm weight gradient: one per workgroup of the
// backward, whose grid is one token per wave up to this many workgroups.
constexpr int kNormParts = 4096;

__device__ __forceinline__ void load8(const void* base, int dtype, int64_t elem, float* v) {
  if (dtype == FMOE_BF16) {
    unpack8(*reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + elem), v);
  } else {
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(base) + elem);
    const float4 a = p[0], b = p[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
}

__device__ __forceinline__ void store8(void* base, int dtype, int64_t elem, const float* v) {
  if (dtype == FMOE_BF16) {
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(base) + elem) = pack8(v);
  } else {
    float4* p = reinterpret_cast<float4*>(static_cast<float*>(base) + elem);
    p[0] = make_float4(v[0], v[1], v[2], v[3]);
    p[1] = make_float4(v[4], v[5], v[6], v[7]);
  }
}

// Sum over the 64 lanes in a fixed xor-butterfly order.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = v + __shfl_xor(v, off, 64);
  return v;
}

template <int NCH>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_fwd_kernel(
    const void* __restrict__ x, int x_dtype, const void* __restrict__ nw, int w_dtype, int64_t T,
    int dim, float eps, uint16_t* __restrict__ xn, float* __restrict__ rstd) {
  const int lane = threadIdx.x & 63;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kNormWaves + (threadIdx.x >> 6);
  if (t >= T) return;
  const int chunks = dim / 8;
  float v[NCH][8];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int c = lane + 64 * i;
    if (c < chunks) {
      load8(x, x_dtype, t * dim + c * 8, v[i]);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = ss + v[i][e] * v[i][e];
    }
  }
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / static_cast<float>(dim) + eps);
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int c = lane + 64 * i;
    if (c < chunks) {
      float w[8] = {1, 1, 1, 1, 1, 1, 1, 1};
      if (nw) load8(nw, w_dtype, c * 8, w);
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (v[i][e] * r) * w[e];
      *reinterpret_cast<uint4*>(xn + t * dim + c * 8) = pack8(o);
    }
  }
  if (lane == 0) rstd[t] = r;
}

template <int NCH>
__global__ __launch_bounds__(kNormThreads) void dx_reduce_norm_kernel(
    const uint16_t* __restrict__ dxr, const int32_t* __restrict__ pos_of_slot,
    const int32_t* __restrict__ idx, const float* __restrict__ dl,
    const uint16_t* __restrict__ gate_w, int64_t T, int dim, int k, int64_t rows_routed,
    int has_shared, const void* __restrict__ x, const float* __restrict__ rstd,
    const void* __restrict__ nw, int w_dtype, const void* __restrict__ d_out, int x_dtype,
    void* __restrict__ dx, float* __restrict__ parts) {
  __shared__ float red[kNormMaxDim];
  const int lane = threadIdx.x & 63;
  // Wave-uniform token index: the token's choices, router gradients and r
  // come through the scalar cache.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int chunks = dim / 8;
  float pw[NCH][8];
#pragma unroll
  for (int i = 0; i < NCH; ++i)
#pragma unroll
    for (int e = 0; e < 8; ++e) pw[i][e] = 0.0f;

  const int64_t stride = static_cast<int64_t>(gridDim.x) * kNormWaves;
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * kNormWaves + wave; t < T; t += stride) {
    Choices ch;
    load_sorted_choices(idx, pos_of_slot, nullptr, t, k, ch);
    float gl[FMOE_MAX_TOPK];
#pragma unroll
    for (int j = 0; j < FMOE_MAX_TOPK; ++j) gl[j] = j < k ? dl[t * k + ch.slot[j]] : 0.0f;
    const float r = rstd[t];
    float g[NCH][8], xh[NCH][8], dov[NCH][8];
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = lane + 64 * i;
      if (c < chunks) {
        load8(d_out, x_dtype, t * dim + c * 8, dov[i]);  // issued early, used after the row sum
        // d_xn: the MoE's input gradient for this chunk, in the order of
        // fmoe_dx_reduce (routed rows by ascending expert, shared, router).
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < FMOE_MAX_TOPK; ++j) {
          if (j < k) {
            float v[8];
            unpack8(reinterpret_cast<const uint4*>(dxr + static_cast<int64_t>(ch.pos[j]) * dim)[c], v);
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[e] = acc[e] + v[e];
          }
        }
        if (has_shared) {
          float v[8];
          unpack8(reinterpret_cast<const uint4*>(dxr + (rows_routed + t) * dim)[c], v);
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[e] = acc[e] + v[e];
        }
#pragma unroll
        for (int j = 0; j < FMOE_MAX_TOPK; ++j) {
          if (j < k) {
            float v[8];
            unpack8(reinterpret_cast<const uint4*>(gate_w + static_cast<int64_t>(ch.e[j]) * dim)[c], v);
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[e] = fmaf(gl[j], v[e], acc[e]);
          }
        }
        float xv[8], w[8] = {1, 1, 1, 1, 1, 1, 1, 1};
        load8(x, x_dtype, t * dim + c * 8, xv);
        if (nw) load8(nw, w_dtype, c * 8, w);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          xh[i][e] = xv[e] * r;
          g[i][e] = acc[e] * w[e];
          s = s + g[i][e] * xh[i][e];
          pw[i][e] = pw[i][e] + acc[e] * xh[i][e];
        }
      }
    }
    const float m = wave_sum(s) / static_cast<float>(dim);
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = lane + 64 * i;
      if (c < chunks) {
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = r * (g[i][e] - xh[i][e] * m) + dov[i][e];
        store8(dx, x_dtype, t * dim + c * 8, o);
      }
    }
  }
  if (!parts) return;  // no norm weight gradient wanted (uniform branch)
  // This workgroup's partial row: waves add into LDS one after the other.
  for (int w = 0; w < kNormWaves; ++w) {
    if (wave == w) {
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        const int c = lane + 64 * i;
        if (c < chunks) {
#pragma unroll
          for (int e = 0; e < 8; ++e) red[c * 8 + e] = (w == 0 ? 0.0f : red[c * 8 + e]) + pw[i][e];
        }
      }
    }
    __syncthreads();
  }
  for (int c = threadIdx.x; c < dim; c += kNormThreads)
    parts[static_cast<int64_t>(blockIdx.x) * dim + c] = red[c];
}

// d_norm_w[c] = sum of the partial rows parts[p, c], as a fixed two-level
// tree: the kNormParts rows are split into kNormGroups groups of 64; in group
// g, wave w adds rows g*64 + w*16 .. +15 in order (16 independent loads in
// flight per lane), the 4 waves' sums are added in wave order into
// level2[g, c]; then the groups are added in order.  Rows past n_parts
// (fewer workgroups than kNormParts) count as zero.
constexpr int kNormGroups = kNormParts / 64;
constexpr int kNormRowsPerWave = kNormParts / (kNormGroups * kNormWaves);

__global__ __launch_bounds__(kNormThreads) void norm_parts_reduce_kernel(
    const float* __restrict__ parts, int n_parts, int dim, float* __restrict__ level2) {
  __shared__ float q[kNormWaves][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c = blockIdx.x * 64 + lane;
  const int p0 = (blockIdx.y * kNormWaves + wave) * kNormRowsPerWave;
  float v[kNormRowsPerWave];
#pragma unroll
  for (int i = 0; i < kNormRowsPerWave; ++i)
    v[i] = (c < dim && p0 + i < n_parts) ? parts[static_cast<int64_t>(p0 + i) * dim + c] : 0.0f;
  float s = v[0];
#pragma unroll
  for (int i = 1; i < kNormRowsPerWave; ++i) s = s + v[i];
  q[wave][lane] = s;
  __syncthreads();
  if (wave == 0 && c < dim) {
    float t = q[0][lane];
#pragma unroll
    for (int w = 1; w < kNormWaves; ++w) t = t + q[w][lane];
    level2[static_cast<int64_t>(blockIdx.y) * dim + c] = t;
  }
}

// Final level: out[c] = sum over the groups g (ascending) of level2[g, c];
// n_groups = 0 writes zeros.
__global__ __launch_bounds__(kNormThreads) void norm_weight_reduce_kernel(
    const float* __restrict__ level2, int n_groups, int dim, void* __restrict__ out, int out_dtype) {
  const int c = blockIdx.x * kNormThreads + threadIdx.x;
  if (c >= dim) return;
  float l2[kNormGroups];  // all loads in flight before the in-order sum
#pragma unroll
  for (int g = 0; g < kNormGroups; ++g) l2[g] = g < n_groups ? level2[static_cast<int64_t>(g) * dim + c] : 0.0f;
  float v = 0.0f;
#pragma unroll
  for (int g = 0; g < kNormGroups; ++g) v = v + l2[g];
  if (out_dtype == FMOE_BF16) static_cast<uint16_t*>(out)[c] = f2bf(v);
  else static_cast<float*>(out)[c] = v;
}

inline int norm_chunks_per_lane(int64_t dim) {
  const int64_t per = ceil_div(dim / 8, 64);
  return per <= 1 ? 1 : per <= 2 ? 2 : per <= 4 ? 4 : 8;
}

}  // namespace fmoe

using namespace fmoe;

extern "C" int fmoe_rmsnorm_fwd(const void* x, int x_dtype, const void* norm_w, int w_dtype,
                                int64_t T, int64_t dim, float eps, void* xn, float* rstd,
                                void* stream) {
  if (T < 0 || dim <= 0) return FMOE_ERR_INVALID_ARG;
  if (dim % 64 != 0 || dim > kNormMaxDim) return FMOE_ERR_SHAPE;
  if ((x_dtype != FMOE_BF16 && x_dtype != FMOE_F32) || (w_dtype != FMOE_BF16 && w_dtype != FMOE_F32))
    return FMOE_ERR_DTYPE;
  if (T == 0) return FMOE_OK;
  if (!x || !xn || !rstd) return FMOE_ERR_INVALID_ARG;
  if (!aligned16(x) || !aligned16(xn) || (norm_w && !aligned16(norm_w))) return FMOE_ERR_ALIGN;
  const dim3 grid(ceil_div(T, kNormWaves)), block(kNormThreads);
  hipStream_t s = as_stream(stream);
  uint16_t* o = static_cast<uint16_t*>(xn);
  switch (norm_chunks_per_lane(dim)) {
    case 1: rmsnorm_fwd_kernel<1><<<grid, block, 0, s>>>(x, x_dtype, norm_w, w_dtype, T, (int)dim, eps, o, rstd); break;
    case 2: rmsnorm_fwd_kernel<2><<<grid, block, 0, s>>>(x, x_dtype, norm_w, w_dtype, T, (int)dim, eps, o, rstd); break;
    case 4: rmsnorm_fwd_kernel<4><<<grid, block, 0, s>>>(x, x_dtype, norm_w, w_dtype, T, (int)dim, eps, o, rstd); break;
    default: rmsnorm_fwd_kernel<8><<<grid, block, 0, s>>>(x, x_dtype, norm_w, w_dtype, T, (int)dim, eps, o, rstd); break;
  }
  return launch_status();
}

extern "C" size_t fmoe_norm_bwd_workspace_bytes(int64_t dim) {
  return dim <= 0 ? 0
                  : static_cast<size_t>(kNormParts + kNormGroups) * static_cast<size_t>(dim) * sizeof(float);
}

extern "C" int fmoe_dx_reduce_norm(const void* dx_rows, const int32_t* pos_of_slot,
                                   const int32_t* idx, const float* d_logits, const void* gate_w,
                                   int64_t T, int64_t dim, int k, int64_t rows_routed,
                                   int has_shared, const void* x, const float* rstd,
                                   const void* norm_w, int w_dtype, const void* d_out, int x_dtype,
                                   void* dx, void* d_norm_w, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  if (T < 0 || dim <= 0 || rows_routed < 0) return FMOE_ERR_INVALID_ARG;
  if (k <= 0 || k > FMOE_MAX_TOPK || dim % 64 != 0 || dim > kNormMaxDim) return FMOE_ERR_SHAPE;
  if ((x_dtype != FMOE_BF16 && x_dtype != FMOE_F32) || (w_dtype != FMOE_BF16 && w_dtype != FMOE_F32))
    return FMOE_ERR_DTYPE;
  if (d_norm_w && !norm_w) return FMOE_ERR_INVALID_ARG;
  if (d_norm_w && workspace_bytes < fmoe_norm_bwd_workspace_bytes(dim)) return FMOE_ERR_WORKSPACE;
  if (T == 0) {
    if (!d_norm_w) return FMOE_OK;
    // No tokens: the norm weight's gradient is zero (a sum over no partial rows).
    norm_weight_reduce_kernel<<<dim3(ceil_div(dim, kNormThreads)), dim3(kNormThreads), 0, as_stream(stream)>>>(
        nullptr, 0, (int)dim, d_norm_w, w_dtype);
    return launch_status();
  }
  if (!dx_rows || !pos_of_slot || !idx || !d_logits || !gate_w || !x || !rstd || !d_out || !dx)
    return FMOE_ERR_INVALID_ARG;
  if (d_norm_w && !workspace) return FMOE_ERR_WORKSPACE;
  if (!aligned16(dx_rows) || !aligned16(gate_w) || !aligned16(x) || !aligned16(d_out) ||
      !aligned16(dx) || (norm_w && !aligned16(norm_w)))
    return FMOE_ERR_ALIGN;
  const int grid = static_cast<int>(std::min<int64_t>(ceil_div(T, kNormWaves), kNormParts));
  float* parts = d_norm_w ? static_cast<float*>(workspace) : nullptr;
  hipStream_t s = as_stream(stream);
  const uint16_t* dr = static_cast<const uint16_t*>(dx_rows);
  const uint16_t* gw = static_cast<const uint16_t*>(gate_w);
#define FMOE_NORM_BWD(N)                                                                        \
  dx_reduce_norm_kernel<N><<<dim3(grid), dim3(kNormThreads), 0, s>>>(                           \
      dr, pos_of_slot, idx, d_logits, gw, T, (int)dim, k, rows_routed, has_shared, x, rstd,     \
      norm_w, w_dtype, d_out, x_dtype, dx, parts)
  switch (norm_chunks_per_lane(dim)) {
    case 1: FMOE_NORM_BWD(1); break;
    case 2: FMOE_NORM_BWD(2); break;
    case 4: FMOE_NORM_BWD(4); break;
    default: FMOE_NORM_BWD(8); break;
  }
#undef FMOE_NORM_BWD
  if (d_norm_w) {
    float* level2 = parts + static_cast<int64_t>(kNormParts) * dim;
    norm_parts_reduce_kernel<<<dim3(ceil_div(dim, 64), kNormGroups), dim3(kNormThreads), 0, s>>>(
        parts, grid, (int)dim, level2);
    norm_weight_reduce_kernel<<<dim3(ceil_div(dim, kNormThreads)), dim3(kNormThreads), 0, s>>>(
        level2, kNormGroups, (int)dim, d_norm_w, w_dtype);
  }
  return launch_status();
}
