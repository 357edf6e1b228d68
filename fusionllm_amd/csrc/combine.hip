// combine.hip — deterministic weighted combine (forward), its backward, and
// the per-token reduction of the input gradient.
//
// Forward replaces y.index_add_(0, token_ids, (expert_out * w).to(fp32)) in
// ascending expert order (FusionLLM models/moe.py:65-76), y.to(x.dtype)
// (moe.py:77) and y_routed + y_shared (moe.py:87).  Instead of scattering
// with atomics, every token gathers its k expert rows (through pos_of_slot)
// and adds them in ascending expert index, each product rounded to fp32
// before the add, which is the reference's rounding sequence.
#include "fmoe_common.h"
#include "choices.h"

namespace fmoe {

// One thread per (token, 8-column chunk).
__global__ __launch_bounds__(256) void combine_fwd_kernel(
    const uint16_t* __restrict__ eo, const int32_t* __restrict__ idx,
    const float* __restrict__ weights, const int32_t* __restrict__ pos_of_slot, int64_t T,
    int dim, int k, int64_t rows_routed, int has_shared, int out_dtype,
    const void* __restrict__ residual, void* __restrict__ y) {
  const int chunks = dim / 8;
  const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (g >= T * chunks) return;
  const int64_t t = g / chunks;
  const int c = static_cast<int>(g - t * chunks);
  Choices ch;
  load_sorted_choices(idx, pos_of_slot, weights, t, k, ch);
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int j = 0; j < FMOE_MAX_TOPK; ++j) {
    if (j < k) {
      float of[8];
      unpack8(reinterpret_cast<const uint4*>(eo + static_cast<int64_t>(ch.pos[j]) * dim)[c], of);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = acc[i] + of[i] * ch.w[j];
    }
  }
  float sh[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  if (has_shared) unpack8(reinterpret_cast<const uint4*>(eo + (rows_routed + t) * dim)[c], sh);
  if (out_dtype == FMOE_BF16) {
    float r[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = bf_round(acc[i]) + sh[i];
    if (residual) {
      // x + moe(x'): the block output rounded to bf16, then the bf16 add.
      float xr[8];
      unpack8(reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(residual) + t * dim)[c], xr);
#pragma unroll
      for (int i = 0; i < 8; ++i) r[i] = xr[i] + bf_round(r[i]);
    }
    reinterpret_cast<uint4*>(static_cast<uint16_t*>(y) + t * dim)[c] = pack8(r);
  } else {
    float r[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = acc[i] + sh[i];
    if (residual) {
      const float4* xp = reinterpret_cast<const float4*>(static_cast<const float*>(residual) + t * dim + c * 8);
      const float4 a = xp[0], b = xp[1];
      const float xr[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int i = 0; i < 8; ++i) r[i] = xr[i] + r[i];
    }
    float* yo = static_cast<float*>(y) + t * dim + c * 8;
    reinterpret_cast<float4*>(yo)[0] = make_float4(r[0], r[1], r[2], r[3]);
    reinterpret_cast<float4*>(yo)[1] = make_float4(r[4], r[5], r[6], r[7]);
  }
}

// One wave per routed row r: reads dy[t] and o[r], writes d_o[r] and the
// weight gradient of slot perm[r] (lane-strided partial sums, then a fixed
// xor butterfly).
__global__ __launch_bounds__(256) void combine_bwd_kernel(
    const void* __restrict__ dy, int dy_dtype, const uint16_t* __restrict__ eo,
    const float* __restrict__ weights, const int32_t* __restrict__ perm, int64_t n_rows, int dim,
    int k, uint16_t* __restrict__ d_eo, float* __restrict__ d_w) {
  const int lane = threadIdx.x & 63;
  const int64_t r = static_cast<int64_t>(blockIdx.x) * (blockDim.x / 64) + (threadIdx.x >> 6);
  if (r >= n_rows) return;
  const int slot = perm[r];
  const int64_t t = slot / k;
  const float w = weights[slot];
  const int chunks = dim / 8;
  float part = 0.0f;
  // two chunks per lane and pass (lane, lane + 64), both rows' loads issued
  // before either is used; the sums keep the chunk order of the lane
  for (int c0 = lane; c0 < chunks; c0 += 128) {
    const int c1 = c0 + 64;
    const bool has1 = c1 < chunks;
    const int cc[2] = {c0, has1 ? c1 : c0};
    float g[2][8], of[2][8];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int c = cc[q];
      if (dy_dtype == FMOE_BF16) {
        unpack8(reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(dy) + t * dim)[c], g[q]);
      } else {
        const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(dy) + t * dim + c * 8);
        const float4 a = p[0], b = p[1];
        g[q][0] = a.x; g[q][1] = a.y; g[q][2] = a.z; g[q][3] = a.w;
        g[q][4] = b.x; g[q][5] = b.y; g[q][6] = b.z; g[q][7] = b.w;
      }
      unpack8(reinterpret_cast<const uint4*>(eo + r * dim)[c], of[q]);
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      if (q == 1 && !has1) break;
      float d[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        d[i] = g[q][i] * w;
        part = part + g[q][i] * of[q][i];
      }
      reinterpret_cast<uint4*>(d_eo + r * dim)[cc[q]] = pack8(d);
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) part = part + __shfl_xor(part, off, 64);
  if (lane == 0) d_w[slot] = part;
}

// One thread per (token, 8-column chunk).
__global__ __launch_bounds__(256) void dx_reduce_kernel(
    const uint16_t* __restrict__ dxr, const int32_t* __restrict__ pos_of_slot,
    const int32_t* __restrict__ idx, const float* __restrict__ dl,
    const uint16_t* __restrict__ gate_w, int64_t T, int dim, int k, int64_t rows_routed,
    int has_shared, int out_dtype, void* __restrict__ dx) {
  const int chunks = dim / 8;
  const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (g >= T * chunks) return;
  const int64_t t = g / chunks;
  const int c = static_cast<int>(g - t * chunks);
  Choices ch;
  load_sorted_choices(idx, pos_of_slot, nullptr, t, k, ch);
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int j = 0; j < FMOE_MAX_TOPK; ++j) {
    if (j < k) {
      float v[8];
      unpack8(reinterpret_cast<const uint4*>(dxr + static_cast<int64_t>(ch.pos[j]) * dim)[c], v);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = acc[i] + v[i];
    }
  }
  if (has_shared) {
    float v[8];
    unpack8(reinterpret_cast<const uint4*>(dxr + (rows_routed + t) * dim)[c], v);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = acc[i] + v[i];
  }
#pragma unroll
  for (int j = 0; j < FMOE_MAX_TOPK; ++j) {
    if (j < k) {
      const float gl = dl[t * k + ch.slot[j]];
      float v[8];
      unpack8(reinterpret_cast<const uint4*>(gate_w + static_cast<int64_t>(ch.e[j]) * dim)[c], v);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = fmaf(gl, v[i], acc[i]);
    }
  }
  if (out_dtype == FMOE_BF16) {
    reinterpret_cast<uint4*>(static_cast<uint16_t*>(dx) + t * dim)[c] = pack8(acc);
  } else {
    float* o = static_cast<float*>(dx) + t * dim + c * 8;
    reinterpret_cast<float4*>(o)[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
    reinterpret_cast<float4*>(o)[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
  }
}

}  // namespace fmoe

using namespace fmoe;

extern "C" int fmoe_combine_fwd(const void* expert_out, const int32_t* idx, const float* weights,
                                const int32_t* pos_of_slot, int64_t T, int64_t dim, int k,
                                int64_t rows_routed, int has_shared, int out_dtype,
                                const void* residual, void* y, void* stream) {
  if (T < 0 || dim <= 0 || rows_routed < 0) return FMOE_ERR_INVALID_ARG;
  if (k <= 0 || k > FMOE_MAX_TOPK || dim % 64 != 0) return FMOE_ERR_SHAPE;
  if (out_dtype != FMOE_BF16 && out_dtype != FMOE_F32) return FMOE_ERR_DTYPE;
  if (T == 0) return FMOE_OK;
  if (!expert_out || !idx || !weights || !pos_of_slot || !y) return FMOE_ERR_INVALID_ARG;
  if (!aligned16(expert_out) || !aligned16(y) || (residual && !aligned16(residual)))
    return FMOE_ERR_ALIGN;
  const int64_t total = T * (dim / 8);
  combine_fwd_kernel<<<dim3(ceil_div(total, 256)), dim3(256), 0, as_stream(stream)>>>(
      static_cast<const uint16_t*>(expert_out), idx, weights, pos_of_slot, T, (int)dim, k,
      rows_routed, has_shared, out_dtype, residual, y);
  return launch_status();
}

extern "C" int fmoe_combine_bwd(const void* dy, int dy_dtype, const void* expert_out,
                                const float* weights, const int32_t* perm, int64_t T, int64_t dim,
                                int k, void* d_expert_out, float* d_weights, void* stream) {
  if (T < 0 || dim <= 0) return FMOE_ERR_INVALID_ARG;
  if (k <= 0 || k > FMOE_MAX_TOPK || dim % 64 != 0) return FMOE_ERR_SHAPE;
  if (dy_dtype != FMOE_BF16 && dy_dtype != FMOE_F32) return FMOE_ERR_DTYPE;
  if (T == 0) return FMOE_OK;
  if (!dy || !expert_out || !weights || !perm || !d_expert_out || !d_weights)
    return FMOE_ERR_INVALID_ARG;
  if (!aligned16(dy) || !aligned16(expert_out) || !aligned16(d_expert_out)) return FMOE_ERR_ALIGN;
  const int64_t rows = T * k;
  combine_bwd_kernel<<<dim3(ceil_div(rows, 4)), dim3(256), 0, as_stream(stream)>>>(
      dy, dy_dtype, static_cast<const uint16_t*>(expert_out), weights, perm, rows, (int)dim, k,
      static_cast<uint16_t*>(d_expert_out), d_weights);
  return launch_status();
}

extern "C" int fmoe_dx_reduce(const void* dx_rows, const int32_t* pos_of_slot, const int32_t* idx,
                              const float* d_logits, const void* gate_w, int64_t T, int64_t dim,
                              int k, int64_t rows_routed, int has_shared, int out_dtype, void* dx,
                              void* stream) {
  if (T < 0 || dim <= 0 || rows_routed < 0) return FMOE_ERR_INVALID_ARG;
  if (k <= 0 || k > FMOE_MAX_TOPK || dim % 64 != 0) return FMOE_ERR_SHAPE;
  if (out_dtype != FMOE_BF16 && out_dtype != FMOE_F32) return FMOE_ERR_DTYPE;
  if (T == 0) return FMOE_OK;
  if (!dx_rows || !pos_of_slot || !idx || !d_logits || !gate_w || !dx) return FMOE_ERR_INVALID_ARG;
  if (!aligned16(dx_rows) || !aligned16(gate_w) || !aligned16(dx)) return FMOE_ERR_ALIGN;
  const int64_t total = T * (dim / 8);
  dx_reduce_kernel<<<dim3(ceil_div(total, 256)), dim3(256), 0, as_stream(stream)>>>(
      static_cast<const uint16_t*>(dx_rows), pos_of_slot, idx, d_logits,
      static_cast<const uint16_t*>(gate_w), T, (int)dim, k, rows_routed, has_shared, out_dtype, dx);
  return launch_status();
}
