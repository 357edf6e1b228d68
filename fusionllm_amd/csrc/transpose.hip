// transpose.hip — transposed copies of the expert weights for the backward
// products of SwiGLUExpert (autograd of FusionLLM models/moe.py:21).
//
// The dX products of the backward multiply by the weights along their output
// dimension: dh = d_out * w2 (w2 is [dim, inter]) and
// dx = [da | db] * [w1; w3] ([w1; w3] is [2*inter, dim]).  The grouped GEMM
// streams both operands K-contiguous, so once per backward pass the weights
// are copied transposed:
//   w2t[g]  = w2[g]^T           [inter, dim]
//   w13t[g] = [w1[g]; w3[g]]^T  [dim, 2*inter]
// for every group g (routed experts, then the shared expert).  HBM-bound:
// 3 * 2 * dim * inter * 2 bytes per group, read once and written once.
#include "fmoe_common.h"

namespace fmoe {

constexpr int kTT = 64;          // tile edge (elements)
constexpr int kTPitch = kTT + 8;  // LDS row pitch (elements): keeps 16-byte rows aligned, spreads banks

struct TransposeArgs {
  const uint16_t* src[3 * (FMOE_MAX_EXPERTS + 1)];  // per group: w1, w3, w2
  int64_t dim, inter;
  uint16_t* w13t;
  uint16_t* w2t;
};

// One workgroup moves one 64 x 64 tile: 16-byte loads of source rows, 2-byte
// transposed writes into LDS, 16-byte reads and stores of destination rows.
__global__ __launch_bounds__(256) void transpose_weights_kernel(const TransposeArgs a, int tiles_per_mat) {
  __shared__ __attribute__((aligned(16))) uint16_t t[kTT * kTPitch];
  const int per_group = 3 * tiles_per_mat;
  const int g = blockIdx.x / per_group;
  const int rem = blockIdx.x - g * per_group;
  const int which = rem / tiles_per_mat;  // 0: w1, 1: w3, 2: w2
  const int tile = rem - which * tiles_per_mat;
  const int64_t dim = a.dim, inter = a.inter;
  // source matrix: w1/w3 are [inter, dim]; w2 is [dim, inter]
  const int64_t rows = which == 2 ? dim : inter;
  const int64_t cols = which == 2 ? inter : dim;
  const int tiles_c = static_cast<int>(cols / kTT);
  const int64_t r0 = static_cast<int64_t>(tile / tiles_c) * kTT;
  const int64_t c0 = static_cast<int64_t>(tile % tiles_c) * kTT;
  const uint16_t* src = a.src[3 * g + which];
  // destination: element (r, c) of the source goes to row c, column r (+ offset)
  uint16_t* dst;
  int64_t dpitch, dcol0;
  if (which == 2) {
    dst = a.w2t + static_cast<int64_t>(g) * inter * dim;
    dpitch = dim;
    dcol0 = 0;
  } else {
    dst = a.w13t + static_cast<int64_t>(g) * dim * 2 * inter;
    dpitch = 2 * inter;
    dcol0 = which == 1 ? inter : 0;
  }
  const int tid = threadIdx.x;
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int idx = p * 256 + tid;  // 512 chunks of 8 elements
    const int r = idx >> 3, ch = idx & 7;
    const uint4 v = *reinterpret_cast<const uint4*>(src + (r0 + r) * cols + c0 + ch * 8);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 8; ++e)
      t[(ch * 8 + e) * kTPitch + r] = static_cast<uint16_t>(w[e >> 1] >> ((e & 1) * 16));
  }
  __syncthreads();
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int idx = p * 256 + tid;
    const int c = idx >> 3, ch = idx & 7;  // destination row c, 8 source rows ch*8 ..
    const uint4 v = *reinterpret_cast<const uint4*>(&t[c * kTPitch + ch * 8]);
    *reinterpret_cast<uint4*>(dst + (c0 + c) * dpitch + dcol0 + r0 + ch * 8) = v;
  }
}

}  // namespace fmoe

using namespace fmoe;

extern "C" int fmoe_transpose_weights(const void* const* w1, const void* const* w3,
                                      const void* const* w2, int n_groups, int64_t dim,
                                      int64_t inter, void* w13t, void* w2t, void* stream) {
  if (n_groups <= 0 || n_groups > FMOE_MAX_EXPERTS + 1) return FMOE_ERR_TOO_MANY_EXPERTS;
  if (dim <= 0 || inter <= 0) return FMOE_ERR_INVALID_ARG;
  if (dim % 64 != 0 || inter % 64 != 0) return FMOE_ERR_SHAPE;
  if (!w1 || !w3 || !w2 || !w13t || !w2t) return FMOE_ERR_INVALID_ARG;
  if (!aligned16(w13t) || !aligned16(w2t)) return FMOE_ERR_ALIGN;
  TransposeArgs a = {};
  for (int g = 0; g < n_groups; ++g) {
    if (!w1[g] || !w3[g] || !w2[g]) return FMOE_ERR_INVALID_ARG;
    if (!aligned16(w1[g]) || !aligned16(w3[g]) || !aligned16(w2[g])) return FMOE_ERR_ALIGN;
    a.src[3 * g + 0] = static_cast<const uint16_t*>(w1[g]);
    a.src[3 * g + 1] = static_cast<const uint16_t*>(w3[g]);
    a.src[3 * g + 2] = static_cast<const uint16_t*>(w2[g]);
  }
  a.dim = dim;
  a.inter = inter;
  a.w13t = static_cast<uint16_t*>(w13t);
  a.w2t = static_cast<uint16_t*>(w2t);
  const int tiles_per_mat = static_cast<int>((dim / kTT) * (inter / kTT));
  const int64_t grid = static_cast<int64_t>(n_groups) * 3 * tiles_per_mat;
  transpose_weights_kernel<<<dim3(grid), dim3(256), 0, as_stream(stream)>>>(a, tiles_per_mat);
  return launch_status();
}
