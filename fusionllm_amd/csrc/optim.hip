// optim.hip — fused NorMuon step for the weight matrices (FusionLLM
// training/optimizer.py:11-58, NorMuon.step), many tensors per launch.
//
// Per element, in the order and with the rounding of the reference's tensor
// operations (each result rounded to the parameter dtype T, arithmetic in
// fp32; "a + s*b" forms as one fused multiply-add):
//   m = T(T(m*b1) + (1-b1)*g)                     exp_avg.mul_(b1).add_(g, alpha=1-b1)
//   v = T(T(v*b2) + (1-b2)*g*g)                   exp_avg_sq.mul_(b2).addcmul_(g, g, value=1-b2)
//   den = T(T(T(sqrt(v)) * i2) + eps)             (exp_avg_sq.sqrt() / bias_corr2**0.5).add_(eps)
//   u = T(T(m * i1) / den)                        exp_avg / bias_corr1 / denom
// matrices (ndim >= 2), per row of the last dimension:
//   r = T(T(T(||u||_2) * ir) + eps), u = T(u / r)  row_norm / (C**0.5 + eps); update / (row_rms + eps)
// A tensor divided by a Python number runs on the GPU as a multiplication by
// the fp32 reciprocal formed on the host (torch's div_true kernel for a CPU
// scalar divisor: inv = 1.0f / float(b)); i1, i2 and ir are those
// reciprocals.  Tensor-by-tensor divisions stay true divisions.
// weight decay (wd > 0): cautious and matrix: p = T(p * T(1 - T(lr*wd*[T(g*p) > 0])))
//                         otherwise:          p = T(p * (1 - lr*wd))
//   p = T(p - lr*u)                               p.add_(update, alpha=-lr)
// One wave per row (a vector counts as one row); the row norm is a sum of
// squares in a fixed lane order, so the step is deterministic.
#include <cmath>

#include "fmoe_common.h"

namespace fmoe {

constexpr int kOptMaxTensors = 32;
constexpr int kOptMaxCols = 4096;  // a row lives in registers: 64 values per lane

struct NormuonArgs {
  void* p[kOptMaxTensors];
  const void* g[kOptMaxTensors];
  void* m[kOptMaxTensors];
  void* v[kOptMaxTensors];
  int row_start[kOptMaxTensors + 1];  // prefix sums of the row counts
  int cols[kOptMaxTensors];
  int matrix[kOptMaxTensors];         // ndim >= 2: row norm and cautious decay
  float inv_rms[kOptMaxTensors];      // 1.0f / float(sqrt(cols) + eps), sqrt(cols) + eps in double
  int n;
  int dtype;
  // The reference's Python scalars as its tensor operations see them: each
  // formed in double on the host, then converted to fp32.
  float b1, om1, b2, om2;      // beta1, 1 - beta1, beta2, 1 - beta2
  float eps, inv_bc1, inv_bc2s;  // eps, 1.0f / float(bias_corr1), 1.0f / float(sqrt(bias_corr2))
  float neg_lr, lrwd, decay;   // -lr, lr * wd, 1 - lr * wd
  int decay_on, cautious;      // wd > 0; cautious_wd
};

template <int DT>
__device__ __forceinline__ float rnd(float x) {
  if constexpr (DT == FMOE_BF16) return bf_round(x);
  return x;
}

// 4 consecutive elements of a row, as floats.
template <int DT>
__device__ __forceinline__ void ld4(const void* base, int64_t e, float* f) {
  if constexpr (DT == FMOE_BF16) {
    const uint2 u = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(base) + e);
    f[0] = __uint_as_float(u.x << 16); f[1] = __uint_as_float(u.x & 0xffff0000u);
    f[2] = __uint_as_float(u.y << 16); f[3] = __uint_as_float(u.y & 0xffff0000u);
  } else {
    const float4 u = *reinterpret_cast<const float4*>(static_cast<const float*>(base) + e);
    f[0] = u.x; f[1] = u.y; f[2] = u.z; f[3] = u.w;
  }
}
template <int DT>
__device__ __forceinline__ void st4(void* base, int64_t e, const float* f) {
  if constexpr (DT == FMOE_BF16) {
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(base) + e) = make_uint2(pack2(f[0], f[1]), pack2(f[2], f[3]));
  } else {
    *reinterpret_cast<float4*>(static_cast<float*>(base) + e) = make_float4(f[0], f[1], f[2], f[3]);
  }
}

template <int DT, int NCH>  // NCH: 4-element chunks per lane, NCH * 256 >= cols
__global__ __launch_bounds__(256) void normuon_kernel(const NormuonArgs a) {
  const int lane = threadIdx.x & 63;
  const int row = static_cast<int>(blockIdx.x) * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (row >= a.row_start[a.n]) return;
  int t = 0;
  while (t + 1 < a.n && a.row_start[t + 1] <= row) ++t;
  const int C = a.cols[t];
  const int64_t base = static_cast<int64_t>(row - a.row_start[t]) * C;
  const int nq = C / 4;
  float u[NCH][4], gg[NCH][4], pp[NCH][4];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int q = lane + 64 * i;
    if (q < nq) {
      const int64_t e = base + 4 * q;
      float m[4], v[4];
      ld4<DT>(a.g[t], e, gg[i]);
      ld4<DT>(a.p[t], e, pp[i]);
      ld4<DT>(a.m[t], e, m);
      ld4<DT>(a.v[t], e, v);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float g = gg[i][j];
        m[j] = rnd<DT>(fmaf(a.om1, g, rnd<DT>(m[j] * a.b1)));
        v[j] = rnd<DT>(fmaf(a.om2 * g, g, rnd<DT>(v[j] * a.b2)));
        const float den = rnd<DT>(rnd<DT>(rnd<DT>(sqrtf(v[j])) * a.inv_bc2s) + a.eps);
        u[i][j] = rnd<DT>(rnd<DT>(m[j] * a.inv_bc1) / den);
        ss = fmaf(u[i][j], u[i][j], ss);
      }
      st4<DT>(a.m[t], e, m);
      st4<DT>(a.v[t], e, v);
    }
  }
  float rd = 1.0f;
  const bool matrix = a.matrix[t] != 0;
  if (matrix) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) ss = ss + __shfl_xor(ss, off, 64);
    const float nrm = rnd<DT>(sqrtf(ss));
    rd = rnd<DT>(rnd<DT>(nrm * a.inv_rms[t]) + a.eps);
  }
  const bool cautious = a.cautious && matrix;
  const float lrwd_t = rnd<DT>(a.lrwd);
  const float fac_on = rnd<DT>(1.0f - lrwd_t);
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int q = lane + 64 * i;
    if (q < nq) {
      float p[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float uu = matrix ? rnd<DT>(u[i][j] / rd) : u[i][j];
        float pv = pp[i][j];
        if (a.decay_on) {
          if (cautious) pv = rnd<DT>(pv * (rnd<DT>(gg[i][j] * pv) > 0.0f ? fac_on : 1.0f));
          else pv = rnd<DT>(pv * a.decay);
        }
        p[j] = rnd<DT>(fmaf(a.neg_lr, uu, pv));
      }
      st4<DT>(a.p[t], base + 4 * q, p);
    }
  }
}

}  // namespace fmoe

using namespace fmoe;

extern "C" int fmoe_normuon_step(void* const* params, const void* const* grads, void* const* exp_avgs,
                                 void* const* exp_avg_sqs, const int64_t* rows, const int64_t* cols,
                                 const int* is_matrix, int n_tensors, int dtype, double lr, double beta1,
                                 double beta2, double eps, double weight_decay, int cautious,
                                 double bias_corr1, double bias_corr2, void* stream) {
  if (n_tensors < 0 || n_tensors > kOptMaxTensors) return FMOE_ERR_INVALID_ARG;
  if (dtype != FMOE_BF16 && dtype != FMOE_F32) return FMOE_ERR_DTYPE;
  if (n_tensors == 0) return FMOE_OK;
  if (!params || !grads || !exp_avgs || !exp_avg_sqs || !rows || !cols || !is_matrix)
    return FMOE_ERR_INVALID_ARG;
  NormuonArgs a = {};
  int64_t total = 0;
  int max_cols = 0;
  for (int i = 0; i < n_tensors; ++i) {
    if (rows[i] < 0 || cols[i] <= 0) return FMOE_ERR_INVALID_ARG;
    if (cols[i] % 4 != 0 || cols[i] > kOptMaxCols) return FMOE_ERR_SHAPE;
    if (!params[i] || !grads[i] || !exp_avgs[i] || !exp_avg_sqs[i]) return FMOE_ERR_INVALID_ARG;
    const size_t al = dtype == FMOE_BF16 ? 8 : 16;
    for (const void* q : {static_cast<const void*>(params[i]), grads[i], static_cast<const void*>(exp_avgs[i]),
                          static_cast<const void*>(exp_avg_sqs[i])})
      if (reinterpret_cast<uintptr_t>(q) % al != 0) return FMOE_ERR_ALIGN;
    a.p[i] = params[i];
    a.g[i] = grads[i];
    a.m[i] = exp_avgs[i];
    a.v[i] = exp_avg_sqs[i];
    a.row_start[i] = static_cast<int>(total);
    a.cols[i] = static_cast<int>(cols[i]);
    a.matrix[i] = is_matrix[i] != 0;
    a.inv_rms[i] = 1.0f / static_cast<float>(std::sqrt(static_cast<double>(cols[i])) + eps);
    total += rows[i];
    if (total > INT32_MAX / 2) return FMOE_ERR_SHAPE;
    max_cols = cols[i] > max_cols ? static_cast<int>(cols[i]) : max_cols;
  }
  a.row_start[n_tensors] = static_cast<int>(total);
  a.n = n_tensors;
  a.dtype = dtype;
  a.b1 = static_cast<float>(beta1);
  a.om1 = static_cast<float>(1.0 - beta1);
  a.b2 = static_cast<float>(beta2);
  a.om2 = static_cast<float>(1.0 - beta2);
  a.eps = static_cast<float>(eps);
  a.inv_bc1 = 1.0f / static_cast<float>(bias_corr1);
  a.inv_bc2s = 1.0f / static_cast<float>(std::sqrt(bias_corr2));
  a.neg_lr = static_cast<float>(-lr);
  a.lrwd = static_cast<float>(lr * weight_decay);
  a.decay = static_cast<float>(1.0 - lr * weight_decay);
  a.decay_on = weight_decay > 0.0;
  a.cautious = cautious;
  if (total == 0) return FMOE_OK;
  const dim3 grid(ceil_div(total, 4)), block(256);
  hipStream_t s = as_stream(stream);
  const int nch = static_cast<int>(ceil_div(max_cols / 4, 64));
#define FMOE_NORMUON(DT, N) normuon_kernel<DT, N><<<grid, block, 0, s>>>(a)
#define FMOE_NORMUON_DT(DT)                        \
  do {                                            \
    if (nch <= 1) FMOE_NORMUON(DT, 1);            \
    else if (nch <= 2) FMOE_NORMUON(DT, 2);       \
    else if (nch <= 4) FMOE_NORMUON(DT, 4);       \
    else if (nch <= 8) FMOE_NORMUON(DT, 8);       \
    else FMOE_NORMUON(DT, 16);                    \
  } while (0)
  if (dtype == FMOE_BF16) FMOE_NORMUON_DT(FMOE_BF16);
  else FMOE_NORMUON_DT(FMOE_F32);
#undef FMOE_NORMUON_DT
#undef FMOE_NORMUON
  return launch_status();
}
