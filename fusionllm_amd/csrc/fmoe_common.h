// fmoe_common.h — helpers shared by the gfx950 kernels of libfusionmoe.so.
//
// The whole library is compiled with -ffp-contract=off: every fused
// multiply-add in the kernels is an explicit fmaf(), so that the rounding
// steps are the ones written here (the router and the combine are
// reproduced bit-for-bit by the CPU oracle).  MFMA instructions are not
// affected by the flag.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/fusionmoe.h"

namespace fmoe {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// ---- bf16 <-> fp32 ---------------------------------------------------------
__device__ __forceinline__ float bf2f(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}
// Round-to-nearest-even (v_cvt_pk_bf16_f32 on gfx950), the rounding torch
// uses for .to(torch.bfloat16).
__device__ __forceinline__ uint16_t f2bf(float f) {
  __bf16 b = static_cast<__bf16>(f);
  return __builtin_bit_cast(uint16_t, b);
}
__device__ __forceinline__ float bf_round(float f) { return bf2f(f2bf(f)); }

// Round two floats to bf16 with one packed conversion (round to nearest
// even) and return them as floats.
__device__ __forceinline__ void bf_round2(float& x, float& y) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const bf16x2 r = __builtin_convertvector((f32x2){x, y}, bf16x2);
  const uint32_t u = __builtin_bit_cast(uint32_t, r);
  x = __uint_as_float(u << 16);
  y = __uint_as_float(u & 0xffff0000u);
}

// Unpack 8 bf16 held in a uint4 into floats.
__device__ __forceinline__ void unpack8(const uint4& v, float* f) {
  f[0] = __uint_as_float(v.x << 16); f[1] = __uint_as_float(v.x & 0xffff0000u);
  f[2] = __uint_as_float(v.y << 16); f[3] = __uint_as_float(v.y & 0xffff0000u);
  f[4] = __uint_as_float(v.z << 16); f[5] = __uint_as_float(v.z & 0xffff0000u);
  f[6] = __uint_as_float(v.w << 16); f[7] = __uint_as_float(v.w & 0xffff0000u);
}
// Two floats to a bf16 pair with one v_cvt_pk_bf16_f32 (round to nearest
// even, as f2bf; two scalar conversions and the shift and or to join them
// took four instructions).
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, bf16x2));
}
__device__ __forceinline__ uint4 pack8(const float* f) {
  uint4 v;
  v.x = pack2(f[0], f[1]); v.y = pack2(f[2], f[3]);
  v.z = pack2(f[4], f[5]); v.w = pack2(f[6], f[7]);
  return v;
}

// ---- wave scans -------------------------------------------------------------
// Inclusive prefix sum over the 64 lanes of a wave.
__device__ __forceinline__ int wave_incl_scan(int v, int lane) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int u = __shfl_up(v, off, 64);
    if (lane >= off) v += u;
  }
  return v;
}

// Expert offsets of a counting sort from per-wave counts (E <= 64):
// start[q] = sum over experts q' < q of sum_w wcount[w][q'], start[E] = the
// total.  Wave 0 does it: lane q adds its expert's W wave counts (independent
// LDS reads), then one exclusive scan over the lanes (a single thread walking
// E x W counts waited for each LDS read in turn: about 3 us at E = 8, W = 8).
template <int W>
__device__ __forceinline__ void scan_wave_counts(const int (*wcount)[FMOE_MAX_EXPERTS], int E, int* start) {
  if (threadIdx.x < 64) {
    const int q = threadIdx.x;
    int t = 0;
    if (q < E)
#pragma unroll
      for (int w = 0; w < W; ++w) t += wcount[w][q];
    const int incl = wave_incl_scan(t, q);
    if (q < E) start[q] = incl - t;
    if (q == 63) start[E] = incl;
  }
}

// ---- exp and sigmoid for the router ----------------------------------------
// e^x by Cody-Waite range reduction x = n*ln2 + r (|r| <= ln2/2) and the
// degree-7 Taylor polynomial of e^r (truncation error < 6e-9 relative), then
// an exact scaling by 2^n done in two halves so that denormal results are
// formed correctly.  Written with explicit fmaf so the CPU oracle
// (oracle/router_ref.c) evaluates the identical sequence.
__host__ __device__ __forceinline__ float fm_pow2i(int n) {  // 2^n, -126 <= n <= 127
  return __uint_as_float(static_cast<uint32_t>(n + 127) << 23);
}
__device__ __forceinline__ float fm_expf(float x) {
  if (x != x) return x;
  if (x > 88.72283935546875f) return __uint_as_float(0x7f800000u);
  if (x < -103.97208404541016f) return 0.0f;
  const float n = rintf(x * 1.4426950216293335f);
  float r = fmaf(n, -0.693145751953125f, x);
  r = fmaf(n, -1.4286067653302598e-06f, r);
  float p = 1.0f / 5040.0f;
  p = fmaf(p, r, 1.0f / 720.0f);
  p = fmaf(p, r, 1.0f / 120.0f);
  p = fmaf(p, r, 1.0f / 24.0f);
  p = fmaf(p, r, 1.0f / 6.0f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  const int ni = static_cast<int>(n);
  const int n1 = ni / 2;
  const int n2 = ni - n1;
  return (p * fm_pow2i(n1)) * fm_pow2i(n2);
}
__device__ __forceinline__ float fm_sigmoid(float l) { return 1.0f / (1.0f + fm_expf(-l)); }

// Fast sigmoid for the SwiGLU epilogues (the result is rounded to bf16, so a
// few fp32 ulps do not matter): v_exp_f32 computes 2^x, v_rcp_f32 1/x (1 ulp).
__device__ __forceinline__ float fast_sigmoid(float a) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-a * 1.4426950408889634f));
}

// Top-k order: a beats b if a is NaN and b is not, or a > b.  Scanning experts
// in ascending order and replacing only on a strict win keeps ties on the
// lowest index.
__device__ __forceinline__ bool score_beats(float a, float b) {
  const bool an = a != a, bn = b != b;
  if (an || bn) return an && !bn;
  return a > b;
}

// Token of a routed slot, floor(n / k) for 0 <= n < 2^29 and 1 <= k <= 8,
// without a division: the high half of n * m with m = ceil(2^32 / k).  With
// m k = 2^32 + e, 0 <= e < k, n m / 2^32 = n / k + n e / (k 2^32); the
// excess stays below 1 / k (n e < 2^32), and the fraction of n / k is at most
// (k - 1) / k, so the floor is exact.  m = 2^32 (k = 1) does not fit 32 bits:
// magic holds m mod 2^32 and the product adds n * (m >> 32), with no branch.
inline uint64_t slot_div_magic(int k) { return ((uint64_t(1) << 32) + k - 1) / k; }
__device__ __forceinline__ uint32_t slot_token(uint32_t n, uint64_t magic) {
  return __umulhi(n, static_cast<uint32_t>(magic)) + n * static_cast<uint32_t>(magic >> 32);
}

// ---- status helpers (host) --------------------------------------------------
inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? FMOE_OK : FMOE_ERR_LAUNCH;
}
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }
inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Tokens per router workgroup, which are also the dispatch blocks of
// fmoe_route_and_dispatch; and its routing launch (router.hip).
constexpr int kRouteBlockTokens = 32;
int launch_router_hist(const uint16_t* xs, const uint16_t* ws, const uint16_t* bs, int64_t T, int64_t dim,
                       int n_experts, int k, float route_scale, int32_t* idx, int64_t* idx64, float* weights,
                       float* topv, int32_t* block_hist, hipStream_t s);

}  // namespace fmoe
