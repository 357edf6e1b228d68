// cast.hip — bf16 copies of several fp32 tensors in one launch.
//
// Under the trainer's bf16 autocast (FusionLLM training/trainer.py:158) every
// nn.Linear of the MoE block casts its fp32 weight to bf16 before the product
// (models/moe.py:16-18 for the experts, moe.py:36,46 for the gate), one cast
// kernel per weight; the module instead casts the block input, the gate and
// all expert weights with one launch.  Round to nearest even, the rounding of
// torch's .to(torch.bfloat16), so the copies are bit-identical to torch's.
#include "fmoe_common.h"

namespace fmoe {

constexpr int kCastThreads = 256;
constexpr int kCastPerBlock = kCastThreads * 8;  // 8 values per thread

struct CastArgs {
  const float* src[FMOE_MAX_CAST];
  uint16_t* dst[FMOE_MAX_CAST];
  int64_t n[FMOE_MAX_CAST];
  int64_t block_start[FMOE_MAX_CAST + 1];  // prefix sums of the blocks per tensor
  int count;
};

__global__ __launch_bounds__(kCastThreads) void cast_bf16_kernel(const CastArgs a) {
  const int64_t b = blockIdx.x;
  int t = 0;
  while (t + 1 < a.count && a.block_start[t + 1] <= b) ++t;
  const int64_t n = a.n[t];
  const int64_t i0 = (b - a.block_start[t]) * kCastPerBlock + static_cast<int64_t>(threadIdx.x) * 8;
  if (i0 + 8 <= n) {
    const float4* s = reinterpret_cast<const float4*>(a.src[t] + i0);
    const float4 u = s[0], v = s[1];
    const float f[8] = {u.x, u.y, u.z, u.w, v.x, v.y, v.z, v.w};
    *reinterpret_cast<uint4*>(a.dst[t] + i0) = pack8(f);
  } else {
    for (int64_t i = i0; i < n; ++i) a.dst[t][i] = f2bf(a.src[t][i]);
  }
}

}  // namespace fmoe

using namespace fmoe;

extern "C" int fmoe_cast_bf16(const void* const* src, void* const* dst, const int64_t* n, int n_tensors,
                              void* stream) {
  if (n_tensors < 0 || n_tensors > FMOE_MAX_CAST) return FMOE_ERR_INVALID_ARG;
  if (n_tensors == 0) return FMOE_OK;
  if (!src || !dst || !n) return FMOE_ERR_INVALID_ARG;
  CastArgs a = {};
  int64_t blocks = 0;
  for (int i = 0; i < n_tensors; ++i) {
    if (n[i] < 0) return FMOE_ERR_INVALID_ARG;
    if (n[i] > 0 && (!src[i] || !dst[i])) return FMOE_ERR_INVALID_ARG;
    if (!aligned16(src[i]) || !aligned16(dst[i])) return FMOE_ERR_ALIGN;
    a.src[i] = static_cast<const float*>(src[i]);
    a.dst[i] = static_cast<uint16_t*>(dst[i]);
    a.n[i] = n[i];
    a.block_start[i] = blocks;
    blocks += ceil_div(n[i], kCastPerBlock);
  }
  a.block_start[n_tensors] = blocks;
  a.count = n_tensors;
  if (blocks == 0) return FMOE_OK;
  cast_bf16_kernel<<<dim3(blocks), dim3(kCastThreads), 0, as_stream(stream)>>>(a);
  return launch_status();
}
