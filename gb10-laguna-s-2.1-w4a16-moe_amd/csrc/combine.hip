// Top-k combine: out[m, k] = bf16( sum_{t=0..topk-1} partial[m*topk+t, k] ).
//
// Reference: _moe_sum_kernel (kernels/w4a16_moe.py:637-670) sums the bf16
// partials (the buffer of :311) in slot order t = 0..topk-1 with an fp32
// accumulator; for M <= 4 it uses fp32 atomics into [M, K] instead
// (:618-625, :763-766), whose order is not fixed.  Here the partials (already
// multiplied by the routing weight) are bf16 like the reference's, or fp32 for
// calls with M <= 4, the sum is always in slot order from +0.0, and pairs
// routed to an expert id outside [0, E) -- which the sort skipped, so their
// partial row was never written -- are left out.  The result is bitwise
// reproducible.
#include "common.hpp"

namespace w4a16 {
namespace {

// Four consecutive partial values of row `row` starting at element 4*k4.
template <bool BF16>
__device__ __forceinline__ float4 load4(const void* partial, int64_t row, int K, int k4) {
  if constexpr (BF16) {
    const uint2 v = reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(partial) +
                                                   row * K)[k4];
    return make_float4(bf16_to_f32(v.x & 0xFFFFu), bf16_to_f32(v.x >> 16),
                       bf16_to_f32(v.y & 0xFFFFu), bf16_to_f32(v.y >> 16));
  } else {
    return reinterpret_cast<const float4*>(static_cast<const float*>(partial) + row * K)[k4];
  }
}

template <bool VEC_STORE, bool BF16>
__global__ __launch_bounds__(256) void combine_kernel(const CombineLaunch a) {
  const int kchunks = (a.K / 4 + 255) / 256;
  const int m = blockIdx.x / kchunks;
  const int k4 = (blockIdx.x - m * kchunks) * 256 + threadIdx.x;  // 4 outputs
  if (k4 * 4 >= a.K) return;
  const int64_t row0 = (int64_t)m * a.topk;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int t = 0; t < a.topk; ++t) {
    const int e = a.ids[row0 + t];
    if (e >= 0 && e < a.num_experts) {
      const float4 v = load4<BF16>(a.partial, row0 + t, a.K, k4);
      acc.x += v.x;
      acc.y += v.y;
      acc.z += v.z;
      acc.w += v.w;
    }
  }
  uint16_t* o = a.out + (int64_t)m * a.ld_out + 4 * k4;
  const uint32_t b0 = f32_to_bf16(acc.x), b1 = f32_to_bf16(acc.y);
  const uint32_t b2 = f32_to_bf16(acc.z), b3 = f32_to_bf16(acc.w);
  if (VEC_STORE) {
    *reinterpret_cast<uint2*>(o) = make_uint2(b0 | (b1 << 16), b2 | (b3 << 16));
  } else {
    o[0] = (uint16_t)b0;
    o[1] = (uint16_t)b1;
    o[2] = (uint16_t)b2;
    o[3] = (uint16_t)b3;
  }
}

template <bool BF16>
void launch_combine_t(const CombineLaunch& a, dim3 grid, bool vec, hipStream_t stream) {
  if (vec)
    hipLaunchKernelGGL((combine_kernel<true, BF16>), grid, dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((combine_kernel<false, BF16>), grid, dim3(256), 0, stream, a);
}

}  // namespace

hipError_t launch_combine(const CombineLaunch& a, hipStream_t stream) {
  if (a.M <= 0) return hipSuccess;
  const int64_t kchunks = (a.K / 4 + 255) / 256;
  const dim3 grid((unsigned)(kchunks * a.M));
  const bool vec = (reinterpret_cast<uintptr_t>(a.out) % 8 == 0) && (a.ld_out % 4 == 0);
  if (a.partial_bf16)
    launch_combine_t<true>(a, grid, vec, stream);
  else
    launch_combine_t<false>(a, grid, vec, stream);
  return hipGetLastError();
}

}  // namespace w4a16
