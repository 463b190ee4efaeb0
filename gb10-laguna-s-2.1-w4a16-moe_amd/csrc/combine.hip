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

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Slots whose partial loads are in flight together.
constexpr int kSlotBatch = 16;
constexpr int kCombineThreads = 128;
// From this many bytes of partial rows the loads are non-temporal: M=4096
// combine 51.3 -> 47.1 us, skewed M=64 (3.9 MB) 3.70 -> 3.54 us; M=16's
// 1 MB, still in L2 from the w2 launch, read 3.12 -> 3.47 us with the hint.
constexpr int64_t kCombineNtBytes = 2 << 20;

// One thread owns VPT consecutive outputs of one token (8 for bf16 partials,
// 4 for fp32: one 16-byte load per slot).  The ids of a batch of slots are
// read with every slot's partial row (a slot with an id outside [0, E) has an
// unwritten row: it is read and left out), all in flight together, and the
// values are added in slot order from +0.0 -- the order of the reference's
// sum, so the result does not depend on the batching.
template <bool VEC_STORE, bool BF16, bool NT>
__global__ __launch_bounds__(kCombineThreads) void combine_kernel(const CombineLaunch a) {
  constexpr int VPT = BF16 ? 8 : 4;
  const int per_row = a.K / VPT;
  const int kchunks = (per_row + kCombineThreads - 1) / kCombineThreads;
  const int m = blockIdx.x / kchunks;
  const int c = (blockIdx.x - m * kchunks) * kCombineThreads + threadIdx.x;
  if (c >= per_row) return;
  const int64_t row0 = (int64_t)m * a.topk;
  const size_t row_bytes = (size_t)a.K * (BF16 ? 2 : 4);
  const char* base = static_cast<const char*>(a.partial) + (size_t)c * 16;
  float acc[VPT];
#pragma unroll
  for (int i = 0; i < VPT; ++i) acc[i] = 0.0f;
  for (int t0 = 0; t0 < a.topk; t0 += kSlotBatch) {
    const int nb = min(kSlotBatch, a.topk - t0);
    bool ok[kSlotBatch];
    u32x4_t v[kSlotBatch];
#pragma unroll
    for (int j = 0; j < kSlotBatch; ++j) {
      ok[j] = false;
      v[j] = u32x4_t{0u, 0u, 0u, 0u};
      if (j < nb) {  // uniform
        const int e = a.ids[row0 + t0 + j];
        ok[j] = e >= 0 && e < a.num_experts;
        const u32x4_t* src =
            reinterpret_cast<const u32x4_t*>(base + (size_t)(row0 + t0 + j) * row_bytes);
        v[j] = NT ? __builtin_nontemporal_load(src) : *src;
      }
    }
#pragma unroll
    for (int j = 0; j < kSlotBatch; ++j) {
      if (!ok[j]) continue;
      if constexpr (BF16) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc[2 * i] += bf16_to_f32(v[j][i] & 0xFFFFu);
          acc[2 * i + 1] += bf16_to_f32(v[j][i] >> 16);
        }
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] += __uint_as_float(v[j][i]);
      }
    }
  }
  uint16_t* o = a.out + (int64_t)m * a.ld_out + (int64_t)c * VPT;
  uint32_t b[VPT];
#pragma unroll
  for (int i = 0; i < VPT; ++i) b[i] = f32_to_bf16(acc[i]);
  if (VEC_STORE) {
    if constexpr (VPT == 8)
      *reinterpret_cast<u32x4_t*>(o) =
          u32x4_t{b[0] | (b[1] << 16), b[2] | (b[3] << 16), b[4] | (b[5] << 16), b[6] | (b[7] << 16)};
    else
      *reinterpret_cast<uint2*>(o) = make_uint2(b[0] | (b[1] << 16), b[2] | (b[3] << 16));
  } else {
#pragma unroll
    for (int i = 0; i < VPT; ++i) o[i] = (uint16_t)b[i];
  }
}

template <bool BF16, bool NT>
void launch_combine_t(const CombineLaunch& a, dim3 grid, bool vec, hipStream_t stream) {
  if (vec)
    hipLaunchKernelGGL((combine_kernel<true, BF16, NT>), grid, dim3(kCombineThreads), 0, stream, a);
  else
    hipLaunchKernelGGL((combine_kernel<false, BF16, NT>), grid, dim3(kCombineThreads), 0, stream, a);
}

}  // namespace

hipError_t launch_combine(const CombineLaunch& a, hipStream_t stream) {
  if (a.M <= 0) return hipSuccess;
  const int vpt = a.partial_bf16 ? 8 : 4;
  // 16-byte partial loads: K a multiple of 8 and a 16-byte aligned buffer
  if (a.K % 8 != 0 || reinterpret_cast<uintptr_t>(a.partial) % 16 != 0)
    return hipErrorInvalidValue;
  const int64_t kchunks = (a.K / vpt + kCombineThreads - 1) / kCombineThreads;
  const dim3 grid((unsigned)(kchunks * a.M));
  const bool vec = (reinterpret_cast<uintptr_t>(a.out) % (2 * vpt) == 0) && (a.ld_out % vpt == 0);
  const bool nt = (int64_t)a.M * a.topk * a.K * (a.partial_bf16 ? 2 : 4) >= kCombineNtBytes;
  if (a.partial_bf16) {
    if (nt)
      launch_combine_t<true, true>(a, grid, vec, stream);
    else
      launch_combine_t<true, false>(a, grid, vec, stream);
  } else {
    if (nt)
      launch_combine_t<false, true>(a, grid, vec, stream);
    else
      launch_combine_t<false, false>(a, grid, vec, stream);
  }
  return hipGetLastError();
}

}  // namespace w4a16
