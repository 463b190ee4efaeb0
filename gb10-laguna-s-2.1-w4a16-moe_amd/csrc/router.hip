// Router step: logits [M, E] (fp32 or bf16) -> the top-k experts of each row
// and their softmax weights, the step in front of the MoE layer.
//
// Follows make_routing, bench/bench_moe.py:225-230: torch.topk(logits, k)
// (values in descending order) then torch.softmax over the k selected
// logits.  With renormalize = 0 the weights are instead the softmax over all
// E logits, read at the selected experts.
//
// One wave per row; lane l holds logits l, l+64, l+128, ...  Each of the k
// rounds takes the wave-wide maximum of a 32-bit order key (DPP within rows
// of 16 lanes, then four lane reads), so a selection costs a handful of
// instructions and no LDS.  Ties between equal logits go to the lower expert
// index; NaN ranks above +inf and -0.0 ties with +0.0, as in torch.topk.
#include "common.hpp"

namespace w4a16 {
namespace {

constexpr int kRouterWaves = 4;

// Order-preserving map of a float to uint32 (larger value -> larger key).
// Real values map to keys >= 0x007FFFFF, so 0 marks a taken or absent slot.
__device__ __forceinline__ uint32_t order_key(float v) {
  if (v != v) return 0xFFFFFFFFu;
  const uint32_t b = __float_as_uint(v == 0.0f ? 0.0f : v);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}

__device__ __forceinline__ uint32_t readlane_u32(uint32_t v, int lane) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, lane);
}

// Maximum over the 64 lanes, returned uniform.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp_u32<0xB1>(v));
  v = max(v, dpp_u32<0x4E>(v));
  v = max(v, dpp_u32<0x141>(v));
  v = max(v, dpp_u32<0x140>(v));
  return max(max(readlane_u32(v, 0), readlane_u32(v, 16)),
             max(readlane_u32(v, 32), readlane_u32(v, 48)));
}

__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  v = min(v, dpp_u32<0xB1>(v));
  v = min(v, dpp_u32<0x4E>(v));
  v = min(v, dpp_u32<0x141>(v));
  v = min(v, dpp_u32<0x140>(v));
  return min(min(readlane_u32(v, 0), readlane_u32(v, 16)),
             min(readlane_u32(v, 32), readlane_u32(v, 48)));
}

// Sum over the 64 lanes in a fixed order, returned uniform.
__device__ __forceinline__ float wave_sum(float v) {
  v = oct_sum(v);
  v += dpp_f32<0x140>(v);
  const float a = __uint_as_float(readlane_u32(__float_as_uint(v), 0));
  const float b = __uint_as_float(readlane_u32(__float_as_uint(v), 16));
  const float c = __uint_as_float(readlane_u32(__float_as_uint(v), 32));
  const float d = __uint_as_float(readlane_u32(__float_as_uint(v), 48));
  return (a + b) + (c + d);
}

template <bool BF16>
__device__ __forceinline__ float load_logit(const void* base, int64_t off) {
  if constexpr (BF16) {
    return bf16_to_f32(static_cast<const uint16_t*>(base)[off]);
  } else {
    return static_cast<const float*>(base)[off];
  }
}

// VPL = logits per lane (E <= 64 * VPL).
template <int VPL, bool BF16>
__global__ __launch_bounds__(64 * kRouterWaves) void router_kernel(const RouterLaunch a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRouterWaves + (threadIdx.x >> 6);
  if (row >= a.M) return;  // uniform per wave

  const int64_t base = row * a.ld;
  float v[VPL];
  uint32_t key[VPL];
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    // clamped, unconditional loads: all VPL of them are in flight at once
    const int e = j * 64 + lane;
    v[j] = load_logit<BF16>(a.logits, base + min(e, a.E - 1));
  }
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    key[j] = j * 64 + lane < a.E ? order_key(v[j]) : 0u;
  }

  // Best remaining slot of this lane: largest key, lowest j among equals.
  uint32_t bk = 0;
  int bj = 0;
  float bv = 0.0f;
  auto lane_best = [&]() {
    bk = 0;
    bj = 0;
    bv = 0.0f;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      if (key[j] > bk) {
        bk = key[j];
        bj = j;
        bv = v[j];
      }
    }
  };
  lane_best();

  int my_idx = 0;      // lane t < topk keeps the expert of rank t
  float my_val = 0.0f;  // and its logit
  for (int t = 0; t < a.topk; ++t) {
    const uint32_t wk = wave_max_u32(bk);
    const bool mine = bk == wk;
    const uint64_t tied = ballot(mine);
    const uint32_t cand = mine ? (uint32_t)(bj * 64 + lane) : 0xFFFFFFFFu;
    uint32_t widx;
    if (__popcll(tied) == 1) {
      widx = readlane_u32(cand, __ffsll((long long)tied) - 1);
    } else {
      widx = wave_min_u32(cand);  // equal logits: lowest expert index wins
    }
    const int wlane = (int)(widx & 63);
    const float wv = __uint_as_float(readlane_u32(__float_as_uint(bv), wlane));
    if (lane == t) {
      my_idx = (int)widx;
      my_val = wv;
    }
    if (lane == wlane) {
      const int wj = (int)(widx >> 6);
#pragma unroll
      for (int j = 0; j < VPL; ++j) {
        if (j == wj) key[j] = 0u;
      }
      lane_best();
    }
  }

  // Softmax.  The rank-0 logit is the maximum of the row (of the selection
  // and of all E logits alike).
  const float m = __uint_as_float(readlane_u32(__float_as_uint(my_val), 0));
  const bool sel = lane < a.topk;
  const float ex = sel ? expf(my_val - m) : 0.0f;
  float part;
  if (a.renormalize) {
    part = ex;
  } else {
    part = 0.0f;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      if (j * 64 + lane < a.E) part += expf(v[j] - m);
    }
  }
  const float s = wave_sum(part);
  if (sel) {
    const int64_t o = row * a.topk + lane;
    a.ids[o] = my_idx;
    a.weights[o] = ex / s;
  }
}

template <int VPL>
hipError_t launch_vpl(const RouterLaunch& a, hipStream_t stream) {
  const dim3 grid((unsigned)((a.M + kRouterWaves - 1) / kRouterWaves));
  const dim3 block(64 * kRouterWaves);
  if (a.bf16) {
    hipLaunchKernelGGL((router_kernel<VPL, true>), grid, block, 0, stream, a);
  } else {
    hipLaunchKernelGGL((router_kernel<VPL, false>), grid, block, 0, stream, a);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_router(const RouterLaunch& a, hipStream_t stream) {
  if (a.M <= 0) return hipSuccess;
  const int vpl = (a.E + 63) / 64;
  if (vpl <= 1) return launch_vpl<1>(a, stream);
  if (vpl <= 2) return launch_vpl<2>(a, stream);
  if (vpl <= 4) return launch_vpl<4>(a, stream);
  if (vpl <= 8) return launch_vpl<8>(a, stream);
  return launch_vpl<16>(a, stream);
}

}  // namespace w4a16
