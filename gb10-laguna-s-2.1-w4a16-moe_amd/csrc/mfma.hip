// Grouped dequant-GEMM on bf16 MFMA for experts with many tokens: the
// MFMA-only launches (the work item is in mfma_item.hpp).
#include <type_traits>

#include "common.hpp"
#include "mfma_item.hpp"

namespace w4a16 {
namespace {

using namespace mfma_dev;

template <int MODE, int GSHIFT, class G>
__global__ __launch_bounds__(G::kWaves * 64, G::kWgsPerCu)
__attribute__((amdgpu_waves_per_eu(G::kWgsPerCu * G::kWaves / 4, G::kWgsPerCu * G::kWaves / 4)))
void mfma_kernel(const MfmaLaunch a) {
  extern __shared__ __align__(16) unsigned char lds[];
  __shared__ int s_f[G::kTM];
  __shared__ float s_wt[G::kTM];
  mfma_item<MODE, GSHIFT, G>(a, (int)blockIdx.x, lds, s_f, s_wt);
}

template <int MODE, class G>
hipError_t launch_geo(const MfmaLaunch& a, hipStream_t stream) {
  const int64_t grid = mfma_grid<MODE, G>(a);
  if (grid <= 0) return hipSuccess;
  const dim3 g((unsigned)grid), b(G::kWaves * 64);
  switch (a.group) {
    case 32: hipLaunchKernelGGL((mfma_kernel<MODE, 0, G>), g, b, G::kLdsTotal, stream, a); break;
    case 64: hipLaunchKernelGGL((mfma_kernel<MODE, 1, G>), g, b, G::kLdsTotal, stream, a); break;
    case 128: hipLaunchKernelGGL((mfma_kernel<MODE, 2, G>), g, b, G::kLdsTotal, stream, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int MODE>
hipError_t launch_mfma_t(const MfmaLaunch& a, hipStream_t stream) {
  // Tiles of at most 64 slots run on 128-row workgroups, two per CU (an
  // item is row_tiles of those row tiles).
  if (a.tile_m <= SmallTile::kTM) {
    if (!mfma_fits<MODE, SmallTile>(a)) return hipErrorInvalidValue;
    return launch_geo<MODE, SmallTile>(a, stream);
  }
  if (!mfma_fits<MODE, BigTile>(a)) return hipErrorInvalidValue;
  return launch_geo<MODE, BigTile>(a, stream);
}

}  // namespace

hipError_t launch_w13_mfma(const MfmaLaunch& a, hipStream_t stream) {
  return launch_mfma_t<0>(a, stream);
}

hipError_t launch_w2_mfma(const MfmaLaunch& a, hipStream_t stream) {
  return launch_mfma_t<1>(a, stream);
}

}  // namespace w4a16
