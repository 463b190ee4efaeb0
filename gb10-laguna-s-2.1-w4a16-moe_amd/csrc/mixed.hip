// One launch per GEMM for the split dispatch: the MFMA work items of the
// experts with many pairs and the GEMV work items of the experts with few.
//
// With separate launches each path pays its own start-up and its own tail:
// the MFMA launch of a skewed decode batch holds a few hundred long items
// (1-2 rounds over the CUs), the GEMV launch a few thousand short ones, and
// each drains before the next starts.  Here both sit in one grid, MFMA items
// first: a workgroup slot that finishes an MFMA item takes the next GEMV
// workgroup, so the GEMV items fill the MFMA launch's tail.
//
// Block b < mfma_blocks runs MFMA item b exactly as the MFMA-only kernel of
// the 128-row geometry does (the same block-to-XCD dealing, from block 0);
// block b >= mfma_blocks runs GEMV workgroup b - mfma_blocks exactly as the
// GEMV-only kernel does.  mfma_blocks covers the tiles the align kernel
// listed (header[2]) in whole rounds of one tile per XCD, so no block of the
// grid is spent on the MFMA range's unused tail.  Both work items compute
// what their own launches compute, bit for bit; only the launch is shared.
//
// Resources: the larger LDS of the two (the MFMA item's), and at most 168
// VGPRs (three waves per SIMD, three workgroups per CU -- the occupancy of
// the 4-token GEMV item).
#include <algorithm>

#include "common.hpp"
#include "gemv_item.hpp"
#include "mfma_item.hpp"

namespace w4a16 {
namespace {

using mfma_dev::SmallTile;

template <int MODE, int GSHIFT, int RPL, int PF, int TC, int NIT>
__global__ __launch_bounds__(SmallTile::kWaves * 64)
__attribute__((amdgpu_waves_per_eu(3, 3)))
void mixed_kernel(const MfmaLaunch m, const GemvLaunch g) {
  extern __shared__ __align__(16) unsigned char lds[];
  __shared__ int s_f[SmallTile::kTM];
  __shared__ float s_wt[SmallTile::kTM];
  const int n_mfma = (int)mfma_dev::mfma_blocks<MODE, SmallTile>(m, m.header[2]);
  const int bid = (int)blockIdx.x;
  if (bid < n_mfma)
    mfma_dev::mfma_item<MODE, GSHIFT, SmallTile>(m, bid, lds, s_f, s_wt);
  else
    gemv_dev::gemv_item<MODE, RPL, PF, TC, SmallTile::kWaves, NIT, false, 1, 8>(
        g, bid - n_mfma, reinterpret_cast<gemv_dev::u32x4_t*>(lds));
}

// Unrolled GEMV step counts of the mixed kernels (8 lanes per row, 256
// reduction elements per step): K = 3072 for w13, N = 1024 for w2.
constexpr int kNitW13 = 12;
constexpr int kNitW2 = 4;

// GEMV output rows per lane of the mixed kernels, by token rows per pass.
constexpr int mixed_rpl(int mode, int tc) {
  return mode == 0 ? (tc == 4 ? W4A16_W13_RPL_T4 : W4A16_W13_RPL)
                   : (tc == 4 ? W4A16_W2_RPL_T4 : W4A16_W2_RPL);
}

// Token rows per GEMV pass the call would use, or 0 when no mixed kernel
// covers its GEMV launch.
int mixed_tc(int mode, const MfmaLaunch& m, const GemvLaunch& g) {
  using namespace gemv_dev;
  if (m.tile_m > SmallTile::kTM) return 0;
  if (mode == 0 ? !mfma_dev::mfma_fits<0, SmallTile>(m) : !mfma_dev::mfma_fits<1, SmallTile>(m))
    return 0;
  const int tc = pick_tc(g, g.num_experts);
  if ((tc != 2 && tc != 4) || pick_lpr(g, tc, mode) != 8 || g.upw > 1 || g.ids || !g.block_list)
    return 0;
  if (((g.kdim >> 5) + 7) / 8 != (mode == 0 ? kNitW13 : kNitW2)) return 0;
  if (g.n_out % (8 * mixed_rpl(mode, tc)) != 0) return 0;
  if (m.group != 32 && m.group != 64 && m.group != 128) return 0;
  return tc;
}

// RPL, PF: GEMV rows per lane and steps in flight of two-row passes; RPL4,
// PF4: those of four-row passes.
template <int MODE, int RPL, int PF, int RPL4, int PF4, int NIT>
hipError_t launch_mixed_t(const MfmaLaunch& m, const GemvLaunch& g_in, hipStream_t stream) {
  using namespace gemv_dev;
  static_assert(kGemvWaves == SmallTile::kWaves, "GEMV and MFMA workgroups of one size");
  static_assert(mixed_rpl(MODE, 2) == RPL && mixed_rpl(MODE, 4) == RPL4, "rows per lane");
  const int tc = mixed_tc(MODE, m, g_in);
  if (tc == 0) return hipErrorInvalidValue;
  GemvLaunch g = g_in;
  g.nib_mask = 0x000F000Fu;
  g.nib_magic = 0x43004300u;  // bf16 (128, 128)
  const int chunks = g.n_out / (8 * (tc == 4 ? RPL4 : RPL));
  const int groups = (chunks + kGemvWaves - 1) / kGemvWaves;
  const int64_t grid = mfma_dev::mfma_grid<MODE, SmallTile>(m) + (int64_t)g.max_blocks * groups;
  if (grid <= 0) return hipSuccess;
  if (grid > INT32_MAX) return hipErrorInvalidValue;
  const size_t lds = std::max<size_t>(SmallTile::kLdsTotal, gemv_lds_bytes(tc, g.kdim));
  const dim3 gr((unsigned)grid), b(SmallTile::kWaves * 64);
#define W4A16_MIXED(GS, R_, P_, TC_)                                                         \
  hipLaunchKernelGGL((mixed_kernel<MODE, GS, R_, P_, TC_, NIT>), gr, b, lds, stream, m, g); \
  break;
  if (tc == 4) {
    switch (m.group) {
      case 32: W4A16_MIXED(0, RPL4, PF4, 4)
      case 64: W4A16_MIXED(1, RPL4, PF4, 4)
      default: W4A16_MIXED(2, RPL4, PF4, 4)
    }
  } else {
    switch (m.group) {
      case 32: W4A16_MIXED(0, RPL, PF, 2)
      case 64: W4A16_MIXED(1, RPL, PF, 2)
      default: W4A16_MIXED(2, RPL, PF, 2)
    }
  }
#undef W4A16_MIXED
  return hipGetLastError();
}

}  // namespace

bool mixed_fits(int mode, const MfmaLaunch& m, const GemvLaunch& g) {
  return mixed_tc(mode, m, g) != 0;
}

hipError_t launch_w13_mixed(const MfmaLaunch& m, const GemvLaunch& g, hipStream_t stream) {
  return launch_mixed_t<0, W4A16_W13_RPL, W4A16_W13_PF, W4A16_W13_RPL_T4, W4A16_W13_PF_T4,
                        kNitW13>(m, g, stream);
}

hipError_t launch_w2_mixed(const MfmaLaunch& m, const GemvLaunch& g, hipStream_t stream) {
  return launch_mixed_t<1, W4A16_W2_RPL, W4A16_W2_PF, W4A16_W2_RPL_T4, W4A16_W2_PF_T4, kNitW2>(
      m, g, stream);
}

}  // namespace w4a16
