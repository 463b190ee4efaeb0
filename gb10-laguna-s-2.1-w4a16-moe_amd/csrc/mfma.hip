// Grouped dequant-GEMM on bf16 MFMA for experts with many tokens (prefill).
//
// Reference kernels: _w4a16_moe_w1_fused_kernel (kernels/w4a16_moe.py:374-499)
// and _w4a16_moe_w2_kernel (:502-634): per 16-token block x 64-column tile,
// tl.dot of bf16 activations with bf16(dequantized weights), fp32 accumulate.
// Here one workgroup (4 waves) owns a tile of up to 128 sorted token slots of
// one expert x 256 weight rows and walks the reduction axis 32 at a time:
//   * the 32-element group of each of the 256 rows (one dwordx4 + one scale)
//     is dequantized once per tile to bf16((code-8) * scale) -- the product
//     is exact in fp32, so this is the reference's rounding -- and stored in
//     LDS as [row][k];
//   * the gathered activation rows are copied to LDS as [token][k];
//   * each wave multiplies a 64-token x 128-row quarter with
//     v_mfma_f32_32x32x16_bf16 (8 accumulator blocks of 32x32 fp32).
// LDS is double-buffered and global loads run two steps ahead, so one
// barrier per step separates the writers of step s+1 from the readers of s.
// Rows of LDS are padded to 80 bytes: the 8 lanes served together by a
// 16-byte LDS read hit 8 distinct 4-bank groups.
//
// w13 (MODE 0): the 256 weight rows are 128 gate rows and the matching 128 up
// rows, so every lane holds gate and up of the same output column and the
// epilogue writes bf16(SiLU(gate) * up) -- the reference's rounding point.
// w2 (MODE 1): the epilogue multiplies by the routing weight and writes the
// fp32 partial row of the (token, slot) pair.
//
// Workgroup ids are remapped so that the N-tiles of one token tile run on one
// XCD (consecutive hardware ids round-robin over the 8 XCDs) and share its L2
// for the activation rows.
#include "common.hpp"

namespace w4a16 {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
// Native 128-bit vector: whole-value copies of HIP's union-based 4-vector
// structs end up in scratch memory instead of registers.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kTM = kMfmaTileM;    // token slots per tile (4 blocks of 32)
constexpr int kTN = kMfmaTileN;    // weight rows per tile (8 blocks of 32)
constexpr int kBK = 32;            // reduction step
constexpr int kRowBytes = kBK * 2 + 16;
constexpr int kABytes = kTM * kRowBytes;
constexpr int kBBytes = kTN * kRowBytes;
constexpr int kStage = kABytes + kBBytes;
constexpr int kXcds = 8;

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// 32 codes of one group -> 32 bf16 (code - 8) * s in k order.
__device__ __forceinline__ void dequant_group(const u32x4_t w, float s, u32x4_t (&o)[4]) {
  const float b = -8.0f * s;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t lo = w[j] & 0x0F0F0F0Fu;         // codes 0,2,4,6
    const uint32_t hi = (w[j] >> 4) & 0x0F0F0F0Fu;  // codes 1,3,5,7
    const float v0 = fmaf((float)(lo & 0xFFu), s, b);
    const float v1 = fmaf((float)(hi & 0xFFu), s, b);
    const float v2 = fmaf((float)((lo >> 8) & 0xFFu), s, b);
    const float v3 = fmaf((float)((hi >> 8) & 0xFFu), s, b);
    const float v4 = fmaf((float)((lo >> 16) & 0xFFu), s, b);
    const float v5 = fmaf((float)((hi >> 16) & 0xFFu), s, b);
    const float v6 = fmaf((float)(lo >> 24), s, b);
    const float v7 = fmaf((float)(hi >> 24), s, b);
    o[j] = u32x4_t{pack_bf16x2(v0, v1), pack_bf16x2(v2, v3), pack_bf16x2(v4, v5),
                   pack_bf16x2(v6, v7)};
  }
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + __expf(-g)); }

__device__ __forceinline__ int xcd_remap(int bid, int n) {
  const int per = n / kXcds;
  if (bid >= per * kXcds) return bid;
  return (bid % kXcds) * per + bid / kXcds;
}

template <int MODE>
__global__ __launch_bounds__(256, 2) void mfma_kernel(const MfmaLaunch a) {
  extern __shared__ __align__(16) unsigned char lds[];
  __shared__ int s_f[kTM];

  const int rows_total = MODE == 0 ? 2 * a.n_out : a.n_out;
  const int n_tiles_n = rows_total / kTN;
  const int bid = xcd_remap(blockIdx.x, gridDim.x);
  const int tile = bid / n_tiles_n;
  const int nt = bid - tile * n_tiles_n;
  if (tile >= a.header[2]) return;
  const int4 info = a.tiles[tile];
  const int e = info.x, start = info.y, count = info.z;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // Wave index in an SGPR: the per-wave branches below are then scalar.
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wid & 1, wn = wid >> 1;

  for (int i = tid; i < kTM; i += 256) s_f[i] = i < count ? a.sorted[start + i] : a.n_tok;
  __syncthreads();

  const int kdim = a.kdim;
  const int G = kdim >> 5;
  const int gpr = kdim / a.group;
  const int gshift = a.group == 32 ? 0 : (a.group == 64 ? 1 : 2);
  const int nsteps = G;

  // Activation rows: 128 rows x 4 octets per step, two octets per thread.
  // Rows past the tile's count read row 0 (their results are discarded).
  const u32x4_t* a_src[2];
  int a_lds[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int u = tid + 256 * i;
    const int row = u >> 2, part = u & 3;
    const int f = s_f[row];
    int64_t arow = 0;
    if (f < a.n_tok) arow = MODE == 0 ? f / a.topk : f;
    a_src[i] = reinterpret_cast<const u32x4_t*>(a.act + arow * a.ld_act) + part;
    a_lds[i] = row * kRowBytes + part * 16;
  }
  // Weight rows: one per thread.
  int grow;
  if (MODE == 0) {
    const int half = kTN / 2;
    grow = tid < half ? nt * half + tid : a.n_out + nt * half + (tid - half);
  } else {
    grow = nt * kTN + tid;
  }
  const int64_t growg = (int64_t)e * rows_total + grow;
  const u32x4_t* b_src = reinterpret_cast<const u32x4_t*>(a.w) + growg * G;
  const uint16_t* s_src = a.s + growg * gpr;
  const int b_lds = tid * kRowBytes;

  const int mb0 = 2 * wm;
  const bool act0 = 32 * mb0 < count;
  const bool act1 = 32 * (mb0 + 1) < count;

  f32x16_t acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int n = 0; n < 4; ++n)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][n][r] = 0.0f;

  // Global loads of one reduction step, kept in registers until stored.
  struct Stage {
    u32x4_t a0, a1;  // two activation octets
    u32x4_t b;       // one packed group of this thread's weight row
    uint32_t s;    // its raw bf16 scale
  };
  // Unconditional (clamped) loads keep the in-flight count path-independent.
  auto gload = [&](Stage& st, int step) {
    const int k = min(step, nsteps - 1);
    st.a0 = a_src[0][k * 4];
    st.a1 = a_src[1][k * 4];
    st.b = b_src[k];
    st.s = s_src[k >> gshift];
  };

  const int lrow = lane & 31;
  const int lk = (lane >> 5) * 16;  // byte offset of this lane's 8 k-values

  auto step_body = [&](Stage& st, unsigned char* A, int step) {
    unsigned char* B = A + kABytes;
    *reinterpret_cast<u32x4_t*>(A + a_lds[0]) = st.a0;
    *reinterpret_cast<u32x4_t*>(A + a_lds[1]) = st.a1;
    u32x4_t o[4];
    dequant_group(st.b, bf16_to_f32(st.s), o);
#pragma unroll
    for (int j = 0; j < 4; ++j) *reinterpret_cast<u32x4_t*>(B + b_lds + 16 * j) = o[j];
    __syncthreads();
    gload(st, step + 2);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      bf16x8_t bf[4];
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const int nsub = MODE == 0 ? (n < 2 ? 2 * wn + n : 4 + 2 * wn + (n - 2)) : 4 * wn + n;
        bf[n] = *reinterpret_cast<const bf16x8_t*>(B + (nsub * 32 + lrow) * kRowBytes +
                                                   kk * 32 + lk);
      }
      if (act0) {
        const bf16x8_t af =
            *reinterpret_cast<const bf16x8_t*>(A + (mb0 * 32 + lrow) * kRowBytes + kk * 32 + lk);
#pragma unroll
        for (int n = 0; n < 4; ++n)
          acc[0][n] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, bf[n], acc[0][n], 0, 0, 0);
      }
      if (act1) {
        const bf16x8_t af = *reinterpret_cast<const bf16x8_t*>(
            A + ((mb0 + 1) * 32 + lrow) * kRowBytes + kk * 32 + lk);
#pragma unroll
        for (int n = 0; n < 4; ++n)
          acc[1][n] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, bf[n], acc[1][n], 0, 0, 0);
      }
    }
  };

  Stage st0, st1;
  gload(st0, 0);
  // Keep stage 0's loads ahead of stage 1's: the loop expects that order and
  // would otherwise wait for every load at its head.
  __builtin_amdgcn_sched_barrier(0);
  gload(st1, 1);
  // nsteps is even: the MFMA path needs K % 256 == 0 and N % 128 == 0.
  for (int step = 0; step < nsteps; step += 2) {
    step_body(st0, lds, step);
    step_body(st1, lds + kStage, step + 1);
  }

  // Epilogue.  Accumulator register r of a 32x32 block holds row
  // 8*(r/4) + 4*(lane/32) + r%4 and column lane%32.
  const int rq = lane >> 5;
#pragma unroll
  for (int mi = 0; mi < 2; ++mi) {
    if (!(mi == 0 ? act0 : act1)) continue;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int trow = (mb0 + mi) * 32 + 8 * (r >> 2) + 4 * rq + (r & 3);
      const int f = s_f[trow];
      if (f >= a.n_tok) continue;
      if (MODE == 0) {
        uint16_t* out = static_cast<uint16_t*>(a.out) + (int64_t)f * a.n_out;
#pragma unroll
        for (int n = 0; n < 2; ++n) {
          const float h = silu(acc[mi][n][r]) * acc[mi][n + 2][r];
          out[nt * (kTN / 2) + (2 * wn + n) * 32 + lrow] = (uint16_t)f32_to_bf16(h);
        }
      } else {
        const float wt = a.topk_w[f];
        float* out = static_cast<float*>(a.out) + (int64_t)f * a.n_out;
#pragma unroll
        for (int n = 0; n < 4; ++n) out[nt * kTN + (4 * wn + n) * 32 + lrow] = acc[mi][n][r] * wt;
      }
    }
  }
}

template <int MODE>
hipError_t launch_mfma_t(const MfmaLaunch& a, hipStream_t stream) {
  const int rows_total = MODE == 0 ? 2 * a.n_out : a.n_out;
  if (rows_total % kTN != 0) return hipErrorInvalidValue;
  const int64_t grid = (int64_t)a.max_tiles * (rows_total / kTN);
  if (grid <= 0) return hipSuccess;
  hipLaunchKernelGGL(mfma_kernel<MODE>, dim3((unsigned)grid), dim3(256), 2 * kStage, stream,
                     a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_w13_mfma(const MfmaLaunch& a, hipStream_t stream) {
  return launch_mfma_t<0>(a, stream);
}

hipError_t launch_w2_mfma(const MfmaLaunch& a, hipStream_t stream) {
  return launch_mfma_t<1>(a, stream);
}

}  // namespace w4a16
