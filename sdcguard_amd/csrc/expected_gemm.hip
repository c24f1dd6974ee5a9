// Expected side of the column-block checksum: E = x @ (block sums of W), on MFMA.
//
// The block sums B2 (k x 2nb fp32) reach the kernel as NP low-precision parts (NP = 3: hi + mid + lo, whose
// sum is B2 to ~2^-27; serve.py:185-186, checksum.py:160-166), stored k-contiguous per checksum column ("parts
// transposed": element (part p, column c, depth kk) at P[(p * N + c) * spc + kk]).  Every part multiplies the
// same x tile and accumulates into one fp32 accumulator, so E comes out summed over parts.  The same pass
// over x also adds |x_row|_2^2 and |x_row|_1 (the norms the noise model needs), in the workgroups of the first
// column tile, so x is read for the norms only once more than the GEMM reads it.
//
// Tiling (gfx950, wave64): a workgroup of 4 waves owns a 128-row x 64-column tile of E and a slice of depth
// (split-K when the tiles alone cannot fill 256 CUs; partial results go to separate planes of the
// workspace and are added by the scoring kernel).  Depth steps of 32 are staged through LDS; each wave
// computes a 64 x 32 sub-tile with v_mfma_f32_32x32x16_{bf16,f16}: per step 2 row fragments x NP parts.
#include "common.h"
#include "profile.h"

namespace {

constexpr int GM = 128;   // rows of E per workgroup
constexpr int GN = 64;    // columns of E per workgroup
constexpr int GK = 32;    // depth per LDS stage
constexpr int LDSK = GK + 8;   // padded LDS row (elements): 80-byte rows spread the banks

template <int DT>
__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (DT == SDC_BF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                  0, 0, 0);
  }
}

// 8 consecutive 16-bit elements, or zeros past `lim` (element-wise when the row is not 16-byte loadable)
template <bool VEC>
__device__ __forceinline__ u32x4 load8(const uint16_t* p, int64_t kk, int64_t lim, bool row_ok) {
  u32x4 v = {0u, 0u, 0u, 0u};
  if (!row_ok || kk >= lim) return v;
  if constexpr (VEC) {
    return *reinterpret_cast<const u32x4*>(p + kk);
  } else {
    uint16_t e[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) e[i] = (kk + i < lim) ? p[kk + i] : (uint16_t)0;
    v.x = e[0] | ((uint32_t)e[1] << 16);
    v.y = e[2] | ((uint32_t)e[3] << 16);
    v.z = e[4] | ((uint32_t)e[5] << 16);
    v.w = e[6] | ((uint32_t)e[7] << 16);
    return v;
  }
}

template <int DT>
__device__ __forceinline__ void norm_acc(u32x4 v, float& sq, float& ab) {
  uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float a = lo_of<DT>(w[i]), b = hi_of<DT>(w[i]);
    sq = fmaf(a, a, sq);
    sq = fmaf(b, b, sq);
    ab += fabsf(a);
    ab += fabsf(b);
  }
}

// X: x rows (k contiguous), row stride sxm.  P: parts transposed (k contiguous), column stride spc.
// E: [split][m][N] fp32.  XN: [split][2][m] fp32 (sum of squares, sum of |x|), written by column tile 0.
template <int DT, int NP, bool VEC>
__global__ __launch_bounds__(256) void expected_gemm_kernel(const uint16_t* __restrict__ X, int64_t sxm,
                                                            const uint16_t* __restrict__ P, int64_t spc,
                                                            int64_t m, int64_t k, int64_t N, int64_t kchunk,
                                                            float* __restrict__ E, float* __restrict__ XN) {
  __shared__ __attribute__((aligned(16))) uint16_t As[GM * LDSK];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[NP * GN * LDSK];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int wm = w >> 1, wn = w & 1;
  const int64_t r0 = (int64_t)blockIdx.x * GM, c0 = (int64_t)blockIdx.y * GN;
  const int64_t split = blockIdx.z;
  const int64_t kbeg = split * kchunk;
  const int64_t kend = kbeg + kchunk < k ? kbeg + kchunk : k;
  const bool norms = blockIdx.y == 0;

  // what this thread stages: two rows of x, one column of each part, 8 deep each
  const int lr = t >> 2, lk = (t & 3) * 8;
  const int64_t ar0 = r0 + lr, ar1 = r0 + lr + 64;
  const uint16_t* xa0 = X + (ar0 < m ? ar0 : 0) * sxm;
  const uint16_t* xa1 = X + (ar1 < m ? ar1 : 0) * sxm;
  const int64_t bc = c0 + lr;
  const bool bc_ok = bc < N;

  u32x4 ra0, ra1, rb[NP];
  float sq0 = 0.f, ab0 = 0.f, sq1 = 0.f, ab1 = 0.f;
  auto load_regs = [&](int64_t k0) {
    ra0 = load8<VEC>(xa0, k0 + lk, kend, ar0 < m);
    ra1 = load8<VEC>(xa1, k0 + lk, kend, ar1 < m);
#pragma unroll
    for (int p = 0; p < NP; ++p) rb[p] = load8<VEC>(P + ((int64_t)p * N + (bc_ok ? bc : 0)) * spc, k0 + lk, kend, bc_ok);
  };

  f32x16 acc[2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;

  if (kbeg < kend) load_regs(kbeg);
  for (int64_t k0 = kbeg; k0 < kend; k0 += GK) {
    __syncthreads();
    *reinterpret_cast<u32x4*>(&As[lr * LDSK + lk]) = ra0;
    *reinterpret_cast<u32x4*>(&As[(lr + 64) * LDSK + lk]) = ra1;
#pragma unroll
    for (int p = 0; p < NP; ++p) *reinterpret_cast<u32x4*>(&Bs[(p * GN + lr) * LDSK + lk]) = rb[p];
    if (norms) {
      norm_acc<DT>(ra0, sq0, ab0);
      norm_acc<DT>(ra1, sq1, ab1);
    }
    __syncthreads();
    if (k0 + GK < kend) load_regs(k0 + GK);
#pragma unroll
    for (int kk = 0; kk < GK; kk += 16) {
      const int ko = kk + (lane >> 5) * 8;
      u32x4 a0 = *reinterpret_cast<const u32x4*>(&As[(wm * 64 + (lane & 31)) * LDSK + ko]);
      u32x4 a1 = *reinterpret_cast<const u32x4*>(&As[(wm * 64 + 32 + (lane & 31)) * LDSK + ko]);
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        u32x4 b = *reinterpret_cast<const u32x4*>(&Bs[(p * GN + wn * 32 + (lane & 31)) * LDSK + ko]);
        acc[0] = mfma32<DT>(a0, b, acc[0]);
        acc[1] = mfma32<DT>(a1, b, acc[1]);
      }
    }
  }

  // C[i][j] of a 32x32 MFMA tile sits in lane j + 32 * ((i / 4) % 2), register (i / 8) * 4 + i % 4
  float* Es = E + split * m * N;
  const int64_t col = c0 + wn * 32 + (lane & 31);
  if (col < N) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = r0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row < m) Es[row * N + col] = acc[i][r];
      }
  }
  if (norms) {
    sq0 = quad_sum(sq0); ab0 = quad_sum(ab0);
    sq1 = quad_sum(sq1); ab1 = quad_sum(ab1);
    if ((t & 3) == 0) {
      float* xs = XN + split * 2 * m;
      if (ar0 < m) { xs[ar0] = sq0; xs[m + ar0] = ab0; }
      if (ar1 < m) { xs[ar1] = sq1; xs[m + ar1] = ab1; }
    }
  }
}

}  // namespace

// Split of the depth so that tiles x splits fill the GPU (256 CUs, 2 workgroups each), in multiples of GK.
extern "C" int64_t sdc_expected_splits(int64_t m, int64_t k, int64_t ncols) {
  if (m <= 0 || k <= 0 || ncols <= 0) return 1;
  const int64_t tiles = sdc_cdiv(m, GM) * sdc_cdiv(ncols, GN);
  int64_t s = sdc_cdiv(512, tiles);
  const int64_t smax = k / 512 > 1 ? k / 512 : 1;
  if (s > smax) s = smax;
  if (s > SDC_MAX_SPLITS) s = SDC_MAX_SPLITS;
  if (s < 1) s = 1;
  return s;
}

// Shared by the serving and the training checks: E[split][m][ncols] and XN[split][2][m] into workspace planes.
int sdc_expected_launch(int dtype, const void* x, int64_t sxm, int64_t sxk, const void* parts, int64_t spk,
                        int64_t spc, int nparts, int64_t m, int64_t k, int64_t ncols, int64_t splits, float* E,
                        float* XN, hipStream_t stream) {
  if (sxk != 1 || spk != 1) return SDC_EUNSUPPORTED;        // both operands must be k-contiguous
  if (nparts != 3) return SDC_EUNSUPPORTED;
  int64_t kchunk = sdc_cdiv(sdc_cdiv(k, splits), GK) * GK;
  const bool vec = (k % 8 == 0) && (sxm % 8 == 0) && (spc % 8 == 0) && ((uintptr_t)x % 16 == 0) &&
                   ((uintptr_t)parts % 16 == 0);
  dim3 grid((unsigned)sdc_cdiv(m, GM), (unsigned)sdc_cdiv(ncols, GN), (unsigned)splits);
  const uint16_t* X = (const uint16_t*)x;
  const uint16_t* P = (const uint16_t*)parts;
  SdcProf prof("expected_gemm", stream);
#define SDC_EG(DT, V) \
  hipLaunchKernelGGL((expected_gemm_kernel<DT, 3, V>), grid, dim3(256), 0, stream, X, sxm, P, spc, m, k, ncols, kchunk, E, XN)
  if (dtype == SDC_BF16) {
    if (vec) SDC_EG(SDC_BF16, true); else SDC_EG(SDC_BF16, false);
  } else {
    if (vec) SDC_EG(SDC_FP16, true); else SDC_EG(SDC_FP16, false);
  }
#undef SDC_EG
  SDC_LAUNCH_CHECK();
  return SDC_OK;
}

// Self-test of the MFMA operand layout this file assumes: C (32 x 32) = A (32 x 16) @ B (16 x 32), bf16 in,
// fp32 out, A given row-major (k contiguous) and B given column-major (k contiguous), one wave.
__global__ void mfma_layout_kernel(const uint16_t* A, const uint16_t* B, float* C) {
  const int lane = threadIdx.x;
  u32x4 a = *reinterpret_cast<const u32x4*>(A + (lane & 31) * 16 + (lane >> 5) * 8);
  u32x4 b = *reinterpret_cast<const u32x4*>(B + (lane & 31) * 16 + (lane >> 5) * 8);
  f32x16 c;
#pragma unroll
  for (int r = 0; r < 16; ++r) c[r] = 0.f;
  c = mfma32<SDC_BF16>(a, b, c);
#pragma unroll
  for (int r = 0; r < 16; ++r) C[(8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * 32 + (lane & 31)] = c[r];
}

extern "C" int sdc_mfma_layout_selftest(const void* A, const void* B, float* C, hipStream_t stream) {
  hipLaunchKernelGGL(mfma_layout_kernel, dim3(1), dim3(64), 0, stream, (const uint16_t*)A, (const uint16_t*)B, C);
  SDC_LAUNCH_CHECK();
  return SDC_OK;
}
