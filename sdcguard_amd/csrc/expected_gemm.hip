// Expected side of the column-block checksum: E = A @ (block sums of B), on MFMA.
//
// The block sums B2 (k x 2nb fp32 per batch) multiply A as three low-precision parts (hi + mid + lo, whose sum is
// B2 to ~2^-27; checksum.py:160-166, :313-343, serve.py:185-186), so A (bf16/fp16) is never widened and the
// tensor-core products stay exact; every part accumulates into one fp32 accumulator, so E comes out summed over
// parts.  The parts come either
//   BSRC 0: precomputed (serving: LayerChecksums.parts, a (3 x 2nb) x k matrix stored k-contiguous per column), or
//   BSRC 1: split on the fly from fp32 block sums B2^T (training: made by the B-side kernel for this call), after
//           division by a per-column power of two (fp16's range; _matmul_fp32 scales the same way).
// The same pass over A adds |a_row|_2^2 and |a_row|_1 (the noise model's row norms), in the workgroups of the
// first column tile.
//
// Tiling (gfx950, wave64): a workgroup of 4 waves owns a 128-row x 64-column tile of E and a slice of the depth
// (split-K when the tiles alone cannot fill 256 CUs: the partial results go to separate planes that the scoring
// kernel adds).  Depth steps of 32 are staged through LDS; each wave computes a 64 x 32 sub-tile with
// v_mfma_f32_32x32x16_{bf16,f16}: per 16-deep step 2 row fragments x 3 parts.
#include "common.h"
#include "gemm.h"
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

// 8 consecutive (in depth) 16-bit elements at p[kk * sk], or zeros past `lim`
template <bool VEC>
__device__ __forceinline__ u32x4 load8(const uint16_t* p, int64_t sk, int64_t kk, int64_t lim, bool ok) {
  u32x4 v = {0u, 0u, 0u, 0u};
  if (!ok || kk >= lim) return v;
  if constexpr (VEC) {
    return *reinterpret_cast<const u32x4*>(p + kk);
  } else {
    uint16_t e[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) e[i] = (kk + i < lim) ? p[(kk + i) * sk] : (uint16_t)0;
    v.x = e[0] | ((uint32_t)e[1] << 16);
    v.y = e[2] | ((uint32_t)e[3] << 16);
    v.z = e[4] | ((uint32_t)e[5] << 16);
    v.w = e[6] | ((uint32_t)e[7] << 16);
    return v;
  }
}

__device__ __forceinline__ uint32_t to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 16) | 0x40u;       // NaN stays NaN (quiet)
  u += 0x7FFFu + ((u >> 16) & 1u);                                    // round to nearest even
  return u >> 16;
}

template <int DT>
__device__ __forceinline__ uint32_t round_bits(float f) {
  if constexpr (DT == SDC_BF16) return to_bf16_bits(f);
  else return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}

template <int DT>
__device__ __forceinline__ float bits_value(uint32_t b) {
  return half_to_f32<DT>((uint16_t)b);
}

// fp32 -> hi, mid, lo parts of 8 values (checksum._split3), packed as three u32x4
template <int DT>
__device__ __forceinline__ void split8(const float* v, u32x4* parts) {
  uint32_t h[8], md[8], lo[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    h[i] = round_bits<DT>(v[i]);
    const float r = v[i] - bits_value<DT>(h[i]);
    md[i] = round_bits<DT>(r);
    lo[i] = round_bits<DT>(r - bits_value<DT>(md[i]));
  }
  uint32_t* o0 = reinterpret_cast<uint32_t*>(&parts[0]);
  uint32_t* o1 = reinterpret_cast<uint32_t*>(&parts[1]);
  uint32_t* o2 = reinterpret_cast<uint32_t*>(&parts[2]);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o0[i] = h[2 * i] | (h[2 * i + 1] << 16);
    o1[i] = md[2 * i] | (md[2 * i + 1] << 16);
    o2[i] = lo[2 * i] | (lo[2 * i + 1] << 16);
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

template <int DT, int BSRC, bool VEC>
__global__ __launch_bounds__(256) void expected_gemm_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) uint16_t As[GM * LDSK];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[3 * GN * LDSK];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int wm = w >> 1, wn = w & 1;
  const int64_t r0 = (int64_t)blockIdx.x * GM, c0 = (int64_t)blockIdx.y * GN;
  const int64_t batch = blockIdx.z / g.splits, split = blockIdx.z - batch * g.splits;
  const int64_t kbeg = split * g.kchunk;
  const int64_t kend = kbeg + g.kchunk < g.k ? kbeg + g.kchunk : g.k;
  const bool norms = blockIdx.y == 0;
  const int64_t m = g.m, N = g.N;

  // what this thread stages: two rows of A, one column of each part, 8 deep each
  const int lr = t >> 2, lk = (t & 3) * 8;
  const int64_t ar0 = r0 + lr, ar1 = r0 + lr + 64;
  const uint16_t* Ab = g.A + batch * g.sab;
  const uint16_t* xa0 = Ab + (ar0 < m ? ar0 : 0) * g.sam;
  const uint16_t* xa1 = Ab + (ar1 < m ? ar1 : 0) * g.sam;
  const int64_t bc = c0 + lr;
  const bool bc_ok = bc < N;
  const int64_t bcc = bc_ok ? bc : 0;
  float inv_scale = 1.f;
  if constexpr (BSRC == 1) inv_scale = 1.f / g.scale[batch * g.sscb + bcc * g.scale_stride];   // (a power of two: exact)

  u32x4 ra0, ra1, rb[3];
  float sq0 = 0.f, ab0 = 0.f, sq1 = 0.f, ab1 = 0.f;
  auto load_regs = [&](int64_t k0) {
    ra0 = load8<VEC>(xa0, g.sak, k0 + lk, kend, ar0 < m);
    ra1 = load8<VEC>(xa1, g.sak, k0 + lk, kend, ar1 < m);
    if constexpr (BSRC == 0) {
      const uint16_t* P = (const uint16_t*)g.B + batch * g.sbb;
#pragma unroll
      for (int p = 0; p < 3; ++p) rb[p] = load8<VEC>(P + ((int64_t)p * N + bcc) * g.sbc, 1, k0 + lk, kend, bc_ok);
    } else {
      const float* Bt = (const float*)g.B + batch * g.sbb + bcc * g.sbc;
      float v[8];
      const int64_t kk = k0 + lk;
      if (VEC && bc_ok && kk + 8 <= kend) {
        const f32x4 a = *reinterpret_cast<const f32x4*>(Bt + kk);
        const f32x4 b = *reinterpret_cast<const f32x4*>(Bt + kk + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = (bc_ok && kk + i < kend) ? Bt[kk + i] : 0.f;
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] *= inv_scale;
      split8<DT>(v, rb);
    }
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
    for (int p = 0; p < 3; ++p) *reinterpret_cast<u32x4*>(&Bs[(p * GN + lr) * LDSK + lk]) = rb[p];
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
      for (int p = 0; p < 3; ++p) {
        u32x4 b = *reinterpret_cast<const u32x4*>(&Bs[(p * GN + wn * 32 + (lane & 31)) * LDSK + ko]);
        acc[0] = mfma32<DT>(a0, b, acc[0]);
        acc[1] = mfma32<DT>(a1, b, acc[1]);
      }
    }
  }

  // C[i][j] of a 32x32 MFMA tile sits in lane j + 32 * ((i / 4) % 2), register (i / 8) * 4 + i % 4
  float* Es = g.E + (batch * g.splits + split) * m * N;
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
      float* xs = g.XN + (batch * g.splits + split) * 2 * m;
      if (ar0 < m) { xs[ar0] = sq0; xs[m + ar0] = ab0; }
      if (ar1 < m) { xs[ar1] = sq1; xs[m + ar1] = ab1; }
    }
  }
}

template <int DT, int BSRC>
int launch_dt(GemmArgs g, bool vec, dim3 grid, hipStream_t stream) {
  if (vec) hipLaunchKernelGGL((expected_gemm_kernel<DT, BSRC, true>), grid, dim3(256), 0, stream, g);
  else hipLaunchKernelGGL((expected_gemm_kernel<DT, BSRC, false>), grid, dim3(256), 0, stream, g);
  SDC_LAUNCH_CHECK();
  return SDC_OK;
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

int sdc_gemm_launch(int dtype, int bsrc, GemmArgs g, int64_t batches, hipStream_t stream) {
  if (g.splits < 1 || g.splits > SDC_MAX_SPLITS || batches < 1) return SDC_EINVAL;
  g.kchunk = sdc_cdiv(sdc_cdiv(g.k, g.splits), GK) * GK;
  bool vec = g.sak == 1 && (g.k % 8 == 0) && (g.sam % 8 == 0) && (g.sab % 8 == 0) && ((uintptr_t)g.A % 16 == 0);
  if (bsrc == 0) vec = vec && (g.sbc % 8 == 0) && (g.sbb % 8 == 0) && ((uintptr_t)g.B % 16 == 0);
  else vec = vec && (g.sbc % 4 == 0) && (g.sbb % 4 == 0) && ((uintptr_t)g.B % 16 == 0);
  dim3 grid((unsigned)sdc_cdiv(g.m, GM), (unsigned)sdc_cdiv(g.N, GN), (unsigned)(batches * g.splits));
  SdcProf prof("expected_gemm", stream);
  if (dtype == SDC_BF16)
    return bsrc == 0 ? launch_dt<SDC_BF16, 0>(g, vec, grid, stream) : launch_dt<SDC_BF16, 1>(g, vec, grid, stream);
  return bsrc == 0 ? launch_dt<SDC_FP16, 0>(g, vec, grid, stream) : launch_dt<SDC_FP16, 1>(g, vec, grid, stream);
}

// The serving check's call: one batch, precomputed parts (k-contiguous columns).
int sdc_expected_launch(int dtype, const void* x, int64_t sxm, int64_t sxk, const void* parts, int64_t spk,
                        int64_t spc, int nparts, int64_t m, int64_t k, int64_t ncols, int64_t splits, float* E,
                        float* XN, hipStream_t stream) {
  if (sxk != 1 || spk != 1) return SDC_EUNSUPPORTED;        // both operands must be k-contiguous
  if (nparts != 3) return SDC_EUNSUPPORTED;
  GemmArgs g{};
  g.A = (const uint16_t*)x; g.sab = 0; g.sam = sxm; g.sak = sxk;
  g.B = parts; g.sbb = 0; g.sbc = spc;
  g.scale = nullptr; g.sscb = 0;
  g.m = m; g.k = k; g.N = ncols; g.splits = splits;
  g.E = E; g.XN = XN;
  return sdc_gemm_launch(dtype, 0, g, 1, stream);
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
  SDC_CLEAR_ERRORS();
  hipLaunchKernelGGL(mfma_layout_kernel, dim3(1), dim3(64), 0, stream, (const uint16_t*)A, (const uint16_t*)B, C);
  SDC_LAUNCH_CHECK();
  return SDC_OK;
}
