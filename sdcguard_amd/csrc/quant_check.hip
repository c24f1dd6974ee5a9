// Column-block checks of quantized GEMMs (modes.py:231-291, `judge`):
//   int8 W8A8   C (int32) = A (int8) @ B (int8): the plain and signed sums of every (row, 128-column block) must
//               equal A @ (the same sums of B's columns) exactly; integers throughout (int64 sums).
//   fp8 e4m3    C (fp32 or bf16) = sa_i * sb_j * sum_k Aq[i,k] Bq[k,j]: sum_j w_j C[i,j] against
//               sa_i * Aq_i . (sum_j w_j sb_j Bq[:,j]) with modes.judge's fp32-accumulator noise
//               u (C1 |sa_i Aq_i| |Bs_blk|_F + (C2 sqrt(k) + C3 k / nfma) |C_blk|) (+ 2^-8 |C_blk| for a bf16 C), and
//               its Inf/NaN and Cauchy-Schwarz (|c_ij| > 2 |a_i| |b_j|) rules.  With sa = sb = 1 and an fp32 C
//               this is modes.judge("fp8") itself.
// Two launches, no host synchronisation: the expected side on MFMA (expected_gemm.hip: int8 A with the block
// sums' two base-128 digits, or fp8 A widened exactly to bf16 with the three bf16 parts of the scaled block sums),
// then one persistent pass over C: 16 lanes per (row, block) pair, 8 elements per lane, the sums in int64 or fp64,
// one verdict per pair, a wave / workgroup reduction and one set of atomics per workgroup.
#include "common.h"
#include "gemm.h"
#include "profile.h"

extern "C" int64_t sdc_expected_splits(int64_t m, int64_t k, int64_t ncols);

namespace {

enum CType { C_F32 = 0, C_BF16 = 1, C_I32 = 2 };

struct QuantArgs {
  const void* C;
  int64_t scm, scn;
  int64_t m, n, nb, bs, rem, npairs;
  int vec;                           // 16-byte loads along rows
  const float* s_full;
  const float* s_last;
  const float* E;                    // fp8: [split][m][ncols] fp32; int8: [split][2][m][ncols] int32 bits
  const float* XN;                   // fp8: [split][2][m]: sum of squares (and of |.|) of Aq's rows
  int64_t splits, ncols;
  const float* sa;                   // fp8: per-row scale, or null (1)
  const float* bfrob;                // fp8: |Bs_blk|_F per block
  const float* bcol;                 // fp8: |Bs_j|_2 per column
  float unit, per_out, zt;
  int c_bf16;
  int64_t* result;                   // [4]: worst key, key with its noise, wrong blocks, blocks with non-finite values
  float* zdump;                      // (m, nb) z per block, or null
};

struct QBest {
  int64_t key = 0, keyd = 0;
  int wrong = 0, nonfin = 0;
};

__device__ __forceinline__ double shfl_xor_d(double v, int m) { return __shfl_xor(v, m, 64); }

__device__ __forceinline__ int64_t shfl_xor_i64(int64_t v, int m) {
  const int lo = __shfl_xor((int)(uint32_t)v, m, 64), hi = __shfl_xor((int)(v >> 32), m, 64);
  return (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}

// 8 consecutive elements of C (row r, columns c0 .. c0 + 7, those < lim) as doubles / int64
template <int CT>
__device__ __forceinline__ void load8c(const QuantArgs& a, int64_t r, int64_t c0, int64_t lim, double* x,
                                       int64_t* xi) {
  const uint8_t* base = (const uint8_t*)a.C;
  constexpr int ES = CT == C_BF16 ? 2 : 4;
  if (a.vec && c0 + 8 <= lim) {
    const uint8_t* p = base + (r * a.scm + c0) * ES;
    if constexpr (CT == C_BF16) {
      const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        x[2 * i] = (double)bf16_lo(v[i]);
        x[2 * i + 1] = (double)bf16_hi(v[i]);
      }
    } else {
      const u32x4 v0 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
      const u32x4 v1 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p + 16));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (CT == C_I32) {
          xi[i] = (int32_t)v0[i];
          xi[4 + i] = (int32_t)v1[i];
        } else {
          x[i] = (double)__uint_as_float(v0[i]);
          x[4 + i] = (double)__uint_as_float(v1[i]);
        }
      }
    }
    return;
  }
#pragma unroll 1
  for (int i = 0; i < 8; ++i) {
    const int64_t c = c0 + i;
    if (c < lim) {
      const uint8_t* p = base + (r * a.scm + c * a.scn) * ES;
      if constexpr (CT == C_BF16) x[i] = (double)half_to_f32<SDC_BF16>(*(const uint16_t*)p);
      else if constexpr (CT == C_I32) xi[i] = *(const int32_t*)p;
      else x[i] = (double)*(const float*)p;
    } else {
      x[i] = 0.0;
      xi[i] = 0;
    }
  }
}

// fp8: one pair's verdict from the 16-lane sums (every lane holds them); returns z (inf = wrong on the rules)
__device__ __forceinline__ float judge_fp8(const QuantArgs& a, int64_t r, int64_t jb, double pl, double sg,
                                           double sq, bool imposs, float& noise_out) {
  double e0 = 0.0, e1 = 0.0, asq = 0.0;
#pragma unroll
  for (int s = 0; s < SDC_MAX_SPLITS; ++s)
    if (s < a.splits) {
      const float* ep = a.E + (s * a.m + r) * a.ncols + 2 * jb;
      e0 += (double)ep[0];
      e1 += (double)ep[1];
      asq += (double)a.XN[s * 2 * a.m + r];
    }
  const double sa = a.sa ? (double)a.sa[r] : 1.0;
  e0 *= sa;
  e1 *= sa;
  const double a_norm = sa * sqrt(asq);
  const double c_norm = sqrt(sq);
  double noise = (double)a.unit * (a_norm * (double)a.bfrob[jb] + (double)a.per_out * c_norm);
  if (a.c_bf16) noise += 0.00390625 * c_norm;
  noise += 1e-300;
  noise_out = (float)noise;
  const double z = fmax(fabs(e0 - pl), fabs(e1 - sg)) / noise;
  const bool fin = isfinite(pl) && isfinite(sg);
  const bool bad = !fin || imposs || !isfinite(noise) || isnan(z);
  return bad ? __builtin_inff() : (float)z;
}

template <int KIND, int CT>
__global__ __launch_bounds__(256) void quant_score_kernel(QuantArgs a) {
  __shared__ int64_t red_k[4], red_d[4];
  __shared__ int red_w[4], red_n[4];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int g = lane >> 4, e = lane & 15;              // pair within the wave, 8-element segment within the pair
  QBest best;
  const int64_t groups = (a.npairs + 3) / 4;
  for (int64_t grp = (int64_t)blockIdx.x * 4 + w; grp < groups; grp += (int64_t)gridDim.x * 4) {
    const int64_t p = grp * 4 + g;
    const bool live = p < a.npairs;
    const int64_t pp = live ? p : 0;
    const int64_t r = pp / a.nb, jb = pp - r * a.nb;
    const bool last = (jb == a.nb - 1) && (a.rem > 0);
    const int64_t wid = last ? a.rem : a.bs;
    const float* sp = last ? a.s_last : a.s_full;
    const int64_t c0 = jb * a.bs + 8 * e, lim = jb * a.bs + wid;
    double x[8];
    int64_t xi[8];
    load8c<CT>(a, r, c0, (live && 8 * e < wid) ? lim : c0, x, xi);
    float sgn[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) sgn[i] = 8 * e + i < wid ? sp[8 * e + i] : 0.f;
    if constexpr (KIND == 0) {
      // int8: exact integer sums
      int64_t pl = 0, sg = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        pl += xi[i];
        sg += sgn[i] > 0.f ? xi[i] : -xi[i];
      }
#pragma unroll
      for (int msk = 1; msk < 16; msk <<= 1) {
        pl += shfl_xor_i64(pl, msk);
        sg += shfl_xor_i64(sg, msk);
      }
      if (live && e == 0) {
        int64_t e0 = 0, e1 = 0;
#pragma unroll
        for (int s = 0; s < SDC_MAX_SPLITS; ++s)
          if (s < a.splits) {
            const int32_t* hi = reinterpret_cast<const int32_t*>(a.E) + ((s * 2) * a.m + r) * a.ncols + 2 * jb;
            const int32_t* lo = hi + a.m * a.ncols;
            e0 += 128 * (int64_t)hi[0] + (int64_t)lo[0];
            e1 += 128 * (int64_t)hi[1] + (int64_t)lo[1];
          }
        const bool bad = e0 != pl || e1 != sg;
        const float z = bad ? __builtin_inff() : 0.f;
        if (a.zdump) a.zdump[p] = z;
        if (bad) {
          best.wrong += 1;
          const int64_t k1 = ((int64_t)__float_as_uint(z) << 32) | (p & 0xFFFFFFFFll);
          best.key = k1 > best.key ? k1 : best.key;
          best.keyd = best.key;
        }
      }
    } else {
      double pl = 0.0, sg = 0.0, sq = 0.0;
      bool imp = false;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        pl += x[i];
        sg = fma(x[i], (double)sgn[i], sg);
        sq = fma(x[i], x[i], sq);
      }
#pragma unroll
      for (int msk = 1; msk < 16; msk <<= 1) {
        pl += shfl_xor_d(pl, msk);
        sg += shfl_xor_d(sg, msk);
        sq += shfl_xor_d(sq, msk);
      }
      // Cauchy-Schwarz per output: |c_ij| > 2 |sa_i Aq_i| |sb_j Bq_j|
      if (live) {
        double asq = 0.0;
#pragma unroll
        for (int s = 0; s < SDC_MAX_SPLITS; ++s)
          if (s < a.splits) asq += (double)a.XN[s * 2 * a.m + r];
        const double an = (a.sa ? (double)a.sa[r] : 1.0) * sqrt(asq);
#pragma unroll
        for (int i = 0; i < 8; ++i)
          if (8 * e + i < wid) imp = imp || (fabs(x[i]) > 2.0 * an * (double)a.bcol[c0 + i] + 1e-300);
      }
      int impi = imp ? 1 : 0;                               // combined over the pair's 16 lanes
#pragma unroll
      for (int msk = 1; msk < 16; msk <<= 1) impi |= __shfl_xor(impi, msk, 64);
      if (live && e == 0) {
        float noise;
        const float z = judge_fp8(a, r, jb, pl, sg, sq, impi != 0, noise);
        if (a.zdump) a.zdump[p] = z;
        const bool fin = isfinite(pl) && isfinite(sg);
        best.wrong += z > a.zt;
        best.nonfin += !fin;
        const int64_t zb = (int64_t)__float_as_uint(fmaxf(z, 0.f));
        const int64_t k1 = (zb << 32) | (p & 0xFFFFFFFFll);
        const int64_t k2 = (zb << 32) | (int64_t)__float_as_uint(noise);
        best.key = k1 > best.key ? k1 : best.key;
        best.keyd = k2 > best.keyd ? k2 : best.keyd;
      }
    }
  }
  const int64_t key = wave_max_i64(best.key), keyd = wave_max_i64(best.keyd);
  const int wr = wave_sum_i32(best.wrong), nf = wave_sum_i32(best.nonfin);
  if (lane == 0) { red_k[w] = key; red_d[w] = keyd; red_w[w] = wr; red_n[w] = nf; }
  __syncthreads();
  if (t == 0) {
    int64_t k0 = red_k[0], d0 = red_d[0];
    int wsum = red_w[0], nsum = red_n[0];
    for (int i = 1; i < 4; ++i) {
      k0 = red_k[i] > k0 ? red_k[i] : k0;
      d0 = red_d[i] > d0 ? red_d[i] : d0;
      wsum += red_w[i];
      nsum += red_n[i];
    }
    int64_t* res = a.result;
    const int64_t s0 = __atomic_load_n(res, __ATOMIC_RELAXED), s1 = __atomic_load_n(res + 1, __ATOMIC_RELAXED);
    if (k0 > s0) atomicMax((unsigned long long*)res, (unsigned long long)k0);
    if (d0 > s1) atomicMax((unsigned long long*)(res + 1), (unsigned long long)d0);
    if (wsum > 0) atomicAdd((unsigned long long*)(res + 2), (unsigned long long)wsum);
    if (nsum > 0) atomicAdd((unsigned long long*)(res + 3), (unsigned long long)nsum);
  }
}

struct QLayout {
  int64_t nb, rem, ncols, splits, nacc, off_e, off_xn, total;
};

QLayout qlayout(int kind, int64_t m, int64_t k, int64_t n, int64_t bs) {
  QLayout L{};
  L.nb = sdc_cdiv(n, bs);
  L.rem = n % bs;
  L.ncols = 2 * L.nb;
  L.nacc = kind == 0 ? 2 : 1;
  L.splits = sdc_expected_splits(m, kind == 0 ? k / 2 : k, L.ncols);
  auto al = [](int64_t x) { return (x + 63) / 64 * 64; };
  int64_t o = 0;
  L.off_e = o; o += al(L.splits * L.nacc * m * L.ncols);
  L.off_xn = o; o += al(L.splits * 2 * m);
  L.total = o;
  return L;
}

template <int KIND, int CT>
void launch_score(const QuantArgs& qa, unsigned grid, hipStream_t stream) {
  hipLaunchKernelGGL((quant_score_kernel<KIND, CT>), dim3(grid), dim3(256), 0, stream, qa);
}

}  // namespace

extern "C" int64_t sdc_quant_check_workspace(int kind, int64_t m, int64_t k, int64_t n, int64_t bs) {
  if ((kind != 0 && kind != 1) || m <= 0 || k <= 0 || n <= 0 || bs <= 0) return 0;
  return qlayout(kind, m, k, n, bs).total * (int64_t)sizeof(float) + 256;
}

extern "C" int sdc_quant_check(int kind, const void* A, int64_t sam, const void* parts, int64_t spc, const float* sa,
                               const void* C, int64_t scm, int64_t scn, int c_dtype, int64_t m, int64_t k, int64_t n,
                               int64_t bs, const float* sign_table, const float* bfrob, const float* bcol, float unit,
                               float nfma, float z, int64_t* result, void* workspace, int64_t workspace_bytes,
                               float* scores_out, hipStream_t stream) {
  SDC_CLEAR_ERRORS();
  if (kind != 0 && kind != 1) return SDC_EINVAL;
  if (m < 1 || n < 1 || k < 1 || !A || !parts || !C || !sign_table || !result) return SDC_EINVAL;
  if (bs < 1 || bs > 128) return SDC_EUNSUPPORTED;
  if (kind == 0 && c_dtype != C_I32) return SDC_EINVAL;
  if (kind == 1 && c_dtype != C_F32 && c_dtype != C_BF16) return SDC_EINVAL;
  if (kind == 1 && (!bfrob || !bcol)) return SDC_EINVAL;
  // int8 runs the GEMM on pairs of bytes: even depth and row strides
  if (kind == 0 && ((k % 2) || (sam % 2) || (spc % 2) || ((uintptr_t)A % 2) || ((uintptr_t)parts % 2)))
    return SDC_EUNSUPPORTED;
  const QLayout L = qlayout(kind, m, k, n, bs);
  if (m * L.nb > 0xFFFFFFFFll) return SDC_EUNSUPPORTED;
  if (!workspace || workspace_bytes < L.total * (int64_t)sizeof(float) + 256) return SDC_EWORKSPACE;
  float* ws = (float*)(((uintptr_t)workspace + 255) & ~(uintptr_t)255);
  const float* s_full = sign_table + (bs - 1) * 128;
  const float* s_last = L.rem ? sign_table + (L.rem - 1) * 128 : s_full;

  GemmArgs g{};
  g.A = (const uint16_t*)A;
  g.sab = 0;
  g.sam = kind == 0 ? sam / 2 : sam;
  g.sak = 1;
  g.B = parts; g.sbb = 0; g.sbc = kind == 0 ? spc / 2 : spc;
  g.m = m; g.k = kind == 0 ? k / 2 : k; g.N = L.ncols; g.splits = L.splits;
  g.E = ws + L.off_e; g.XN = ws + L.off_xn;
  g.prof_name = kind == 0 ? "quant_gemm_i8" : "quant_gemm_fp8";
  int rc = sdc_gemm_launch(kind == 0 ? SDC_I8 : SDC_FP8, g, 1, stream);
  if (rc != SDC_OK) return rc;

  QuantArgs qa{};
  qa.C = C; qa.scm = scm; qa.scn = scn;
  qa.m = m; qa.n = n; qa.nb = L.nb; qa.bs = bs; qa.rem = L.rem; qa.npairs = m * L.nb;
  const int es = c_dtype == C_BF16 ? 2 : 4;
  qa.vec = scn == 1 && ((scm * es) % 16 == 0) && ((bs * es) % 16 == 0) && ((uintptr_t)C % 16 == 0);
  qa.s_full = s_full; qa.s_last = s_last;
  qa.E = ws + L.off_e; qa.XN = ws + L.off_xn; qa.splits = L.splits; qa.ncols = L.ncols;
  qa.sa = sa; qa.bfrob = bfrob; qa.bcol = bcol;
  qa.unit = unit;
  qa.per_out = (float)(sqrt((double)k) + (nfma > 0.f ? (double)k / (double)nfma : 0.0));
  qa.zt = z;
  qa.c_bf16 = c_dtype == C_BF16;
  qa.result = result; qa.zdump = scores_out;
  const int64_t groups = sdc_cdiv(qa.npairs, 4);
  const unsigned grid = (unsigned)(sdc_cdiv(groups, 4) < 2048 ? sdc_cdiv(groups, 4) : 2048);
  SdcProf prof(kind == 0 ? "quant_score_i8" : "quant_score_fp8", stream);
  if (kind == 0) launch_score<0, C_I32>(qa, grid, stream);
  else if (c_dtype == C_F32) launch_score<1, C_F32>(qa, grid, stream);
  else launch_score<1, C_BF16>(qa, grid, stream);
  SDC_LAUNCH_CHECK();
  return SDC_OK;
}
