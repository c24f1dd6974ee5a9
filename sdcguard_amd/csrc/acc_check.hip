// Precise column-block check of C = beta * bias + alpha * (A @ B) with C the fp32 product itself (the accumulator,
// not rounded to 16 bits): checksum.py:537-692 (`matmul_zscores_acc`, `_acc_zscores`, `check_matmul_acc`).
//
// Both sides of every checksum are float64: the block sums of B and of C, and E = A @ B2.  The noise is the fp32
// accumulation's own rounding,
//     u (C1 sqrt(k) |alpha| |a_row|_2 |B_block|_F + (C2 sqrt(k) + C3 k / nfma + sqrt(width)) |C_block|_2),  u = 2^-24,
// judged with the Inf/NaN rules of `_judge_nonfinite` (fp32 outputs, no subnormal step).  MI355X runs float64 FMAs
// on its vector units at the same rate as its fp64 matrix cores, so the expected side is a tiled VALU GEMM.
// Five launches, no host synchronisation:
//   1. acc_bsums: B2 (fp64 plain and signed block sums of every row of B, stored depth-contiguous per checksum
//      column) and per 64-row slice the partial |B|^2 and max |B| of every block;
//   2. acc_finish: |B_block|_F and max |B_block| from those partials, and a bias vector's block sums (fp64) and
//      largest |bias| per block;
//   3. acc_anorm: |a_row|_2 and |a_row|_1 (fp32);
//   4. acc_gemm: E = A @ B2 in float64, 64 x 64 tiles, depth split over workgroups when the tiles alone cannot fill
//      the GPU (each split its own plane, added by the scorer);
//   5. acc_score: one pass over C, 16 lanes per (batch, row, block): fp64 plain and signed sums, |C_block|_2 and
//      |C_block|_1 (fp32), then one lane scores the pair; worst keys and the unjudged count go to the result row.
// sdc_matmul_check_acc_stats scores the same check from the block statistics the fused GEMM leaves instead of C
// (fused.py:181-235, `zscores_from_stats`: 2-D, bias vector, alpha = beta = 1; |C_block|_2 is the square root of
// the float64 sum of squares).
#include "common.h"
#include "profile.h"

namespace {

constexpr int SLICE = 64;          // rows of B per acc_bsums workgroup
constexpr int MAX_SPLITS = 8;      // depth splits of acc_gemm
constexpr double ACC_U = 5.9604644775390625e-08;         // 2^-24, checksum.py:558
constexpr double ACC_C1 = 0.6, ACC_C2 = 1.0, ACC_C3 = 1.0;

__device__ __forceinline__ float nan_abs(float v) { return v == v ? fabsf(v) : __builtin_inff(); }

template <int DT>
__device__ __forceinline__ float elem(const void* p, int64_t i) {
  return half_to_f32<DT>(reinterpret_cast<const uint16_t*>(p)[i]);
}

__device__ __forceinline__ double shfl_xor_f64(double v, int m) { return __shfl_xor(v, m, SDC_WAVE); }

// sum over the 16 lanes of an aligned group (lanes 16 g .. 16 g + 15)
__device__ __forceinline__ double sum16_f64(double v) {
#pragma unroll
  for (int m = 1; m < 16; m <<= 1) v += shfl_xor_f64(v, m);
  return v;
}
__device__ __forceinline__ float sum16_f32(float v) {
#pragma unroll
  for (int m = 1; m < 16; m <<= 1) v += __shfl_xor(v, m, SDC_WAVE);
  return v;
}
__device__ __forceinline__ float max16_f32(float v) {
#pragma unroll
  for (int m = 1; m < 16; m <<= 1) v = fmaxf(v, __shfl_xor(v, m, SDC_WAVE));
  return v;
}

struct AccArgs {
  const void* A;                   // (batch_a, m, k) of dtype
  int64_t sab, sam, sak, batch_a;
  const void* B;                   // (batch_b, k, n) of dtype
  int64_t sbb, sbk, sbn, batch_b;
  const float* C;                  // (batch_c, m, n) fp32
  int64_t scb, scm, scn, batch_c;
  int64_t m, k, n, bs, nb, rem, nslice, splits, kchunk;
  const void* bias;                // dtype (or fp32 with bias_f32), kind 1: (n), kind 2: (batch, m, n) strides
  int bias_kind, bias_f32;
  int64_t sbias_b, sbias_m, sbias_n;
  double alpha, beta;
  double steps;                    // k / nfma (0: no tensor-core truncation steps)
  float z, abs_floor;
  const float* sign_table;         // 128 x 128, row w - 1 = the pattern of width w
  double* B2T;                     // [batch_b][2 nb][k]
  float* part;                     // [batch_b][nslice][nb][2]: sum of squares, max |B|
  float* bstat;                    // [batch_b][nb][2]: |B_block|_F, max |B_block|
  double* bsum;                    // [nb][2]: bias vector block sums (kind 1)
  float* bmax;                     // [nb]: max |bias| of the block (kind 1)
  float* an;                       // [batch_a][2][m]: |a|_2, |a|_1
  double* E;                       // [splits][batch_c][m][2 nb]
  int64_t* result;
  float* scores;                   // (batch_c, m, nb, 2) or null
  const double* stats;             // instead of C: (m, nb, 4) plain, signed, squared, absolute block sums of C
  int64_t sst_m, sst_b;            //   (row and block strides, in doubles)
};

__device__ __forceinline__ int64_t bwidth(const AccArgs& a, int64_t jb) {
  return (jb == a.nb - 1 && a.rem > 0) ? a.rem : a.bs;
}

__device__ __forceinline__ float bias_at(const AccArgs& a, int dt, int64_t i) {
  if (a.bias_f32) return reinterpret_cast<const float*>(a.bias)[i];
  const uint16_t w = reinterpret_cast<const uint16_t*>(a.bias)[i];
  return dt == SDC_BF16 ? half_to_f32<SDC_BF16>(w) : half_to_f32<SDC_FP16>(w);
}

// ---------------------------------------------------------------------------------------------- 1. B-side sums
// Workgroup (slice of 64 rows of B, block jb, batch bb); 16 lanes per row, lane c16 takes the block's columns
// c16, c16 + 16, ... (float64 sums of the bf16/fp16 values, exact up to the sum's size), 16 rows per pass.
template <int DT>
__global__ __launch_bounds__(256) void acc_bsums_kernel(AccArgs a) {
  __shared__ float red[4][2];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, c16 = t & 15, r16 = t >> 4;
  const int64_t sl = blockIdx.x, jb = blockIdx.y, bb = blockIdx.z;
  const int64_t wid = bwidth(a, jb);
  const float* sp = a.sign_table + (wid - 1) * 128;
  float sq = 0.f, mx = 0.f;
  for (int rr = 0; rr < SLICE; rr += 16) {
    const int64_t kk = sl * SLICE + rr + r16;
    double pl = 0.0, sg = 0.0;
    if (kk < a.k) {
      const int64_t base = bb * a.sbb + kk * a.sbk + jb * a.bs * a.sbn;
      for (int64_t c = c16; c < wid; c += 16) {
        const float x = elem<DT>(a.B, base + c * a.sbn);
        pl += (double)x;
        sg += (double)x * (double)sp[c];
        sq = fmaf(x, x, sq);
        mx = fmaxf(mx, nan_abs(x));
      }
    }
    pl = sum16_f64(pl);
    sg = sum16_f64(sg);
    if (c16 == 0 && kk < a.k) {
      double* col = a.B2T + (bb * 2 * a.nb + 2 * jb) * a.k;
      col[kk] = pl;
      col[a.k + kk] = sg;
    }
  }
#pragma unroll
  for (int msk = 1; msk < 64; msk <<= 1) {
    sq += __shfl_xor(sq, msk, SDC_WAVE);
    mx = fmaxf(mx, __shfl_xor(mx, msk, SDC_WAVE));
  }
  if (lane == 0) {
    red[w][0] = sq;
    red[w][1] = mx;
  }
  __syncthreads();
  if (t == 0) {
    float s = red[0][0], m = red[0][1];
    for (int i = 1; i < 4; ++i) {
      s += red[i][0];
      m = fmaxf(m, red[i][1]);
    }
    float* p = a.part + ((bb * a.nslice + sl) * a.nb + jb) * 2;
    p[0] = s;
    p[1] = m;
  }
}

// ------------------------------------------------------------------------- 2. block norms and bias block sums
// One thread per (batch of B, block): the slices' partials added in slice order.  Thread blocks past those: the
// bias vector's per-block fp64 sums and largest |bias| (kind 1).
template <int DT>
__global__ __launch_bounds__(256) void acc_finish_kernel(AccArgs a) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t nbb = a.batch_b * a.nb;
  if (i < nbb) {
    const int64_t bb = i / a.nb, jb = i % a.nb;
    float s = 0.f, m = 0.f;
    for (int64_t sl = 0; sl < a.nslice; ++sl) {
      const float* p = a.part + ((bb * a.nslice + sl) * a.nb + jb) * 2;
      s += p[0];
      m = fmaxf(m, p[1]);
    }
    a.bstat[i * 2] = sqrtf(s);
    a.bstat[i * 2 + 1] = m;
  } else if (a.bias_kind == 1 && i < nbb + a.nb) {
    const int64_t jb = i - nbb, wid = bwidth(a, jb);
    const float* sp = a.sign_table + (wid - 1) * 128;
    double pl = 0.0, sg = 0.0;
    float mx = 0.f;
    for (int64_t c = 0; c < wid; ++c) {
      const float v = bias_at(a, DT, (jb * a.bs + c) * a.sbias_n);
      pl += (double)v;
      sg += (double)v * (double)sp[c];
      mx = fmaxf(mx, nan_abs(v));
    }
    a.bsum[jb * 2] = pl;
    a.bsum[jb * 2 + 1] = sg;
    a.bmax[jb] = mx;
  }
}

// ---------------------------------------------------------------------------------------------- 3. A row norms
template <int DT>
__global__ __launch_bounds__(256) void acc_anorm_kernel(AccArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6), ba = blockIdx.y;
  if (row >= a.m) return;
  const int64_t base = ba * a.sab + row * a.sam;
  float sq = 0.f, l1 = 0.f;
  for (int64_t kk = lane; kk < a.k; kk += 64) {
    const float x = elem<DT>(a.A, base + kk * a.sak);
    sq = fmaf(x, x, sq);
    l1 += fabsf(x);
  }
  sq = wave_sum_f32(sq);
  l1 = wave_sum_f32(l1);
  if (lane == 0) {
    a.an[(ba * 2) * a.m + row] = sqrtf(sq);
    a.an[(ba * 2 + 1) * a.m + row] = l1;
  }
}

// ------------------------------------------------------------------------------------- 4. E = A @ B2 (float64)
// Workgroup: 64 rows x 64 checksum columns of one batch and one depth split; thread (tr, tc) = (t / 16, t % 16)
// owns rows 4 tr .. 4 tr + 3 and columns tc, tc + 16, tc + 32, tc + 48.  Depth advances 16 at a time through LDS
// (A converted to float64 on the way in); columns and rows past the ends read as zero and are not stored.
constexpr int GT = 64, GK = 16;

template <int DT>
__global__ __launch_bounds__(256) void acc_gemm_kernel(AccArgs a) {
  __shared__ double As[GK][GT + 1];
  __shared__ double Bs[GK][GT + 1];
  const int t = threadIdx.x, tr = t >> 4, tc = t & 15;
  const int64_t nc = 2 * a.nb;
  const int64_t ctiles = sdc_cdiv(nc, GT);
  const int64_t ct = blockIdx.x % ctiles, rt = blockIdx.x / ctiles;
  const int64_t split = blockIdx.y, bc = blockIdx.z;
  const int64_t ba = a.batch_a == 1 ? 0 : bc, bb = a.batch_b == 1 ? 0 : bc;
  const int64_t r0 = rt * GT, c0 = ct * GT;
  const int64_t kb = split * a.kchunk, ke = kb + a.kchunk < a.k ? kb + a.kchunk : a.k;
  double acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.0;
  const double* B2 = a.B2T + bb * nc * a.k;
  for (int64_t k0 = kb; k0 < ke; k0 += GK) {
    // A tile: 64 rows x 16 depths (4 per thread); B2 tile: 16 depths x 64 columns (4 per thread)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int e = t + 256 * q, r = e >> 4, d = e & 15;
      const int64_t row = r0 + r, kk = k0 + d;
      As[d][r] = (row < a.m && kk < ke) ? (double)elem<DT>(a.A, ba * a.sab + row * a.sam + kk * a.sak) : 0.0;
      const int c = e >> 4;
      const int64_t col = c0 + c;
      Bs[d][c] = (col < nc && kk < ke) ? B2[col * a.k + kk] : 0.0;
    }
    __syncthreads();
#pragma unroll
    for (int d = 0; d < GK; ++d) {
      double av[4], bv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = As[d][4 * tr + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) bv[j] = Bs[d][tc + 16 * j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fma(av[i], bv[j], acc[i][j]);
    }
    __syncthreads();
  }
  double* Ep = a.E + ((split * a.batch_c + bc) * a.m) * nc;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t row = r0 + 4 * tr + i;
    if (row >= a.m) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t col = c0 + tc + 16 * j;
      if (col < nc) Ep[row * nc + col] = acc[i][j];
    }
  }
}

// ------------------------------------------------------------------------------------------------ 5. scoring
// One checksum of the precise check, scored as checksum.py:640-670 scores it: z = |expected - actual| / (noise +
// abs_floor) in float64 (the plain one also against the L1 bound), then `_judge_nonfinite` with fp32 outputs.
__device__ __forceinline__ float acc_judge(double e, double act, float noise, float worst, float bound, float cn,
                                           float wf, bool plain, const AccArgs& a, float& den32) {
  const float inf = __builtin_inff();
  const float den = noise + a.abs_floor;
  den32 = den;
  const double diff = fabs(e - act);
  double zd = diff / (double)den;
  if (plain) {
    const double zw = diff / (double)worst * (double)a.z;
    zd = (zd == zd && zw == zw) ? fmin(zd, zw) : __builtin_nan("");
  }
  float zf = (float)zd;
  const bool e_bad = !(fabs(e) < __builtin_inf());
  const bool a_bad = !(fabs(act) < __builtin_inf()) && !e_bad;
  const bool big = !(noise < inf) && !e_bad && !a_bad;
  const float lim = bound * 1.01f;
  zf = zf == zf ? zf : -1.f;
  zf = e_bad ? -1.f : zf;
  const float cap = bound * (float)(1.02 + (double)a.k * 2.384185791015625e-07);
  const bool imposs = !e_bad && !a_bad && !big && (lim < 1e18f) && (cn > cap * sqrtf(wf));
  zf = imposs ? inf : zf;
  zf = a_bad ? (lim < 1e18f ? inf : -1.f) : zf;
  zf = big ? (lim < 1e18f ? inf : -1.f) : zf;
  return zf;
}

// 16 pairs per workgroup: lanes 16 g .. 16 g + 15 of a wave take one (batch, row, block) pair; lane c16 adds the
// block's columns c16, c16 + 16, ... (full 128-wide blocks of a row-contiguous C: 8 columns, two 16-byte loads).
template <int DT>
__global__ __launch_bounds__(256) void acc_score_kernel(AccArgs a) {
  __shared__ int64_t rk[4], rd[4];
  __shared__ int ru[4];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, c16 = t & 15;
  const int64_t npairs = a.batch_c * a.m * a.nb;
  const int64_t p = (int64_t)blockIdx.x * 16 + (t >> 4);
  const bool live = p < npairs;
  const int64_t pp = live ? p : 0;
  const int64_t jb = pp % a.nb, row = (pp / a.nb) % a.m, bc = pp / (a.nb * a.m);
  const int64_t wid = bwidth(a, jb);
  const float* sp = a.sign_table + (wid - 1) * 128;
  const int64_t cbase = bc * a.scb + row * a.scm + jb * a.bs * a.scn;
  double pl = 0.0, sg = 0.0, bpl = 0.0, bsg = 0.0;
  float sq = 0.f, l1 = 0.f, bmx = 0.f;
  double sqd = 0.0;
  if (live && a.stats) {                    // the fused kernel's block statistics (fused.py:205-207)
    if (c16 == 0) {
      const double* st = a.stats + row * a.sst_m + jb * a.sst_b;
      pl = st[0];
      sg = st[1];
      sqd = st[2];
      l1 = (float)st[3];
    }
  } else if (live) {
    if (a.scn == 1 && wid == 128 && ((uintptr_t)(a.C + cbase) & 15) == 0) {
      const f32x4 v0 = *reinterpret_cast<const f32x4*>(a.C + cbase + 8 * c16);
      const f32x4 v1 = *reinterpret_cast<const f32x4*>(a.C + cbase + 8 * c16 + 4);
      const f32x4 s0 = *reinterpret_cast<const f32x4*>(sp + 8 * c16);
      const f32x4 s1 = *reinterpret_cast<const f32x4*>(sp + 8 * c16 + 4);
      const float x[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
      const float s[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        pl += (double)x[e];
        sg += (double)x[e] * (double)s[e];
        sq = fmaf(x[e], x[e], sq);
        l1 += fabsf(x[e]);
      }
    } else {
      for (int64_t c = c16; c < wid; c += 16) {
        const float x = a.C[cbase + c * a.scn];
        pl += (double)x;
        sg += (double)x * (double)sp[c];
        sq = fmaf(x, x, sq);
        l1 += fabsf(x);
      }
    }
    if (a.bias_kind == 2 && !a.stats) {
      const int64_t bb0 = bc * a.sbias_b + row * a.sbias_m + jb * a.bs * a.sbias_n;
      for (int64_t c = c16; c < wid; c += 16) {
        const float v = bias_at(a, DT, bb0 + c * a.sbias_n);
        bpl += (double)v;
        bsg += (double)v * (double)sp[c];
        bmx = fmaxf(bmx, nan_abs(v));
      }
    }
  }
  pl = sum16_f64(pl);
  sg = sum16_f64(sg);
  sq = sum16_f32(sq);
  l1 = sum16_f32(l1);
  if (a.bias_kind == 2) {
    bpl = sum16_f64(bpl);
    bsg = sum16_f64(bsg);
    bmx = max16_f32(bmx);
  }
  int64_t key = 0, keyd = 0;
  int unk = 0;
  if (live && c16 == 0) {
    const int64_t ba = a.batch_a == 1 ? 0 : bc, bb = a.batch_b == 1 ? 0 : bc;
    const int64_t nc = 2 * a.nb;
    double e0 = 0.0, e1 = 0.0;
    for (int64_t s = 0; s < a.splits; ++s) {
      const double* Ep = a.E + ((s * a.batch_c + bc) * a.m + row) * nc + 2 * jb;
      e0 += Ep[0];
      e1 += Ep[1];
    }
    const float anorm = a.an[(ba * 2) * a.m + row], al1 = a.an[(ba * 2 + 1) * a.m + row];
    const float bfrob = a.bstat[(bb * a.nb + jb) * 2], bmaxb = a.bstat[(bb * a.nb + jb) * 2 + 1];
    float bound = al1 * bmaxb;
    if (a.alpha != 1.0) {
      e0 *= a.alpha;
      e1 *= a.alpha;
      bound = bound * (float)fabs(a.alpha);
    }
    if (a.bias_kind != 0 && a.beta != 0.0) {
      if (a.bias_kind == 1) {
        bpl = a.bsum[jb * 2];
        bsg = a.bsum[jb * 2 + 1];
        bmx = a.bmax[jb];
      }
      e0 += a.beta * bpl;
      e1 += a.beta * bsg;
      bound = bound + (float)fabs(a.beta) * bmx;
    }
    const float wf = (float)wid;
    // from statistics: sqrt of the float64 sum of squares (a NaN stays NaN), rounded to fp32
    const float cn = a.stats ? (float)sqrt(sqd < 0.0 ? 0.0 : sqd) : sqrtf(sq);
    const float per_out_u = (float)((ACC_C2 * sqrt((double)a.k) + ACC_C3 * a.steps + sqrt((double)wid)) * ACC_U);
    float prod = (anorm * bfrob) * (float)(ACC_C1 * sqrt((double)a.k) * fabs(a.alpha) * ACC_U);
    prod = fabsf(prod) < __builtin_inff() ? prod : bound * (float)(ACC_U * 128.0);
    const float noise = cn * per_out_u + prod;
    const float worst = (l1 * per_out_u + prod) + a.abs_floor;
    float d0, d1;
    const float z0 = acc_judge(e0, pl, noise, worst, bound, cn, wf, true, a, d0);
    const float z1 = acc_judge(e1, sg, noise, worst, bound, cn, wf, false, a, d1);
    const int64_t flat = ((bc * a.m + row) * a.nb + jb);
    if (a.scores) {
      a.scores[2 * flat] = z0;
      a.scores[2 * flat + 1] = z1;
    }
    unk = (z0 < 0.f) + (z1 < 0.f);
    const bool sec = z1 > z0;
    const float zc = sec ? z1 : z0, dc = sec ? d1 : d0;
    const int64_t zb = fbits64(fmaxf(zc, 0.f));
    key = (zb << 32) | ((flat * 2 + (sec ? 1 : 0)) & 0xFFFFFFFFll);
    keyd = (zb << 32) | (fbits64(dc) & 0xFFFFFFFFll);
  }
  key = wave_max_i64(key);
  keyd = wave_max_i64(keyd);
  unk = wave_sum_i32(unk);
  if (lane == 0) {
    rk[w] = key;
    rd[w] = keyd;
    ru[w] = unk;
  }
  __syncthreads();
  if (t == 0) {
    int64_t k0 = rk[0], d0 = rd[0];
    int u = ru[0];
    for (int i = 1; i < 4; ++i) {
      k0 = rk[i] > k0 ? rk[i] : k0;
      d0 = rd[i] > d0 ? rd[i] : d0;
      u += ru[i];
    }
    if (k0 > __atomic_load_n(a.result, __ATOMIC_RELAXED)) atomicMax((unsigned long long*)a.result, (unsigned long long)k0);
    if (d0 > __atomic_load_n(a.result + 1, __ATOMIC_RELAXED))
      atomicMax((unsigned long long*)(a.result + 1), (unsigned long long)d0);
    if (u > 0) atomicAdd((unsigned long long*)(a.result + 2), (unsigned long long)u);
  }
}

struct AccLayout {
  int64_t nb, nslice, splits, kchunk;
  int64_t off_b2, off_part, off_bstat, off_bsum, off_bmax, off_an, off_e, total;   // bytes
};

AccLayout acc_layout(int64_t batch_a, int64_t batch_b, int64_t batch_c, int64_t m, int64_t k, int64_t n,
                     int64_t bs) {
  AccLayout L{};
  L.nb = sdc_cdiv(n, bs);
  L.nslice = sdc_cdiv(k, SLICE);
  const int64_t tiles = sdc_cdiv(m, GT) * sdc_cdiv(2 * L.nb, GT) * batch_c;
  int64_t s = sdc_cdiv(256, tiles);
  const int64_t smax = k / 256 > 1 ? k / 256 : 1;
  s = s < smax ? s : smax;
  s = s < MAX_SPLITS ? s : MAX_SPLITS;
  L.splits = s < 1 ? 1 : s;
  L.kchunk = sdc_cdiv(sdc_cdiv(k, L.splits), GK) * GK;
  auto al = [](int64_t x) { return (x + 255) / 256 * 256; };
  int64_t o = 0;
  L.off_b2 = o; o += al(batch_b * 2 * L.nb * k * 8);
  L.off_part = o; o += al(batch_b * L.nslice * L.nb * 2 * 4);
  L.off_bstat = o; o += al(batch_b * L.nb * 2 * 4);
  L.off_bsum = o; o += al(L.nb * 2 * 8);
  L.off_bmax = o; o += al(L.nb * 4);
  L.off_an = o; o += al(batch_a * 2 * m * 4);
  L.off_e = o; o += al(L.splits * batch_c * m * 2 * L.nb * 8);
  L.total = o;
  return L;
}

template <int DT>
int acc_run(AccArgs a, const AccLayout& L, int64_t batch_a, hipStream_t stream) {
  {
    SdcProf prof("acc_bsums", stream);
    hipLaunchKernelGGL(acc_bsums_kernel<DT>, dim3((unsigned)L.nslice, (unsigned)L.nb, (unsigned)a.batch_b), dim3(256),
                       0, stream, a);
    SDC_LAUNCH_CHECK();
  }
  {
    SdcProf prof("acc_finish", stream);
    const int64_t nthr = a.batch_b * L.nb + L.nb;
    hipLaunchKernelGGL(acc_finish_kernel<DT>, dim3((unsigned)sdc_cdiv(nthr, 256)), dim3(256), 0, stream, a);
    SDC_LAUNCH_CHECK();
  }
  {
    SdcProf prof("acc_anorm", stream);
    hipLaunchKernelGGL(acc_anorm_kernel<DT>, dim3((unsigned)sdc_cdiv(a.m, 4), (unsigned)batch_a), dim3(256), 0, stream, a);
    SDC_LAUNCH_CHECK();
  }
  {
    SdcProf prof("acc_gemm", stream);
    const int64_t tiles = sdc_cdiv(a.m, GT) * sdc_cdiv(2 * L.nb, GT);
    hipLaunchKernelGGL(acc_gemm_kernel<DT>, dim3((unsigned)tiles, (unsigned)L.splits, (unsigned)a.batch_c), dim3(256),
                       0, stream, a);
    SDC_LAUNCH_CHECK();
  }
  {
    SdcProf prof("acc_score", stream);
    const int64_t npairs = a.batch_c * a.m * L.nb;
    hipLaunchKernelGGL(acc_score_kernel<DT>, dim3((unsigned)sdc_cdiv(npairs, 16)), dim3(256), 0, stream, a);
    SDC_LAUNCH_CHECK();
  }
  return SDC_OK;
}

}  // namespace

extern "C" int64_t sdc_matmul_check_acc_workspace(int64_t batch_a, int64_t batch_b, int64_t batch_c, int64_t m,
                                                  int64_t k, int64_t n, int64_t bs) {
  if (batch_a < 1 || batch_b < 1 || batch_c < 1 || m < 1 || k < 1 || n < 1 || bs < 1) return 0;
  return acc_layout(batch_a, batch_b, batch_c, m, k, n, bs < 128 ? bs : 128).total + 256;
}

extern "C" int sdc_matmul_check_acc_stats(int dtype, const void* A, int64_t sam, int64_t sak, const void* B,
                                          int64_t sbk, int64_t sbn, const double* stats, int64_t sst_m,
                                          int64_t sst_b, int64_t m, int64_t k, int64_t n, const void* bias,
                                          int bias_f32, float nfma, float z, float abs_floor,
                                          const float* sign_table, int64_t* result, void* workspace,
                                          int64_t workspace_bytes, float* scores_out, hipStream_t stream) {
  SDC_CLEAR_ERRORS();
  if (dtype != SDC_BF16 && dtype != SDC_FP16) return SDC_EUNSUPPORTED;
  if (!A || !B || !stats || !sign_table || !result) return SDC_EINVAL;
  if (m < 1 || k < 1 || n < 1) return SDC_EINVAL;
  const int64_t bw = n < 128 ? n : 128;
  const AccLayout L = acc_layout(1, 1, 1, m, k, n, bw);
  if (m * L.nb * 2 > 0xFFFFFFFFll) return SDC_EUNSUPPORTED;
  if (!workspace || workspace_bytes < L.total + 256) return SDC_EWORKSPACE;
  uint8_t* ws = (uint8_t*)(((uintptr_t)workspace + 255) & ~(uintptr_t)255);
  AccArgs a{};
  a.A = A; a.sab = 0; a.sam = sam; a.sak = sak; a.batch_a = 1;
  a.B = B; a.sbb = 0; a.sbk = sbk; a.sbn = sbn; a.batch_b = 1;
  a.C = nullptr; a.batch_c = 1;
  a.stats = stats; a.sst_m = sst_m; a.sst_b = sst_b;
  a.m = m; a.k = k; a.n = n; a.bs = bw; a.nb = L.nb; a.rem = n % bw; a.nslice = L.nslice;
  a.splits = L.splits; a.kchunk = L.kchunk;
  a.bias = bias; a.bias_kind = bias ? 1 : 0; a.bias_f32 = bias_f32; a.sbias_n = 1;
  a.alpha = 1.0; a.beta = 1.0; a.steps = nfma > 0.f ? (double)k / (double)nfma : 0.0;
  a.z = z; a.abs_floor = abs_floor; a.sign_table = sign_table;
  a.B2T = (double*)(ws + L.off_b2); a.part = (float*)(ws + L.off_part); a.bstat = (float*)(ws + L.off_bstat);
  a.bsum = (double*)(ws + L.off_bsum); a.bmax = (float*)(ws + L.off_bmax); a.an = (float*)(ws + L.off_an);
  a.E = (double*)(ws + L.off_e); a.result = result; a.scores = scores_out;
  return dtype == SDC_BF16 ? acc_run<SDC_BF16>(a, L, 1, stream) : acc_run<SDC_FP16>(a, L, 1, stream);
}

extern "C" int sdc_matmul_check_acc(int dtype, const void* A, int64_t sab, int64_t sam, int64_t sak, int64_t batch_a,
                                    const void* B, int64_t sbb, int64_t sbk, int64_t sbn, int64_t batch_b,
                                    const float* C, int64_t scb, int64_t scm, int64_t scn, int64_t batch_c, int64_t m,
                                    int64_t k, int64_t n, int64_t bs, const void* bias, int bias_kind, int64_t sbias_b,
                                    int64_t sbias_m, int64_t sbias_n, float alpha, float beta, float nfma, float z,
                                    float abs_floor, const float* sign_table, int64_t* result, void* workspace,
                                    int64_t workspace_bytes, float* scores_out, hipStream_t stream) {
  SDC_CLEAR_ERRORS();
  if (dtype != SDC_BF16 && dtype != SDC_FP16) return SDC_EUNSUPPORTED;
  if (!A || !B || !C || !sign_table || !result) return SDC_EINVAL;
  if (m < 1 || k < 1 || n < 1 || bs < 1 || bs > 128) return SDC_EINVAL;
  if (batch_c < 1 || (batch_a != 1 && batch_a != batch_c) || (batch_b != 1 && batch_b != batch_c)) return SDC_EINVAL;
  const int kind = bias_kind & 3, bias32 = (bias_kind & 4) != 0;
  if (kind > 2 || (kind && !bias)) return SDC_EINVAL;
  const int64_t bw = bs < n ? bs : n;
  const AccLayout L = acc_layout(batch_a, batch_b, batch_c, m, k, n, bw);
  if (m * L.nb * batch_c * 2 > 0xFFFFFFFFll) return SDC_EUNSUPPORTED;      // flat indexes fit the key's 32 bits
  if (!workspace || workspace_bytes < L.total + 256) return SDC_EWORKSPACE;
  uint8_t* ws = (uint8_t*)(((uintptr_t)workspace + 255) & ~(uintptr_t)255);
  AccArgs a{};
  a.A = A; a.sab = sab; a.sam = sam; a.sak = sak; a.batch_a = batch_a;
  a.B = B; a.sbb = sbb; a.sbk = sbk; a.sbn = sbn; a.batch_b = batch_b;
  a.C = C; a.scb = scb; a.scm = scm; a.scn = scn; a.batch_c = batch_c;
  a.m = m; a.k = k; a.n = n; a.bs = bw; a.nb = L.nb; a.rem = n % bw; a.nslice = L.nslice;
  a.splits = L.splits; a.kchunk = L.kchunk;
  a.bias = bias; a.bias_kind = kind; a.bias_f32 = bias32; a.sbias_b = sbias_b; a.sbias_m = sbias_m; a.sbias_n = sbias_n;
  a.alpha = alpha; a.beta = beta; a.steps = nfma > 0.f ? (double)k / (double)nfma : 0.0;
  a.z = z; a.abs_floor = abs_floor; a.sign_table = sign_table;
  a.B2T = (double*)(ws + L.off_b2); a.part = (float*)(ws + L.off_part); a.bstat = (float*)(ws + L.off_bstat);
  a.bsum = (double*)(ws + L.off_bsum); a.bmax = (float*)(ws + L.off_bmax); a.an = (float*)(ws + L.off_an);
  a.E = (double*)(ws + L.off_e); a.result = result; a.scores = scores_out;
  return dtype == SDC_BF16 ? acc_run<SDC_BF16>(a, L, batch_a, stream) : acc_run<SDC_FP16>(a, L, batch_a, stream);
}
