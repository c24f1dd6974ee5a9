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
// then one pass over C: for blocks of 128 and rows read in 16-byte pieces, the tile pass (quant_tile_kernel:
// 128 (bf16 C) or 64 rows x one block per workgroup, sums in int64 or fp32 across 16 lanes, one lane per pair
// judging); otherwise a persistent pass with 16 lanes per (row, block) pair, the sums in int64 or fp64.
#include "common.h"
#include "gemm.h"
#include "profile.h"


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
#pragma unroll 4
  for (int s = 0; s < a.splits; ++s) {
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
#pragma unroll 4
        for (int s = 0; s < a.splits; ++s) {
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
#pragma unroll 4
        for (int s = 0; s < a.splits; ++s) asq += (double)a.XN[s * 2 * a.m + r];
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

// The tile pass (blocks of 128 columns, C read along rows in 16-byte pieces): one workgroup owns 64 rows x one
// column block.  Thread t = 16 rg + cg reads rows 4 rg .. 4 rg + 3, columns 8 cg .. 8 cg + 7 (a wave's load covers
// 4 rows x a whole block); its partial sums of each row go to the row's 16 lanes by DPP steps, and to LDS.  Wave 0
// prepares the rows' norms (fp8: |sa_i Aq_i| for the Cauchy-Schwarz rule, which every element checks) and then
// judges the 64 pairs, one lane each, reading the expected sums from transposed planes (consecutive rows).
__device__ __forceinline__ float sum16(float v) {
  v += dpp_xor1(v);
  v += dpp_xor2(v);
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));  // half mirror
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));  // row mirror
  return v;
}

// int32 sum over the 16 lanes of a DPP row (every lane holding it)
__device__ __forceinline__ int sum16_i32(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, true);    // xor 1
  v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, true);    // xor 2
  v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, true);   // half mirror
  v += __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, true);   // row mirror
  return v;
}

__device__ __forceinline__ int64_t sum16_i64(int64_t v) {
#pragma unroll
  for (int msk = 1; msk < 16; msk <<= 1) v += shfl_xor_i64(v, msk);
  return v;
}

// FEW: at most SDC_MAX_SPLITS depth splits (the launch picks the instance: each holds only its own way of adding
// the splits, which measured faster than one kernel holding both)
// NS: the most planes the instance adds with all loads in flight (2: the tall-tile GEMM's pair)
// RPT: rows per thread; the tile is 16 RPT rows (64 or 128) x 128 columns, and its RPT / 4 first waves load the
// expected sums of one row each and score them
template <int KIND, int CT, bool FEW, int NS = SDC_MAX_SPLITS, int RPT = 4>
__global__ __launch_bounds__(256) void quant_tile_kernel(QuantArgs a) {
  constexpr int ES = CT == C_BF16 ? 2 : 4;                  // bytes per C element
  constexpr int NL = 8 * ES / 16;                           // 16-byte loads per row piece (1 or 2)
  constexpr int TRW = 16 * RPT, NSW = TRW / 64;             // tile rows, scoring waves
  static_assert(RPT == 4 || RPT == 8, "64- or 128-row tiles");
  __shared__ float an_s[TRW];                               // fp8: 2 |sa_i Aq_i| per row (the rule's limit)
  __shared__ float imp_s[TRW];                              // fp8: lanes of the row that broke the rule
  __shared__ float srow[TRW][4];                            // fp8: plain, signed, squares, |sa_i Aq_i|
  __shared__ int64_t irow[TRW][2];                          // int8: plain, signed
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int rg = t >> 4, cg = t & 15;
  const int64_t jb = blockIdx.x, r0 = (int64_t)blockIdx.y * TRW;
  const int64_t c0 = jb * 128 + 8 * cg;
  const bool scorer = w < NSW;
  // the result row's worst keys as they stand now, read first so the read's latency hides under the tile's (a key
  // at or below them needs no atomic at the end; keys only grow, so a stale value only lets an unneeded one through)
  int64_t seen0 = 0, seen1 = 0;
  if (scorer && lane == 0) {
    seen0 = __atomic_load_n(a.result, __ATOMIC_RELAXED);
    seen1 = __atomic_load_n(a.result + 1, __ATOMIC_RELAXED);
  }
  // C: RPT rows x 8 columns, clamped to row m - 1 (rows past m are never judged); the last block's columns past n
  // are masked at use
  u32x4 v[RPT][NL];
  const uint8_t* base = (const uint8_t*)a.C;
  const int64_t cl = c0 + 8 <= a.n ? c0 : a.n - 8;
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int64_t r = r0 + RPT * rg + i < a.m ? r0 + RPT * rg + i : a.m - 1;
#pragma unroll
    for (int l = 0; l < NL; ++l)
      v[i][l] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(base + (r * a.scm + cl) * ES + 16 * l));
  }
  const int wid = (int)((jb == a.nb - 1 && a.rem > 0) ? a.rem : 128);
  const float* sp = wid == 128 ? a.s_full : a.s_last;
  float sgn[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) sgn[e] = 8 * cg + e < wid ? sp[8 * cg + e] : 0.f;
  const bool on = 8 * cg < wid;                              // this thread's columns exist (a whole piece or none)
  // the scoring waves: the expected sums and (fp8) the row norms of the lane's row
  const int64_t rl = 64 * w + lane;                          // (a scoring wave's row in the tile)
  const int64_t rr = r0 + rl < a.m ? r0 + rl : a.m - 1;
  double e0 = 0.0, e1 = 0.0;
  int64_t i0 = 0, i1 = 0;
  if (scorer) {
    // up to SDC_MAX_SPLITS splits: every split's loads issued at once (an index past a.splits reads split 0 and is
    // not added), then added in split order; more splits (short fp8 GEMMs): four at a time
    if constexpr (KIND == 0) {
      const int32_t* E = reinterpret_cast<const int32_t*>(a.E);
      if constexpr (FEW) {
        int32_t hv[NS][2], lv[NS][2];
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          const int64_t sc = s < a.splits ? s : 0;
          const int32_t* hi = E + ((int64_t)(2 * sc) * a.ncols + 2 * jb) * a.m + rr;
          const int32_t* lo = E + ((int64_t)(2 * sc + 1) * a.ncols + 2 * jb) * a.m + rr;
          hv[s][0] = hi[0]; hv[s][1] = hi[a.m];
          lv[s][0] = lo[0]; lv[s][1] = lo[a.m];
        }
#pragma unroll
        for (int s = 0; s < NS; ++s)
          if (s < a.splits) {
            i0 += 128 * (int64_t)hv[s][0] + (int64_t)lv[s][0];
            i1 += 128 * (int64_t)hv[s][1] + (int64_t)lv[s][1];
          }
      } else {
#pragma unroll 4
        for (int s = 0; s < a.splits; ++s) {
          const int32_t* hi = E + ((int64_t)(2 * s) * a.ncols + 2 * jb) * a.m + rr;
          const int32_t* lo = E + ((int64_t)(2 * s + 1) * a.ncols + 2 * jb) * a.m + rr;
          i0 += 128 * (int64_t)hi[0] + (int64_t)lo[0];
          i1 += 128 * (int64_t)hi[a.m] + (int64_t)lo[a.m];
        }
      }
    } else {
      double asq = 0.0;
      if constexpr (FEW) {
        float ev[NS][3];
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          const int64_t sc = s < a.splits ? s : 0;
          const float* ep = a.E + ((int64_t)sc * a.ncols + 2 * jb) * a.m + rr;
          ev[s][0] = ep[0];
          ev[s][1] = ep[a.m];
          ev[s][2] = a.XN[sc * 2 * a.m + rr];
        }
#pragma unroll
        for (int s = 0; s < NS; ++s)
          if (s < a.splits) {
            e0 += (double)ev[s][0];
            e1 += (double)ev[s][1];
            asq += (double)ev[s][2];
          }
      } else {
#pragma unroll 4
        for (int s = 0; s < a.splits; ++s) {
          const float* ep = a.E + ((int64_t)s * a.ncols + 2 * jb) * a.m + rr;
          e0 += (double)ep[0];
          e1 += (double)ep[a.m];
          asq += (double)a.XN[s * 2 * a.m + rr];
        }
      }
      const double sa = a.sa ? (double)a.sa[rr] : 1.0;
      e0 *= sa;
      e1 *= sa;
      const double an = sa * sqrt(asq);
      an_s[rl] = (float)(2.0 * an);
      srow[rl][3] = (float)an;                               // |sa_i Aq_i| for the noise (e0, e1 stay in registers)
    }
  }
  __syncthreads();
  if constexpr (KIND == 0) {
    // Exact sums of 128 int32 values without 64-bit lane traffic: each value split as x = hi 2^16 + lo (lo in
    // [0, 2^16), hi signed), the halves summed in int32 (|sum| < 2^23 over a block) and over the 16 lanes by DPP
    // adds, then put back together in int64
    int sgi[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) sgi[e] = sgn[e] > 0.f ? 1 : (sgn[e] < 0.f ? -1 : 0);
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      int pl_lo = 0, pl_hi = 0, sg_lo = 0, sg_hi = 0;
      if (on) {
#pragma unroll
        for (int l = 0; l < NL; ++l)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int e = 4 * l + q;
            const int x = (int)v[i][l][q];
            const int lo = x & 0xFFFF, hi = x >> 16;
            pl_lo += lo;
            pl_hi += hi;
            sg_lo += sgi[e] * lo;
            sg_hi += sgi[e] * hi;
          }
      }
      pl_lo = sum16_i32(pl_lo);
      pl_hi = sum16_i32(pl_hi);
      sg_lo = sum16_i32(sg_lo);
      sg_hi = sum16_i32(sg_hi);
      // (the sums finish here, with every lane on: their DPP steps must not move under the store's mask)
      asm volatile("" : "+v"(pl_lo), "+v"(pl_hi), "+v"(sg_lo), "+v"(sg_hi));
      if (cg == 0) {
        irow[RPT * rg + i][0] = (int64_t)pl_hi * 65536 + pl_lo;
        irow[RPT * rg + i][1] = (int64_t)sg_hi * 65536 + sg_lo;
      }
    }
  } else {
    float bc[8];
    {
      const int64_t cc = on ? c0 : 0;
      const f32x4 b0 = *reinterpret_cast<const f32x4*>(a.bcol + cc);
      const f32x4 b1 = *reinterpret_cast<const f32x4*>(a.bcol + cc + 4);
      bc[0] = b0.x; bc[1] = b0.y; bc[2] = b0.z; bc[3] = b0.w; bc[4] = b1.x; bc[5] = b1.y; bc[6] = b1.z; bc[7] = b1.w;
    }
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      float x[8];
      if constexpr (CT == C_BF16) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          x[2 * q] = bf16_lo(v[i][0][q]);
          x[2 * q + 1] = bf16_hi(v[i][0][q]);
        }
      } else {
#pragma unroll
        for (int l = 0; l < 2; ++l)
#pragma unroll
          for (int q = 0; q < 4; ++q) x[4 * l + q] = __uint_as_float(v[i][l][q]);
      }
      const float lim = an_s[RPT * rg + i];
      float pl = 0.f, sg = 0.f, sq = 0.f;
      bool imp = false;
      if (on) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          pl += x[e];
          sg = fmaf(x[e], sgn[e], sg);
          sq = fmaf(x[e], x[e], sq);
          imp = imp || (fabsf(x[e]) > lim * bc[e]);
        }
      }
      pl = sum16(pl);
      sg = sum16(sg);
      sq = sum16(sq);
      float fi = imp ? 1.f : 0.f;
      fi += dpp_xor1(fi);
      fi += dpp_xor2(fi);
      fi += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(fi), 0x141, 0xF, 0xF, false));
      fi += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(fi), 0x140, 0xF, 0xF, false));
      // (the sums finish here, with every lane on: their last DPP steps must not move under the store's mask)
      asm volatile("" : "+v"(pl), "+v"(sg), "+v"(sq), "+v"(fi));
      if (cg == 0) {
        srow[RPT * rg + i][0] = pl;
        srow[RPT * rg + i][1] = sg;
        srow[RPT * rg + i][2] = sq;
        imp_s[RPT * rg + i] = fi;
      }
    }
  }
  __syncthreads();
  QBest best;
  if (scorer && r0 + rl < a.m) {
    const int64_t p = (r0 + rl) * a.nb + jb;
    if constexpr (KIND == 0) {
      const bool bad = i0 != irow[rl][0] || i1 != irow[rl][1];
      const float z = bad ? __builtin_inff() : 0.f;
      if (a.zdump) a.zdump[p] = z;
      if (bad) {
        best.wrong = 1;
        best.key = ((int64_t)__float_as_uint(z) << 32) | (p & 0xFFFFFFFFll);
        best.keyd = best.key;
      }
    } else {
      const double pl = srow[rl][0], sg = srow[rl][1], sq = srow[rl][2];
      const bool imposs = imp_s[rl] > 0.f;
      const double a_norm = srow[rl][3];
      const double c_norm = sqrt(sq);
      double noise = (double)a.unit * (a_norm * (double)a.bfrob[jb] + (double)a.per_out * c_norm);
      if (a.c_bf16) noise += 0.00390625 * c_norm;
      noise += 1e-300;
      const double zd = fmax(fabs(e0 - pl), fabs(e1 - sg)) / noise;
      const bool fin = isfinite(pl) && isfinite(sg);
      const bool bad = !fin || imposs || !isfinite(noise) || isnan(zd);
      const float z = bad ? __builtin_inff() : (float)zd;
      if (a.zdump) a.zdump[p] = z;
      best.wrong = z > a.zt;
      best.nonfin = !fin;
      const int64_t zb = (int64_t)__float_as_uint(fmaxf(z, 0.f));
      best.key = (zb << 32) | (p & 0xFFFFFFFFll);
      best.keyd = (zb << 32) | (int64_t)__float_as_uint((float)noise);
    }
  }
  if (scorer) {                                              // (a whole wave: the reductions by DPP moves)
    const int64_t key = wave_max_i64_dpp(best.key), keyd = wave_max_i64_dpp(best.keyd);
    const int wr = wave_sum_i32_dpp(best.wrong), nf = wave_sum_i32_dpp(best.nonfin);
    if (lane == 0) {
      int64_t* res = a.result;
      if (key > seen0) atomicMax((unsigned long long*)res, (unsigned long long)key);
      if (keyd > seen1) atomicMax((unsigned long long*)(res + 1), (unsigned long long)keyd);
      if (wr > 0) atomicAdd((unsigned long long*)(res + 2), (unsigned long long)wr);
      if (nf > 0) atomicAdd((unsigned long long*)(res + 3), (unsigned long long)nf);
    }
  }
}

// Depth splits of the quantized checks' GEMM: sdc_expected_splits' (tiles x splits covering the 256 CUs, at most
// SDC_MAX_SPLITS planes), except that an fp8 GEMM of few row tiles (2048 tokens make four) takes up to
// SDC_MAX_GEMM_SPLITS splits of at least 128 depths: its planes are small, and MFMA work is its cost.  (int8 keeps
// the planes few: each split writes two digit planes the scoring pass reads back.)
int64_t quant_splits(int kind, int64_t m, int64_t k, int64_t ncols) {
  const int wgn = ncols > 64 ? 2 : 1;
  const int64_t tiles = sdc_cdiv(m, 64 * (8 / wgn)) * sdc_cdiv(ncols, 64 * wgn);
  if (kind == 0 || tiles > 8) return sdc_expected_splits(m, k, ncols);
  int64_t s = sdc_cdiv(256, tiles);
  const int64_t smax = k / 128 > 1 ? k / 128 : 1;
  if (s > smax) s = smax;
  if (s > SDC_MAX_GEMM_SPLITS) s = SDC_MAX_GEMM_SPLITS;
  return s < 1 ? 1 : s;
}

struct QLayout {
  int64_t nb, rem, ncols, splits, nacc, kpad, off_e, off_xn, off_apad, off_ppad, off_frag, total;   // in floats
  bool tall;                       // the tall-tile register-streamed GEMM where the shape allows
  bool short_rows;                 // (its 64-row tiles, for a short A)
  int64_t tsplits;                 // (its depth parts: planes of E)
};

QLayout qlayout(int kind, int64_t m, int64_t k, int64_t n, int64_t bs) {
  QLayout L{};
  L.nb = sdc_cdiv(n, bs);
  L.rem = n % bs;
  L.ncols = 2 * L.nb;
  L.nacc = kind == 0 ? 2 : 1;
  L.splits = quant_splits(kind, m, kind == 0 ? (k + 1) / 2 : k, L.ncols);
  // the GEMM on the register-streamed tall-tile kernel (depth a multiple of 1024, the parts in fragment order):
  // fp8 takes 128 x 64 tiles over two depth halves where they fill the GPU (192 workgroups or more), else (a short
  // A, and int8 always) 64 x 64 tiles over as many depth parts, up to SDC_MAX_SPLITS, as keep within two workgroups
  // a CU
  const int64_t nct = sdc_cdiv(L.ncols, 64);
  if (k % 1024 == 0) {
    // (int8: two int32 digit planes a part)
    if (kind == 1 && 2 * sdc_cdiv(m, 128) * nct >= 192) {
      L.tall = true;
      L.tsplits = 2;
    } else {
      for (int64_t s = SDC_MAX_SPLITS; s >= 2; --s)
        if (k % (512 * s) == 0 && s * sdc_cdiv(m, 64) * nct <= 512) {
          L.tall = L.short_rows = true;
          L.tsplits = s;
          break;
        }
    }
  }
  const int64_t esplits = L.tall && L.splits < L.tsplits ? L.tsplits : L.splits;
  L.kpad = kind == 0 ? (k + 63) / 64 * 64 : 0;           // int8: depth of the zero-padded copies (bytes)
  auto al = [](int64_t x) { return (x + 63) / 64 * 64; };
  int64_t o = 0;
  L.off_e = o; o += al(esplits * L.nacc * m * L.ncols);
  L.off_xn = o; o += al(esplits * 2 * m);
  L.off_apad = o; o += al(sdc_cdiv(m * L.kpad, 4));
  L.off_ppad = o; o += al(sdc_cdiv(2 * L.ncols * L.kpad, 4));
  L.off_frag = o;
  o += L.tall ? al((kind == 0 ? sdc_digit_fragments_bytes(L.ncols, k) : sdc_parts_fragments_bytes(L.ncols, k)) / 4) : 0;
  L.total = o;
  return L;
}

// rows x cols bytes at src (row stride s_row) -> rows x dcols at dst, zero past cols; 4 destination bytes per
// thread (dcols a multiple of 4, dst 4-byte aligned)
__global__ __launch_bounds__(256) void pad_bytes_kernel(const uint8_t* src, int64_t s_row, int64_t rows, int64_t cols,
                                                        uint8_t* dst, int64_t dcols) {
  const int64_t words = rows * (dcols / 4);
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < words; i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / (dcols / 4), c = 4 * (i % (dcols / 4));
    const uint8_t* row = src + r * s_row;
    uint32_t v = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b)
      if (c + b < cols) v |= (uint32_t)row[c + b] << (8 * b);
    reinterpret_cast<uint32_t*>(dst + r * dcols)[c / 4] = v;
  }
}

int pad_bytes(const void* src, int64_t s_row, int64_t rows, int64_t cols, void* dst, int64_t dcols,
              hipStream_t stream) {
  const int64_t words = rows * (dcols / 4);
  const unsigned grid = (unsigned)(sdc_cdiv(words, 256) < 4096 ? sdc_cdiv(words, 256) : 4096);
  hipLaunchKernelGGL(pad_bytes_kernel, dim3(grid), dim3(256), 0, stream, (const uint8_t*)src, s_row, rows, cols,
                     (uint8_t*)dst, dcols);
  SDC_LAUNCH_CHECK();
  return SDC_OK;
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

extern "C" int sdc_quant_check(int kind, const void* A, int64_t sam, const void* parts, int64_t spc,
                               const void* parts_frag, const float* sa,
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
  const QLayout L = qlayout(kind, m, k, n, bs);
  if (m * L.nb > 0xFFFFFFFFll) return SDC_EUNSUPPORTED;
  if (!workspace || workspace_bytes < L.total * (int64_t)sizeof(float) + 256) return SDC_EWORKSPACE;
  float* ws = (float*)(((uintptr_t)workspace + 255) & ~(uintptr_t)255);
  // int8 runs the GEMM on pairs of bytes: an odd depth, odd row strides or odd addresses are copied first into
  // zero-padded buffers of the workspace (depth rounded up to 64 bytes, so the copy also loads 16 bytes at a time)
  int64_t kg = kind == 0 ? k / 2 : k;                     // the GEMM's depth (int8: in pairs)
  if (kind == 0 && ((k % 2) || (sam % 2) || (spc % 2) || ((uintptr_t)A % 2) || ((uintptr_t)parts % 2))) {
    uint8_t* apad = (uint8_t*)(ws + L.off_apad);
    uint8_t* ppad = (uint8_t*)(ws + L.off_ppad);
    int rc = pad_bytes(A, sam, m, k, apad, L.kpad, stream);
    if (rc == SDC_OK) rc = pad_bytes(parts, spc, 2 * L.ncols, k, ppad, L.kpad, stream);
    if (rc != SDC_OK) return rc;
    A = apad;
    sam = L.kpad;
    parts = ppad;
    spc = L.kpad;
    kg = L.kpad / 2;
  }
  const float* s_full = sign_table + (bs - 1) * 128;
  const float* s_last = L.rem ? sign_table + (L.rem - 1) * 128 : s_full;

  const int es = c_dtype == C_BF16 ? 2 : 4;
  const bool vec = scn == 1 && ((scm * es) % 16 == 0) && ((bs * es) % 16 == 0) && ((uintptr_t)C % 16 == 0);
  const bool tiles = vec && bs == 128 && n % 8 == 0 && sdc_cdiv(m, 64) <= 65535;   // the tile pass (transposed E)
  GemmArgs g{};
  g.et = tiles ? 1 : 0;
  g.A = (const uint16_t*)A;
  g.sab = 0;
  g.sam = kind == 0 ? sam / 2 : sam;
  g.sak = 1;
  g.B = parts; g.sbb = 0; g.sbc = kind == 0 ? spc / 2 : spc;
  g.m = m; g.k = kg; g.N = L.ncols; g.splits = L.splits;
  g.E = ws + L.off_e; g.XN = ws + L.off_xn;
  g.prof_name = kind == 0 ? "quant_gemm_i8" : "quant_gemm_fp8";
  int rc = SDC_EUNSUPPORTED;
  int64_t splits = L.splits;
  if (L.tall && tiles && sam % 16 == 0 && (uintptr_t)A % 16 == 0 && spc % 8 == 0 && spc >= k &&
      (uintptr_t)parts % 16 == 0) {
    // the parts in fragment order (given, or made here), then the tall-tile GEMM (fp8: with the row norms; int8:
    // on bytes, both digits)
    const void* frag = parts_frag;
    if (!frag) {
      frag = ws + L.off_frag;
      rc = kind == 0 ? sdc_digit_fragments(parts, spc, L.ncols, k, ws + L.off_frag, stream)
                     : sdc_parts_fragments(parts, spc, L.ncols, k, ws + L.off_frag, stream);
      if (rc != SDC_OK) return rc;
    }
    GemmArgs gt = g;
    gt.B = frag;
    gt.splits = L.tsplits;
    gt.short_rows = L.short_rows ? 1 : 0;
    gt.et = 1;
    if (kind == 0) {
      gt.sam = sam; gt.k = k; gt.XN = nullptr;                 // (bytes, not the staged GEMM's pairs)
    }
    rc = sdc_rs_gemm_tall_launch(kind == 0 ? SDC_I8 : SDC_FP8, gt, 0, stream);
    if (rc == SDC_OK) splits = L.tsplits;
  }
  if (rc == SDC_EUNSUPPORTED) rc = sdc_gemm_launch(kind == 0 ? SDC_I8 : SDC_FP8, g, 1, stream);
  if (rc != SDC_OK) return rc;

  QuantArgs qa{};
  qa.C = C; qa.scm = scm; qa.scn = scn;
  qa.m = m; qa.n = n; qa.nb = L.nb; qa.bs = bs; qa.rem = L.rem; qa.npairs = m * L.nb;
  qa.vec = vec;
  qa.s_full = s_full; qa.s_last = s_last;
  qa.E = ws + L.off_e; qa.XN = ws + L.off_xn; qa.splits = splits; qa.ncols = L.ncols;
  qa.sa = sa; qa.bfrob = bfrob; qa.bcol = bcol;
  qa.unit = unit;
  qa.per_out = (float)(sqrt((double)k) + (nfma > 0.f ? (double)k / (double)nfma : 0.0));
  qa.zt = z;
  qa.c_bf16 = c_dtype == C_BF16;
  qa.result = result; qa.zdump = scores_out;
  SdcProf prof(kind == 0 ? "quant_score_i8" : "quant_score_fp8", stream);
  if (tiles) {
    // bf16 C: 128-row tiles (32 KB; measured 13% faster than 64 rows at 4096 x 14336); 4-byte C
    // (int32, fp32): 64-row tiles, already two loads a row piece (128 rows measured 9% slower)
    constexpr int MS = SDC_MAX_SPLITS;
    const int rows = c_dtype == C_BF16 ? 128 : 64;
    const dim3 grid((unsigned)L.nb, (unsigned)sdc_cdiv(m, rows));
    const bool few = qa.splits <= SDC_MAX_SPLITS;
    if (kind == 0 && few) hipLaunchKernelGGL((quant_tile_kernel<0, C_I32, true, MS, 4>), grid, dim3(256), 0, stream, qa);
    else if (kind == 0) hipLaunchKernelGGL((quant_tile_kernel<0, C_I32, false, MS, 4>), grid, dim3(256), 0, stream, qa);
    else if (c_dtype == C_F32 && qa.splits <= 2)
      hipLaunchKernelGGL((quant_tile_kernel<1, C_F32, true, 2, 4>), grid, dim3(256), 0, stream, qa);
    else if (qa.splits <= 2)
      hipLaunchKernelGGL((quant_tile_kernel<1, C_BF16, true, 2, 8>), grid, dim3(256), 0, stream, qa);
    else if (c_dtype == C_F32 && few)
      hipLaunchKernelGGL((quant_tile_kernel<1, C_F32, true, MS, 4>), grid, dim3(256), 0, stream, qa);
    else if (c_dtype == C_F32)
      hipLaunchKernelGGL((quant_tile_kernel<1, C_F32, false, MS, 4>), grid, dim3(256), 0, stream, qa);
    else if (few) hipLaunchKernelGGL((quant_tile_kernel<1, C_BF16, true, MS, 8>), grid, dim3(256), 0, stream, qa);
    else hipLaunchKernelGGL((quant_tile_kernel<1, C_BF16, false, MS, 8>), grid, dim3(256), 0, stream, qa);
  } else {
    const int64_t groups = sdc_cdiv(qa.npairs, 4);
    const unsigned grid = (unsigned)(sdc_cdiv(groups, 4) < 2048 ? sdc_cdiv(groups, 4) : 2048);
    if (kind == 0) launch_score<0, C_I32>(qa, grid, stream);
    else if (c_dtype == C_F32) launch_score<1, C_F32>(qa, grid, stream);
    else launch_score<1, C_BF16>(qa, grid, stream);
  }
  SDC_LAUNCH_CHECK();
  return SDC_OK;
}
