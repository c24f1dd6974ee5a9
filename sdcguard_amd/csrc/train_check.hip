// Column-block check of one matmul C = beta * bias + alpha * (A @ B), answered on the device (the training check).
//
// Reference: checksum.py:435-530 (`_zscores`: the arithmetic), :349-383 (`_complete_score`, `_judge_nonfinite`:
// the Inf/NaN rules with unjudged checksums scoring -1), _group.py:386-746 (the device version it replaces: B-side
// stage, comparison, worst-z search).  Four launches, no host synchronisation:
//   1. b_stage: the plain and signed block sums of every row of B (B2, fp32, stored transposed so the GEMM reads
//      depth-contiguous columns) and, per 64-row slice, partial sums of squares / maxima of B2's columns and the
//      largest |B| of every block;
//   2. b_finish: those partials added up (|checksum column|_2, its largest entry, the per-column power of two that
//      keeps fp16 parts in range, the block's largest |B|) and the bias vector's block sums;
//   3. split + expected_gemm (expected_gemm.hip): B2 as three parts, E = A @ B2 on MFMA, plus A's row norms;
//   4. train_score: one persistent pass over C scoring every (batch, row, block) pair, worst key and unjudged count
//      into the check's result row with atomics.
#include "blocksums.h"
#include "judge.h"
#include "gemm.h"
#include "profile.h"

extern "C" int64_t sdc_expected_splits(int64_t m, int64_t k, int64_t ncols);

namespace {

constexpr int BROWS = 64;          // rows of B per b_stage workgroup
constexpr int NSTAT = 5;           // partial stats per (slice, block): sq0, sq1, max0, max1, bmax

struct BStageArgs {
  const uint16_t* B;
  int64_t sbb, sbk, sbn;
  int64_t k, n, nb, bs, rem, nkc;
  const float* s_full;
  const float* s_last;
  float* B2T;                      // [bB][2nb][k]
  float* part;                     // [bB][nkc][nb][NSTAT]
  int vec;
};

__device__ __forceinline__ float nan_inf(float v) { return v == v ? fabsf(v) : __builtin_inff(); }

template <int DT>
__global__ __launch_bounds__(256) void b_stage_kernel(BStageArgs a) {
  __shared__ float red[4][NSTAT];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, q = t & 3;
  const int64_t kc = blockIdx.x, jb = blockIdx.y, bb = blockIdx.z;
  const int64_t kk = kc * BROWS + (t >> 2);
  const bool last = (jb == a.nb - 1) && (a.rem > 0);
  const int64_t wid = last ? a.rem : a.bs;
  const float* sp = last ? a.s_last : a.s_full;
  float pl = 0.f, sg = 0.f, mx = 0.f;
  if (kk < a.k) {
    const uint16_t* row = a.B + bb * a.sbb + kk * a.sbk + jb * a.bs * a.sbn;
    if (a.vec && wid == 128) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int c0 = 8 * (q + 4 * j);
        const u32x4 v = *reinterpret_cast<const u32x4*>(row + c0);
        const f32x4 s0 = *reinterpret_cast<const f32x4*>(sp + c0);
        const f32x4 s1 = *reinterpret_cast<const f32x4*>(sp + c0 + 4);
        const float x[8] = {lo_of<DT>(v.x), hi_of<DT>(v.x), lo_of<DT>(v.y), hi_of<DT>(v.y),
                            lo_of<DT>(v.z), hi_of<DT>(v.z), lo_of<DT>(v.w), hi_of<DT>(v.w)};
        const float s[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          pl += x[e];
          sg = fmaf(x[e], s[e], sg);
          mx = fmaxf(mx, nan_inf(x[e]));
        }
      }
    } else {
#pragma unroll 1
      for (int j = 0; j < 4; ++j)
#pragma unroll 1
        for (int e = 0; e < 8; ++e) {
          const int c = 8 * (q + 4 * j) + e;
          if (c < wid) {
            const float x = half_to_f32<DT>(row[c * a.sbn]);
            pl += x;
            sg = fmaf(x, sp[c], sg);
            mx = fmaxf(mx, nan_inf(x));
          }
        }
    }
  }
  pl = quad_sum(pl);
  sg = quad_sum(sg);
  mx = fmaxf(mx, dpp_xor1(mx));
  mx = fmaxf(mx, dpp_xor2(mx));
  const bool mine = q == 0 && kk < a.k;
  if (mine) {
    float* col = a.B2T + (bb * 2 * a.nb + 2 * jb) * a.k;
    col[kk] = pl;
    col[a.k + kk] = sg;
  }
  // this slice's partial |column|^2, largest |entry| of both checksum columns, largest |B| of the block
  float st[NSTAT] = {mine ? pl * pl : 0.f, mine ? sg * sg : 0.f, mine ? nan_inf(pl) : 0.f, mine ? nan_inf(sg) : 0.f,
                     mine ? mx : 0.f};
#pragma unroll
  for (int i = 0; i < NSTAT; ++i) {
    float v = st[i];
#pragma unroll
    for (int msk = 1; msk < 64; msk <<= 1) {
      const float o = __shfl_xor(v, msk, 64);
      v = i < 2 ? v + o : fmaxf(v, o);
    }
    if (lane == 0) red[w][i] = v;
  }
  __syncthreads();
  if (t < NSTAT) {
    float v = red[0][t];
    for (int i = 1; i < 4; ++i) v = t < 2 ? v + red[i][t] : fmaxf(v, red[i][t]);
    a.part[((bb * a.nkc + kc) * a.nb + jb) * NSTAT + t] = v;
  }
}

// The same stage for a B whose rows are contiguous across k (sbk == 1: a weight passed as W.t(), or the activations
// x^T of a row-block check).  A workgroup takes 256 consecutive rows of B and one block of columns: each thread reads
// 16 bytes (8 rows of B) of one column per step, the eight column groups of a workgroup take every eighth column,
// and LDS adds their sums.  Partial stats are written per 64-row slice, as b_stage_kernel writes them.
template <int DT>
__global__ __launch_bounds__(256) void b_stage_t_kernel(BStageArgs a) {
  __shared__ float red[2][8][256 + 4];
  __shared__ float redm[4];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int kg = t & 31, cg = t >> 5;
  const int64_t kc = blockIdx.x, jb = blockIdx.y, bb = blockIdx.z;
  const int64_t kk0 = kc * 256 + 8 * kg;
  const bool last = (jb == a.nb - 1) && (a.rem > 0);
  const int wid = (int)(last ? a.rem : a.bs);
  const float* sp = last ? a.s_last : a.s_full;
  float pl[8], sg[8], mx = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) pl[e] = sg[e] = 0.f;
  const uint16_t* base = a.B + bb * a.sbb + jb * a.bs * a.sbn + kk0;
  auto add8 = [&](const u32x4 v, float s) {
    const float x[8] = {lo_of<DT>(v.x), hi_of<DT>(v.x), lo_of<DT>(v.y), hi_of<DT>(v.y),
                        lo_of<DT>(v.z), hi_of<DT>(v.z), lo_of<DT>(v.w), hi_of<DT>(v.w)};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      pl[e] += x[e];
      sg[e] = fmaf(x[e], s, sg[e]);
      mx = fmaxf(mx, nan_inf(x[e]));
    }
  };
  if (a.vec && kk0 + 8 <= a.k && wid == 128) {
    // a full block: all 16 loads of this thread in flight before the first add
    u32x4 v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i)
      v[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(base + (cg + 8 * i) * a.sbn));
#pragma unroll
    for (int i = 0; i < 16; ++i) add8(v[i], sp[cg + 8 * i]);
  } else if (a.vec && kk0 + 8 <= a.k) {
#pragma unroll 4
    for (int c = cg; c < wid; c += 8)
      add8(__builtin_nontemporal_load(reinterpret_cast<const u32x4*>(base + c * a.sbn)), sp[c]);
  } else if (kk0 < a.k) {
    const int ne = a.k - kk0 < 8 ? (int)(a.k - kk0) : 8;
#pragma unroll 1
    for (int c = cg; c < wid; c += 8) {
      const float s = sp[c];
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (e < ne) {
          const float x = half_to_f32<DT>(base[c * a.sbn + e]);
          pl[e] += x;
          sg[e] = fmaf(x, s, sg[e]);
          mx = fmaxf(mx, nan_inf(x));
        }
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    red[0][cg][8 * kg + e] = pl[e];
    red[1][cg][8 * kg + e] = sg[e];
  }
#pragma unroll
  for (int msk = 1; msk < 64; msk <<= 1) mx = fmaxf(mx, __shfl_xor(mx, msk, 64));
  if (lane == 0) redm[w] = mx;
  __syncthreads();
  float P = 0.f, S = 0.f;
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    P += red[0][g][t];
    S += red[1][g][t];
  }
  const float bm = fmaxf(fmaxf(redm[0], redm[1]), fmaxf(redm[2], redm[3]));
  const int64_t kk = kc * 256 + t;
  const bool mine = kk < a.k;
  if (mine) {
    float* col = a.B2T + (bb * 2 * a.nb + 2 * jb) * a.k;
    col[kk] = P;
    col[a.k + kk] = S;
  }
  float st[NSTAT] = {mine ? P * P : 0.f, mine ? S * S : 0.f, mine ? nan_inf(P) : 0.f, mine ? nan_inf(S) : 0.f, bm};
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int msk = 1; msk < 64; msk <<= 1) {
      const float o = __shfl_xor(st[i], msk, 64);
      st[i] = i < 2 ? st[i] + o : fmaxf(st[i], o);
    }
  const int64_t slice = kc * 4 + w;           // 64-row slice of this wave's rows
  if (lane < NSTAT && slice < a.nkc) a.part[((bb * a.nkc + slice) * a.nb + jb) * NSTAT + lane] = st[lane];
}

struct BFinishArgs {
  const float* part;
  int64_t nkc, nb, bs, rem;
  int fp16;
  float* colstat;                  // [bB][2nb][3]: |column|_2, largest |entry|, power-of-two scale
  float* bmaxf;                    // [bB][nb]
  const uint16_t* bias;            // vector bias (n,) or null
  int64_t sbias;
  const float* s_full;
  const float* s_last;
  float* bias_out;                 // [nb][3]: plain sum, signed sum, largest |value|
};

// ceil(log2 x) as a power of two, exactly (frexp: x = f 2^e, f in [0.5, 1))
__device__ __forceinline__ float pow2_ceil(float x) {
  int e;
  const float f = frexpf(x, &e);
  return ldexpf(1.f, f == 0.5f ? e - 1 : e);
}

template <int DT>
__global__ __launch_bounds__(64) void b_finish_kernel(BFinishArgs a) {
  const int lane = threadIdx.x;
  const int64_t jb = blockIdx.x, bb = blockIdx.y;
  float st[NSTAT] = {0.f, 0.f, 0.f, 0.f, 0.f};
  for (int64_t kc = lane; kc < a.nkc; kc += 64) {
    const float* p = a.part + ((bb * a.nkc + kc) * a.nb + jb) * NSTAT;
    st[0] += p[0];
    st[1] += p[1];
    st[2] = fmaxf(st[2], p[2]);
    st[3] = fmaxf(st[3], p[3]);
    st[4] = fmaxf(st[4], p[4]);
  }
#pragma unroll
  for (int i = 0; i < NSTAT; ++i)
#pragma unroll
    for (int msk = 1; msk < 64; msk <<= 1) {
      const float o = __shfl_xor(st[i], msk, 64);
      st[i] = i < 2 ? st[i] + o : fmaxf(st[i], o);
    }
  if (lane == 0) {
    float* cs = a.colstat + (bb * 2 * a.nb + 2 * jb) * 3;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const float amax = st[2 + c];
      cs[3 * c + 0] = sqrtf(st[c]);
      cs[3 * c + 1] = amax;
      // fp16 parts stay in range divided by a power of two (checksum._matmul_fp32); bf16 needs none
      cs[3 * c + 2] = (a.fp16 && amax > 0.f && amax < __builtin_inff()) ? pow2_ceil(amax) : 1.f;
    }
    a.bmaxf[bb * a.nb + jb] = st[4];
  }
  if (a.bias && bb == 0) {
    const bool last = (jb == a.nb - 1) && (a.rem > 0);
    const int64_t wid = last ? a.rem : a.bs;
    const float* sp = last ? a.s_last : a.s_full;
    float pl = 0.f, sg = 0.f, mx = 0.f;
    for (int64_t c = lane; c < wid; c += 64) {
      const float x = half_to_f32<DT>(a.bias[(jb * a.bs + c) * a.sbias]);
      pl += x;
      sg = fmaf(x, sp[c], sg);
      mx = fmaxf(mx, nan_inf(x));
    }
#pragma unroll
    for (int msk = 1; msk < 64; msk <<= 1) {
      pl += __shfl_xor(pl, msk, 64);
      sg += __shfl_xor(sg, msk, 64);
      mx = fmaxf(mx, __shfl_xor(mx, msk, 64));
    }
    if (lane == 0) {
      a.bias_out[3 * jb] = pl;
      a.bias_out[3 * jb + 1] = sg;
      a.bias_out[3 * jb + 2] = mx;
    }
  }
}

struct TrainArgs {
  YView cv;                        // C
  int64_t k, splits, nbt, ncols;
  int b_batched;                   // B (and its stats) has one entry per batch
  int e_batched;                   // E / XN have one plane set per batch
  int et;                          // E planes transposed (the column-read scoring pass)
  const float* E;
  const float* XN;
  const float* colstat;
  const float* bmaxf;
  int bias_kind;                   // 0 none, 1 vector (block sums in bias_vec), 2 matrix (read per pair)
  const float* bias_vec;
  const uint16_t* bias_mat;
  int64_t sbias_b, sbias_m, sbias_n;
  float alpha, beta, u, h, abs_floor, l1c, zt, lim_a, capk;
  int64_t* result;                 // [key, key of the noise, unjudged]
  float* zdump;
  const int64_t* goffs;            // grouped rows: cumulative group ends (device), or null
  int64_t ngroups;
};

struct TrainBest {
  int64_t key = 0, keyd = 0;
  int unk = 0;
};

// A pair's expected sums and its row's norms, the GEMM's split planes added in split order.  eb: the E / XN batch.
struct PairE {
  float e0, e1, asq, asum;
};

template <int NS = SDC_MAX_SPLITS>
__device__ __forceinline__ PairE pair_expected(const TrainArgs& a, int64_t eb, int64_t r, int64_t jb) {
  // E planes row-major ([m][ncols]: plain and signed adjacent) or transposed ([ncols][m]: adjacent rows)
  const float* ep = a.et ? a.E + ((eb * a.splits) * a.ncols + 2 * jb) * a.cv.m + r
                         : a.E + ((eb * a.splits) * a.cv.m + r) * a.ncols + 2 * jb;
  const float* xp = a.XN + (eb * a.splits) * 2 * a.cv.m + r;
  const int64_t estep = a.cv.m * a.ncols, xstep = 2 * a.cv.m;
  float2 ev[NS];
  float xa[NS], xb[NS];
  // loads unconditional, so all are in flight at once (a split index past a.splits reads split 0, not added)
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int64_t sc = s < a.splits ? s : 0;
    if (a.et) ev[s] = make_float2(ep[sc * estep], ep[sc * estep + a.cv.m]);
    else ev[s] = *reinterpret_cast<const float2*>(ep + sc * estep);
    xa[s] = xp[sc * xstep];
    xb[s] = xp[sc * xstep + a.cv.m];
  }
  PairE pe{ev[0].x, ev[0].y, xa[0], xb[0]};
#pragma unroll
  for (int s = 1; s < NS; ++s)
    if (s < a.splits) {
      pe.e0 += ev[s].x;
      pe.e1 += ev[s].y;
      pe.asq += xa[s];
      pe.asum += xb[s];
    }
  return pe;
}

// pe: the pair's expected sums when the caller has them (loaded ahead of C), else null
template <int DT>
__device__ __forceinline__ void train_pair(const TrainArgs& a, int64_t p, float pl, float sg, float sq, float l1,
                                           TrainBest& best, int64_t grp = -1, const PairE* pe = nullptr) {
  if (p >= a.cv.npairs) return;
  int64_t bc, r, jb;
  pair_index(a.cv, p, bc, r, jb);
  const bool last = (jb == a.cv.nb - 1) && (a.cv.rem > 0);
  const float wf = (float)(last ? a.cv.rem : a.cv.bs);
  const int64_t eb = (a.e_batched && grp < 0) ? bc : 0, bbi = grp >= 0 ? grp : (a.b_batched ? bc : 0);
  const PairE ex = pe ? *pe : pair_expected(a, eb, r, jb);
  float e0 = ex.e0, e1 = ex.e1;
  const float asq = ex.asq, asum = ex.asum;
  const float* cs = a.colstat + (bbi * a.ncols + 2 * jb) * 3;
  e0 *= cs[2];                                   // the parts were made from B2 / scale
  e1 *= cs[5];
  float bound = asum * a.bmaxf[bbi * a.cv.nb + jb];
  if (a.alpha != 1.f) {
    e0 *= a.alpha;
    e1 *= a.alpha;
    bound *= fabsf(a.alpha);
  }
  if (a.bias_kind == 1) {
    e0 = e0 + a.bias_vec[3 * jb] * a.beta;
    e1 = e1 + a.bias_vec[3 * jb + 1] * a.beta;
    bound = bound + fabsf(a.beta) * a.bias_vec[3 * jb + 2];
  } else if (a.bias_kind == 2) {
    const uint16_t* br = a.bias_mat + bc * a.sbias_b + r * a.sbias_m + jb * a.cv.bs * a.sbias_n;
    const float* sp = last ? a.cv.s_last : a.cv.s_full;
    float bp = 0.f, bsg = 0.f, bmx = 0.f;
    if (a.sbias_n == 0) {
      // a bias constant along the row (a per-output bias of a row-block check): w copies of one value, whose
      // block sums w*b and (sum of signs)*b are exact in fp32 (8-bit significands times w <= 128)
      const float x = half_to_f32<DT>(br[0]);
      float ss = 0.f;
      for (int64_t c = 0; c < (int64_t)wf; ++c) ss += sp[c];
      bp = x * wf;
      bsg = x * ss;
      bmx = nan_inf(x);
    } else {
      for (int64_t c = 0; c < (int64_t)wf; ++c) {
        const float x = half_to_f32<DT>(br[c * a.sbias_n]);
        bp += x;
        bsg = fmaf(x, sp[c], bsg);
        bmx = fmaxf(bmx, nan_inf(x));
      }
    }
    e0 = e0 + bp * a.beta;
    e1 = e1 + bsg * a.beta;
    bound = bound + fabsf(a.beta) * bmx;
  }
  const float cn = fsqrt(sq);
  const float noise = cn * a.u;
  const float xn = fsqrt(asq), aal = fabsf(a.alpha);
  float fl[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const float f_l2 = (xn * cs[3 * c]) * (1e-5f * aal);
    const float f_l1 = (asum * cs[3 * c + 1]) * (a.l1c * aal);
    const float inf = __builtin_inff();
    float f = fminf(fabsf(f_l2) < inf ? f_l2 : inf, fabsf(f_l1) < inf ? f_l1 : inf);
    fl[c] = f < inf ? f : bound * (float)(1e-5 * 128.0);
  }
  float d0, d1;
  bool ok0, ok1;
  float z0 = judge_one_clean(e0, pl, noise, cn, fl[0], bound, wf, l1, true, a, d0, ok0);
  float z1 = judge_one_clean(e1, sg, noise, cn, fl[1], bound, wf, l1, false, a, d1, ok1);
  if (!(ok0 && ok1)) {                           // (non-finite inputs or an "impossible" checksum: the full rules)
    z0 = judge_one(e0, pl, noise, cn, fl[0], bound, wf, l1, true, a, d0);
    z1 = judge_one(e1, sg, noise, cn, fl[1], bound, wf, l1, false, a, d1);
  }
  if (a.zdump) {
    a.zdump[2 * p] = z0;
    a.zdump[2 * p + 1] = z1;
  }
  best.unk += (z0 < 0.f) + (z1 < 0.f);
  const bool sec = z1 > z0;
  const float zc = sec ? z1 : z0;
  const int64_t zb = fbits64(fmaxf(zc, 0.f));
  const int64_t flat = p * 2 + (sec ? 1 : 0);
  const int64_t k1 = (zb << 32) | (flat & 0xFFFFFFFFll);
  const int64_t k2 = (zb << 32) | (fbits64(sec ? d1 : d0) & 0xFFFFFFFFll);
  best.key = k1 > best.key ? k1 : best.key;
  best.keyd = k2 > best.keyd ? k2 : best.keyd;
}

template <int DT>
__global__ __launch_bounds__(256) void train_score_kernel(TrainArgs a) {
  __shared__ int64_t red_k[4], red_d[4];
  __shared__ int red_u[4];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, q = lane & 3;
  uint32_t sg2[16];
  lane_signs<DT>(a.cv, q, sg2);
  TrainBest best;
  const int64_t tiles = (a.cv.npairs + 63) / 64;
  for (int64_t tile = (int64_t)blockIdx.x * 4 + w; tile < tiles; tile += (int64_t)gridDim.x * 4) {
    const int64_t base = tile * 64;
    float pl, sg, sq, ab;
    pair_sums<DT>(a.cv, base, lane, sg2, pl, sg, sq, ab);
    train_pair<DT>(a, base + q * 16 + (lane >> 2), pl, sg, sq, ab, best);
  }
  int64_t key = wave_max_i64_dpp(best.key), keyd = wave_max_i64_dpp(best.keyd);   // (every lane active)
  int unk = wave_sum_i32_dpp(best.unk);
  if (lane == 0) { red_k[w] = key; red_d[w] = keyd; red_u[w] = unk; }
  __syncthreads();
  if (t == 0) {
    int64_t k0 = red_k[0], d0 = red_d[0];
    int un = red_u[0];
    for (int i = 1; i < 4; ++i) {
      k0 = red_k[i] > k0 ? red_k[i] : k0;
      d0 = red_d[i] > d0 ? red_d[i] : d0;
      un += red_u[i];
    }
    int64_t* res = a.result;
    const int64_t s0 = __atomic_load_n(res, __ATOMIC_RELAXED), s1 = __atomic_load_n(res + 1, __ATOMIC_RELAXED);
    if (k0 > s0) atomicMax((unsigned long long*)res, (unsigned long long)k0);
    if (d0 > s1) atomicMax((unsigned long long*)(res + 1), (unsigned long long)d0);
    if (un > 0) atomicAdd((unsigned long long*)(res + 2), (unsigned long long)un);
  }
}

// The scoring pass for a C whose rows are contiguous across each other (scm == 1: C = y^T of a row-block check,
// where a "row" of C is a column of y and a block of C's columns is a block of 128 rows of y).  A workgroup takes
// 512 consecutive rows of C (8 per lane, one 16-byte load) and one block: the four waves split the block's
// columns, each lane accumulates the four sums of its 8 rows, LDS adds the waves' sums, and every thread scores
// two (row, block) pairs with the same arithmetic as train_score_kernel.
template <int DT>
__global__ __launch_bounds__(256) void train_score_t_kernel(TrainArgs a) {
  __shared__ float red[4][4][512];
  __shared__ int64_t red_k[4], red_d[4];
  __shared__ int red_u[4];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int64_t rt = blockIdx.x, jb = blockIdx.y, bc = blockIdx.z;
  const int64_t m = a.cv.m;
  const bool last = (jb == a.cv.nb - 1) && (a.cv.rem > 0);
  const int wid = (int)(last ? a.cv.rem : a.cv.bs);
  const float* sp = last ? a.cv.s_last : a.cv.s_full;
  const int64_t r0 = rt * 512 + 8 * lane;
  float pl[8], sg[8], sq[8], ab[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) pl[e] = sg[e] = sq[e] = ab[e] = 0.f;
  const uint16_t* base = a.cv.y + bc * a.cv.sb + r0 + jb * a.cv.bs * a.cv.sn;
  if (a.cv.vec && r0 + 8 <= m) {
#pragma unroll 8
    for (int c = w; c < wid; c += 4) {
      const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(base + c * a.cv.sn));
      const float s = sp[c];
      const float x[8] = {lo_of<DT>(v.x), hi_of<DT>(v.x), lo_of<DT>(v.y), hi_of<DT>(v.y),
                          lo_of<DT>(v.z), hi_of<DT>(v.z), lo_of<DT>(v.w), hi_of<DT>(v.w)};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        pl[e] += x[e];
        sg[e] = fmaf(x[e], s, sg[e]);
        sq[e] = fmaf(x[e], x[e], sq[e]);
        ab[e] += fabsf(x[e]);
      }
    }
  } else if (r0 < m) {
    const int ne = m - r0 < 8 ? (int)(m - r0) : 8;
#pragma unroll 1
    for (int c = w; c < wid; c += 4) {
      const float s = sp[c];
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (e < ne) {
          const float x = half_to_f32<DT>(base[c * a.cv.sn + e]);
          pl[e] += x;
          sg[e] = fmaf(x, s, sg[e]);
          sq[e] = fmaf(x, x, sq[e]);
          ab[e] += fabsf(x);
        }
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    red[w][0][8 * lane + e] = pl[e];
    red[w][1][8 * lane + e] = sg[e];
    red[w][2][8 * lane + e] = sq[e];
    red[w][3][8 * lane + e] = ab[e];
  }
  __syncthreads();
  TrainBest best;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int i = t + 256 * h;
    const int64_t r = rt * 512 + i;
    if (r < m) {
      float s4[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) s4[q] = (red[0][q][i] + red[1][q][i]) + (red[2][q][i] + red[3][q][i]);
      train_pair<DT>(a, (bc * m + r) * a.cv.nb + jb, s4[0], s4[1], s4[2], s4[3], best);
    }
  }
  int64_t key = wave_max_i64_dpp(best.key), keyd = wave_max_i64_dpp(best.keyd);   // (every lane active)
  int unk = wave_sum_i32_dpp(best.unk);
  if (lane == 0) { red_k[w] = key; red_d[w] = keyd; red_u[w] = unk; }
  __syncthreads();
  if (t == 0) {
    int64_t k0 = red_k[0], d0 = red_d[0];
    int un = red_u[0];
    for (int i = 1; i < 4; ++i) {
      k0 = red_k[i] > k0 ? red_k[i] : k0;
      d0 = red_d[i] > d0 ? red_d[i] : d0;
      un += red_u[i];
    }
    int64_t* res = a.result;
    const int64_t s0 = __atomic_load_n(res, __ATOMIC_RELAXED), s1 = __atomic_load_n(res + 1, __ATOMIC_RELAXED);
    if (k0 > s0) atomicMax((unsigned long long*)res, (unsigned long long)k0);
    if (d0 > s1) atomicMax((unsigned long long*)(res + 1), (unsigned long long)d0);
    if (un > 0) atomicAdd((unsigned long long*)(res + 2), (unsigned long long)un);
  }
}

// The scoring pass of a grouped check (rows grouped by cumulative offsets, each group with its own B): every
// (row, block) pair is scored as train_score_kernel scores it, with the B-side statistics of its row's group, and
// the worst key and unjudged count go to that group's result row.  Rows past the last offset belong to no group and
// are not scored.  A wave's 64 pairs usually share one group: then one set of atomics per wave, else one per lane.
__device__ __forceinline__ int64_t group_of(const int64_t* offs, int64_t ng, int64_t r) {
  int64_t lo = 0, hi = ng;                        // first q with offs[q] > r (offsets are non-decreasing)
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (offs[mid] > r) hi = mid;
    else lo = mid + 1;
  }
  return lo < ng ? lo : -1;
}

__device__ __forceinline__ void flush_group(int64_t* res, const TrainBest& b) {
  if (b.key) atomicMax((unsigned long long*)res, (unsigned long long)b.key);
  if (b.keyd) atomicMax((unsigned long long*)(res + 1), (unsigned long long)b.keyd);
  if (b.unk > 0) atomicAdd((unsigned long long*)(res + 2), (unsigned long long)b.unk);
}

constexpr int GCAP = 1024;                        // group ends a workgroup holds in LDS
constexpr int GSLOT = 64;                         // groups a workgroup gathers its results for in LDS

// One tile of 64 consecutive pairs per wave, the workgroup's four tiles consecutive (no loop: every wave's loads go
// out at once).  The group ends go to LDS first (up to GCAP groups; the row-to-group searches then read LDS), each
// pair's expected sums are loaded before its C.  The waves gather their worst keys and counts per group in LDS (the
// workgroup's rows span few groups), then one thread per group it touched updates that group's result row: device
// atomics on one row serialize, so they are made per workgroup, not per wave.  NS: the most split planes added.
template <int DT, int NS>
__global__ __launch_bounds__(256) void grouped_score_kernel(TrainArgs a) {
  __shared__ int64_t offs_s[GCAP];
  __shared__ unsigned long long s_key[GSLOT], s_keyd[GSLOT];
  __shared__ int s_unk[GSLOT];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, q = lane & 3;
  const bool gl = a.ngroups <= GCAP;
  if (gl)
    for (int64_t i = t; i < a.ngroups; i += 256) offs_s[i] = a.goffs[i];
  if (t < GSLOT) {
    s_key[t] = s_keyd[t] = 0ull;
    s_unk[t] = 0;
  }
  uint32_t sg2[16];
  lane_signs<DT>(a.cv, q, sg2);
  __syncthreads();
  const int64_t* offs = gl ? offs_s : a.goffs;
  const int64_t tiles = (a.cv.npairs + 63) / 64;
  const int64_t tile = (int64_t)blockIdx.x * 4 + w;
  // the group of the workgroup's first row: its pairs' groups are that one and the next few
  const int64_t gfirst = group_of(offs, a.ngroups, ((int64_t)blockIdx.x * 256) / a.cv.nb);
  TrainBest tb;
  int64_t grp = -1, g0 = -1, g1 = -1;
  if (tile < tiles) {
    const int64_t base = tile * 64;
    const int64_t p = base + q * 16 + (lane >> 2);
    const int64_t pc = p < a.cv.npairs ? p : a.cv.npairs - 1;
    int64_t bc, r, jb;
    pair_index(a.cv, pc, bc, r, jb);
    const PairE pe = pair_expected<NS>(a, 0, r, jb);
    float pl, sg, sq, ab;
    pair_sums<DT>(a.cv, base, lane, sg2, pl, sg, sq, ab);
    grp = group_of(offs, a.ngroups, r);
    if (grp >= 0) train_pair<DT>(a, p, pl, sg, sq, ab, tb, grp, &pe);
    const int64_t last = base + 63 < a.cv.npairs ? base + 63 : a.cv.npairs - 1;
    g0 = group_of(offs, a.ngroups, base / a.cv.nb);
    g1 = group_of(offs, a.ngroups, last / a.cv.nb);
  }
  // into the workgroup's slots (a group past the slots, or rows before the first group: straight to its row)
  auto gather = [&](int64_t g, const TrainBest& b) {
    const int64_t sl = gfirst >= 0 ? g - gfirst : -1;
    if (sl >= 0 && sl < GSLOT) {
      if (b.key) atomicMax(&s_key[sl], (unsigned long long)b.key);
      if (b.keyd) atomicMax(&s_keyd[sl], (unsigned long long)b.keyd);
      if (b.unk) atomicAdd(&s_unk[sl], b.unk);
    } else {
      flush_group(a.result + 3 * g, b);
    }
  };
  if (g0 == g1) {
    if (g0 >= 0) {
      // (g0 and g1 are the wave's: the whole wave is here, so the reductions can use DPP moves)
      const int64_t key = wave_max_i64_dpp(tb.key), keyd = wave_max_i64_dpp(tb.keyd);
      const int unk = wave_sum_i32_dpp(tb.unk);
      if (lane == 0) {
        TrainBest w1;
        w1.key = key; w1.keyd = keyd; w1.unk = unk;
        gather(g0, w1);
      }
    }
  } else if (grp >= 0) {
    gather(grp, tb);
  }
  __syncthreads();
  if (t < GSLOT && gfirst >= 0 && gfirst + t < a.ngroups && (s_key[t] | s_keyd[t] | (unsigned long long)s_unk[t])) {
    TrainBest b;
    b.key = (int64_t)s_key[t]; b.keyd = (int64_t)s_keyd[t]; b.unk = s_unk[t];
    flush_group(a.result + 3 * (gfirst + t), b);
  }
}

struct Layout {
  int64_t nb, rem, ncols, nkc, splits, nbt;
  int64_t kp;                      // depth pitch of the parts (k rounded up to 8: 16-byte aligned columns)
  int64_t esplits;                 // E and XN planes the workspace holds (the grouped tall GEMM's two at least)
  int64_t fragb;                   // bytes of one group's parts in fragment order (grouped, depth a multiple of 512)
  int64_t off_b2t, off_part, off_col, off_bmax, off_bias, off_parts, off_frag, off_e, off_xn, total;
};

// The grouped check's expected side runs on the tall-tile GEMM where the depth allows it, over one depth part (the
// whole depth a workgroup: measured 2% faster than two halves for 32768 rows x 2048 deep x 22 columns, and the
// scoring pass then reads one plane; 1 or 2).
constexpr int64_t TALL_K = 512;
#ifndef SDC_GROUPED_TALL_SPLITS
#define SDC_GROUPED_TALL_SPLITS 1
#endif

// grouped: B has batch_b groups but A, C, E and XN are one tall matrix (rows grouped by offsets)
Layout layout(int64_t batch_a, int64_t batch_b, int64_t m, int64_t k, int64_t n, int64_t bs, bool grouped = false) {
  Layout L{};
  L.nb = sdc_cdiv(n, bs);
  L.rem = n % bs;
  L.ncols = 2 * L.nb;
  L.nkc = sdc_cdiv(k, BROWS);
  L.nbt = grouped ? 1 : (batch_a > batch_b ? batch_a : batch_b);
  L.splits = sdc_expected_splits(m, k, L.ncols);
  auto al = [](int64_t x) { return (x + 63) / 64 * 64; };   // floats, 256-byte aligned sections
  int64_t o = 0;
  L.kp = (k + 7) / 8 * 8;
  L.off_b2t = o; o += al(batch_b * L.ncols * k);
  L.off_part = o; o += al(batch_b * L.nkc * L.nb * NSTAT);
  L.off_col = o; o += al(batch_b * L.ncols * 3);
  L.off_bmax = o; o += al(batch_b * L.nb);
  L.off_bias = o; o += al(3 * L.nb);
  L.off_parts = o; o += al((batch_b * 3 * L.ncols * L.kp + 1) / 2);      // 16-bit parts, two per float
  L.fragb = grouped && k % TALL_K == 0 ? sdc_parts_fragments_bytes(L.ncols, k) : 0;
  L.off_frag = o; o += al(batch_b * L.fragb / 4);
  L.esplits = L.fragb ? std::max<int64_t>(L.splits, 2) : L.splits;
  L.off_e = o; o += al(L.nbt * L.esplits * m * L.ncols);
  L.off_xn = o; o += al(L.nbt * L.esplits * 2 * m);
  L.total = o;
  return L;
}

}  // namespace

extern "C" int64_t sdc_matmul_check_workspace(int64_t batch_a, int64_t batch_b, int64_t m, int64_t k, int64_t n,
                                              int64_t bs) {
  if (m <= 0 || n <= 0 || k <= 0 || bs <= 0 || batch_a <= 0 || batch_b <= 0) return 0;
  return layout(batch_a, batch_b, m, k, n, bs).total * (int64_t)sizeof(float) + 256;
}

namespace {

// Where a check's B-side constants live: in the call's workspace (the training checks), or in a per-layer buffer
// made once (the grouped check's serving form, sdc_grouped_constants).
struct BConsts {
  float* colstat;                  // [bB][2nb][3]
  float* bmaxf;                    // [bB][nb]
  float* bias3;                    // [nb][3]
  uint16_t* parts;                 // [bB][3 * 2nb][kp]
  uint16_t* frag;                  // the parts in fragment order, [bB][fragb / 2] (grouped), or null
};

// The B side: block sums of B and their statistics (b_stage, b_finish), the bias's block sums, and the three parts
// of the block sums (split).  b2t and part are scratch of layout()'s sizes.
int stage_b(int dtype, const void* B, int64_t sbb, int64_t sbk, int64_t sbn, int64_t batch_b, int64_t k, int64_t n,
            int64_t bs, const Layout& L, const void* bias, int bias_kind, int64_t sbias_n, const float* s_full,
            const float* s_last, float* b2t, float* part, const BConsts& bc, hipStream_t stream) {
  BStageArgs ba{};
  ba.B = (const uint16_t*)B; ba.sbb = sbb; ba.sbk = sbk; ba.sbn = sbn;
  ba.k = k; ba.n = n; ba.nb = L.nb; ba.bs = bs; ba.rem = L.rem; ba.nkc = L.nkc;
  ba.s_full = s_full; ba.s_last = s_last; ba.B2T = b2t; ba.part = part;
  // B with k-contiguous rows (W.t(), x^T) is read down its columns by b_stage_t_kernel; otherwise across rows
  const bool b_t = sbk == 1 && sbn != 1;
  if (b_t) ba.vec = (sbn % 8 == 0) && (sbb % 8 == 0) && ((uintptr_t)B % 16 == 0);
  else ba.vec = sbn == 1 && (sbk % 8 == 0) && (sbb % 8 == 0) && (bs % 8 == 0) && ((uintptr_t)B % 16 == 0);
  {
    SdcProf prof("b_stage", stream);
    if (b_t) {
      dim3 grid((unsigned)sdc_cdiv(k, 256), (unsigned)L.nb, (unsigned)batch_b);
      if (dtype == SDC_BF16) hipLaunchKernelGGL(b_stage_t_kernel<SDC_BF16>, grid, dim3(256), 0, stream, ba);
      else hipLaunchKernelGGL(b_stage_t_kernel<SDC_FP16>, grid, dim3(256), 0, stream, ba);
    } else {
      dim3 grid((unsigned)L.nkc, (unsigned)L.nb, (unsigned)batch_b);
      if (dtype == SDC_BF16) hipLaunchKernelGGL(b_stage_kernel<SDC_BF16>, grid, dim3(256), 0, stream, ba);
      else hipLaunchKernelGGL(b_stage_kernel<SDC_FP16>, grid, dim3(256), 0, stream, ba);
    }
    SDC_LAUNCH_CHECK();
  }
  BFinishArgs fa{};
  fa.part = part; fa.nkc = L.nkc; fa.nb = L.nb; fa.bs = bs; fa.rem = L.rem; fa.fp16 = dtype == SDC_FP16;
  fa.colstat = bc.colstat; fa.bmaxf = bc.bmaxf;
  fa.bias = bias_kind == 1 ? (const uint16_t*)bias : nullptr; fa.sbias = sbias_n;
  fa.s_full = s_full; fa.s_last = s_last; fa.bias_out = bc.bias3;
  {
    SdcProf prof("b_finish", stream);
    dim3 grid((unsigned)L.nb, (unsigned)batch_b);
    if (dtype == SDC_BF16) hipLaunchKernelGGL(b_finish_kernel<SDC_BF16>, grid, dim3(64), 0, stream, fa);
    else hipLaunchKernelGGL(b_finish_kernel<SDC_FP16>, grid, dim3(64), 0, stream, fa);
    SDC_LAUNCH_CHECK();
  }
  // the three parts of B2 / scale (scale: every third float of colstat, stride 3 per column)
  int rc = sdc_split_launch(dtype, b2t, bc.colstat + 2, L.ncols * 3, 3, L.ncols, k, L.kp, batch_b, bc.parts, stream);
  if (rc != SDC_OK || !bc.frag) return rc;
  // and, for the tall-tile GEMM, in its fragment order (one set per group)
  return sdc_parts_fragments_sets(bc.parts, L.kp, 3 * L.ncols * L.kp, batch_b, L.ncols, k, bc.frag, stream);
}

int check_with(int dtype, const void* A, int64_t sab, int64_t sam, int64_t sak, int64_t batch_a, int64_t batch_b,
               const void* C, int64_t scb, int64_t scm, int64_t scn, int64_t batch_c, int64_t m, int64_t k, int64_t bs,
               const Layout& L, const BConsts& bc, const void* bias, int bias_kind, int64_t sbias_b, int64_t sbias_m,
               int64_t sbias_n, float alpha, float beta, float z, float abs_floor, const float* s_full,
               const float* s_last, int64_t* result, float* E, float* XN, float* scores_out, const int64_t* goffs,
               hipStream_t stream);

// The check of sdc_matmul_check, or (goffs set) of sdc_grouped_check: batch_b groups of B over one tall A / C.
int run_check(int dtype, const void* A, int64_t sab, int64_t sam, int64_t sak, int64_t batch_a, const void* B,
              int64_t sbb, int64_t sbk, int64_t sbn, int64_t batch_b, const void* C, int64_t scb, int64_t scm,
              int64_t scn, int64_t batch_c, int64_t m, int64_t k, int64_t n, int64_t bs, const void* bias,
              int bias_kind, int64_t sbias_b, int64_t sbias_m, int64_t sbias_n, float alpha, float beta, float z,
              float abs_floor, const float* sign_table, int64_t* result, void* workspace, int64_t workspace_bytes,
              float* scores_out, const int64_t* goffs, hipStream_t stream) {
  const bool grouped = goffs != nullptr;
  const Layout L = layout(batch_a, batch_b, m, k, n, bs, grouped);
  if (batch_c * m * L.nb * 2 > 0xFFFFFFFFll) return SDC_EUNSUPPORTED;     // flat index in 32 bits
  if (!workspace || workspace_bytes < L.total * (int64_t)sizeof(float) + 256) return SDC_EWORKSPACE;
  float* ws = (float*)(((uintptr_t)workspace + 255) & ~(uintptr_t)255);
  const float* s_full = sign_table + (bs - 1) * 128;
  const float* s_last = L.rem ? sign_table + (L.rem - 1) * 128 : s_full;
  const BConsts bc{ws + L.off_col, ws + L.off_bmax, ws + L.off_bias, (uint16_t*)(ws + L.off_parts),
                   L.fragb ? (uint16_t*)(ws + L.off_frag) : nullptr};
  int rc = stage_b(dtype, B, sbb, sbk, sbn, batch_b, k, n, bs, L, bias, bias_kind, sbias_n, s_full, s_last,
                   ws + L.off_b2t, ws + L.off_part, bc, stream);
  if (rc != SDC_OK) return rc;
  return check_with(dtype, A, sab, sam, sak, batch_a, batch_b, C, scb, scm, scn, batch_c, m, k, bs, L, bc, bias,
                    bias_kind, sbias_b, sbias_m, sbias_n, alpha, beta, z, abs_floor, s_full, s_last, result,
                    ws + L.off_e, ws + L.off_xn, scores_out, goffs, stream);
}

// The expected-side GEMM and the scoring pass of a check whose B-side constants are made (bc).
int check_with(int dtype, const void* A, int64_t sab, int64_t sam, int64_t sak, int64_t batch_a, int64_t batch_b,
               const void* C, int64_t scb, int64_t scm, int64_t scn, int64_t batch_c, int64_t m, int64_t k, int64_t bs,
               const Layout& L, const BConsts& bc, const void* bias, int bias_kind, int64_t sbias_b, int64_t sbias_m,
               int64_t sbias_n, float alpha, float beta, float z, float abs_floor, const float* s_full,
               const float* s_last, int64_t* result, float* E, float* XN, float* scores_out, const int64_t* goffs,
               hipStream_t stream) {
  const bool grouped = goffs != nullptr;
  const int64_t nbt = grouped ? 1 : (batch_a > batch_b ? batch_a : batch_b);
  GemmArgs g{};
  g.A = (const uint16_t*)A; g.sab = batch_a > 1 ? sab : 0; g.sam = sam; g.sak = sak;
  g.B = bc.parts; g.sbb = batch_b > 1 ? 3 * L.ncols * L.kp : 0; g.sbc = L.kp;
  g.m = m; g.k = k; g.N = L.ncols; g.splits = L.splits;
  g.E = E; g.XN = XN;
  const bool c_t = !grouped && scm == 1 && scn != 1 && L.nb < 65536 && batch_c < 65536;   // C read down columns
  g.et = c_t;
  g.prof_name = "train_gemm";
  g.goffs = goffs; g.ngroups = grouped ? batch_b : 0;
  int rc = SDC_EUNSUPPORTED;
  int64_t splits = L.splits;
  bool e_t = c_t;
  if (grouped && bc.frag) {
    // the tall-tile GEMM over SDC_GROUPED_TALL_SPLITS depth parts: E transposed, the groups' fragments L.fragb bytes
    // apart
    GemmArgs gt = g;
    gt.B = bc.frag; gt.sbb = L.fragb / 2; gt.sbc = 0;
    gt.splits = SDC_GROUPED_TALL_SPLITS; gt.et = 1;
    rc = sdc_rs_gemm_tall_launch(dtype, gt, 0, stream);
    if (rc == SDC_OK) {
      splits = gt.splits;
      e_t = true;
    }
  }
  if (rc == SDC_EUNSUPPORTED) rc = sdc_gemm_launch(dtype, g, nbt, stream);
  if (rc != SDC_OK) return rc;

  TrainArgs ta{};
  ta.cv.y = (const uint16_t*)C; ta.cv.sb = scb; ta.cv.sm = scm; ta.cv.sn = scn; ta.cv.m = m; ta.cv.nb = L.nb;
  ta.cv.bs = bs; ta.cv.rem = L.rem; ta.cv.npairs = batch_c * m * L.nb; ta.cv.s_full = s_full; ta.cv.s_last = s_last;
  ta.cv.vec = scn == 1 && (scm % 8 == 0) && (scb % 8 == 0) && (bs % 8 == 0) && ((uintptr_t)C % 16 == 0);
  ta.k = k; ta.splits = splits; ta.nbt = nbt; ta.ncols = L.ncols;
  ta.b_batched = batch_b > 1; ta.e_batched = nbt > 1;
  ta.E = E; ta.XN = XN; ta.colstat = bc.colstat; ta.bmaxf = bc.bmaxf;
  ta.bias_kind = bias_kind; ta.bias_vec = bc.bias3; ta.bias_mat = (const uint16_t*)bias;
  ta.sbias_b = sbias_b; ta.sbias_m = sbias_m; ta.sbias_n = sbias_n;
  ta.alpha = alpha; ta.beta = beta;
  ta.u = dtype == SDC_BF16 ? 1.f / 256.f : 1.f / 2048.f;
  ta.h = dtype == SDC_BF16 ? 0.f : 1.f / 33554432.f;
  ta.abs_floor = abs_floor;
  ta.l1c = (float)(k * 7.450580596923828e-09 > 1e-5 ? k * 7.450580596923828e-09 : 1e-5);
  ta.zt = z;
  ta.lim_a = dtype == SDC_BF16 ? 1e18f : 65504.f;
  ta.capk = (float)(1.02 + (double)k * 2.384185791015625e-07);
  ta.result = result; ta.zdump = scores_out;
  ta.goffs = goffs; ta.ngroups = grouped ? batch_b : 0;
  SdcProf prof("train_score", stream);
  ta.et = e_t;
  if (grouped) {
    const int64_t tiles = sdc_cdiv(ta.cv.npairs, 64);
    if (sdc_cdiv(tiles, 4) > 0x7FFFFFFF) return SDC_EUNSUPPORTED;
    const unsigned grid = (unsigned)sdc_cdiv(tiles, 4);                // one tile per wave
    if (ta.splits <= 2) {                                              // (the tall grouped GEMM's two planes)
      if (dtype == SDC_BF16) hipLaunchKernelGGL((grouped_score_kernel<SDC_BF16, 2>), dim3(grid), dim3(256), 0, stream, ta);
      else hipLaunchKernelGGL((grouped_score_kernel<SDC_FP16, 2>), dim3(grid), dim3(256), 0, stream, ta);
    } else if (ta.splits <= 4) {
      if (dtype == SDC_BF16) hipLaunchKernelGGL((grouped_score_kernel<SDC_BF16, 4>), dim3(grid), dim3(256), 0, stream, ta);
      else hipLaunchKernelGGL((grouped_score_kernel<SDC_FP16, 4>), dim3(grid), dim3(256), 0, stream, ta);
    } else {
      if (dtype == SDC_BF16)
        hipLaunchKernelGGL((grouped_score_kernel<SDC_BF16, SDC_MAX_SPLITS>), dim3(grid), dim3(256), 0, stream, ta);
      else
        hipLaunchKernelGGL((grouped_score_kernel<SDC_FP16, SDC_MAX_SPLITS>), dim3(grid), dim3(256), 0, stream, ta);
    }
  } else if (c_t) {
    // C with adjacent rows (y^T): read 512 rows at a time down each column
    ta.cv.vec = (scn % 8 == 0) && (scb % 8 == 0) && ((uintptr_t)C % 16 == 0);
    dim3 grid((unsigned)sdc_cdiv(m, 512), (unsigned)L.nb, (unsigned)batch_c);
    if (dtype == SDC_BF16) hipLaunchKernelGGL(train_score_t_kernel<SDC_BF16>, grid, dim3(256), 0, stream, ta);
    else hipLaunchKernelGGL(train_score_t_kernel<SDC_FP16>, grid, dim3(256), 0, stream, ta);
  } else {
    const int64_t tiles = sdc_cdiv(ta.cv.npairs, 64);
    const unsigned grid = (unsigned)(sdc_cdiv(tiles, 4) < 1024 ? sdc_cdiv(tiles, 4) : 1024);
    if (dtype == SDC_BF16) hipLaunchKernelGGL(train_score_kernel<SDC_BF16>, dim3(grid), dim3(256), 0, stream, ta);
    else hipLaunchKernelGGL(train_score_kernel<SDC_FP16>, dim3(grid), dim3(256), 0, stream, ta);
  }
  SDC_LAUNCH_CHECK();
  return SDC_OK;
}

}  // namespace

extern "C" int sdc_matmul_check(int dtype, const void* A, int64_t sab, int64_t sam, int64_t sak, int64_t batch_a,
                                const void* B, int64_t sbb, int64_t sbk, int64_t sbn, int64_t batch_b, const void* C,
                                int64_t scb, int64_t scm, int64_t scn, int64_t batch_c, int64_t m, int64_t k,
                                int64_t n, int64_t bs, const void* bias, int bias_kind, int64_t sbias_b,
                                int64_t sbias_m, int64_t sbias_n, float alpha, float beta, float z, float abs_floor,
                                const float* sign_table, int64_t* result, void* workspace, int64_t workspace_bytes,
                                float* scores_out, hipStream_t stream) {
  SDC_CLEAR_ERRORS();
  if (m < 1 || n < 1 || k < 1 || batch_a < 1 || batch_b < 1 || batch_c < 1) return SDC_EINVAL;
  if (dtype != SDC_BF16 && dtype != SDC_FP16) return SDC_EINVAL;
  if (bs < 1 || bs > 128) return SDC_EUNSUPPORTED;
  if (!A || !B || !C || !sign_table || !result) return SDC_EINVAL;
  if (bias_kind < 0 || bias_kind > 2 || (bias_kind && !bias)) return SDC_EINVAL;
  const int64_t nbt = batch_a > batch_b ? batch_a : batch_b;
  if ((batch_a != 1 && batch_a != nbt) || (batch_b != 1 && batch_b != nbt)) return SDC_EINVAL;
  if (batch_c != nbt && !(nbt == 1)) return SDC_EINVAL;
  return run_check(dtype, A, sab, sam, sak, batch_a, B, sbb, sbk, sbn, batch_b, C, scb, scm, scn, batch_c, m, k, n, bs,
                   bias, bias_kind, sbias_b, sbias_m, sbias_n, alpha, beta, z, abs_floor, sign_table, result, workspace,
                   workspace_bytes, scores_out, nullptr, stream);
}

extern "C" int64_t sdc_grouped_check_workspace(int64_t groups, int64_t rows, int64_t k, int64_t n, int64_t bs) {
  if (groups <= 0 || rows <= 0 || n <= 0 || k <= 0 || bs <= 0) return 0;
  return layout(1, groups, rows, k, n, bs, true).total * (int64_t)sizeof(float) + 256;
}

// ---- the grouped check's serving form: the experts' constants made once per layer, the per-call check without
// a B-side stage.  Constants buffer: colstat [groups][2nb][3] | bmaxf [groups][nb] | bias [nb][3] | parts
// [groups][3 * 2nb][kp] (16-bit), each section 256-byte aligned.
namespace {
struct ConstsLayout {
  int64_t off_col, off_bmax, off_bias, off_parts, off_frag, total;          // bytes
};
ConstsLayout consts_layout(int64_t groups, int64_t k, int64_t n, int64_t bs) {
  const Layout L = layout(1, groups, 1, k, n, bs, true);
  auto al = [](int64_t x) { return (x + 255) / 256 * 256; };
  ConstsLayout c{};
  int64_t o = 0;
  c.off_col = o; o += al(groups * L.ncols * 3 * 4);
  c.off_bmax = o; o += al(groups * L.nb * 4);
  c.off_bias = o; o += al(3 * L.nb * 4);
  c.off_parts = o; o += al(groups * 3 * L.ncols * L.kp * 2);
  c.off_frag = o; o += al(groups * L.fragb);                      // (none where the depth is not a multiple of 512)
  c.total = o;
  return c;
}
BConsts consts_at(void* consts, const ConstsLayout& c) {
  uint8_t* p = (uint8_t*)consts;
  return BConsts{(float*)(p + c.off_col), (float*)(p + c.off_bmax), (float*)(p + c.off_bias),
                 (uint16_t*)(p + c.off_parts), c.total > c.off_frag ? (uint16_t*)(p + c.off_frag) : nullptr};
}
}  // namespace

extern "C" int64_t sdc_grouped_constants_bytes(int64_t groups, int64_t k, int64_t n, int64_t bs) {
  if (groups <= 0 || n <= 0 || k <= 0 || bs <= 0 || bs > 128) return 0;
  return consts_layout(groups, k, n, bs).total;
}

// Scratch of the constants' build (the block sums before their split, per-slice statistics).
extern "C" int64_t sdc_grouped_constants_workspace(int64_t groups, int64_t k, int64_t n, int64_t bs) {
  if (groups <= 0 || n <= 0 || k <= 0 || bs <= 0) return 0;
  const Layout L = layout(1, groups, 1, k, n, bs, true);
  return (L.off_col - L.off_b2t) * (int64_t)sizeof(float) + 512;
}

extern "C" int sdc_grouped_constants(int dtype, const void* B, int64_t sbg, int64_t sbk, int64_t sbn, int64_t groups,
                                     int64_t k, int64_t n, int64_t bs, const void* bias, int64_t sbias,
                                     const float* sign_table, void* consts, int64_t consts_bytes, void* workspace,
                                     int64_t workspace_bytes, hipStream_t stream) {
  SDC_CLEAR_ERRORS();
  if (n < 1 || k < 1 || groups < 1) return SDC_EINVAL;
  if (dtype != SDC_BF16 && dtype != SDC_FP16) return SDC_EINVAL;
  if (bs < 1 || bs > 128) return SDC_EUNSUPPORTED;
  if (!B || !sign_table || !consts) return SDC_EINVAL;
  if ((uintptr_t)consts % 256) return SDC_EINVAL;
  const ConstsLayout c = consts_layout(groups, k, n, bs);
  if (consts_bytes < c.total) return SDC_EWORKSPACE;
  if (!workspace || workspace_bytes < sdc_grouped_constants_workspace(groups, k, n, bs)) return SDC_EWORKSPACE;
  const Layout L = layout(1, groups, 1, k, n, bs, true);
  float* ws = (float*)(((uintptr_t)workspace + 255) & ~(uintptr_t)255);
  const float* s_full = sign_table + (bs - 1) * 128;
  const float* s_last = L.rem ? sign_table + (L.rem - 1) * 128 : s_full;
  return stage_b(dtype, B, sbg, sbk, sbn, groups, k, n, bs, L, bias, bias ? 1 : 0, sbias, s_full, s_last, ws,
                 ws + (L.off_part - L.off_b2t), consts_at(consts, c), stream);
}

extern "C" int64_t sdc_grouped_check_consts_workspace(int64_t groups, int64_t rows, int64_t k, int64_t n,
                                                      int64_t bs) {
  if (groups <= 0 || rows <= 0 || n <= 0 || k <= 0 || bs <= 0) return 0;
  const Layout L = layout(1, groups, rows, k, n, bs, true);
  return (L.total - L.off_e) * (int64_t)sizeof(float) + 256;
}

extern "C" int sdc_grouped_check_consts(int dtype, const void* A, int64_t sam, int64_t sak, const void* consts,
                                        int64_t groups, const void* C, int64_t scm, int64_t scn, int64_t rows,
                                        int64_t k, int64_t n, int64_t bs, const int64_t* offs, int has_bias,
                                        float z, float abs_floor, const float* sign_table, int64_t* results,
                                        void* workspace, int64_t workspace_bytes, float* scores_out,
                                        hipStream_t stream) {
  SDC_CLEAR_ERRORS();
  if (rows < 1 || n < 1 || k < 1 || groups < 1) return SDC_EINVAL;
  if (dtype != SDC_BF16 && dtype != SDC_FP16) return SDC_EINVAL;
  if (bs < 1 || bs > 128) return SDC_EUNSUPPORTED;
  if (!A || !consts || !C || !offs || !sign_table || !results) return SDC_EINVAL;
  if ((uintptr_t)consts % 256) return SDC_EINVAL;
  if (scn != 1 && scm == 1) return SDC_EUNSUPPORTED;
  const Layout L = layout(1, groups, rows, k, n, bs, true);
  if (rows * L.nb * 2 > 0xFFFFFFFFll) return SDC_EUNSUPPORTED;
  if (!workspace || workspace_bytes < sdc_grouped_check_consts_workspace(groups, rows, k, n, bs))
    return SDC_EWORKSPACE;
  float* ws = (float*)(((uintptr_t)workspace + 255) & ~(uintptr_t)255);
  const float* s_full = sign_table + (bs - 1) * 128;
  const float* s_last = L.rem ? sign_table + (L.rem - 1) * 128 : s_full;
  const ConstsLayout c = consts_layout(groups, k, n, bs);
  const BConsts bc = consts_at(const_cast<void*>(consts), c);
  // (the bias's block sums are part of the constants; has_bias says whether the layer has one)
  return check_with(dtype, A, 0, sam, sak, 1, groups, C, 0, scm, scn, 1, rows, k, bs, L, bc, nullptr, has_bias ? 1 : 0,
                    0, 0, 0, 1.f, 1.f, z, abs_floor, s_full, s_last, results, ws, ws + (L.off_xn - L.off_e),
                    scores_out, offs, stream);
}

extern "C" int sdc_grouped_check(int dtype, const void* A, int64_t sam, int64_t sak, const void* B, int64_t sbg,
                                 int64_t sbk, int64_t sbn, int64_t groups, const void* C, int64_t scm, int64_t scn,
                                 int64_t rows, int64_t k, int64_t n, int64_t bs, const int64_t* offs, const void* bias,
                                 int64_t sbias, float z, float abs_floor, const float* sign_table, int64_t* results,
                                 void* workspace, int64_t workspace_bytes, float* scores_out, hipStream_t stream) {
  SDC_CLEAR_ERRORS();
  if (rows < 1 || n < 1 || k < 1 || groups < 1) return SDC_EINVAL;
  if (dtype != SDC_BF16 && dtype != SDC_FP16) return SDC_EINVAL;
  if (bs < 1 || bs > 128) return SDC_EUNSUPPORTED;
  if (!A || !B || !C || !offs || !sign_table || !results) return SDC_EINVAL;
  if (scn != 1 && scm == 1) return SDC_EUNSUPPORTED;          // the grouped pass reads C along its rows
  return run_check(dtype, A, 0, sam, sak, 1, B, sbg, sbk, sbn, groups, C, 0, scm, scn, 1, rows, k, n, bs, bias,
                   bias ? 1 : 0, 0, 0, sbias, 1.f, 1.f, z, abs_floor, sign_table, results, workspace,
                   workspace_bytes, scores_out, offs, stream);
}

// ---------------------------------------------------------------------------------------------------------------
// Per-layer constants of the serving check, built on the device from W (n x k, rows k-contiguous) and an optional
// bias: the B-side stage of the training check run on B = W^T (block sums B2 over 128 output rows of W, their
// column norms and maxima, each block's largest |W|, the bias's block sums), the split of B2 into three parts
// (k-major, depth pitch kp = k rounded up to 8), and one table of per-block constants for the check's scoring pass,
// with and without the bias.

namespace {

struct PackArgs {
  const float* colstat;            // [2nb][3]: |B2 column|_2, largest |entry|, power-of-two scale
  const float* bmaxf;              // [nb]
  const float* bias3;              // [nb][3] or null
  int64_t nb;
  float* with_bias;                // [nb][12]
  float* without_bias;             // [nb][12]
};

// |w|_2^2 and |w|_1 of every row of W (the row-block check's noise model takes them per row of its A = W): one
// wave per row, 16-byte pieces across the row, fp32 sums
template <int DT>
__global__ __launch_bounds__(256) void row_norms_kernel(const uint16_t* W, int64_t swn, int64_t n, int64_t k,
                                                        int vec, float* out) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= n) return;                                   // whole waves leave; no barrier follows
  const uint16_t* p = W + row * swn;
  float sq = 0.f, ab = 0.f;
  int64_t kk = 0;
  if (vec) {
    for (; kk + 512 <= k; kk += 512) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(p + kk + 8 * lane);
      const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float a = lo_of<DT>(w4[q]), b = hi_of<DT>(w4[q]);
        sq = fmaf(a, a, sq);
        sq = fmaf(b, b, sq);
        ab += fabsf(a) + fabsf(b);
      }
    }
  }
  for (int64_t e = kk + lane; e < k; e += 64) {
    const float a = half_to_f32<DT>(p[e]);
    sq = fmaf(a, a, sq);
    ab += fabsf(a);
  }
#pragma unroll
  for (int msk = 1; msk < 64; msk <<= 1) {
    sq += __shfl_xor(sq, msk, 64);
    ab += __shfl_xor(ab, msk, 64);
  }
  if (lane == 0) {
    out[row] = sq;
    out[n + row] = ab;
  }
}

// row of a block: scale(plain, signed), bias sums(plain, signed), |B2|_2(2), max |B2|(2), max |W|, max |bias|, 0, 0
__global__ __launch_bounds__(256) void pack_consts_kernel(PackArgs a) {
  for (int64_t jb = (int64_t)blockIdx.x * 256 + threadIdx.x; jb < a.nb; jb += (int64_t)gridDim.x * 256) {
    const float* c = a.colstat + 6 * jb;
    float row[12] = {c[2], c[5], 0.f, 0.f, c[0], c[3], c[1], c[4], a.bmaxf[jb], 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 12; ++i) a.without_bias[12 * jb + i] = row[i];
    if (a.bias3) {
      row[2] = a.bias3[3 * jb];
      row[3] = a.bias3[3 * jb + 1];
      row[9] = a.bias3[3 * jb + 2];
    }
#pragma unroll
    for (int i = 0; i < 12; ++i) a.with_bias[12 * jb + i] = row[i];
  }
}

}  // namespace

extern "C" int64_t sdc_layer_constants_workspace(int64_t n, int64_t k, int64_t bs) {
  if (n <= 0 || k <= 0 || bs <= 0) return 0;
  return layout(1, 1, 1, k, n, bs).total * (int64_t)sizeof(float) + 256;
}

extern "C" int sdc_layer_constants(int dtype, const void* W, int64_t swn, int64_t n, int64_t k, int64_t bs,
                                   const void* bias, int64_t sbias, const float* sign_table, void* parts,
                                   int64_t parts_pitch, float* consts_bias, float* consts_plain, float* row_norms,
                                   void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  SDC_CLEAR_ERRORS();
  if (n < 1 || k < 1 || swn < k) return SDC_EINVAL;
  if (dtype != SDC_BF16 && dtype != SDC_FP16) return SDC_EINVAL;
  if (bs < 1 || bs > 128) return SDC_EUNSUPPORTED;
  if (!W || !sign_table || !parts || !consts_bias || !consts_plain) return SDC_EINVAL;
  const Layout L = layout(1, 1, 1, k, n, bs);
  if (parts_pitch != L.kp) return SDC_EINVAL;
  if (!workspace || workspace_bytes < L.total * (int64_t)sizeof(float) + 256) return SDC_EWORKSPACE;
  float* ws = (float*)(((uintptr_t)workspace + 255) & ~(uintptr_t)255);
  const float* s_full = sign_table + (bs - 1) * 128;
  const float* s_last = L.rem ? sign_table + (L.rem - 1) * 128 : s_full;

  BStageArgs ba{};
  ba.B = (const uint16_t*)W; ba.sbb = 0; ba.sbk = 1; ba.sbn = swn;      // B = W^T: B[kk][j] = W[j][kk]
  ba.k = k; ba.n = n; ba.nb = L.nb; ba.bs = bs; ba.rem = L.rem; ba.nkc = L.nkc;
  ba.s_full = s_full; ba.s_last = s_last; ba.B2T = ws + L.off_b2t; ba.part = ws + L.off_part;
  {
    SdcProf prof("b_stage", stream);
    if (swn != 1) {
      ba.vec = (swn % 8 == 0) && ((uintptr_t)W % 16 == 0);
      dim3 grid((unsigned)sdc_cdiv(k, 256), (unsigned)L.nb, 1u);
      if (dtype == SDC_BF16) hipLaunchKernelGGL(b_stage_t_kernel<SDC_BF16>, grid, dim3(256), 0, stream, ba);
      else hipLaunchKernelGGL(b_stage_t_kernel<SDC_FP16>, grid, dim3(256), 0, stream, ba);
    } else {                                                            // k == 1: W^T is one contiguous row
      ba.vec = (bs % 8 == 0) && ((uintptr_t)W % 16 == 0);
      dim3 grid((unsigned)L.nkc, (unsigned)L.nb, 1u);
      if (dtype == SDC_BF16) hipLaunchKernelGGL(b_stage_kernel<SDC_BF16>, grid, dim3(256), 0, stream, ba);
      else hipLaunchKernelGGL(b_stage_kernel<SDC_FP16>, grid, dim3(256), 0, stream, ba);
    }
    SDC_LAUNCH_CHECK();
  }
  BFinishArgs fa{};
  fa.part = ws + L.off_part; fa.nkc = L.nkc; fa.nb = L.nb; fa.bs = bs; fa.rem = L.rem; fa.fp16 = dtype == SDC_FP16;
  fa.colstat = ws + L.off_col; fa.bmaxf = ws + L.off_bmax;
  fa.bias = (const uint16_t*)bias; fa.sbias = sbias;
  fa.s_full = s_full; fa.s_last = s_last; fa.bias_out = ws + L.off_bias;
  {
    SdcProf prof("b_finish", stream);
    if (dtype == SDC_BF16) hipLaunchKernelGGL(b_finish_kernel<SDC_BF16>, dim3((unsigned)L.nb, 1u), dim3(64), 0, stream, fa);
    else hipLaunchKernelGGL(b_finish_kernel<SDC_FP16>, dim3((unsigned)L.nb, 1u), dim3(64), 0, stream, fa);
    SDC_LAUNCH_CHECK();
  }
  int rc = sdc_split_launch(dtype, ws + L.off_b2t, ws + L.off_col + 2, L.ncols * 3, 3, L.ncols, k, L.kp, 1,
                            (uint16_t*)parts, stream);
  if (rc != SDC_OK) return rc;
  PackArgs pa{ws + L.off_col, ws + L.off_bmax, bias ? ws + L.off_bias : nullptr, L.nb, consts_bias, consts_plain};
  const unsigned grid = (unsigned)(sdc_cdiv(L.nb, 256) < 1024 ? sdc_cdiv(L.nb, 256) : 1024);
  hipLaunchKernelGGL(pack_consts_kernel, dim3(grid), dim3(256), 0, stream, pa);
  SDC_LAUNCH_CHECK();
  if (row_norms) {
    const int vec = (swn % 8 == 0) && ((uintptr_t)W % 16 == 0);
    const dim3 g4((unsigned)sdc_cdiv(n, 4));
    if (dtype == SDC_BF16)
      hipLaunchKernelGGL(row_norms_kernel<SDC_BF16>, g4, dim3(256), 0, stream, (const uint16_t*)W, swn, n, k, vec,
                         row_norms);
    else
      hipLaunchKernelGGL(row_norms_kernel<SDC_FP16>, g4, dim3(256), 0, stream, (const uint16_t*)W, swn, n, k, vec,
                         row_norms);
    SDC_LAUNCH_CHECK();
  }
  return SDC_OK;
}
