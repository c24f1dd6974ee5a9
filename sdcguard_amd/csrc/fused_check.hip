// A linear layer computed on MFMA with the check of its fp32 accumulator in the same kernel (fused.py:116-176,
// :238-546): C = A @ B + bias rounded to A's dtype, where B is read as W = B^T (a linear layer's weight, rows of
// depth), and, before rounding, for every row of C and block of 128 columns either
//   - statistics mode (`fused_mm`): the float64 plain sum, signed sum (the +-1 pattern of the block's width), sum
//     of squares and sum of absolute values of the fp32 accumulator (bias added), scored later against
//     x . (block sums of W) in float64 (acc_check.hip, sdc_matmul_check_acc_stats); or
//   - check mode (`fused_mm_checked`): the check itself, scored in the epilogue with no float64 on the expected
//     side: each stage of 32 depths multiplies the tile's rows of A by three bf16/fp16 parts of each block sum of
//     W (a narrow 16-column MFMA beside the main ones), and the stage results are added into a running fp32 sum
//     compensated for its rounding (Neumaier's variant of Kahan summation); the score follows precise mode's
//     noise model plus the expected side's own rounding (fused.py:392-450).
// Either way the product is never read back from HBM and the matmul runs once.
//
// Tiles of 256 rows of A by 256 rows of W (two checksum blocks), eight waves of 128 x 64 (2 x 4), 4 x 2 fragments
// of v_mfma_f32_32x32x16 each.  Depth advances 32 at a time through three LDS buffers filled straight from global
// memory (global_load_lds_dwordx4, 16 tile rows per instruction, four per wave per stage, three stages ahead; in
// check mode wave 0 also loads the stage's 16 rows of block-sum parts); every wave reads the fragments of the next
// MFMA step while the current step's MFMAs run.  Workgroups take tiles in groups of four row tiles per XCD, so the
// rows of A and W that a group of concurrent workgroups reads stay in that XCD's L2.
// Epilogue: bias and an optional injected fault (experiments) go into the accumulator, C is rounded and stored,
// then the accumulator passes through LDS in four rounds of 32 rows per wave and four lanes reduce each
// (row, block)'s 128 columns in float64.
//
// Operands that are not depth-contiguous with 16-byte rows (a transposed view such as a weight gradient's dY^T),
// or whose depth is not a multiple of 32, are first copied into zero-padded depth-contiguous workspace copies.
#include "common.h"
#include "mfma_pipe.h"
#include "profile.h"

namespace {

using namespace sdc_pipe;

constexpr int FT = 256;                       // tile rows (of A) and columns (rows of W)
constexpr int FNT = 512;                      // threads per workgroup
constexpr int FBUF = 3;                       // LDS buffers
constexpr int BXR = 16;                       // rows of block-sum parts per column tile: 2 blocks x 6, padded
constexpr int FROWS = 2 * FT + BXR;           // LDS rows per stage: 256 of A, 256 of W, the parts
constexpr int FNIW = 2 * FT / 16 / 8;         // global-to-LDS instructions per wave per stage (rows of A and W)
constexpr int GROUP_M = 4;                    // row tiles per group of the tile order
constexpr int BLK = 128;                      // checksum block width
constexpr int SROW = 2 * (BLK + 16);          // floats per LDS row of the statistics pass: two blocks, 16 apart
constexpr int STG_FLOATS = 64 * SROW;         // one round of the statistics pass
constexpr int E_FLOATS = 2 * FT * BXR;        // narrow-dot sums and their compensations
constexpr int PIPE_BYTES = FBUF * FROWS * KS * 2;
constexpr int EPI_BYTES = (STG_FLOATS + E_FLOATS + 8) * 4;
constexpr int LDS_BYTES = PIPE_BYTES > EPI_BYTES ? PIPE_BYTES : EPI_BYTES;
constexpr int PSLICE = 64;                    // depths per workgroup of the side pass
constexpr float U32 = 5.9604644775390625e-08f;          // 2^-24, checksum.py:558
constexpr float C1 = 0.6f, C2 = 1.0f, C3 = 1.0f;        // checksum.py:559

__device__ __forceinline__ float nan_abs(float v) { return v == v ? fabsf(v) : __builtin_inff(); }

template <int DT>
__device__ __forceinline__ uint16_t round16(float f) {
  if constexpr (DT == SDC_BF16) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
  } else {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
  }
}

// The power of two that puts 128 max|W| (the largest block sum a block can have) in [2^14, 2^15), so fp16 holds the
// three parts of every block sum; 1 when max|W| is not finite (fused.py:263-270)
__device__ __forceinline__ float pow2_scale(float wmax) {
  int e = (int)((__float_as_uint(wmax * 128.0f) >> 23) & 0xFFu);
  e = e == 255 ? 141 : (e > 15 ? e : 15);
  return __uint_as_float((uint32_t)(e - 14) << 23);
}

// ------------------------------------------------------------------------------------------------ operand copies
// dst (rows, kp) depth-contiguous from src (rows, k) with strides (s_row, s_k), depths k .. kp - 1 zero.  64 x 64
// tiles; a source whose rows are contiguous (s_row == 1, a transposed view) goes through LDS so that both the loads
// and the stores are coalesced.
__global__ __launch_bounds__(256) void fused_pack_kernel(const uint16_t* src, int64_t s_row, int64_t s_k,
                                                         int64_t rows, int64_t k, uint16_t* dst, int64_t kp) {
  __shared__ uint16_t tile[64][66];
  const int t = threadIdx.x;
  const int64_t r0 = (int64_t)blockIdx.x * 64, k0 = (int64_t)blockIdx.y * 64;
  if (s_row != 1 || s_k == 1) {
#pragma unroll 4
    for (int i = 0; i < 16; ++i) {
      const int e = t + 256 * i, r = e >> 6, c = e & 63;
      const int64_t row = r0 + r, kk = k0 + c;
      if (row < rows && kk < kp) dst[row * kp + kk] = kk < k ? src[row * s_row + kk * s_k] : (uint16_t)0;
    }
  } else {
#pragma unroll 4
    for (int i = 0; i < 16; ++i) {
      const int e = t + 256 * i, c = e >> 6, r = e & 63;
      const int64_t row = r0 + r, kk = k0 + c;
      tile[c][r] = (row < rows && kk < k) ? src[row + kk * s_k] : (uint16_t)0;
    }
    __syncthreads();
#pragma unroll 4
    for (int i = 0; i < 16; ++i) {
      const int e = t + 256 * i, r = e >> 6, c = e & 63;
      const int64_t row = r0 + r, kk = k0 + c;
      if (row < rows && kk < kp) dst[row * kp + kk] = tile[c][r];
    }
  }
}

// --------------------------------------------------------------------------------------------- the side pass
// Check mode's inputs besides the operands (fused.py:272-316, and the row norms of fused.py:513-515):
//   bx    [ntp][16][kp]: per column tile (two blocks) and depth, rows 6 h + 3 s + p = part p (hi, mid, lo) of the
//         plain (s = 0) or signed (s = 1) block sum of block 2 tile + h; the block sums are float64 sums rounded
//         once to fp32 (fp16: divided first by pow2_scale(max|W| of the block)); rows 12 .. 15 zero;
//   wpart [nslice][nb][4]: per slice of 64 depths and block, sum of W^2, of plain block sums^2, of signed block
//         sums^2 (the fp32 sums), and max |W| (NaN counts as Inf);
//   an    [2][m]: |a_row|_2 and |a_row|_1;   bsum [nb][4]: the bias's plain and signed block sums, max |bias|.
// PASS 0 makes all of it (bf16); fp16 runs PASS 1 (everything but bx) and then PASS 2 (bx, scaled by the block's
// max |W| from PASS 1's partials).
struct SideArgs {
  const uint16_t* w;                          // (n, kp)
  int64_t swn;
  const uint16_t* x;                          // (m, kp)
  int64_t sxm;
  const void* bias;
  int bias_f32;
  const float* sign_table;
  uint16_t* bx;
  double* wpart;
  double* bsum;
  float* an;
  int64_t m, kp, n, nb, rem, nslice;
  int64_t side_blocks, an_blocks;
};

template <int DT, int PASS>
__global__ __launch_bounds__(256) void fused_side_kernel(SideArgs a) {
  __shared__ double red_pl[4][64], red_sg[4][64];
  __shared__ double red_q[4][2];
  __shared__ float red_s;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int64_t bid = blockIdx.x;
  if (bid < a.side_blocks) {
    const int64_t jb = bid % a.nb, sl = bid / a.nb;
    const int64_t wid = (jb == a.nb - 1 && a.rem > 0) ? a.rem : BLK;
    const float* sp = a.sign_table + (wid - 1) * 128;
    float sc = 1.0f;
    if constexpr (PASS == 2) {                  // the block's max |W| from the first pass's partials
      double mx = 0.0;
      for (int64_t s = t; s < a.nslice; s += 256) mx = fmax(mx, a.wpart[(s * a.nb + jb) * 4 + 3]);
#pragma unroll
      for (int msk = 1; msk < 64; msk <<= 1) mx = fmax(mx, __shfl_xor(mx, msk, SDC_WAVE));
      if (lane == 0) red_q[w][0] = mx;
      __syncthreads();
      if (t == 0) red_s = pow2_scale((float)fmax(fmax(red_q[0][0], red_q[1][0]), fmax(red_q[2][0], red_q[3][0])));
      __syncthreads();
      sc = red_s;
    }
    // thread: depth sl * 64 + lane, rows 32 w .. 32 w + 31 of the block (64 lanes read 128 contiguous bytes)
    const int64_t kk = sl * PSLICE + lane;
    const bool live = kk < a.kp;
    double pl = 0.0, sg = 0.0, sq = 0.0;
    float mx = 0.f;
    if (live) {
      const uint16_t* col = a.w + (jb * BLK) * a.swn + kk;
      for (int j = 32 * w; j < 32 * w + 32; ++j) {
        if (j >= wid) break;
        const float v = half_to_f32<DT>(col[(int64_t)j * a.swn]);
        pl += (double)v;
        sg += (double)v * (double)sp[j];
        sq += (double)v * (double)v;
        mx = fmaxf(mx, nan_abs(v));
      }
    }
    red_pl[w][lane] = pl;
    red_sg[w][lane] = sg;
    if constexpr (PASS != 2) {
#pragma unroll
      for (int msk = 1; msk < 64; msk <<= 1) {
        sq += __shfl_xor(sq, msk, SDC_WAVE);
        mx = fmaxf(mx, __shfl_xor(mx, msk, SDC_WAVE));
      }
      if (lane == 0) {
        red_q[w][0] = sq;
        red_q[w][1] = (double)mx;
      }
    }
    __syncthreads();
    if (w == 0) {
      const double P = (red_pl[0][lane] + red_pl[1][lane]) + (red_pl[2][lane] + red_pl[3][lane]);
      const double S = (red_sg[0][lane] + red_sg[1][lane]) + (red_sg[2][lane] + red_sg[3][lane]);
      const float bp = (float)P, bs = (float)S;
      if constexpr (PASS != 1) {
        if (live) {
          uint16_t* base = a.bx + ((jb >> 1) * BXR + 6 * (jb & 1)) * a.kp + kk;
          const float xs[2] = {bp / sc, bs / sc};
#pragma unroll
          for (int s = 0; s < 2; ++s) {
            const uint16_t hi = round16<DT>(xs[s]);
            const float r = xs[s] - half_to_f32<DT>(hi);
            const uint16_t mid = round16<DT>(r);
            const uint16_t lo = round16<DT>(r - half_to_f32<DT>(mid));
            base[(3 * s) * a.kp] = hi;
            base[(3 * s + 1) * a.kp] = mid;
            base[(3 * s + 2) * a.kp] = lo;
          }
          if ((jb & 1) == 0) {                  // the tile's padding rows, and a missing second block
            uint16_t* pair = a.bx + (jb >> 1) * BXR * a.kp + kk;
            for (int r = (jb == a.nb - 1 ? 6 : 12); r < BXR; ++r) pair[r * a.kp] = 0;
          }
        }
      }
      if constexpr (PASS != 2) {
        double q1 = live ? (double)bp * (double)bp : 0.0, q2 = live ? (double)bs * (double)bs : 0.0;
#pragma unroll
        for (int msk = 1; msk < 64; msk <<= 1) {
          q1 += __shfl_xor(q1, msk, SDC_WAVE);
          q2 += __shfl_xor(q2, msk, SDC_WAVE);
        }
        if (lane == 0) {
          double* o = a.wpart + (sl * a.nb + jb) * 4;
          o[0] = (red_q[0][0] + red_q[1][0]) + (red_q[2][0] + red_q[3][0]);
          o[1] = q1;
          o[2] = q2;
          o[3] = fmax(fmax(red_q[0][1], red_q[1][1]), fmax(red_q[2][1], red_q[3][1]));
        }
      }
    }
    return;
  }
  if constexpr (PASS == 2) return;
  if (bid < a.side_blocks + a.an_blocks) {      // |a_row|_2 and |a_row|_1, one wave per row
    const int64_t row = (bid - a.side_blocks) * 4 + w;
    if (row >= a.m) return;
    const uint16_t* xr = a.x + row * a.sxm;
    double sq = 0.0, l1 = 0.0;
    for (int64_t kk = lane; kk < a.kp; kk += 64) {
      const double v = (double)half_to_f32<DT>(xr[kk]);
      sq += v * v;
      l1 += fabs(v);
    }
#pragma unroll
    for (int msk = 1; msk < 64; msk <<= 1) {
      sq += __shfl_xor(sq, msk, SDC_WAVE);
      l1 += __shfl_xor(l1, msk, SDC_WAVE);
    }
    if (lane == 0) {
      a.an[row] = (float)sqrt(sq);
      a.an[a.m + row] = (float)l1;
    }
    return;
  }
  // the bias's block sums: one thread per block
  const int64_t jb = (bid - a.side_blocks - a.an_blocks) * 256 + t;
  if (!a.bias || jb >= a.nb) return;
  const int64_t wid = (jb == a.nb - 1 && a.rem > 0) ? a.rem : BLK;
  const float* sp = a.sign_table + (wid - 1) * 128;
  double pl = 0.0, sg = 0.0;
  float mx = 0.f;
  for (int64_t c = 0; c < wid; ++c) {
    const int64_t i = jb * BLK + c;
    const float v = a.bias_f32 ? reinterpret_cast<const float*>(a.bias)[i]
                               : half_to_f32<DT>(reinterpret_cast<const uint16_t*>(a.bias)[i]);
    pl += (double)v;
    sg += (double)v * (double)sp[c];
    mx = fmaxf(mx, nan_abs(v));
  }
  a.bsum[jb * 4] = pl;
  a.bsum[jb * 4 + 1] = sg;
  a.bsum[jb * 4 + 2] = (double)mx;
  a.bsum[jb * 4 + 3] = 0.0;
}

// -------------------------------------------------------------------------------------------- the fused GEMM
struct FusedArgs {
  const uint16_t* x;                          // (m, kp), row stride sxm
  int64_t sxm;
  const uint16_t* w;                          // (n, kp), row stride swn
  int64_t swn;
  const uint16_t* bx;                         // check mode: block-sum parts (the side pass)
  const void* bias;                           // (n) of dtype, or fp32 with bias_f32, or null
  int bias_f32;
  uint16_t* y;                                // (m, n), row stride sym
  int64_t sym;
  double* stats;                              // statistics mode: (m, nb, 4)
  const float* sign_table;                    // 128 x 128, row w - 1 = the pattern of width w
  const double* wpart;                        // check mode: the side pass's outputs
  const double* bsum;
  const float* an;
  int64_t nslice;
  int64_t m, kp, k, n, nb, rem;
  float steps, zthr, abs_floor;
  int64_t* result;                            // check mode: worst key, key with its noise, unjudged count
  float* scores;                              // check mode, optional: (m, nb, 2)
  double* expected;                           // check mode, optional: (m, nb, 2) expected sides (bias included)
  int64_t inj_m, inj_n;                       // inject: add inj_v to the accumulator at (inj_m, inj_n)
  float inj_v;
  int inject;
};

// One checksum pair of check mode, scored as fused.py:419-458 scores it (fp32 noise terms; the differences are
// taken between float64 sums, and overflow of either side is judged at fp32's range).
struct PairScore {
  float z0, z1, den;
};

__device__ __forceinline__ PairScore score_pair(const FusedArgs& a, double ep, double es, double ap, double as,
                                                float cn, float cl1, float an, float al1, float bfro2, float bsp2,
                                                float bss2, float bmax, float bound_b, float wf) {
  const float inf = __builtin_inff();
  const float kf = (float)a.k;
  const float sk = sqrtf(kf);
  const float per_out = C2 * sk + C3 * a.steps + sqrtf(wf);
  const float bound = al1 * bmax + bound_b;
  const float stand_in = bound * (U32 * 128.0f);
  float prod = an * sqrtf(bfro2) * (C1 * sk * U32);
  prod = (prod == prod && fabsf(prod) < inf) ? prod : stand_in;
  const float noise = cn * (per_out * U32) + prod;
  const float skc = sqrtf(kf < 32.f ? kf : 32.f);
  const float ep32 = (float)ep, es32 = (float)es;
  float exp_ = an * sqrtf(bsp2) * (C1 * skc * U32) + 4.0f * U32 * fabsf(ep32);
  float exs = an * sqrtf(bss2) * (C1 * skc * U32) + 4.0f * U32 * fabsf(es32);
  exp_ = fabsf(exp_) < inf ? exp_ : stand_in;
  exs = fabsf(exs) < inf ? exs : stand_in;
  const float noise_p = noise + exp_, noise_s = noise + exs;
  const float den_p = noise_p + a.abs_floor, den_s = noise_s + a.abs_floor;
  const double dp = fabs(ep - ap), ds = fabs(es - as);
  float zp = (float)(dp / (double)den_p), zs = (float)(ds / (double)den_s);
  const float worst = cl1 * (per_out * U32) + prod + exp_ + a.abs_floor;
  const float zw = (float)(dp / (double)worst * (double)a.zthr);
  zp = (zp == zp && zw == zw) ? fminf(zp, zw) : __builtin_nanf("");
  const float lim = bound * 1.01f;
  const bool e_bad = !(fabsf(ep32) < inf) || !(fabsf(es32) < inf);
  const bool a_bad = (!(fabsf((float)ap) < inf) || !(fabsf((float)as) < inf)) && !e_bad;
  const bool n_bad = (!(noise_p < inf) || !(noise_s < inf)) && !e_bad && !a_bad;
  const float cap = bound * (1.02f + kf * 2.384185791015625e-07f);
  const bool imposs = !e_bad && !a_bad && !n_bad && (lim < 1e18f) && (cn > cap * sqrtf(wf));
  const float for_bad = lim < 1e18f ? inf : -1.f;
  zp = zp == zp ? zp : -1.f;
  zs = zs == zs ? zs : -1.f;
  zp = imposs ? inf : zp;
  zs = imposs ? inf : zs;
  zp = (a_bad || n_bad) ? for_bad : zp;
  zs = (a_bad || n_bad) ? for_bad : zs;
  zp = e_bad ? -1.f : zp;
  zs = e_bad ? -1.f : zs;
  return {zp, zs, zp >= zs ? den_p : den_s};
}

template <int DT, bool CHECK>
__global__ __launch_bounds__(FNT) void fused_mm_kernel(FusedArgs a) {
  // one LDS object: with several, the compiler's wait-count pass makes every LDS read wait for all loads into LDS
  __shared__ __attribute__((aligned(16))) uint8_t smem[LDS_BYTES + 160];
  int64_t* red_k = reinterpret_cast<int64_t*>(smem + LDS_BYTES);
  int64_t* red_d = red_k + 8;
  int* red_u = reinterpret_cast<int*>(red_d + 8);
  uint16_t(*lds)[FROWS * KS] = reinterpret_cast<uint16_t(*)[FROWS * KS]>(smem);
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int wm = w >> 2, wn = w & 3;
  const int64_t nrt = sdc_cdiv(a.m, FT), nct = sdc_cdiv(a.n, FT);
  // XCD-aware order (block b runs on XCD b % 8: XCD x takes the x-th eighth of the tiles), grouped by GROUP_M rows
  const int64_t G = (int64_t)gridDim.x, b = blockIdx.x;
  const int64_t wid = (G % 8 == 0) ? (b % 8) * (G / 8) + b / 8 : b;
  const int64_t per_group = GROUP_M * nct, group = wid / per_group;
  const int64_t first = group * GROUP_M;
  const int64_t gm = nrt - first < GROUP_M ? nrt - first : GROUP_M;
  const int64_t rt = first + (wid % per_group) % gm, ct = (wid % per_group) / gm;
  const int64_t r0 = rt * FT, c0 = ct * FT;

  // this wave's load instructions: LDS rows 16 I .. 16 I + 15 of a stage; lane L loads the chunk the swizzle puts
  // at position L % 4 of row L / 4 (rows past m or n read row 0: their results are never stored)
  const uint8_t* src[FNIW];
  int dst[FNIW];
#pragma unroll
  for (int j = 0; j < FNIW; ++j) {
    const int I = w + 8 * j;
    const int R = 16 * I + lane / 4, P = lane % 4;
    const int q = P ^ ((R >> 1) & 3);
    dst[j] = 16 * I * KS;
    if (R < FT) {
      const int64_t row = r0 + R;
      src[j] = reinterpret_cast<const uint8_t*>(a.x + (row < a.m ? row : 0) * a.sxm) + 16 * q;
    } else {
      const int64_t row = c0 + R - FT;
      src[j] = reinterpret_cast<const uint8_t*>(a.w + (row < a.n ? row : 0) * a.swn) + 16 * q;
    }
  }
  const uint8_t* bsrc = nullptr;              // check mode, wave 0: the tile's 16 rows of block-sum parts
  if constexpr (CHECK) {
    const int R = lane / 4, q = (lane % 4) ^ ((R >> 1) & 3);
    bsrc = reinterpret_cast<const uint8_t*>(a.bx + (ct * BXR + R) * a.kp) + 16 * q;
  }
  auto issue = [&](int st, int buf) {
    const int64_t off = (int64_t)st * KS * 2;
    if constexpr (CHECK) {
      if (w == 0) lds_load16(bsrc + off, &lds[buf][2 * FT * KS]);
    }
#pragma unroll
    for (int j = 0; j < FNIW; ++j) lds_load16(src[j] + off, &lds[buf][dst[j]]);
  };

  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][n][r] = 0.f;
  // check mode: this wave's rows 128 wm + 32 wn + 16 g + (0 .. 15) times the 16 part columns; sx the running sums,
  // cx their compensations, part the last stage's product (added in the next stage)
  f32x4 sx[2], cx[2], part[2];
#pragma unroll
  for (int g = 0; g < 2; ++g)
#pragma unroll
    for (int r = 0; r < 4; ++r) sx[g][r] = cx[g][r] = part[g][r] = 0.f;

  struct Frag {
    u32x4 a[4], b[2];
  };
  struct NFrag {
    u32x4 a[2], b;
  };
  auto read = [&](Frag& f, int buf, int step) {
    const uint16_t* L = lds[buf];
    const int q = 2 * step + (lane >> 5);
#pragma unroll
    for (int i = 0; i < 4; ++i) f.a[i] = *reinterpret_cast<const u32x4*>(&L[lds_at(wm * 128 + 32 * i + (lane & 31), q)]);
#pragma unroll
    for (int n = 0; n < 2; ++n) f.b[n] = *reinterpret_cast<const u32x4*>(&L[lds_at(FT + wn * 64 + 32 * n + (lane & 31), q)]);
  };
  auto read_n = [&](NFrag& f, int buf) {
    const uint16_t* L = lds[buf];
    const int q = lane >> 4;
#pragma unroll
    for (int g = 0; g < 2; ++g)
      f.a[g] = *reinterpret_cast<const u32x4*>(&L[lds_at(wm * 128 + 32 * wn + 16 * g + (lane & 15), q)]);
    f.b = *reinterpret_cast<const u32x4*>(&L[lds_at(2 * FT + (lane & 15), q)]);
  };
  auto mma = [&](const Frag& f) {
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i][n] = mfma32<DT>(f.a[i], f.b[n], acc[i][n]);
  };
  auto mma_n = [&](const NFrag& f) {
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int g = 0; g < 2; ++g) part[g] = mfma16<DT>(f.a[g], f.b, zero);
  };
  auto neumaier = [&]() {
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float s = sx[g][r], p = part[g][r], tt = s + p;
        cx[g][r] += fabsf(s) >= fabsf(p) ? (s - tt) + p : (p - tt) + s;
        sx[g][r] = tt;
      }
  };

  const int nst = (int)(a.kp / KS);
  {
    const int last = nst - 1;
    issue(0, 0);
    issue(1 < last ? 1 : last, 1);
    issue(2 < last ? 2 : last, 2);
    // stage 0 in LDS (stages 1, 2 may be in flight; wave 0's one more load per stage only makes it wait longer)
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * FNIW));
    __syncthreads();
    Frag fx, fy;
    NFrag nf;
    read(fx, 0, 0);
    __builtin_amdgcn_s_waitcnt(lgkmcnt0_imm());
    int b0 = 0, b1 = 1;
    for (int s = 0; s < nst; ++s) {
      read(fy, b0, 1);
      if constexpr (CHECK) read_n(nf, b0);
      __builtin_amdgcn_sched_barrier(0);
      mma(fx);
      if constexpr (CHECK) neumaier();                          // the previous stage's narrow product
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(FNIW));           // stage s + 1 in LDS (stage s + 2 may be in flight)
      __syncthreads();
      issue(s + 3 < last ? s + 3 : last, b0);
      read(fx, b1, 0);
      __builtin_amdgcn_sched_barrier(0);
      mma(fy);
      if constexpr (CHECK) mma_n(nf);
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_waitcnt(lgkmcnt0_imm());
      b0 = b1;
      b1 = b1 == FBUF - 1 ? 0 : b1 + 1;
    }
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));               // no load into LDS outlives the main loop
    if constexpr (CHECK) neumaier();
  }

  // ---- epilogue: bias, injection, C
  // fragment (i, n), register r: row r0 + 128 wm + 32 i + 8 (r / 4) + 4 (lane / 32) + r % 4,
  // column c0 + 64 wn + 32 n + lane % 32 (rows and columns fit 31 bits: checked at the entry point)
  const int mrow = (int)a.m, ncol = (int)a.n;
  const int rowb = (int)r0 + wm * 128 + 4 * (lane >> 5);
#pragma unroll
  for (int n = 0; n < 2; ++n) {
    const int col = (int)c0 + wn * 64 + 32 * n + (lane & 31);
    float bv = 0.f;
    if (a.bias && col < ncol)
      bv = a.bias_f32 ? reinterpret_cast<const float*>(a.bias)[col]
                      : half_to_f32<DT>(reinterpret_cast<const uint16_t*>(a.bias)[col]);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][n][r] += bv;
    if (a.inject && col == (int)a.inj_n) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (rowb + 32 * i + 8 * (r >> 2) + (r & 3) == (int)a.inj_m) acc[i][n][r] += a.inj_v;
    }
    if (col < ncol) {
      uint16_t* yc = a.y + (int64_t)rowb * a.sym + col;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int dr = 32 * i + 8 * (r >> 2) + (r & 3);
          if (rowb + dr < mrow) yc[(int64_t)dr * a.sym] = round16<DT>(acc[i][n][r]);
        }
    }
  }

  // ---- block sums of the accumulator: round i puts every wave's rows 32 i .. 32 i + 31 in LDS (row 32 wm + rr of
  // the round, block wn / 2 at float (wn / 2) * (BLK + 16), column 64 (wn % 2) + 32 n + lane % 32 of the block);
  // then thread t adds chunks c4, c4 + 4, ..., c4 + 28 (16 bytes each) of (row t / 8, block (t / 4) % 2), c4 = t % 4
  float* stg = reinterpret_cast<float*>(smem);
  float* es = stg + STG_FLOATS;               // check mode: [256][16] narrow-dot sums, then [256][16] compensations
  float* aux = es + E_FLOATS;                 // check mode: [2 blocks][4] the W-side norms and max |W|
  const int pr = t >> 3, pb = (t >> 2) & 1, c4 = t & 3;
  const int64_t blk = c0 / BLK + pb;
  const int64_t wid_b = (blk == a.nb - 1 && a.rem > 0) ? a.rem : BLK;
  const float* sp = a.sign_table + (wid_b - 1) * 128;
  int64_t key = 0, keyd = 0;
  int unk = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {                                 // (unrolled: acc is indexed by constants only)
    __syncthreads();                                            // (the main loop's and the last round's readers)
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int rr = 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        stg[(wm * 32 + rr) * SROW + (wn >> 1) * (BLK + 16) + (wn & 1) * 64 + 32 * n + (lane & 31)] = acc[i][n][r];
      }
    if constexpr (CHECK) {
      if (i == 0) {
        // the narrow dot's results: lane holds column lane % 16 of rows 128 wm + 32 wn + 16 g + 4 (lane / 16) + r
#pragma unroll
        for (int g = 0; g < 2; ++g)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int rl = wm * 128 + 32 * wn + 16 * g + 4 * (lane >> 4) + r;
            es[rl * BXR + (lane & 15)] = sx[g][r];
            es[FT * BXR + rl * BXR + (lane & 15)] = cx[g][r];
          }
        // wave w: quantity w % 4 of block w / 4 of the tile, from the side pass's per-slice partials
        const int64_t ab = c0 / BLK + (w >> 2);
        const int qn = w & 3;
        double v = 0.0;
        if (ab < a.nb)
          for (int64_t s = lane; s < a.nslice; s += 64) {
            const double pv = a.wpart[(s * a.nb + ab) * 4 + qn];
            v = qn == 3 ? fmax(v, pv) : v + pv;
          }
#pragma unroll
        for (int msk = 1; msk < 64; msk <<= 1) {
          const double o = __shfl_xor(v, msk, SDC_WAVE);
          v = qn == 3 ? fmax(v, o) : v + o;
        }
        if (lane == 0) aux[w] = (float)v;
      }
    }
    __syncthreads();
    double pl = 0.0, sg = 0.0, sq = 0.0, ab = 0.0;
    const float* rowp = stg + pr * SROW + pb * (BLK + 16);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int cc = 4 * (c4 + 4 * j);                         // column of the block
      const f32x4 v = *reinterpret_cast<const f32x4*>(rowp + cc);
      const f32x4 s = *reinterpret_cast<const f32x4*>(sp + cc);
      const float vv[4] = {v.x, v.y, v.z, v.w};
      const float ss[4] = {s.x, s.y, s.z, s.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const double c = (cc + e < wid_b) ? (double)vv[e] : 0.0;
        pl += c;
        sg += c * (double)ss[e];
        sq += c * c;
        ab += fabs(c);
      }
    }
#pragma unroll
    for (int msk = 1; msk < 4; msk <<= 1) {
      pl += __shfl_xor(pl, msk, SDC_WAVE);
      sg += __shfl_xor(sg, msk, SDC_WAVE);
      sq += __shfl_xor(sq, msk, SDC_WAVE);
      ab += __shfl_xor(ab, msk, SDC_WAVE);
    }
    const int rl = (pr >> 5) * 128 + 32 * i + (pr & 31);
    const int row = (int)r0 + rl;
    if (c4 == 0 && row < mrow && blk < a.nb) {
      if constexpr (!CHECK) {
        double* o = a.stats + ((int64_t)row * a.nb + blk) * 4;
        o[0] = pl;
        o[1] = sg;
        o[2] = sq;
        o[3] = ab;
      } else {
        const float* e0 = es + rl * BXR + 6 * pb;
        const float* k0 = e0 + FT * BXR;
        double ep = ((double)e0[0] + (double)e0[1] + (double)e0[2]) + ((double)k0[0] + (double)k0[1] + (double)k0[2]);
        double esg = ((double)e0[3] + (double)e0[4] + (double)e0[5]) + ((double)k0[3] + (double)k0[4] + (double)k0[5]);
        const float* ax = aux + 4 * pb;
        if constexpr (DT == SDC_FP16) {                          // the parts were made from block sums / this
          const double sc = (double)pow2_scale(ax[3]);
          ep *= sc;
          esg *= sc;
        }
        float bound_b = 0.f;
        if (a.bias) {
          ep += a.bsum[blk * 4];
          esg += a.bsum[blk * 4 + 1];
          bound_b = (float)a.bsum[blk * 4 + 2];
        }
        const PairScore ps = score_pair(a, ep, esg, pl, sg, (float)sqrt(sq), (float)ab, a.an[row], a.an[a.m + row],
                                        ax[0], ax[1], ax[2], ax[3], bound_b, (float)wid_b);
        const int64_t flat = (int64_t)row * a.nb + blk;
        if (a.scores) {
          a.scores[2 * flat] = ps.z0;
          a.scores[2 * flat + 1] = ps.z1;
        }
        if (a.expected) {
          a.expected[2 * flat] = ep;
          a.expected[2 * flat + 1] = esg;
        }
        unk += (ps.z0 < 0.f) + (ps.z1 < 0.f);
        const bool sec = ps.z1 > ps.z0;
        const int64_t zb = fbits64(fmaxf(sec ? ps.z1 : ps.z0, 0.f));
        const int64_t kk = (zb << 32) | ((flat * 2 + (sec ? 1 : 0)) & 0xFFFFFFFFll);
        const int64_t kd = (zb << 32) | (fbits64(ps.den) & 0xFFFFFFFFll);
        key = kk > key ? kk : key;
        keyd = kd > keyd ? kd : keyd;
      }
    }
  }
  if constexpr (CHECK) {
    key = wave_max_i64(key);
    keyd = wave_max_i64(keyd);
    unk = wave_sum_i32(unk);
    if (lane == 0) {
      red_k[w] = key;
      red_d[w] = keyd;
      red_u[w] = unk;
    }
    __syncthreads();
    if (t == 0) {
      int64_t k0 = red_k[0], d0 = red_d[0];
      int u = red_u[0];
      for (int j = 1; j < 8; ++j) {
        k0 = red_k[j] > k0 ? red_k[j] : k0;
        d0 = red_d[j] > d0 ? red_d[j] : d0;
        u += red_u[j];
      }
      if (k0 > __atomic_load_n(a.result, __ATOMIC_RELAXED))
        atomicMax((unsigned long long*)a.result, (unsigned long long)k0);
      if (d0 > __atomic_load_n(a.result + 1, __ATOMIC_RELAXED))
        atomicMax((unsigned long long*)(a.result + 1), (unsigned long long)d0);
      if (u > 0) atomicAdd((unsigned long long*)(a.result + 2), (unsigned long long)u);
    }
  }
}

// ------------------------------------------------------------------------------------------------ host side
struct FusedPlan {
  bool pack_x, pack_w;
  int64_t kp, nb, nslice, ntp;
  int64_t off_x, off_w, off_bx, off_wpart, off_bsum, off_an, total;        // bytes
};

bool direct_ok(const void* p, int64_t s_row, int64_t s_k, int64_t k) {
  return s_k == 1 && s_row % 8 == 0 && k % KS == 0 && k > 0 && ((uintptr_t)p & 15) == 0;
}

FusedPlan fused_plan(const void* A, int64_t sam, int64_t sak, const void* B, int64_t sbk, int64_t sbn, int64_t m,
                     int64_t k, int64_t n, bool check) {
  FusedPlan P{};
  P.kp = k > 0 ? sdc_cdiv(k, KS) * KS : KS;
  P.pack_x = !direct_ok(A, sam, sak, k);
  P.pack_w = !direct_ok(B, sbn, sbk, k);                  // W = B^T: row stride sbn, depth stride sbk
  P.nb = sdc_cdiv(n, BLK);
  P.nslice = sdc_cdiv(P.kp, PSLICE);
  P.ntp = sdc_cdiv(n, FT);
  auto al = [](int64_t x) { return (x + 255) / 256 * 256; };
  int64_t o = 0;
  P.off_x = o; o += P.pack_x ? al(m * P.kp * 2) : 0;
  P.off_w = o; o += P.pack_w ? al(n * P.kp * 2) : 0;
  if (check) {
    P.off_bx = o; o += al(P.ntp * BXR * P.kp * 2);
    P.off_wpart = o; o += al(P.nslice * P.nb * 4 * 8);
    P.off_bsum = o; o += al(P.nb * 4 * 8);
    P.off_an = o; o += al(2 * m * 4);
  }
  P.total = o;
  return P;
}

int validate(int dtype, const void* A, const void* B, const void* C, int64_t m, int64_t k, int64_t n) {
  if (dtype != SDC_BF16 && dtype != SDC_FP16) return SDC_EUNSUPPORTED;
  if (!C || m < 1 || n < 1 || k < 0 || (k > 0 && (!A || !B))) return SDC_EINVAL;    // (k = 0: never read)
  const int64_t tiles = sdc_cdiv(m, FT) * sdc_cdiv(n, FT);
  if (tiles > 0x7FFFFFFF || m >= (1ll << 31) - FT || n >= (1ll << 31) - FT) return SDC_EUNSUPPORTED;
  if (m * sdc_cdiv(n, BLK) * 2 > 0xFFFFFFFFll) return SDC_EUNSUPPORTED;    // flat indexes fit the key's 32 bits
  return SDC_OK;
}

// the operands as the kernel reads them: direct, or packed into the workspace
int prepare(const FusedPlan& P, uint8_t* ws, const void* A, int64_t sam, int64_t sak, const void* B, int64_t sbk,
            int64_t sbn, int64_t m, int64_t k, int64_t n, FusedArgs& a, hipStream_t stream) {
  a.x = (const uint16_t*)A;
  a.sxm = sam;
  a.w = (const uint16_t*)B;
  a.swn = sbn;
  if (P.pack_x || P.pack_w) {
    SdcProf prof("fused_pack", stream);
    if (P.pack_x) {
      uint16_t* d = (uint16_t*)(ws + P.off_x);
      hipLaunchKernelGGL(fused_pack_kernel, dim3((unsigned)sdc_cdiv(m, 64), (unsigned)sdc_cdiv(P.kp, 64)), dim3(256),
                         0, stream, (const uint16_t*)A, sam, sak, m, k, d, P.kp);
      SDC_LAUNCH_CHECK();
      a.x = d;
      a.sxm = P.kp;
    }
    if (P.pack_w) {
      uint16_t* d = (uint16_t*)(ws + P.off_w);
      hipLaunchKernelGGL(fused_pack_kernel, dim3((unsigned)sdc_cdiv(n, 64), (unsigned)sdc_cdiv(P.kp, 64)), dim3(256),
                         0, stream, (const uint16_t*)B, sbn, sbk, n, k, d, P.kp);
      SDC_LAUNCH_CHECK();
      a.w = d;
      a.swn = P.kp;
    }
  }
  return SDC_OK;
}

template <int DT, bool CHECK>
int launch(const FusedArgs& a, hipStream_t stream) {
  const int64_t tiles = sdc_cdiv(a.m, FT) * sdc_cdiv(a.n, FT);
  SdcProf prof(CHECK ? "fused_mm_checked" : "fused_mm", stream);
  hipLaunchKernelGGL((fused_mm_kernel<DT, CHECK>), dim3((unsigned)tiles), dim3(FNT), 0, stream, a);
  SDC_LAUNCH_CHECK();
  return SDC_OK;
}

template <int DT>
int run_side(const FusedPlan& P, SideArgs s, hipStream_t stream) {
  SdcProf prof("fused_side", stream);
  const int64_t bias_blocks = s.bias ? sdc_cdiv(P.nb, 256) : 0;
  const unsigned all = (unsigned)(s.side_blocks + s.an_blocks + bias_blocks);
  if constexpr (DT == SDC_BF16) {
    hipLaunchKernelGGL((fused_side_kernel<DT, 0>), dim3(all), dim3(256), 0, stream, s);
    SDC_LAUNCH_CHECK();
  } else {
    hipLaunchKernelGGL((fused_side_kernel<DT, 1>), dim3(all), dim3(256), 0, stream, s);
    SDC_LAUNCH_CHECK();
    hipLaunchKernelGGL((fused_side_kernel<DT, 2>), dim3((unsigned)s.side_blocks), dim3(256), 0, stream, s);
    SDC_LAUNCH_CHECK();
  }
  return SDC_OK;
}

}  // namespace

extern "C" int64_t sdc_fused_mm_workspace(const void* A, int64_t sam, int64_t sak, const void* B, int64_t sbk,
                                          int64_t sbn, int64_t m, int64_t k, int64_t n, int checked) {
  if (m < 1 || n < 1 || k < 0) return 0;
  return fused_plan(A, sam, sak, B, sbk, sbn, m, k, n, checked != 0).total + 256;
}

extern "C" int sdc_fused_mm(int dtype, const void* A, int64_t sam, int64_t sak, const void* B, int64_t sbk,
                            int64_t sbn, int64_t m, int64_t k, int64_t n, const void* bias, int bias_f32,
                            const float* sign_table, void* C, int64_t scm, double* stats, int64_t inj_m,
                            int64_t inj_n, float inj_v, int inject, void* workspace, int64_t workspace_bytes,
                            hipStream_t stream) {
  SDC_CLEAR_ERRORS();
  int rc = validate(dtype, A, B, C, m, k, n);
  if (rc != SDC_OK) return rc;
  if (!stats || !sign_table) return SDC_EINVAL;
  const FusedPlan P = fused_plan(A, sam, sak, B, sbk, sbn, m, k, n, false);
  if (P.total > 0 && (!workspace || workspace_bytes < P.total + 256)) return SDC_EWORKSPACE;
  uint8_t* ws = (uint8_t*)(((uintptr_t)workspace + 255) & ~(uintptr_t)255);
  FusedArgs a{};
  rc = prepare(P, ws, A, sam, sak, B, sbk, sbn, m, k, n, a, stream);
  if (rc != SDC_OK) return rc;
  a.bias = bias; a.bias_f32 = bias_f32; a.y = (uint16_t*)C; a.sym = scm; a.stats = stats; a.sign_table = sign_table;
  a.m = m; a.kp = P.kp; a.k = k; a.n = n; a.nb = P.nb; a.rem = n % BLK;
  a.inj_m = inj_m; a.inj_n = inj_n; a.inj_v = inj_v; a.inject = inject;
  return dtype == SDC_BF16 ? launch<SDC_BF16, false>(a, stream) : launch<SDC_FP16, false>(a, stream);
}

extern "C" int sdc_fused_mm_checked(int dtype, const void* A, int64_t sam, int64_t sak, const void* B, int64_t sbk,
                                    int64_t sbn, int64_t m, int64_t k, int64_t n, const void* bias, int bias_f32,
                                    const float* sign_table, void* C, int64_t scm, float nfma, float z,
                                    float abs_floor, int64_t* result, float* scores_out, double* expected_out,
                                    int64_t inj_m, int64_t inj_n, float inj_v, int inject, void* workspace,
                                    int64_t workspace_bytes, hipStream_t stream) {
  SDC_CLEAR_ERRORS();
  int rc = validate(dtype, A, B, C, m, k, n);
  if (rc != SDC_OK) return rc;
  if (!result || !sign_table) return SDC_EINVAL;
  const FusedPlan P = fused_plan(A, sam, sak, B, sbk, sbn, m, k, n, true);
  if (!workspace || workspace_bytes < P.total + 256) return SDC_EWORKSPACE;
  uint8_t* ws = (uint8_t*)(((uintptr_t)workspace + 255) & ~(uintptr_t)255);
  FusedArgs a{};
  rc = prepare(P, ws, A, sam, sak, B, sbk, sbn, m, k, n, a, stream);
  if (rc != SDC_OK) return rc;
  SideArgs s{};
  s.w = a.w; s.swn = a.swn; s.x = a.x; s.sxm = a.sxm; s.bias = bias; s.bias_f32 = bias_f32; s.sign_table = sign_table;
  s.bx = (uint16_t*)(ws + P.off_bx); s.wpart = (double*)(ws + P.off_wpart); s.bsum = (double*)(ws + P.off_bsum);
  s.an = (float*)(ws + P.off_an);
  s.m = m; s.kp = P.kp; s.n = n; s.nb = P.nb; s.rem = n % BLK; s.nslice = P.nslice;
  s.side_blocks = P.nslice * P.nb; s.an_blocks = sdc_cdiv(m, 4);
  rc = dtype == SDC_BF16 ? run_side<SDC_BF16>(P, s, stream) : run_side<SDC_FP16>(P, s, stream);
  if (rc != SDC_OK) return rc;
  a.bx = s.bx; a.wpart = s.wpart; a.bsum = s.bsum; a.an = s.an; a.nslice = P.nslice;
  a.bias = bias; a.bias_f32 = bias_f32; a.y = (uint16_t*)C; a.sym = scm; a.sign_table = sign_table;
  a.m = m; a.kp = P.kp; a.k = k; a.n = n; a.nb = P.nb; a.rem = n % BLK;
  a.steps = nfma > 0.f ? (float)((double)k / (double)nfma) : 0.f;
  a.zthr = z; a.abs_floor = abs_floor; a.result = result; a.scores = scores_out; a.expected = expected_out;
  a.inj_m = inj_m; a.inj_n = inj_n; a.inj_v = inj_v; a.inject = inject;
  return dtype == SDC_BF16 ? launch<SDC_BF16, true>(a, stream) : launch<SDC_FP16, true>(a, stream);
}
