// Both block checksums of one linear layer y = x @ W^T (+ b), with one pass over y.
//
// Column-block check (the serving check, serve.py:301-396 / _serve_fast.py:102-526): for every row i of y and
// block of 128 output columns, sum_j y_ij against x_i . B2 (B2: the layer's block sums of W, three parts, made once
// per layer), scored as the serving check scores it (unjudged checksums count, score 0).
// Row-block check (the column-block check of y^T = W x^T, checksum.py:435-530 on
// transposed operands): for every column j and block of 128 rows, sum_i y_ij against W_j . (sum_i x_i), scored as
// the training check scores it (unjudged checksums score -1).
//
// Five launches, no host synchronisation:
//   1. xstage: the plain and signed sums of every 128-row block of x, split into three bf16 parts (the B operand
//      of the row check's GEMM), and per 256-deep chunk partials of those sums' statistics and of x's row norms;
//   2. xfinish, on a side stream beside 3: those partials added up in chunk order (the column check's |x_i|_2^2 and
//      |x_i|_1, the row blocks' statistics and sign-pattern sums);
//   3. the row check's GEMM E_row = W @ (x block sums) on MFMA (expected_gemm.hip; W's row norms are the layer's,
//      made once by sdc_layer_constants);
//   4. the column check's GEMM E_col = x @ B2 on MFMA -- independent of 1 to 3, so it can run on the side stream
//      concurrently with them;
//   5. ypass: one read of y.  A workgroup owns a 128 x 128 tile (one row block by one column block): every thread
//      reads 8 rows x 8 columns (eight 16-byte loads, all in flight), adds the four sums (plain, signed, squares,
//      |values|) of its rows with packed dot products and those of its columns by pairing two rows' values of a
//      column into one packed operand; the 16 lanes sharing the rows add theirs with DPP steps, the column partials
//      go through LDS; then two waves score the tile's 128 (row, column block) pairs and two its 128 (column,
//      row block) pairs, and the workgroup's worst keys go to the two result rows with one atomic maximum each.
#include <algorithm>

#include "blocksums.h"
#include "gemm.h"
#include "judge.h"
#include "profile.h"
#include "streams.h"
#include "xfinish.h"


namespace {

constexpr int BS = 128;            // block width of both checks
constexpr int RS_K = 256;          // depth multiple of the register-streamed GEMM (expected_gemm.hip)
constexpr int XK = 128;            // depth per xstage workgroup
#ifndef SDC_YTPW
#define SDC_YTPW 1
#endif
constexpr int YTPW = SDC_YTPW;     // column blocks per y-pass workgroup

__device__ __forceinline__ float nan_abs(float v) { return v == v ? fabsf(v) : __builtin_inff(); }

__device__ __forceinline__ uint16_t bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));

// sum over the 16 lanes of a DPP row
template <int DT>
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_xor1(v);
  v += dpp_xor2(v);
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, true));   // half mirror
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, true));   // row mirror
  return v;
}

// One reduce-scatter step over the lanes of a DPP row: the lane holds NV values (v[0 .. NV)), its partner under
// the DPP pattern CTRL the same ones; `low` lanes keep the first half, the others the second (moved to the front),
// each adding the partner's copy of what it keeps (which the partner sends: the half it does not keep).  Every lane
// active.
template <int CTRL, int NV>
__device__ __forceinline__ void row_scatter(float* v, bool low) {
  constexpr int H = NV / 2;
#pragma unroll
  for (int j = 0; j < H; ++j) {
    const float keep = low ? v[j] : v[H + j], send = low ? v[H + j] : v[j];
    v[j] = keep + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(send), CTRL, 0xF, 0xF, true));
  }
}

// ---------------------------------------------------------------------------------------- 1. x block sums

// One workgroup: one row block (128 rows) by 128 consecutive depths (32 KB of x).  Thread t = 16 rg + dc reads
// depths 8 dc .. 8 dc + 7 of rows rg + 16 i (i < 8): eight 16-byte loads, a wave covering four rows of 256
// contiguous bytes each.  Per row, its |x|_2^2 and |x|_1 over the thread's 8 depths (packed dot products), added
// over the row's 16 lanes (one DPP row) and written per depth chunk for xfinish_kernel.  Per depth, the plain and
// signed sums over the thread's 8 rows by packed dot products that pick one half of each word (exact: +-1 times a
// bf16 value); lane swaps add the four row groups of a wave and LDS the four waves, and thread t < 128 owns depth
// t: its two sums become three bf16 parts
// (checksum._split3), stored k-contiguous per checksum column or in the register-streamed GEMM's fragment order.
// max |x| of the tile as the packed 16-bit maximum of the magnitudes' bits (NaN above infinity, read as infinity).
__global__ __launch_bounds__(256) void xstage_kernel(XStageArgs a) {
  __shared__ f32x4 red[4][4][16];                 // each wave's depth sums [wave][lane / 16][lane % 16]
  __shared__ float wst[4][NXS];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int dc = t & 15, rg = t >> 4;
  const int64_t kc = blockIdx.x, ib = blockIdx.y;
  const int64_t k0 = kc * XK + 8 * dc;
  const int wid = (int)((ib == a.mb - 1 && a.rem > 0) ? a.rem : BS);
  const float* sp = (ib == a.mb - 1 && a.rem > 0) ? a.s_last : a.s_full;
  const uint16_t* base = a.x + (ib * BS) * a.sxm + k0;
  constexpr uint32_t ONES = 0x3F803F80u, HI1 = 0x3F800000u;
  // (1, 0) as a bf16 pair, kept in a register: as an immediate the compiler encodes 0x00003F80 as the inline
  // constant 1.0, which v_dot2c_f32_bf16 does not read as that pair
  uint32_t LO1;
  asm volatile("v_mov_b32 %0, 0x3f80" : "=v"(LO1));
  float pl[8], sg[8], rsq[8], rab[8];
  uint32_t mxb = 0;                                // packed max of the magnitudes' bits
#pragma unroll
  for (int e = 0; e < 8; ++e) pl[e] = sg[e] = rsq[e] = rab[e] = 0.f;
  if (k0 + 8 <= a.k) {
    // loads unconditional (a guarded load makes the compiler wait for it inside the guard); rows past a narrower
    // last block read row 0 of the block and are weighted 0
    u32x4 v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = rg + 16 * i;
      v[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(base + (int64_t)(r < wid ? r : 0) * a.sxm));
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = rg + 16 * i;
      const float s = sp[r];                      // (0 past the pattern's width)
      if (r >= wid) v[i] = u32x4{0u, 0u, 0u, 0u};
      const uint32_t sb = __float_as_uint(s) >> 16;                   // s as bf16 (+-1 or 0: exact)
      const uint32_t slo = sb, shi = sb << 16;
      const uint32_t ww[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        rsq[i] = dot2<SDC_BF16>(ww[q], ww[q], rsq[i]);
        const uint32_t mag = ww[q] & 0x7FFF7FFFu;
        rab[i] = dot2<SDC_BF16>(mag, ONES, rab[i]);
        mxb = __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2, mxb),
                                                                     __builtin_bit_cast(u16x2, mag)));
        pl[2 * q] = dot2<SDC_BF16>(ww[q], LO1, pl[2 * q]);
        pl[2 * q + 1] = dot2<SDC_BF16>(ww[q], HI1, pl[2 * q + 1]);
        sg[2 * q] = dot2<SDC_BF16>(ww[q], slo, sg[2 * q]);
        sg[2 * q + 1] = dot2<SDC_BF16>(ww[q], shi, sg[2 * q + 1]);
      }
    }
  } else if (k0 < a.k) {
    const int ne = (int)(a.k - k0);
#pragma unroll 1
    for (int i = 0; i < 8; ++i) {
      const int r = rg + 16 * i;
      if (r >= wid) continue;
      const float s = sp[r];
      for (int e = 0; e < ne; ++e) {
        const uint16_t b = base[(int64_t)r * a.sxm + e];
        const float xv = bf16_lo(b);
        pl[e] += xv;
        sg[e] = fmaf(xv, s, sg[e]);
        const uint32_t mag = b & 0x7FFFu;
        mxb = (mxb & 0xFFFFu) >= mag ? mxb : ((mxb & 0xFFFF0000u) | mag);
        rsq[i] = fmaf(xv, xv, rsq[i]);
        rab[i] += fabsf(xv);
      }
    }
  }
  // the wave's four row groups (lanes dc, dc + 16, dc + 32, dc + 48) add their depth sums by lane swaps:
  // permlane32_swap pairs lanes q and q + 2, permlane16_swap then q and q + 1; value i of lane (q, dc) (pl[0 .. 7],
  // then sg[0 .. 7]) ends as the wave's sum of value i + 4 q, so lane (q, dc) holds depths 8 dc + 4 (q % 2) .. + 3
  // of the plain (q < 2) or signed (q >= 2) sums
  {
    float t1[8], u[4];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(pl[j]), __float_as_uint(sg[j]), false, false);
      t1[j] = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(t1[j]), __float_as_uint(t1[j + 4]), false,
                                                      false);
      u[j] = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    }
    red[w][lane >> 4][lane & 15] = f32x4{u[0], u[1], u[2], u[3]};
  }
  // the row's 16 lanes (a DPP row) add its norms in lane order; lane dc < 8 keeps row rg + 16 dc
  {
    float keep_sq = 0.f, keep_ab = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float q = row16_sum<SDC_BF16>(rsq[i]), b = row16_sum<SDC_BF16>(rab[i]);
      if (dc == i) {
        keep_sq = q;
        keep_ab = b;
      }
    }
    const int r = rg + 16 * dc;
    if (dc < 8 && r < wid) {
      const int64_t row = ib * BS + r;
      a.xnp[(kc * 2 + 0) * a.m + row] = keep_sq;
      a.xnp[(kc * 2 + 1) * a.m + row] = keep_ab;
    }
  }
  // max |x|: the larger half, as a float (NaN's bits are above infinity's: read as infinity)
  uint32_t mb16 = (mxb & 0xFFFFu) > (mxb >> 16) ? (mxb & 0xFFFFu) : (mxb >> 16);
  float mx = mb16 > 0x7F80u ? __builtin_inff() : __uint_as_float(mb16 << 16);
  mx = wave_max_f32_dpp(mx);                      // (every lane active: DPP moves, no LDS round trips)
  __syncthreads();
  float st[4] = {0.f, 0.f, 0.f, 0.f};
  if (t < XK) {
    // depth t = 8 dc + e: plain sums at slot (e / 4, dc), signed at (2 + e / 4, dc), element e % 4
    const float* rf = reinterpret_cast<const float*>(&red[0][0][0]);
    const int e4 = (t & 7) >> 2, dcr = t >> 3, ec = t & 3;
    float P = 0.f, S = 0.f;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      P += rf[((g * 4 + e4) * 16 + dcr) * 4 + ec];
      S += rf[((g * 4 + 2 + e4) * 16 + dcr) * 4 + ec];
    }
    const int64_t kk = kc * XK + t;
    const bool mine = kk < a.k;
    if (kk < a.kp) {
      // three parts of each sum (hi + mid + lo reproduces it to ~2^-27); depths past k are zero
      const float v2[2] = {mine ? P : 0.f, mine ? S : 0.f};
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const uint16_t h = bf16_rne(v2[c]);
        const float r1 = v2[c] - bf16_lo(h);
        const uint16_t md = bf16_rne(r1);
        const uint16_t lo = bf16_rne(r1 - bf16_lo(md));
        const int64_t col = 2 * ib + c;
        if (a.frag) {
          // element e of lane l of fragment (step s, part p, column fragment f): column 32 f + l % 32, depth
          // 64 (s / 4) + 32 (l / 32) + 8 (s % 4) + e
          const int64_t fs = 4 * (kk >> 6) + ((kk & 31) >> 3);
          const int64_t ln = (col & 31) + 32 * ((kk & 63) >> 5);
          const int64_t fb = (fs * 3 * a.ncf + (col >> 5)) * 512 + ln * 8 + (kk & 7);
          a.parts[fb] = h;
          a.parts[fb + a.ncf * 512] = md;
          a.parts[fb + 2 * a.ncf * 512] = lo;
        } else {
          a.parts[(0 * 2 * a.mb + col) * a.kp + kk] = h;
          a.parts[(1 * 2 * a.mb + col) * a.kp + kk] = md;
          a.parts[(2 * 2 * a.mb + col) * a.kp + kk] = lo;
        }
      }
    }
    st[0] = mine ? P * P : 0.f;
    st[1] = mine ? S * S : 0.f;
    st[2] = mine ? nan_abs(P) : 0.f;
    st[3] = mine ? nan_abs(S) : 0.f;
  }
  st[0] = wave_sum_f32_dpp(st[0]);
  st[1] = wave_sum_f32_dpp(st[1]);
  st[2] = wave_max_f32_dpp(st[2]);
  st[3] = wave_max_f32_dpp(st[3]);
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) wst[w][i] = st[i];
    wst[w][4] = mx;
  }
  __syncthreads();
  if (t < NXS) {
    float v = wst[0][t];
    for (int i = 1; i < 4; ++i) v = t < 2 ? v + wst[i][t] : fmaxf(v, wst[i][t]);
    a.stats[(kc * a.mb + ib) * NXS + t] = v;
  }
}


// The finishing step as its own launch (where the row check's GEMM has no spare workgroups to run it).
__global__ __launch_bounds__(256) void xfinish_kernel(XStageArgs a) { xfinish_block(a, blockIdx.x, threadIdx.x); }

// --------------------------------------------------------------------------------------------- 4. the y pass
struct YArgs {
  const uint16_t* y;
  int64_t sym, m, n, k, nb, mb, rem_n, rem_m;
  const float* sign_table;         // 128 x 128, row w - 1 = the pattern of width w
  // column-block check (serving flavour)
  const float* Ecol;               // [scol][2 nb][m] (transposed planes)
  const float* xn;                 // [2][m]: |x_i|_2^2, |x_i|_1
  int64_t scol;
  const f32x4* consts;             // (nb, 12) packed per-block constants of the layer
  int64_t* state;                  // int64[4]: key, key with noise, checks, unjudged
  float* zcol;                     // (m, nb, 2) scores or null
  // row-block check (training flavour)
  const float* Erow;               // [srow][2 mb][n]
  const float* wn;                 // [2][n]: |w_j|_2^2, |w_j|_1
  int64_t srow;
  const float* rstat;              // [mb][RST]: the row blocks' statistics (xstage)
  const uint16_t* bias;            // (n) or null
  int64_t* result;                 // int64[3]: key, key with noise, unjudged
  float* zrow;                     // (n, mb, 2) scores or null
  // constants of both noise models
  float u, h, abs_floor, l1c, zt, lim_a, lim_big, capk;
};


struct Best {
  int64_t key = 0, keyd = 0;
  int unk = 0;
};

__device__ __forceinline__ void keep_best(Best& b, float zc, bool sec, float dc, int64_t p) {
  const int64_t zb = fbits64(fmaxf(zc, 0.f));
  const int64_t k1 = (zb << 32) | ((p * 2 + (sec ? 1 : 0)) & 0xFFFFFFFFll);
  const int64_t k2 = (zb << 32) | (fbits64(dc) & 0xFFFFFFFFll);
  b.key = k1 > b.key ? k1 : b.key;
  b.keyd = k2 > b.keyd ? k2 : b.keyd;
}

// Signs of a pattern as packed pairs of 16-bit +-1 (entries past the width read as +1: they only ever meet zeros)
template <int DT>
__device__ __forceinline__ uint32_t pack_signs(float s0, float s1) {
  constexpr uint32_t ONE = DT == SDC_BF16 ? 0x3F80u : 0x3C00u;
  return (ONE | ((__float_as_uint(s0) >> 16) & 0x8000u)) | ((ONE << 16) | (__float_as_uint(s1) & 0x80000000u));
}


// A workgroup takes TPW tiles of one row block: 128 rows x 128 columns each (one column block), column blocks
// TPW bx .. TPW bx + TPW - 1.  Every tile's loads (y and what its scoring reads) are issued first, so the later
// tiles' reads stream in while the first tile is summed and scored.  Per tile, thread t = 16 rg + cg owns rows
// 8 rg .. 8 rg + 7 and columns 8 cg .. 8 cg + 7 (each load instruction of a wave reads 4 rows x 256 contiguous
// bytes).  Waves 0 and 1 score the tile's 128 column-block pairs (one row each), waves 2 and 3 its 128 row-block
// pairs (one column each).  Each wave keeps its worst keys over the tiles; one atomic maximum per check and
// workgroup at the end.
// NS: the most planes of E either check has (1 or 2: the register-streamed GEMMs; else up to SDC_MAX_SPLITS), added
// in plane order
template <int DT, int NS, int TPW>
__global__ __launch_bounds__(256) void ypass_kernel(YArgs a) {
  __shared__ f32x4 colw[4][2][64];              // each wave's column sums [wave][column parity][lane]
  __shared__ f32x4 rows[BS];                    // the tile's row sums
  __shared__ int64_t red_k[4], red_d[4];
  __shared__ int red_u[4];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int rg = t >> 4, cg = t & 15;
  const int ib = blockIdx.y, jb0 = blockIdx.x * TPW;
  const int r0 = ib * BS;
  const int wr = (int)((ib == a.mb - 1 && a.rem_m > 0) ? a.rem_m : BS);     // rows in this row block
  const int m = (int)a.m, n = (int)a.n;
  const bool colside = w < 2;
  const int R = r0 + 64 * w + lane;                                          // (column side) this lane's row
  constexpr uint32_t ONES = DT == SDC_BF16 ? 0x3F803F80u : 0x3C003C00u;
  // the result rows' worst keys as they stand now (thread 0: the column check's, thread 64: the row check's), read
  // first so the read's latency hides under the tile's: at the end a key at or below them needs no atomic (keys
  // only grow, so a stale value only lets an unneeded atomic through)
  int64_t seen0 = 0, seen1 = 0;
  if (t == 0 || t == 64) {
    const int64_t* res = t == 0 ? a.state : a.result;
    seen0 = __atomic_load_n(res, __ATOMIC_RELAXED);
    seen1 = __atomic_load_n(res + 1, __ATOMIC_RELAXED);
  }

  // ---- what every tile shares: the row block's pattern (this thread's 8 rows), statistics, the rows' norms
  uint32_t srow2[4];
  {
    const float* spr = a.sign_table + (wr - 1) * 128;
    const f32x4 ra = *reinterpret_cast<const f32x4*>(spr + 8 * rg);
    const f32x4 rb = *reinterpret_cast<const f32x4*>(spr + 8 * rg + 4);
    srow2[0] = pack_signs<DT>(ra.x, ra.y); srow2[1] = pack_signs<DT>(ra.z, ra.w);
    srow2[2] = pack_signs<DT>(rb.x, rb.y); srow2[3] = pack_signs<DT>(rb.z, rb.w);
  }
  const f32x4 rst0 = *reinterpret_cast<const f32x4*>(a.rstat + (int64_t)ib * RST);
  const f32x4 rst1 = *reinterpret_cast<const f32x4*>(a.rstat + (int64_t)ib * RST + 4);
  const float rstat[NXS] = {rst0.x, rst0.y, rst0.z, rst0.w, rst1.x};
  const float rsign = rst1.y;
  const int Rc = R < m ? R : m - 1;
  const float xsq = colside ? a.xn[Rc] : 0.f, xsum = colside ? a.xn[a.m + Rc] : 0.f;

  // ---- every tile's loads: y (eight 16-byte pieces, unconditional on a full tile), its column block's pattern,
  //      E, and (row side) W's row norms and the bias
  u32x4 v[TPW][8];
  float ev[TPW][NS][2], wsq[TPW], wsum[TPW], bjv[TPW];
  uint32_t scol2[TPW][4];
#pragma unroll
  for (int tt = 0; tt < TPW; ++tt) {
    const int jbt = jb0 + tt < a.nb ? jb0 + tt : (int)a.nb - 1;   // (a tile past the last is skipped below)
    const int c0 = jbt * BS;
    const int wc = (int)((jbt == a.nb - 1 && a.rem_n > 0) ? a.rem_n : BS);
    if (wr == BS && wc == BS) {
      const uint16_t* p0 = a.y + (int64_t)(r0 + 8 * rg) * a.sym + c0 + 8 * cg;
#pragma unroll
      for (int i = 0; i < 8; ++i)
        v[tt][i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p0 + i * a.sym));
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int r = 8 * rg + i;
        v[tt][i] = (r < wr && 8 * cg < wc) ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
                                                 a.y + (int64_t)(r0 + r) * a.sym + c0 + 8 * cg))
                                           : u32x4{0u, 0u, 0u, 0u};
      }
    }
    {
      const float* spc = a.sign_table + (wc - 1) * 128;
      const f32x4 ca = *reinterpret_cast<const f32x4*>(spc + 8 * cg);
      const f32x4 cb = *reinterpret_cast<const f32x4*>(spc + 8 * cg + 4);
      scol2[tt][0] = pack_signs<DT>(ca.x, ca.y); scol2[tt][1] = pack_signs<DT>(ca.z, ca.w);
      scol2[tt][2] = pack_signs<DT>(cb.x, cb.y); scol2[tt][3] = pack_signs<DT>(cb.z, cb.w);
    }
    const float* ebase;
    int64_t estride, pstride, splits;
    if (colside) {
      ebase = a.Ecol + (int64_t)(2 * jbt) * a.m + Rc; estride = a.m; pstride = 2 * a.nb * a.m; splits = a.scol;
      wsq[tt] = wsum[tt] = bjv[tt] = 0.f;
    } else {
      const int J = c0 + 64 * (w - 2) + lane, Jc = J < n ? J : n - 1;
      ebase = a.Erow + (int64_t)(2 * ib) * a.n + Jc; estride = a.n; pstride = 2 * a.mb * a.n; splits = a.srow;
      wsq[tt] = a.wn[Jc];
      wsum[tt] = a.wn[a.n + Jc];
      bjv[tt] = a.bias ? half_to_f32<DT>(a.bias[Jc]) : 0.f;
    }
#pragma unroll
    for (int sp = 0; sp < NS; ++sp) {
      const int64_t sc = sp < splits ? sp : 0;
      ev[tt][sp][0] = ebase[sc * pstride];
      ev[tt][sp][1] = ebase[sc * pstride + estride];
    }
  }

  Best best;
#pragma unroll
  for (int tt = 0; tt < TPW; ++tt) {
    const int jb = jb0 + tt;
    if (jb >= a.nb) break;                                       // (uniform over the workgroup)
    if (tt > 0) __syncthreads();                                 // the previous tile's LDS reads are done
    const int c0 = jb * BS;
    const int wc = (int)((jb == a.nb - 1 && a.rem_n > 0) ? a.rem_n : BS);
    // ---- column direction: two rows' values of one column packed into one operand
    // (the first row pair starts each sum with the three-operand dot2: no cleared accumulators)
    float cs[8][4];
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
      const uint32_t w0[4] = {v[tt][i].x, v[tt][i].y, v[tt][i].z, v[tt][i].w};
      const uint32_t w1[4] = {v[tt][i + 1].x, v[tt][i + 1].y, v[tt][i + 1].z, v[tt][i + 1].w};
      const uint32_t sr = srow2[i / 2];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t plo = __builtin_amdgcn_perm(w1[q], w0[q], 0x05040100u);     // column 2q of rows i, i + 1
        const uint32_t phi = __builtin_amdgcn_perm(w1[q], w0[q], 0x07060302u);     // column 2q + 1
        const uint32_t op[2] = {plo, phi};
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const uint32_t pv = op[hh], pa = pv & 0x7FFF7FFFu;
          float* c = cs[2 * q + hh];
          if (i == 0) {
            c[0] = dot2_first<DT>(pv, ONES);
            c[1] = dot2_first<DT>(pv, sr);
            c[2] = dot2_first<DT>(pv, pv);
            c[3] = dot2_first<DT>(pa, ONES);
          } else {
            c[0] = dot2<DT>(pv, ONES, c[0]);
            c[1] = dot2<DT>(pv, sr, c[1]);
            c[2] = dot2<DT>(pv, pv, c[2]);
            c[3] = dot2<DT>(pa, ONES, c[3]);
          }
        }
      }
    }
    // the four row groups of the wave (lanes cg, cg + 16, cg + 32, cg + 48) add their column sums by lane swaps:
    // permlane32_swap pairs lanes q and q + 2, permlane16_swap then q and q + 1; value i = 4 e + s of lane (q, cg)
    // ends as the wave's sum of value i + 8 q, so lane (q, cg) holds the four sums of columns 8 cg + 2 q (u[0 .. 3])
    // and 8 cg + 2 q + 1 (u[4 .. 7]).  Into LDS by lane (consecutive 16-byte slots); the reader adds the four waves.
    {
      float t1[16], u[8];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(cs[j / 4][j % 4]),
                                                        __float_as_uint(cs[(j + 16) / 4][j % 4]), false, false);
        t1[j] = __uint_as_float(p[0]) + __uint_as_float(p[1]);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(t1[j]), __float_as_uint(t1[j + 8]), false,
                                                        false);
        u[j] = __uint_as_float(p[0]) + __uint_as_float(p[1]);
      }
      colw[w][0][lane] = f32x4{u[0], u[1], u[2], u[3]};
      colw[w][1][lane] = f32x4{u[4], u[5], u[6], u[7]};
    }
    // ---- row direction: four sums of each of the eight rows over this thread's eight columns (32 values a lane,
    //      value 4 i + kind), added over the 16 lanes of the row group by a reduce-scatter: at each of four DPP
    //      steps a lane and its partner (lane xor 8, 7, 3, 1: the same values held, one bit of the lane apart) keep
    //      opposite halves, each adding the partner's copy of its half.  Lane cg ends with values 2 cg, 2 cg + 1:
    //      row cg / 2, kinds 2 (cg & 1) and 2 (cg & 1) + 1, stored as one pair.
    float rv[32];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t ww[4] = {v[tt][i].x, v[tt][i].y, v[tt][i].z, v[tt][i].w};
      float pl = dot2_first<DT>(ww[0], ONES), sg = dot2_first<DT>(ww[0], scol2[tt][0]);
      float sq = dot2_first<DT>(ww[0], ww[0]), ab = dot2_first<DT>(ww[0] & 0x7FFF7FFFu, ONES);
#pragma unroll
      for (int q = 1; q < 4; ++q) {
        pl = dot2<DT>(ww[q], ONES, pl);
        sg = dot2<DT>(ww[q], scol2[tt][q], sg);
        sq = dot2<DT>(ww[q], ww[q], sq);
        ab = dot2<DT>(ww[q] & 0x7FFF7FFFu, ONES, ab);
      }
      rv[4 * i] = pl; rv[4 * i + 1] = sg; rv[4 * i + 2] = sq; rv[4 * i + 3] = ab;
    }
    row_scatter<0x128, 32>(rv, (cg & 8) == 0);        // row_ror:8 (lane xor 8)
    row_scatter<0x141, 16>(rv, (cg & 4) == 0);        // row_half_mirror (lane xor 7)
    row_scatter<0x1B, 8>(rv, (cg & 2) == 0);          // quad_perm [3, 2, 1, 0] (lane xor 3)
    row_scatter<0xB1, 4>(rv, (cg & 1) == 0);          // quad_perm [1, 0, 3, 2] (lane xor 1)
    *reinterpret_cast<float2*>(reinterpret_cast<float*>(&rows[8 * rg + (cg >> 1)]) + 2 * (cg & 1)) =
        float2{rv[0], rv[1]};
    __syncthreads();

    // ---- scoring
    float e0 = ev[tt][0][0], e1 = ev[tt][0][1];
#pragma unroll
    for (int sp = 1; sp < NS; ++sp)
      if (sp < (colside ? a.scol : a.srow)) {
        e0 += ev[tt][sp][0];
        e1 += ev[tt][sp][1];
      }
    if (colside) {
      // column-block check of row R, block jb (serving flavour)
      const int rr = 64 * w + lane;
      if (rr < wr) {
        const f32x4 s4 = rows[rr];
        const f32x4 q0 = a.consts[3 * jb], q1 = a.consts[3 * jb + 1], q2 = a.consts[3 * jb + 2];
        bool ok;
        PairScore ps = judge_serve_clean(s4.x, s4.y, s4.z, s4.w, fsqrt(xsq), xsum, e0, e1, q0.x, q0.y, q0.z, q0.w,
                                         q2.x, q2.y, q1.x, q1.y, q1.z, q1.w, (float)wc, a, ok);
        if (!ok)                                 // (non-finite inputs or an "impossible" pair: the full rules)
          ps = judge_serve(s4.x, s4.y, s4.z, s4.w, fsqrt(xsq), xsum, e0, e1, q0.x, q0.y, q0.z, q0.w, q2.x, q2.y,
                           q1.x, q1.y, q1.z, q1.w, (float)wc, a);
        const int64_t p = (int64_t)R * a.nb + jb;
        if (a.zcol) {
          a.zcol[2 * p] = ps.z0;
          a.zcol[2 * p + 1] = ps.z1;
        }
        keep_best(best, ps.zc, ps.sec, ps.dc, p);
        best.unk += ps.unk;
      }
    } else {
      // row-block check of column J, row block ib (training flavour, y^T = W x^T + b)
      const int cc = 64 * (w - 2) + lane, J = c0 + cc;
      if (cc < wc) {
        // column cc = 8 cg + 2 q + parity sits at lane 16 q + cg of every wave's slot
        const int cl = 16 * ((cc & 7) >> 1) + (cc >> 3), par = cc & 1;
        float pl = 0.f, sg = 0.f, sq = 0.f, ab = 0.f;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 q = colw[g][par][cl];
          pl += q.x; sg += q.y; sq += q.z; ab += q.w;
        }
        const float wf = (float)wr, asum = wsum[tt], bj = bjv[tt];
        float bound = asum * rstat[4];
        if (a.bias) {
          // a bias constant along the block: w copies of b_j, whose sums w b_j and (sum of signs) b_j are exact
          e0 = e0 + bj * wf;
          e1 = e1 + bj * rsign;
          bound = bound + nan_abs(bj);
        }
        const float cn = fsqrt(sq), noise = cn * a.u, xn = fsqrt(wsq[tt]);
        const float inf = __builtin_inff();
        const float nrm[2] = {fsqrt(rstat[0]), fsqrt(rstat[1])};
        float fl[2];
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const float f_l2 = (xn * nrm[c]) * 1e-5f;
          const float f_l1 = (asum * rstat[2 + c]) * a.l1c;
          const float f = fminf(fabsf(f_l2) < inf ? f_l2 : inf, fabsf(f_l1) < inf ? f_l1 : inf);
          fl[c] = f < inf ? f : bound * (float)(1e-5 * 128.0);
        }
        float d0, d1;
        bool ok0, ok1;
        float z0 = judge_one_clean(e0, pl, noise, cn, fl[0], bound, wf, ab, true, a, d0, ok0);
        float z1 = judge_one_clean(e1, sg, noise, cn, fl[1], bound, wf, ab, false, a, d1, ok1);
        if (!(ok0 && ok1)) {                     // (non-finite inputs or an "impossible" checksum: the full rules)
          z0 = judge_one(e0, pl, noise, cn, fl[0], bound, wf, ab, true, a, d0);
          z1 = judge_one(e1, sg, noise, cn, fl[1], bound, wf, ab, false, a, d1);
        }
        const int64_t p = (int64_t)J * a.mb + ib;
        if (a.zrow) {
          a.zrow[2 * p] = z0;
          a.zrow[2 * p + 1] = z1;
        }
        best.unk += (z0 < 0.f) + (z1 < 0.f);
        const bool sec = z1 > z0;
        keep_best(best, sec ? z1 : z0, sec, sec ? d1 : d0, p);
      }
    }
  }
  // (every lane of the wave active here: the reductions by DPP moves, no LDS round trips)
  const int64_t key = wave_max_i64_dpp(best.key), keyd = wave_max_i64_dpp(best.keyd);
  const int unk = wave_sum_i32_dpp(best.unk);
  if (lane == 0) {
    red_k[w] = key;
    red_d[w] = keyd;
    red_u[w] = unk;
  }
  __syncthreads();
  if (t == 0 || t == 64) {
    // thread 0: the column check (waves 0, 1); thread 64: the row check (waves 2, 3)
    const int w0 = t == 0 ? 0 : 2;
    const int64_t k0 = red_k[w0] > red_k[w0 + 1] ? red_k[w0] : red_k[w0 + 1];
    const int64_t d0 = red_d[w0] > red_d[w0 + 1] ? red_d[w0] : red_d[w0 + 1];
    const int un = red_u[w0] + red_u[w0 + 1];
    int64_t* res = t == 0 ? a.state : a.result;
    if (k0 > seen0) atomicMax((unsigned long long*)res, (unsigned long long)k0);
    if (d0 > seen1) atomicMax((unsigned long long*)(res + 1), (unsigned long long)d0);
    if (t == 0) {
      if (blockIdx.x == 0 && blockIdx.y == 0) atomicAdd((unsigned long long*)(res + 2), 1ull);
      if (un > 0) atomicAdd((unsigned long long*)(res + 3), (unsigned long long)un);
    } else if (un > 0) {
      atomicAdd((unsigned long long*)(res + 2), (unsigned long long)un);
    }
  }
}

struct Layout {
  int64_t nb, mb, rem_n, rem_m, nkc, kp, scol, srow;
  bool rs_col, rs_row, tall_col, tall_row;
  int64_t off_parts, off_stats, off_xnp, off_xn, off_rstat, off_erow, off_ecol, off_fcol, total;   // in floats
};

Layout layout(int64_t m, int64_t k, int64_t n) {
  Layout L{};
  L.nb = sdc_cdiv(n, BS);
  L.mb = sdc_cdiv(m, BS);
  L.rem_n = n % BS;
  L.rem_m = m % BS;
  L.nkc = sdc_cdiv(k, XK);
  L.kp = (k + 7) / 8 * 8;
  // one plane from the register-streamed GEMM where the depth allows it and its tiles fill the GPU (64 of them
  // at least), else depth splits of the staged GEMM
  L.rs_col = k % RS_K == 0 && sdc_cdiv(m, 64) * sdc_cdiv(2 * L.nb, 64) >= 64;
  L.rs_row = k % RS_K == 0 && sdc_cdiv(n, 64) * sdc_cdiv(2 * L.mb, 64) >= 64;
  // the tall-tile variant (128-row tiles over depth halves, two planes) where its workgroups still fill the GPU
  L.tall_col = L.rs_col && k % (2 * RS_K) == 0 && 2 * sdc_cdiv(m, 128) * sdc_cdiv(2 * L.nb, 64) >= 192;
  L.tall_row = L.rs_row && k % (2 * RS_K) == 0 && 2 * sdc_cdiv(n, 128) * sdc_cdiv(2 * L.mb, 64) >= 192;
  L.scol = L.rs_col ? (L.tall_col ? 2 : 1) : sdc_expected_splits(m, k, 2 * L.nb);
  L.srow = L.rs_row ? (L.tall_row ? 2 : 1) : sdc_expected_splits(n, k, 2 * L.mb);
  auto al = [](int64_t x) { return (x + 63) / 64 * 64; };
  int64_t o = 0;
  // x's block-sum parts: [3][2 mb][kp], or (register-streamed row GEMM) fragment order, whichever is larger
  L.off_parts = o;
  o += al(std::max((3 * 2 * L.mb * L.kp + 1) / 2, L.rs_row ? sdc_parts_fragments_bytes(2 * L.mb, k) / 4 : 0));
  L.off_stats = o; o += al(L.nkc * L.mb * NXS);
  L.off_xnp = o; o += al(L.nkc * 2 * m);
  L.off_xn = o; o += al(2 * m);
  L.off_rstat = o; o += al(L.mb * RST);
  L.off_erow = o; o += al(L.srow * 2 * L.mb * n);
  L.off_ecol = o; o += al(L.scol * 2 * L.nb * m);
  // (the layer's parts in fragment order, made here when the caller passes none)
  L.off_fcol = o; o += L.rs_col ? al(sdc_parts_fragments_bytes(2 * L.nb, k) / 4) : 0;
  L.total = o;
  return L;
}

int queue_both(const void* x, int64_t sxm, const void* W, int64_t swn, const void* y, int64_t sym, const void* bias,
               int64_t m, int64_t k, int64_t n, const void* parts, int64_t spc, const void* parts_frag,
               const float* block_consts, const float* w_norms, const float* sign_table, int64_t* state,
               int64_t* row_result, float z, float abs_floor, float* ws, float* col_scores, float* row_scores,
               const Layout& L, hipStream_t stream, hipStream_t side);

}  // namespace

extern "C" int64_t sdc_linear_check_workspace(int64_t m, int64_t k, int64_t n) {
  if (m <= 0 || k <= 0 || n <= 0) return 0;
  return layout(m, k, n).total * (int64_t)sizeof(float) + 256;
}

extern "C" int sdc_linear_check(int dtype, const void* x, int64_t sxm, const void* W, int64_t swn, const void* y,
                                int64_t sym, const void* bias, int64_t m, int64_t k, int64_t n, const void* parts,
                                int64_t spc, const void* parts_frag, const float* block_consts, const float* w_norms, const float* sign_table,
                                int64_t* state, int64_t* row_result, float z, float abs_floor, void* workspace,
                                int64_t workspace_bytes, float* col_scores, float* row_scores, int flags,
                                hipStream_t stream) {
  SDC_CLEAR_ERRORS();
  if (m < 1 || n < 1 || k < 1) return SDC_EINVAL;
  if (dtype != SDC_BF16) return SDC_EUNSUPPORTED;               // (fp16: the separate checks)
  if (!x || !W || !y || !parts || !block_consts || !w_norms || !sign_table || !state || !row_result)
    return SDC_EINVAL;
  if (n % 8 || sym % 8 || sxm % 8 || ((uintptr_t)y | (uintptr_t)x | (uintptr_t)block_consts) % 16)
    return SDC_EUNSUPPORTED;                                    // x and y are read in 16-byte pieces
  const Layout L = layout(m, k, n);
  if (m * L.nb * 2 > 0xFFFFFFFFll || n * L.mb * 2 > 0xFFFFFFFFll) return SDC_EUNSUPPORTED;
  if (!workspace || workspace_bytes < L.total * (int64_t)sizeof(float) + 256) return SDC_EWORKSPACE;
  float* ws = (float*)(((uintptr_t)workspace + 255) & ~(uintptr_t)255);
  hipStream_t side = stream;
  if ((flags & 1) && !(side = sdc_fork(stream))) return SDC_ELAUNCH;
  const int rc = queue_both(x, sxm, W, swn, y, sym, bias, m, k, n, parts, spc, parts_frag, block_consts, w_norms,
                            sign_table, state, row_result, z, abs_floor, ws, col_scores, row_scores, L, stream, side);
  // a call that fails after the fork still makes the caller's stream wait for the side stream, so nothing queued
  // there can be reading the workspace when the caller reuses it
  if (rc != SDC_OK && side != stream) sdc_join(stream, side);
  return rc;
}

namespace {

// The five launches of sdc_linear_check.  side: the stream of the column check's GEMM and of xfinish (the
// caller's stream itself for the one-stream variant, in which every kernel runs on the caller's stream).
int queue_both(const void* x, int64_t sxm, const void* W, int64_t swn, const void* y, int64_t sym, const void* bias,
               int64_t m, int64_t k, int64_t n, const void* parts, int64_t spc, const void* parts_frag,
               const float* block_consts, const float* w_norms, const float* sign_table, int64_t* state,
               int64_t* row_result, float z, float abs_floor, float* ws, float* col_scores, float* row_scores,
               const Layout& L, hipStream_t stream, hipStream_t side) {
  const float* s_full = sign_table + (BS - 1) * 128;

  // 3. (side stream when asked) the column check's GEMM: E_col = x @ B2 parts (x's row norms come from xstage)
  GemmArgs gc{};
  gc.A = (const uint16_t*)x; gc.sab = 0; gc.sam = sxm; gc.sak = 1;
  gc.B = parts; gc.sbb = 0; gc.sbc = spc;
  gc.m = m; gc.k = k; gc.N = 2 * L.nb; gc.splits = L.scol;
  gc.E = ws + L.off_ecol; gc.XN = nullptr; gc.et = 1;
  gc.prof_name = "col_gemm";
  int rc = SDC_EUNSUPPORTED;
  if (L.rs_col && (parts_frag ||
                   sdc_parts_fragments(parts, spc, 2 * L.nb, k, ws + L.off_fcol, side) == SDC_OK)) {
    GemmArgs gf = gc;
    gf.B = parts_frag ? parts_frag : ws + L.off_fcol;
    rc = L.tall_col ? sdc_rs_gemm_tall_launch(SDC_BF16, gf, 0, side) : sdc_rs_gemm_launch(SDC_BF16, gf, 0, side);
  }
  if (rc == SDC_EUNSUPPORTED) rc = sdc_gemm_launch(SDC_BF16, gc, 1, side);   // (alignment: the staged GEMM)
  if (rc != SDC_OK) return rc;

  // 1. the block sums of x (as three parts, in fragment order when the row GEMM is the register-streamed one), their
  //    statistics and x's row norms
  const bool rs_row = L.rs_row && swn % 8 == 0 && (uintptr_t)W % 16 == 0;
  XStageArgs xa{};
  xa.frag = rs_row ? 1 : 0;
  xa.ncf = sdc_cdiv(2 * L.mb, 32);
  xa.x = (const uint16_t*)x; xa.sxm = sxm; xa.m = m; xa.k = k; xa.kp = L.kp; xa.mb = L.mb; xa.rem = L.rem_m;
  xa.nkc = L.nkc;
  xa.s_full = s_full; xa.s_last = L.rem_m ? sign_table + (L.rem_m - 1) * 128 : s_full;
  xa.parts = (uint16_t*)(ws + L.off_parts); xa.stats = ws + L.off_stats; xa.xnp = ws + L.off_xnp;
  xa.xn = ws + L.off_xn; xa.rstat = ws + L.off_rstat;
  {
    SdcProf prof("xstage", stream);
    hipLaunchKernelGGL(xstage_kernel, dim3((unsigned)L.nkc, (unsigned)L.mb), dim3(256), 0, stream, xa);
    SDC_LAUNCH_CHECK();
  }
  // 2, 3. the row check's GEMM: E_row = W @ (x block sums), each XCD taking every depth slice of its rows (W's row
  //    norms are the layer's, made once); the tall-tile GEMM runs xfinish in spare workgroups of its grid (one per
  //    row block), else xfinish is a launch of its own (on the side stream when there is one)
  GemmArgs gr{};
  gr.A = (const uint16_t*)W; gr.sab = 0; gr.sam = swn; gr.sak = 1;
  gr.B = ws + L.off_parts; gr.sbb = 0; gr.sbc = L.kp;
  gr.m = n; gr.k = k; gr.N = 2 * L.mb; gr.splits = L.srow;
  gr.E = ws + L.off_erow; gr.XN = nullptr; gr.et = 1; gr.rows_per_xcd = 1;
  gr.prof_name = "row_gemm";
  rc = SDC_EUNSUPPORTED;
  bool finished = false;
  if (rs_row && L.tall_row && side == stream) {
    GemmArgs gx = gr;
    gx.xf = xa;
    gx.xf_blocks = (int)L.mb;
    rc = sdc_rs_gemm_tall_launch(SDC_BF16, gx, 1, stream);
    finished = rc == SDC_OK;
  }
  hipStream_t fin = stream;
  if (!finished) {
    if (side != stream && !(fin = sdc_fork(stream))) return SDC_ELAUNCH;
    SdcProf prof("xfinish", fin);
    hipLaunchKernelGGL(xfinish_kernel, dim3((unsigned)L.mb), dim3(256), 0, fin, xa);
    SDC_LAUNCH_CHECK();
  }
  if (rc == SDC_EUNSUPPORTED) {
    if (!rs_row) rc = sdc_gemm_launch(SDC_BF16, gr, 1, stream);     // (W not 16-byte aligned: the staged GEMM)
    else if (L.tall_row) rc = sdc_rs_gemm_tall_launch(SDC_BF16, gr, 1, stream);
    else rc = sdc_rs_gemm_launch(SDC_BF16, gr, 1, stream);
  }
  if (rc != SDC_OK) return rc;
  if (side != stream && (rc = sdc_join(stream, side)) != SDC_OK) return rc;   // (the column GEMM, and xfinish)

  // 4. one pass over y: both checks
  YArgs ya{};
  ya.y = (const uint16_t*)y; ya.sym = sym; ya.m = m; ya.n = n; ya.k = k; ya.nb = L.nb; ya.mb = L.mb;
  ya.rem_n = L.rem_n; ya.rem_m = L.rem_m; ya.sign_table = sign_table;
  ya.Ecol = ws + L.off_ecol; ya.xn = ws + L.off_xn; ya.scol = L.scol; ya.consts = (const f32x4*)block_consts;
  ya.state = state; ya.zcol = col_scores;
  ya.Erow = ws + L.off_erow; ya.wn = w_norms; ya.srow = gr.splits; ya.rstat = ws + L.off_rstat;
  ya.bias = (const uint16_t*)bias; ya.result = row_result; ya.zrow = row_scores;
  ya.u = 1.f / 256.f; ya.h = 0.f; ya.abs_floor = abs_floor;
  ya.l1c = (float)(k * 7.450580596923828e-09 > 1e-5 ? k * 7.450580596923828e-09 : 1e-5);   // checksum.py:95-104
  ya.zt = z; ya.lim_a = 1e18f; ya.lim_big = 1e18f;
  ya.capk = (float)(1.02 + (double)k * 2.384185791015625e-07);
  SdcProf prof("ypass", stream);
  const int64_t ns = std::max(L.scol, gr.splits);
  const dim3 yg((unsigned)sdc_cdiv(L.nb, YTPW), (unsigned)L.mb);
  if (ns == 1) hipLaunchKernelGGL((ypass_kernel<SDC_BF16, 1, YTPW>), yg, dim3(256), 0, stream, ya);
  else if (ns == 2) hipLaunchKernelGGL((ypass_kernel<SDC_BF16, 2, YTPW>), yg, dim3(256), 0, stream, ya);
  else hipLaunchKernelGGL((ypass_kernel<SDC_BF16, SDC_MAX_SPLITS, YTPW>), yg, dim3(256), 0, stream, ya);
  SDC_LAUNCH_CHECK();
  return SDC_OK;
}

}  // namespace
