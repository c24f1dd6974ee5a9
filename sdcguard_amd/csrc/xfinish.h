// The x pass's statistics of sdc_linear_check (linear_check.hip) and their finishing step, which the row check's
// GEMM (expected_gemm.hip) can run in workgroups that would otherwise be idle.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

constexpr int NXS = 5;             // partial stats per (depth chunk, row block): sq0, sq1, max0, max1, max|x|
constexpr int RST = 8;             // final stats per row block: the NXS above, then the sum of its sign pattern
constexpr int XF_BS = 128;         // rows per row block

struct XStageArgs {
  const uint16_t* x;
  int64_t sxm, m, k, kp, mb, rem, nkc;
  int frag;                        // parts in the register-streamed GEMM's fragment order (else [3][2 mb][kp])
  int64_t ncf;                     // (fragment order) 32-column fragments of the 2 mb checksum columns
  const float* s_full;             // sign pattern of a full row block (128), and of the last (rem) one
  const float* s_last;
  uint16_t* parts;                 // [3][2 mb][kp] bf16: hi, mid, lo of (plain, signed) per row block
  float* stats;                    // [nkc][mb][NXS] partial statistics of the sums, per depth chunk
  float* xnp;                      // [nkc][2][m] partial |x_i|_2^2, |x_i|_1 per depth chunk
  float* xn;                       // [2][m] |x_i|_2^2, |x_i|_1 (the column check's A norms)
  float* rstat;                    // [mb][RST]: sq0, sq1, max0, max1, max |x|, sum of the block's pattern
};

// The depth chunks' partials of one row block added up in chunk order (so the result is the same on every run):
// the rows' |x|_2^2 and |x|_1 (thread t: row t / 2, t % 2 the statistic), the block sums' statistics (wave 1), the
// sum of the block's sign pattern (wave 2).  Each thread has XF_BATCH chunks' loads in flight at once (its time is
// the loads' latency, not their bytes).
// 256 threads; no barrier, no LDS (so idle workgroups of another kernel can run it).
constexpr int XF_BATCH = 32;
__device__ __forceinline__ void xfinish_block(const XStageArgs& a, int64_t ib, int t) {
  const int lane = t & 63, w = t >> 6;
  const int wid = (int)((ib == a.mb - 1 && a.rem > 0) ? a.rem : XF_BS);
  const float* sp = (ib == a.mb - 1 && a.rem > 0) ? a.s_last : a.s_full;
  {
    const int r = t >> 1, c = t & 1;
    const int64_t row = ib * XF_BS + (r < wid ? r : 0);
    float acc = 0.f;
    for (int64_t q0 = 0; q0 < a.nkc; q0 += XF_BATCH) {
      float p[XF_BATCH];
#pragma unroll
      for (int j = 0; j < XF_BATCH; ++j) p[j] = a.xnp[((q0 + j < a.nkc ? q0 + j : a.nkc - 1) * 2 + c) * a.m + row];
#pragma unroll
      for (int j = 0; j < XF_BATCH; ++j)
        if (q0 + j < a.nkc) acc += p[j];
    }
    if (r < wid) a.xn[c * a.m + row] = acc;
  }
  if (w == 1) {
    const int i = lane < NXS ? lane : 0;
    float v = 0.f;
    for (int64_t q0 = 0; q0 < a.nkc; q0 += XF_BATCH) {
      float p[XF_BATCH];
#pragma unroll
      for (int j = 0; j < XF_BATCH; ++j)
        p[j] = a.stats[((q0 + j < a.nkc ? q0 + j : a.nkc - 1) * a.mb + ib) * NXS + i];
#pragma unroll
      for (int j = 0; j < XF_BATCH; ++j)
        if (q0 + j < a.nkc) v = i < 2 ? v + p[j] : fmaxf(v, p[j]);
    }
    if (lane < NXS) a.rstat[ib * RST + lane] = v;
  } else if (w == 2) {
    const float ss = wave_sum_f32((lane < wid ? sp[lane] : 0.f) + (lane + 64 < wid ? sp[lane + 64] : 0.f));
    if (lane == 0) a.rstat[ib * RST + NXS] = ss;
  }
}
