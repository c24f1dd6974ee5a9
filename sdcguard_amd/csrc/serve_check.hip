// Serving check of one linear layer (the sdcguard::check_static op): y = x @ W^T (+ b), W's block sums known.
//
// Reference: serve.py:301-396 (`_check_static_impl`, the arithmetic and the state row), _serve_fast.py:102-262
// (`_check`), :334-452 (`_judge`, `_report`: scoring order, Inf/NaN rules, unjudged counts, the capture of an
// alarming row), :454-526 (`_sums`, `_score`).  Two launches:
//   1. expected_gemm (expected_gemm.hip): E = x @ parts on MFMA, plus |x_row|_2^2 and |x_row|_1;
//   2. serve_score (here): one pass over y.  A wave owns 64 (row, block) pairs; four lanes share a pair (each
//      reads 4 x 16 bytes of the 256-byte block, in runs of 64 bytes), accumulate its four sums (plain, signed,
//      of squares, of |values|) and add them up with two DPP steps; over four rounds each lane keeps one pair's
//      sums, then scores it with the reference's noise model.  The workgroup's worst key goes into the layer's
//      state row with one integer atomic maximum (only when it raises the row), counts with atomic adds.
#include "blocksums.h"
#include "judge.h"
#include "gemm.h"
#include "profile.h"
#include "streams.h"

int sdc_expected_launch(int dtype, const void* x, int64_t sxm, int64_t sxk, const void* parts, int64_t spk,
                        int64_t spc, int nparts, int64_t m, int64_t k, int64_t ncols, int64_t splits, float* E,
                        float* XN, hipStream_t stream);
extern "C" int64_t sdc_expected_splits(int64_t m, int64_t k, int64_t ncols);

namespace {

struct ScoreArgs {
  YView yv;
  const uint16_t* x; int64_t sxm, sxk;
  const uint16_t* y; int64_t sym, syn;
  int64_t m, k, n, nb, bs, rem, npairs;
  const float* E; int64_t ncols; int64_t splits;
  const float* XN;
  const float* s_full; const float* s_last;       // sign patterns of widths bs and rem (rows of the table)
  const float* scale; const float* b2n; const float* b2max; const float* bmax; const float* bmb; const float* bsum;
  int64_t* state; int counts;
  float u, h, abs_floor, l1c, zt, lim_a, lim_big, capk;
  int64_t* capm; float* capd; int64_t cst, cw, ctag, cfo, ncap, slot;
  int vec;
  float* zdump;      // optional: every checksum's score, (m, nb, 2) fp32 (tests)
  const f32x4* packed;   // optional: the per-block constants as 3 float4 per block (see sdc_check_static)
};

// Scores this lane's pairs (NP of them: p0, p0 + 256, ...; those >= npairs are skipped) from their four sums, then
// the workgroup's worst key into the layer's state row (one atomic maximum, only when it raises the row), the
// counts, and the capture of a row over the line (_serve_fast.py:404-452).  Every thread of the workgroup calls it.
struct LaneBest {
  int64_t key = 0, keyd = 0;
  int unk = 0;
};

// Pair p's expected sums and x row norms over the GEMM's NS depth-split planes (NS at most SDC_MAX_SPLITS), all
// loads issued before any is used and unconditional: a split index past a.splits reads split 0 (added nowhere), a
// pair past the last reads the last pair's (scored nowhere).
template <int NS>
struct PairE {
  float2 ev[NS];
  float xa[NS], xb[NS];
};

template <int NS>
__device__ __forceinline__ PairE<NS> load_pair_e(const ScoreArgs& a, int64_t p) {
  const int64_t pc = p < a.npairs ? p : a.npairs - 1;
  const int64_t r = (uint32_t)pc / (uint32_t)a.nb, jb = (uint32_t)pc - (uint32_t)r * (uint32_t)a.nb;
  const float* ep = a.E + r * a.ncols + 2 * jb;
  const float* xp = a.XN + r;
  const int64_t estep = a.m * a.ncols, xstep = 2 * a.m;
  PairE<NS> e;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int64_t sc = s < a.splits ? s : 0;
    e.ev[s] = *reinterpret_cast<const float2*>(ep + sc * estep);
    e.xa[s] = xp[sc * xstep];
    e.xb[s] = xp[sc * xstep + a.m];
  }
  return e;
}

// Scores pair p (skipped when p >= npairs) from its four sums and its loaded planes into the lane's running worst.
template <int DT, int NS>
__device__ __forceinline__ void score_pair_e(const ScoreArgs& a, int64_t p, float pl, float sg, float sq, float ab,
                                             const PairE<NS>& pe, LaneBest& best) {
  if (p >= a.npairs) return;
  const int64_t r = (uint32_t)p / (uint32_t)a.nb, jb = (uint32_t)p - (uint32_t)r * (uint32_t)a.nb;
  const bool last = (jb == a.nb - 1) && (a.rem > 0);
  const float wf = (float)(last ? a.rem : a.bs);
  // the planes added in split order
  float e0 = pe.ev[0].x, e1 = pe.ev[0].y, asq = pe.xa[0], asum = pe.xb[0];
#pragma unroll
  for (int s = 1; s < NS; ++s) {
    if (s < a.splits) {
      e0 += pe.ev[s].x;
      e1 += pe.ev[s].y;
      asq += pe.xa[s];
      asum += pe.xb[s];
    }
  }
  PairScore ps;
  if (a.packed) {
    const f32x4 c0 = a.packed[3 * jb], c1 = a.packed[3 * jb + 1], c2 = a.packed[3 * jb + 2];
    bool ok;
    ps = judge_serve_clean(pl, sg, sq, ab, fsqrt(asq), asum, e0, e1, c0.x, c0.y, c0.z, c0.w, c2.x, c2.y, c1.x, c1.y,
                           c1.z, c1.w, wf, a, ok);
    if (!ok)                                   // (non-finite inputs or an "impossible" pair: the full rules)
      ps = judge_serve(pl, sg, sq, ab, fsqrt(asq), asum, e0, e1, c0.x, c0.y, c0.z, c0.w, c2.x, c2.y, c1.x, c1.y,
                       c1.z, c1.w, wf, a);
  } else {
    ps = judge_serve(pl, sg, sq, ab, fsqrt(asq), asum, e0, e1, a.scale[2 * jb], a.scale[2 * jb + 1],
                     a.bsum[2 * jb], a.bsum[2 * jb + 1], a.bmax[jb], a.bmb[jb], a.b2n[2 * jb], a.b2n[2 * jb + 1],
                     a.b2max[2 * jb], a.b2max[2 * jb + 1], wf, a);
  }
  if (a.zdump) {
    a.zdump[2 * p] = ps.z0;
    a.zdump[2 * p + 1] = ps.z1;
  }
  const int64_t zb = fbits64(fmaxf(ps.zc, 0.f));
  const int64_t flat = p * 2 + (ps.sec ? 1 : 0);
  const int64_t k1 = (zb << 32) | (flat & 0xFFFFFFFFll);
  const int64_t d1 = (zb << 32) | (fbits64(ps.dc) & 0xFFFFFFFFll);
  best.key = k1 > best.key ? k1 : best.key;
  best.keyd = d1 > best.keyd ? d1 : best.keyd;
  best.unk += ps.unk;
}

// The same with the planes loaded here.
template <int DT>
__device__ __forceinline__ void score_pair(const ScoreArgs& a, int64_t p, float pl, float sg, float sq, float ab,
                                           LaneBest& best) {
  if (p >= a.npairs) return;
  score_pair_e<DT, SDC_MAX_SPLITS>(a, p, pl, sg, sq, ab, load_pair_e<SDC_MAX_SPLITS>(a, p), best);
}

// The workgroup's worst key into the layer's state row (one atomic maximum, only when it raises the row), the
// counts, and the capture of a row over the line (_serve_fast.py:404-452).  Every thread of the workgroup calls it.
template <int DT>
__device__ __forceinline__ void report_wg(const ScoreArgs& a, LaneBest best) {
  __shared__ int64_t red_k[4], red_d[4];
  __shared__ int red_u[4];
  __shared__ int64_t cap_slot;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  int64_t key = wave_max_i64_dpp(best.key);        // (every lane of the wave calls this: DPP reductions)
  int64_t keyd = wave_max_i64_dpp(best.keyd);
  int unk = wave_sum_i32_dpp(best.unk);
  if (lane == 0) { red_k[w] = key; red_d[w] = keyd; red_u[w] = unk; }
  __syncthreads();
  int64_t* st = a.state;
  if (t == 0) {
    int64_t k0 = red_k[0], d0 = red_d[0];
    int un = red_u[0];
    for (int i = 1; i < 4; ++i) {
      k0 = red_k[i] > k0 ? red_k[i] : k0;
      d0 = red_d[i] > d0 ? red_d[i] : d0;
      un += red_u[i];
    }
    red_k[0] = k0;
    // most workgroups cannot raise the layer's worst score: read first, take the atomic only when it can
    const int64_t s0 = __atomic_load_n(st, __ATOMIC_RELAXED), s1 = __atomic_load_n(st + 1, __ATOMIC_RELAXED);
    if (k0 > s0) atomicMax((unsigned long long*)st, (unsigned long long)k0);
    if (d0 > s1) atomicMax((unsigned long long*)(st + 1), (unsigned long long)d0);
    if (a.counts) {
      if (blockIdx.x == 0) atomicAdd((unsigned long long*)(st + 2), 1ull);
      if (un > 0) atomicAdd((unsigned long long*)(st + 3), (unsigned long long)un);
    }
    cap_slot = -1;
    if (a.capm) {
      const int64_t zbits = k0 >> 32;
      const float bz = __uint_as_float((uint32_t)zbits);
      if (bz > a.zt) {
        unsigned long long taken = atomicExch((unsigned long long*)(a.capm + a.cfo + a.slot), 1ull);
        if (taken == 0) {
          int64_t c = (int64_t)atomicAdd((unsigned long long*)a.capm, 1ull);
          if (c < a.ncap) {
            const int64_t best_i = k0 & 0xFFFFFFFFll;
            const int64_t bi = best_i / 2, crow = bi / a.nb, cblk = bi % a.nb;
            int64_t* rec = a.capm + 2 + c * 6;
            rec[0] = a.ctag; rec[1] = crow; rec[2] = cblk; rec[3] = best_i; rec[4] = zbits;
            rec[5] = __atomic_load_n(a.capm + 1, __ATOMIC_RELAXED);
            cap_slot = c;
          }
        }
      }
    }
  }
  __syncthreads();
  if (a.capm && cap_slot >= 0) {
    const int64_t k0 = red_k[0];
    const int64_t bi = (k0 & 0xFFFFFFFFll) / 2, crow = bi / a.nb, cblk = bi % a.nb;
    const int64_t cwid = (cblk == a.nb - 1 && a.rem > 0) ? a.rem : a.bs;
    float* dst = a.capd + cap_slot * a.cst;
    for (int64_t i = t; i < cwid; i += 256) dst[i] = half_to_f32<DT>(a.y[crow * a.sym + (cblk * a.bs + i) * a.syn]);
    for (int64_t i = t; i < a.k; i += 256) dst[a.cw + i] = half_to_f32<DT>(a.x[crow * a.sxm + i * a.sxk]);
  }
}

// v1 (one launch after the GEMM): sums and scores in the same pass over y.  Each wave walks tiles of 64 pairs
// with a grid stride and keeps its worst key; the workgroup reports once at the end.  A tile's expected sums (NS
// planes: 2 from the tall-tile GEMM) are loaded before its outputs, so both arrive in one round trip.
template <int DT, int NS>
__global__ __launch_bounds__(256) void serve_fused_kernel(ScoreArgs a) {
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, q = lane & 3;
  uint32_t sg2[16];
  lane_signs<DT>(a.yv, q, sg2);
  LaneBest best;
  const int64_t tiles = (a.npairs + 63) / 64;
  for (int64_t tile = (int64_t)blockIdx.x * 4 + w; tile < tiles; tile += (int64_t)gridDim.x * 4) {
    const int64_t base = tile * 64, p = base + q * 16 + (lane >> 2);
    const PairE<NS> pe = load_pair_e<NS>(a, p);
    float pl, sg, sq, ab;
    pair_sums<DT>(a.yv, base, lane, sg2, pl, sg, sq, ab);
    score_pair_e<DT, NS>(a, p, pl, sg, sq, ab, pe, best);
  }
  report_wg<DT>(a, best);
}

// v3, part 1 (concurrent with the GEMM, on a side stream): the four sums of every pair, (4, npairs) fp32.  Each
// wave walks tiles of 64 pairs with a grid stride, so a workgroup's set-up (the sign pairs) is paid once.
template <int DT>
__global__ __launch_bounds__(256) void serve_sums_kernel(ScoreArgs a, float* __restrict__ sums) {
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, q = lane & 3;
  uint32_t sg2[16];
  lane_signs<DT>(a.yv, q, sg2);
  const int64_t tiles = (a.npairs + 63) / 64;
  for (int64_t tile = (int64_t)blockIdx.x * 4 + w; tile < tiles; tile += (int64_t)gridDim.x * 4) {
    const int64_t base = tile * 64;
    float pl, sg, sq, ab;
    pair_sums<DT>(a.yv, base, lane, sg2, pl, sg, sq, ab);
    const int64_t p = base + q * 16 + (lane >> 2);
    if (p < a.npairs) {
      sums[p] = pl;
      sums[a.npairs + p] = sg;
      sums[2 * a.npairs + p] = sq;
      sums[3 * a.npairs + p] = ab;
    }
  }
}

// v3, part 2 (after both): pairs scored with a grid stride, one report per workgroup.
template <int DT>
__global__ __launch_bounds__(256) void serve_pairs_kernel(ScoreArgs a, const float* __restrict__ sums) {
  LaneBest best;
  for (int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x; p < a.npairs; p += (int64_t)gridDim.x * 256)
    score_pair<DT>(a, p, sums[p], sums[a.npairs + p], sums[2 * a.npairs + p], sums[3 * a.npairs + p], best);
  report_wg<DT>(a, best);
}

}  // namespace

extern "C" int64_t sdc_check_static_workspace(int64_t m, int64_t k, int64_t n, int64_t bs) {
  if (m <= 0 || n <= 0 || bs <= 0) return 0;
  const int64_t nb = sdc_cdiv(n, bs), ncols = 2 * nb;
  const int64_t splits = sdc_expected_splits(m, k, ncols);
  // E planes, row-norm planes, then the (4, m * nb) pair sums of the split design
  return (splits * m * ncols + splits * 2 * m + 4 * m * nb) * (int64_t)sizeof(float) + 512;
}

extern "C" int sdc_check_static(int dtype, const void* x, int64_t sxm, int64_t sxk, const void* y, int64_t sym,
                                int64_t syn, int64_t m, int64_t k, int64_t n, int64_t bs, const void* parts,
                                int64_t spk, int64_t spc, int nparts, const float* sign_table, const float* scale,
                                const float* b2n, const float* b2max, const float* bmax, const float* bmax_bias,
                                const float* bsum, int64_t* state, int counts, int64_t slot, float z,
                                float abs_floor, int64_t* cap_meta, float* cap_data, int64_t cap_stride,
                                int64_t cap_w, int64_t cap_tag, int64_t cap_flags, int64_t cap_slots,
                                void* workspace, int64_t workspace_bytes, float* scores_out, int kernel,
                                const float* block_consts, const void* parts_frag, hipStream_t stream) {
  SDC_CLEAR_ERRORS();
  if (m < 0 || n < 0 || k < 0) return SDC_EINVAL;
  if (m == 0 || n == 0) return SDC_OK;                     // nothing to check, not counted (serve.py:435)
  if (dtype != SDC_BF16 && dtype != SDC_FP16) return SDC_EINVAL;
  if (bs < 1 || bs > 128) return SDC_EUNSUPPORTED;         // the sign table holds widths 1..128
  if (k < 1) return SDC_EUNSUPPORTED;
  if (!x || !y || !parts || !sign_table || !scale || !b2n || !b2max || !bmax || !bmax_bias || !bsum || !state)
    return SDC_EINVAL;
  if (m * (sdc_cdiv(n, bs)) * 2 > 0xFFFFFFFFll) return SDC_EUNSUPPORTED;   // flat index in 32 bits
  const int64_t need = sdc_check_static_workspace(m, k, n, bs);
  if (!workspace || workspace_bytes < need) return SDC_EWORKSPACE;
  const int64_t nb = sdc_cdiv(n, bs), rem = n % bs, ncols = 2 * nb;
  const int64_t splits = sdc_expected_splits(m, k, ncols);
  float* E = (float*)(((uintptr_t)workspace + 255) & ~(uintptr_t)255);
  float* XN = E + splits * m * ncols;
  float* SUMS = (float*)(((uintptr_t)(XN + splits * 2 * m) + 255) & ~(uintptr_t)255);
  // (the fused persistent pass measured fastest at every batch size on MI355X; v3 stays available on request)
  const bool split_design = kernel == 3 || kernel == 4;
  const double u = dtype == SDC_BF16 ? 1.0 / 256.0 : 1.0 / 2048.0;
  const double h = dtype == SDC_BF16 ? 0.0 : 1.0 / 33554432.0;             // 2^-25
  const double dmax = dtype == SDC_BF16 ? 3.3895313892515355e38 : 65504.0;
  ScoreArgs a;
  a.x = (const uint16_t*)x; a.sxm = sxm; a.sxk = sxk;
  a.y = (const uint16_t*)y; a.sym = sym; a.syn = syn;
  a.m = m; a.k = k; a.n = n; a.nb = nb; a.bs = bs; a.rem = rem; a.npairs = m * nb;
  a.E = E; a.ncols = ncols; a.splits = splits; a.XN = XN;
  a.s_full = sign_table + (bs - 1) * 128;
  a.s_last = rem ? sign_table + (rem - 1) * 128 : a.s_full;
  a.scale = scale; a.b2n = b2n; a.b2max = b2max; a.bmax = bmax; a.bmb = bmax_bias; a.bsum = bsum;
  a.state = state + 0; a.counts = counts;
  a.u = (float)u; a.h = (float)h; a.abs_floor = abs_floor;
  a.l1c = (float)(k * 7.450580596923828e-09 > 1e-5 ? k * 7.450580596923828e-09 : 1e-5);   // checksum.py:95-104
  a.zt = z; a.lim_a = (float)(dmax < 1e18 ? dmax : 1e18); a.lim_big = 1e18f;
  a.capk = (float)(1.02 + (double)k * 2.384185791015625e-07);
  a.capm = cap_meta; a.capd = cap_data; a.cst = cap_stride; a.cw = cap_w; a.ctag = cap_tag; a.cfo = cap_flags;
  a.ncap = cap_slots; a.slot = slot;
  a.yv.y = a.y; a.yv.sb = 0; a.yv.sm = sym; a.yv.sn = syn; a.yv.m = m; a.yv.nb = nb; a.yv.bs = bs;
  a.yv.rem = rem; a.yv.npairs = m * nb; a.yv.s_full = a.s_full; a.yv.s_last = a.s_last;
  a.zdump = scores_out;
  a.packed = (const f32x4*)block_consts;
  if (block_consts && ((uintptr_t)block_consts % 16)) return SDC_EINVAL;
  a.vec = (syn == 1) && (sym % 8 == 0) && (bs % 8 == 0) && ((uintptr_t)y % 16 == 0);
  a.yv.vec = a.vec;
  if (cap_meta && (!cap_data || cap_w < bs)) return SDC_EINVAL;
  // The expected side: the register-streamed tall-tile GEMM (two depth halves, row-major planes, x's row norms in
  // the same pass) where the parts come in fragment order and the shape suits it, else the staged GEMM
  auto expected = [&]() -> int {
    if (parts_frag && nparts == 3 && spk == 1 && sxk == 1 && splits >= 2 && k % 512 == 0 &&
        2 * sdc_cdiv(m, 128) * sdc_cdiv(ncols, 64) >= 192) {
      GemmArgs g{};
      g.A = (const uint16_t*)x; g.sam = sxm; g.sak = 1;
      g.B = parts_frag; g.m = m; g.k = k; g.N = ncols; g.splits = 2;
      g.E = E; g.XN = XN; g.et = 0;
      g.prof_name = "expected_gemm";
      const int rc = sdc_rs_gemm_tall_launch(dtype, g, 0, stream);
      if (rc != SDC_EUNSUPPORTED) {
        a.splits = 2;
        return rc;
      }
    }
    return sdc_expected_launch(dtype, x, sxm, sxk, parts, spk, spc, nparts, m, k, ncols, splits, E, XN, stream);
  };
  // persistent grids: about four workgroups per CU (256 CUs), fewer for small batches
  const int64_t tiles = sdc_cdiv(m * nb, 64);
  const unsigned grid = (unsigned)(sdc_cdiv(tiles, 4) < 1024 ? sdc_cdiv(tiles, 4) : 1024);
  if (!split_design) {
    int rc = expected();
    if (rc != SDC_OK) return rc;
    SdcProf prof("serve_fused", stream);
    constexpr int MS = SDC_MAX_SPLITS;
    if (dtype == SDC_BF16 && a.splits <= 2)
      hipLaunchKernelGGL((serve_fused_kernel<SDC_BF16, 2>), dim3(grid), dim3(256), 0, stream, a);
    else if (dtype == SDC_BF16)
      hipLaunchKernelGGL((serve_fused_kernel<SDC_BF16, MS>), dim3(grid), dim3(256), 0, stream, a);
    else if (a.splits <= 2)
      hipLaunchKernelGGL((serve_fused_kernel<SDC_FP16, 2>), dim3(grid), dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL((serve_fused_kernel<SDC_FP16, MS>), dim3(grid), dim3(256), 0, stream, a);
    SDC_LAUNCH_CHECK();
    return SDC_OK;
  }
  // the block sums of y need nothing from the GEMM: they stream from HBM on a side stream while the GEMM runs
  // (kernel 4: the same design without the fork, every launch on the caller's stream, for measurements)
  hipStream_t side = stream;                   // (the caller's stream may be the null stream)
  if (kernel != 4 && !(side = sdc_fork(stream))) return SDC_ELAUNCH;
  {
    SdcProf prof("serve_sums", side);
    if (dtype == SDC_BF16)
      hipLaunchKernelGGL(serve_sums_kernel<SDC_BF16>, dim3(grid), dim3(256), 0, side, a, SUMS);
    else
      hipLaunchKernelGGL(serve_sums_kernel<SDC_FP16>, dim3(grid), dim3(256), 0, side, a, SUMS);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
      sdc_note_error(e);
      if (kernel != 4) sdc_join(stream, side);    // (the caller's stream waits for the side stream even so)
      return SDC_ELAUNCH;
    }
  }
  int rc = expected();
  if (kernel != 4) {
    const int jc = sdc_join(stream, side);
    if (rc == SDC_OK) rc = jc;
  }
  if (rc != SDC_OK) return rc;
  SdcProf prof("serve_score", stream);
  const unsigned pgrid = (unsigned)(sdc_cdiv(m * nb, 1024) < 512 ? sdc_cdiv(m * nb, 1024) : 512);
  if (dtype == SDC_BF16)
    hipLaunchKernelGGL(serve_pairs_kernel<SDC_BF16>, dim3(pgrid), dim3(256), 0, stream, a, (const float*)SUMS);
  else
    hipLaunchKernelGGL(serve_pairs_kernel<SDC_FP16>, dim3(pgrid), dim3(256), 0, stream, a, (const float*)SUMS);
  SDC_LAUNCH_CHECK();
  return SDC_OK;
}
