// The check of a serving layer's FP8 input quantization (serve_fp8.py:63-164, `quant_check_torch`): were the FP8
// values the GEMM got, and their scale, made from this step's real rows by the layer's recipe?
//   recipe 0 static:         the scale against its value at load; the sampled rows' values;
//   recipe 1 per-tensor:     max |x| over the step's real rows / 448 against the scale (and, when it differs, whether
//                            the scale is the maximum over every row, padding included); the sampled rows' values;
//   recipe 2 per-token:      each sampled row's own max |x| / 448 (capped by scale_ub, at least 1 / (448 * 512))
//                            against its scale; its values.
// The values: the sampled rows quantized as the layer's kernels do (x / scale per token, x * (1 / scale) otherwise,
// clamped to +-448, rounded to nearest even E4M3) against the codes the GEMM got, in the codes' value order; two or
// more FP8 steps apart is wrong, one step is counted (fast-math kernels).  Results accumulate into the layer's
// 8-column int64 state row (calls, wrong scales, scales from outside rows, rows with wrong values, values one step
// off, last finding, worst scale ratio, static scale changed); nothing is judged while the step's real row count
// on the device is 0.  No host synchronisation; no memory set (graph-safe).
//
// Two launches: fp8q_amax (per-tensor recipe only): per workgroup the largest |x| over the real rows and over every
// row, as IEEE bits (a NaN's bits exceed Inf's, so the maximum of the bits propagates NaN as amax does); and
// fp8q_judge, one workgroup: the two sampled rows, the reductions and the state update.
#include "common.h"
#include "profile.h"

namespace {

constexpr int DT_F32 = 4;                         // an fp32 input (the library's 16-bit codes are 0 and 1)
constexpr float FP8_MAX = 448.0f;
constexpr int SAMPLES = 2;                        // rows sampled per call (serve_fp8.py:44)
constexpr int64_t ROW_A = 7919, ROW_B = 104729;   // their positions: (step * ROW_A + j * ROW_B) % rows
constexpr int64_t M32 = 0xFFFFFFFFll, S31 = 0x7FFFFFFFll, EVERY_ROW = 0xFFFFFF;
enum { C_CALLS, C_SCALE, C_OUTSIDE, C_VALUES, C_ONE, C_LAST, C_RATIO, C_STATIC };
enum { KIND_SCALE = 1, KIND_OUTSIDE = 2, KIND_VALUES = 3, KIND_STATIC = 4 };
constexpr int AMAX_BLOCKS = 1024;                 // workgroups of fp8q_amax (at most)
constexpr int AMAX_ROWS = 4;                      // rows a workgroup of fp8q_amax has in flight

template <int DT>
__device__ __forceinline__ float load_x(const void* p, int64_t i) {
  if constexpr (DT == DT_F32) {
    return reinterpret_cast<const float*>(p)[i];
  } else {
    return half_to_f32<DT>(reinterpret_cast<const uint16_t*>(p)[i]);
  }
}

// fp32 -> FP8 E4M3 (OCP "fn": no infinities, S.1111.111 is NaN) code, rounding to nearest even, for |v| <= 448
// (the caller clamps); NaN keeps its sign
__device__ __forceinline__ uint32_t to_e4m3(float v) {
  const uint32_t u = __float_as_uint(v), sign = (u >> 24) & 0x80u, a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return sign | 0x7Fu;
  if (a < 0x3C800000u) {                                     // |v| < 2^-6: multiples of 2^-9 (8 rounds up to 2^-6)
    return sign | (uint32_t)rintf(__uint_as_float(a) * 512.0f);
  }
  const uint32_t r = (a + 0x7FFFFu + ((a >> 20) & 1u)) >> 20;  // exponent and 3 mantissa bits, rounded
  return sign | (r - (120u << 3));                            // rebias 127 -> 7
}

// a code's position in value order: one representable step apart = 1 apart (+0 and -0 both 0)
__device__ __forceinline__ int fp8_order(uint32_t c) { return (c & 0x80u) ? -(int)(c & 0x7Fu) : (int)(c & 0x7Fu); }

__device__ __forceinline__ uint32_t abs_bits(float v) { return __float_as_uint(v) & 0x7FFFFFFFu; }

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    const uint32_t o = __shfl_xor(v, m, SDC_WAVE);
    v = o > v ? o : v;
  }
  return v;
}

struct Fp8Args {
  const void* x;                                  // (m, k) layer input
  int64_t sxm, sxk, m, k;
  const uint8_t* xq;                              // (mq >= m, k) FP8 codes the GEMM got
  int64_t sqm, sqk, mq;
  const float* xs;                                // scale(s): xs[i * sxs], i < xs_n
  int64_t xs_n, sxs;
  int recipe;
  const float* ub;                                // per-token cap of max |x| (or null)
  const float* sref;                              // static: the scale at load (or null)
  const int64_t* rows_buf;                        // [0]: this step's real rows (0: outside a step)
  const int64_t* stepbuf;                         // [0]: the step
  int64_t mult;                                   // input rows per token
  int64_t* state;                                 // the layer's 8 columns
  uint32_t* partial;                              // fp8q_amax: [blocks][2] bits of the maxima
  int nblk;
};

__device__ __forceinline__ int64_t real_rows(const Fp8Args& a) {
  int64_t r = a.rows_buf[0] * a.mult;
  return r < 0 ? 0 : (r > a.m ? a.m : r);
}

template <int DT>
__global__ __launch_bounds__(256) void fp8q_amax_kernel(Fp8Args a) {
  __shared__ uint32_t red[4][2];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int64_t real = real_rows(a);
  uint32_t mi = 0, ma = 0;
  const bool vec = DT != DT_F32 && a.sxk == 1 && a.k % 8 == 0 && a.sxm % 8 == 0 && ((uintptr_t)a.x & 15) == 0;
  // AMAX_ROWS rows a workgroup at a time, every 16-byte load of a thread's share of them (two pieces a row) issued
  // before any is used
  for (int64_t r0 = (int64_t)blockIdx.x * AMAX_ROWS; r0 < a.m; r0 += (int64_t)gridDim.x * AMAX_ROWS) {
    if (vec) {
      const int64_t cpr = a.k / 8;                                  // 16-byte pieces a row
      for (int64_t c0 = t; c0 < cpr; c0 += 512) {
        uint4 q[AMAX_ROWS][2];
#pragma unroll
        for (int i = 0; i < AMAX_ROWS; ++i)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int64_t row = r0 + i, c = c0 + 256 * h;
            q[i][h] = row < a.m && c < cpr ? reinterpret_cast<const uint4*>(
                                                 reinterpret_cast<const uint16_t*>(a.x) + row * a.sxm)[c]
                                           : uint4{0u, 0u, 0u, 0u};
          }
#pragma unroll
        for (int i = 0; i < AMAX_ROWS; ++i) {
          uint32_t rm = 0;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const uint32_t ws[4] = {q[i][h].x, q[i][h].y, q[i][h].z, q[i][h].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const uint32_t lo = abs_bits(lo_of<DT>(ws[e])), hi = abs_bits(hi_of<DT>(ws[e]));
              rm = lo > rm ? lo : rm;
              rm = hi > rm ? hi : rm;
            }
          }
          ma = rm > ma ? rm : ma;
          if (r0 + i < real) mi = rm > mi ? rm : mi;
        }
      }
    } else {
      for (int i = 0; i < AMAX_ROWS; ++i) {
        const int64_t row = r0 + i;
        if (row >= a.m) break;
        uint32_t rm = 0;
        for (int64_t kk = t; kk < a.k; kk += 256) {
          const uint32_t v = abs_bits(load_x<DT>(a.x, row * a.sxm + kk * a.sxk));
          rm = v > rm ? v : rm;
        }
        ma = rm > ma ? rm : ma;
        if (row < real) mi = rm > mi ? rm : mi;
      }
    }
  }
  mi = wave_max_u32_dpp(mi);
  ma = wave_max_u32_dpp(ma);
  if (lane == 0) {
    red[w][0] = mi;
    red[w][1] = ma;
  }
  __syncthreads();
  if (t == 0) {
    uint32_t x0 = red[0][0], x1 = red[0][1];
    for (int i = 1; i < 4; ++i) {
      x0 = red[i][0] > x0 ? red[i][0] : x0;
      x1 = red[i][1] > x1 ? red[i][1] : x1;
    }
    a.partial[2 * blockIdx.x] = x0;
    a.partial[2 * blockIdx.x + 1] = x1;
  }
}

__device__ __forceinline__ float scale_at(const Fp8Args& a, int64_t i) {
  return a.xs[(i < a.xs_n ? i : a.xs_n - 1) * a.sxs];
}

template <int DT>
__global__ __launch_bounds__(256) void fp8q_judge_kernel(Fp8Args a) {
  __shared__ uint32_t ru[4][2 + SAMPLES];
  __shared__ int ri[4][SAMPLES + 1];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int64_t real = real_rows(a);
  const bool armed = real > 0;
  const int64_t step = a.stepbuf[0] & M32;
  const int64_t rmod = real > 0 ? real : 1;
  int64_t rows[SAMPLES];
#pragma unroll
  for (int j = 0; j < SAMPLES; ++j) rows[j] = (step * ROW_A + j * ROW_B) % rmod;
  const bool per_token = a.recipe == 2, per_tensor = a.recipe == 1;
  // the scale each sampled row is quantized with, and how
  float use[SAMPLES];
#pragma unroll
  for (int j = 0; j < SAMPLES; ++j) use[j] = per_token ? scale_at(a, rows[j]) : a.xs[0];
  const bool divide = per_token;
  // per-tensor: the maxima from fp8q_amax
  uint32_t mi = 0, ma = 0;
  if (per_tensor)
    for (int i = t; i < a.nblk; i += 256) {
      mi = a.partial[2 * i] > mi ? a.partial[2 * i] : mi;
      ma = a.partial[2 * i + 1] > ma ? a.partial[2 * i + 1] : ma;
    }
  // the sampled rows: their max |x| and their values against the GEMM's codes
  uint32_t am[SAMPLES];
  int nbad[SAMPLES], none = 0;
  float inv[SAMPLES];
#pragma unroll
  for (int j = 0; j < SAMPLES; ++j) {
    am[j] = 0;
    nbad[j] = 0;
    inv[j] = 1.0f / use[j];
  }
  // one value of sampled row j against the GEMM's code for it
  auto judge_one = [&](int j, float x, uint32_t code) {
    const uint32_t xb = abs_bits(x);
    am[j] = xb > am[j] ? xb : am[j];
    float v = divide ? x / use[j] : x * inv[j];
    v = v != v ? v : fminf(fmaxf(v, -FP8_MAX), FP8_MAX);
    const int d = abs(fp8_order(to_e4m3(v)) - fp8_order(code));
    nbad[j] += d >= 2;
    none += d == 1;
  };
  const bool vec = DT != DT_F32 && a.sxk == 1 && a.sqk == 1 && a.k % 8 == 0 && a.sxm % 8 == 0 && a.sqm % 8 == 0 &&
                   ((uintptr_t)a.x & 15) == 0 && ((uintptr_t)a.xq & 7) == 0;
  if (vec) {
    // 8 values a load (16 bytes of x, 8 of codes); both rows' loads of U chunks issued before any is used
    constexpr int U = 2;
    const int64_t nch = a.k / 8;
    for (int64_t c0 = t; c0 < nch; c0 += 256 * U) {
      uint4 xv[SAMPLES][U];
      uint2 qv[SAMPLES][U];
#pragma unroll
      for (int j = 0; j < SAMPLES; ++j)
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int64_t c = c0 + 256 * u;
          if (c < nch) {
            xv[j][u] = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(a.x) + rows[j] * a.sxm + 8 * c);
            qv[j][u] = *reinterpret_cast<const uint2*>(a.xq + rows[j] * a.sqm + 8 * c);
          }
        }
#pragma unroll
      for (int j = 0; j < SAMPLES; ++j)
#pragma unroll
        for (int u = 0; u < U; ++u) {
          if (c0 + 256 * u >= nch) continue;
          const uint32_t ws[4] = {xv[j][u].x, xv[j][u].y, xv[j][u].z, xv[j][u].w};
          const uint32_t qs[2] = {qv[j][u].x, qv[j][u].y};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t qw = qs[e / 2] >> (16 * (e & 1));
            judge_one(j, lo_of<DT>(ws[e]), qw & 0xFFu);
            judge_one(j, hi_of<DT>(ws[e]), (qw >> 8) & 0xFFu);
          }
        }
    }
  } else {
#pragma unroll
    for (int j = 0; j < SAMPLES; ++j)
      for (int64_t kk = t; kk < a.k; kk += 256)
        judge_one(j, load_x<DT>(a.x, rows[j] * a.sxm + kk * a.sxk), a.xq[rows[j] * a.sqm + kk * a.sqk]);
  }
  mi = wave_max_u32_dpp(mi);
  ma = wave_max_u32_dpp(ma);
#pragma unroll
  for (int j = 0; j < SAMPLES; ++j) {
    am[j] = wave_max_u32_dpp(am[j]);
    nbad[j] = wave_sum_i32_dpp(nbad[j]);
  }
  none = wave_sum_i32_dpp(none);
  if (lane == 0) {
    ru[w][0] = mi;
    ru[w][1] = ma;
#pragma unroll
    for (int j = 0; j < SAMPLES; ++j) {
      ru[w][2 + j] = am[j];
      ri[w][j] = nbad[j];
    }
    ri[w][SAMPLES] = none;
  }
  __syncthreads();
  if (t != 0) return;
  for (int i = 1; i < 4; ++i) {
    mi = ru[i][0] > ru[0][0] ? ru[i][0] : ru[0][0];
    ru[0][0] = mi;
    ma = ru[i][1] > ru[0][1] ? ru[i][1] : ru[0][1];
    ru[0][1] = ma;
#pragma unroll
    for (int j = 0; j < SAMPLES; ++j) {
      ru[0][2 + j] = ru[i][2 + j] > ru[0][2 + j] ? ru[i][2 + j] : ru[0][2 + j];
      ri[0][j] += ri[i][j];
    }
    ri[0][SAMPLES] += ri[i][SAMPLES];
  }
  mi = ru[0][0];
  ma = ru[0][1];
  const float tol = 0.00390625f;                              // 2^-8, one bf16 rounding (serve_fp8.py:45)
  const float tiny = 1e-38f;
  bool scale_bad = false, outside = false, static_bad = false;
  float ratio = 1.0f;
  int64_t scale_row = EVERY_ROW;
  if (per_tensor) {
    const float ks = a.xs[0];
    const float ref = __uint_as_float(mi) / FP8_MAX, every = __uint_as_float(ma) / FP8_MAX;
    scale_bad = fabsf(ks - ref) > tol * fabsf(ref) + tiny;
    outside = scale_bad && (fabsf(ks - every) <= tol * fabsf(every) + tiny) && (every > ref);
    ratio = ks / (ref != ref ? ref : fmaxf(ref, tiny));
  } else if (per_token) {
    const float min_scale = (float)(1.0 / (448.0 * 512.0));
    int sel = 0;
    bool found = false;
    float r_sel = 1.0f;
#pragma unroll
    for (int j = 0; j < SAMPLES; ++j) {
      float amax = __uint_as_float(ru[0][2 + j]);
      if (a.ub) {
        const float ub = a.ub[0];
        amax = (amax != amax || ub != ub) ? __builtin_nanf("") : fminf(amax, ub);
      }
      float ref = amax / FP8_MAX;
      ref = ref != ref ? ref : fmaxf(ref, min_scale);
      const float ks = use[j];
      const bool diff = fabsf(ks - ref) > tol * fabsf(ref) + tiny;
      const float rj = ks / (ref != ref ? ref : fmaxf(ref, tiny));
      if (j == 0) r_sel = rj;
      if (diff && !found) {
        found = true;
        sel = j;
        r_sel = rj;
      }
    }
    scale_bad = found;
    ratio = r_sel;
    scale_row = rows[sel] / (a.mult > 1 ? a.mult : 1);
  } else if (a.sref) {
    static_bad = !(a.xs[0] == a.sref[0]);
  }
  bool vb[SAMPLES], any_vb = false;
  int nvb = 0, first_vb = 0;
#pragma unroll
  for (int j = 0; j < SAMPLES; ++j) {
    vb[j] = ri[0][j] > 0 && armed;
    if (vb[j] && !any_vb) first_vb = j;
    any_vb = any_vb || vb[j];
    nvb += vb[j];
  }
  const bool sb = scale_bad && armed;
  const int kind = (outside && armed) ? KIND_OUTSIDE : sb ? KIND_SCALE : any_vb ? KIND_VALUES
                 : (static_bad && armed) ? KIND_STATIC : 0;
  const int64_t val_row = rows[first_vb] / (a.mult > 1 ? a.mult : 1);
  const int64_t bad_row = kind == KIND_VALUES ? val_row : kind == KIND_SCALE ? scale_row : EVERY_ROW;
  const int64_t rec = ((step & S31) << 32) | ((int64_t)kind << 24) | (bad_row & 0xFFFFFF);
  unsigned long long* s = reinterpret_cast<unsigned long long*>(a.state);
  if (armed) {
    atomicAdd(s + C_CALLS, 1ull);
    if (sb) atomicAdd(s + C_SCALE, 1ull);
    if (outside) atomicAdd(s + C_OUTSIDE, 1ull);
    if (nvb) atomicAdd(s + C_VALUES, (unsigned long long)nvb);
    if (ri[0][SAMPLES]) atomicAdd(s + C_ONE, (unsigned long long)ri[0][SAMPLES]);
    if (static_bad) atomicMax(s + C_STATIC, 1ull);
  }
  if (kind > 0) atomicMax(s + C_LAST, (unsigned long long)rec);
  if (sb) {
    float r = fabsf(ratio);
    r = r != r ? r : fminf(r, 3e38f);
    atomicMax(s + C_RATIO, (unsigned long long)__float_as_uint(r));
  }
}

template <int DT>
int run(Fp8Args a, hipStream_t stream) {
  if (a.recipe == 1) {
    SdcProf prof("fp8q_amax", stream);
    hipLaunchKernelGGL(fp8q_amax_kernel<DT>, dim3((unsigned)a.nblk), dim3(256), 0, stream, a);
    SDC_LAUNCH_CHECK();
  }
  SdcProf prof("fp8q_judge", stream);
  hipLaunchKernelGGL(fp8q_judge_kernel<DT>, dim3(1), dim3(256), 0, stream, a);
  SDC_LAUNCH_CHECK();
  return SDC_OK;
}

int64_t amax_blocks(int64_t m) {
  const int64_t b = (m + AMAX_ROWS - 1) / AMAX_ROWS;
  return b < 1 ? 1 : (b < AMAX_BLOCKS ? b : AMAX_BLOCKS);
}

}  // namespace

extern "C" int64_t sdc_fp8_quant_check_workspace(int64_t m) { return amax_blocks(m) * 8 + 256; }

extern "C" int sdc_fp8_quant_check(int dtype, const void* x, int64_t sxm, int64_t sxk, int64_t m, int64_t k,
                                   const uint8_t* xq, int64_t sqm, int64_t sqk, int64_t mq, const float* xs,
                                   int64_t xs_n, int64_t sxs, int recipe, const float* scale_ub,
                                   const float* static_ref, const int64_t* rows_buf, const int64_t* stepbuf,
                                   int64_t mult, int64_t* state_row, void* workspace, int64_t workspace_bytes,
                                   hipStream_t stream) {
  SDC_CLEAR_ERRORS();
  if (dtype != SDC_BF16 && dtype != SDC_FP16 && dtype != DT_F32) return SDC_EUNSUPPORTED;
  if (!x || !xq || !xs || !rows_buf || !stepbuf || !state_row) return SDC_EINVAL;
  if (m < 1 || k < 1 || mq < m || xs_n < 1 || recipe < 0 || recipe > 2 || mult < 1) return SDC_EINVAL;
  const int64_t nblk = amax_blocks(m);
  if (recipe == 1 && (!workspace || workspace_bytes < nblk * 8)) return SDC_EWORKSPACE;
  Fp8Args a{};
  a.x = x; a.sxm = sxm; a.sxk = sxk; a.m = m; a.k = k;
  a.xq = xq; a.sqm = sqm; a.sqk = sqk; a.mq = mq;
  a.xs = xs; a.xs_n = xs_n; a.sxs = sxs; a.recipe = recipe; a.ub = scale_ub; a.sref = static_ref;
  a.rows_buf = rows_buf; a.stepbuf = stepbuf; a.mult = mult; a.state = state_row;
  a.partial = (uint32_t*)workspace; a.nblk = (int)nblk;
  if (dtype == SDC_BF16) return run<SDC_BF16>(a, stream);
  if (dtype == SDC_FP16) return run<SDC_FP16>(a, stream);
  return run<DT_F32>(a, stream);
}
