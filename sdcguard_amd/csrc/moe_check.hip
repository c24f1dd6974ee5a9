// The sampled recompute of a fused MoE layer's output (serve_moe.py:127-506, `recompute`, `scores`,
// `moe_check_torch`): at each step one MoE layer (the one whose index is the step modulo the number of layers)
// recomputes the output of SAMPLES rows of its batch from the layer's own input, routing and expert weights,
//     y = sum_k g_k W2_e (act(W1_e x) * (W3_e x)),
// rounded where the fused kernel rounds (the first matmul in fp32 rounded to the dtype, the activation rounded,
// the product rounded, the second matmul in fp32 times the routing weight and rounded, the experts summed in fp32),
// and scores every output against
//     u |r| + 2 (2u) max_k |c_k| + u sqrt(sum_k g_k^2 sum_i (W2_ni h_i)^2) + max_k,i |g_k W2_ni| s_i + spacing.
// It also reads the expert ids of every known real row of the step: a real row with all (or some) experts -1 is
// counted.  Results go into the layer's 11-column state row (worst keys z << 32 | row, column, output bits,
// recompute bits, step; active calls; rows checked; unjudged outputs; unrouted and partly routed real rows; the last
// such row), and the first sampled row over the line is kept (input, output, experts, routing weights).
//
// Four launches, each returning at once unless its layer is the active one this step (read from the step buffer on
// the device: no host synchronisation, graph-safe): moe_up (one wave per row of W13: 16-byte loads of the expert's
// weights against the sampled input row, wave reduction), moe_act (h and its rounding sensitivity s per sampled
// (row, expert) into scratch), moe_down (one wave per output row of W2: the sum, the sum of squares and the worst
// |w| s), moe_compare (one workgroup per sampled row: experts summed, scored, keys, capture; NSCAN more scan the
// real rows' expert ids).
#include "common.h"
#include "profile.h"

namespace {

constexpr int SAMPLES = 2;                       // rows recomputed per active call (serve_moe.py:51)
constexpr int64_t ROW_A = 7919, ROW_B = 104729;
constexpr int64_t M32 = 0xFFFFFFFFll;
enum { C_ROW, C_COL, C_OUT, C_REF, C_STEP, C_CALLS, C_ROWS, C_UNJ, C_UNROUTED, C_PARTIAL, C_BADROW, COLS };
constexpr int WPB = 4;                           // waves per workgroup (256 threads)
constexpr int RPW = 4;                           // matrix rows per wave
constexpr int NSCAN = 8;                         // workgroups of moe_compare scanning the real rows' expert ids

struct MoeArgs {
  const void* x;                                 // (m, H) layer input
  int64_t sx;
  const void* out;                               // (m, H) layer output
  int64_t so;
  const void* gw;                                // (m, K) routing weights (dtype gdt)
  int gdt;                                       // 0 bf16, 1 fp16, 4 fp32
  const int32_t* ids;                            // (m, K) expert ids (int32)
  const void* w13;                               // (E, 2I, H)
  int64_t s13e, s13n;
  const void* w2;                                // (E, H, I)
  int64_t s2e, s2n;
  const int32_t* emap;                           // expert map or null
  int64_t E, maplen;                             // experts held (w13 / w2), entries of the expert map
  int64_t m, H, I, K;
  int act;                                       // 0 silu, 1 gelu
  int routed_first;
  const int64_t* stepbuf;                        // [0]: step (low 32 bits) | real rows << 32
  int64_t nl, idx;                               // layers taking turns, this layer's index
  float u, spacing, fmax, line;
  float* A;                                      // scratch (SAMPLES K, 2I)
  float* Hs;                                     // scratch (SAMPLES K, 2, I): h, s
  float* C;                                      // scratch (SAMPLES K, 3, H): c, sq, mx
  int64_t* state;                                // the layer's COLS
  int32_t* capm;                                 // the layer's capture: claimed, row, step, z bits
  float* capx;
  float* capy;
  int64_t* capi;
  float* capg;
  float* scores;                                 // optional (SAMPLES, H): every output's score
};

template <int DT>
__device__ __forceinline__ float ld(const void* p, int64_t i) {
  if constexpr (DT == 4) {
    return reinterpret_cast<const float*>(p)[i];
  } else {
    return half_to_f32<DT>(reinterpret_cast<const uint16_t*>(p)[i]);
  }
}

__device__ __forceinline__ float gweight(const MoeArgs& a, int64_t i) {
  return a.gdt == 4 ? reinterpret_cast<const float*>(a.gw)[i]
                    : (a.gdt == 0 ? half_to_f32<SDC_BF16>(reinterpret_cast<const uint16_t*>(a.gw)[i])
                                  : half_to_f32<SDC_FP16>(reinterpret_cast<const uint16_t*>(a.gw)[i]));
}

// fp32 rounded to the dtype and back (ties to even; NaN kept)
template <int DT>
__device__ __forceinline__ float rnd(float v) {
  if constexpr (DT == SDC_BF16) {
    if (v != v) return v;
    uint32_t b = __float_as_uint(v);
    b = (b + 0x7FFFu + ((b >> 16) & 1u)) & 0xFFFF0000u;
    return __uint_as_float(b);
  } else {
    return (float)(_Float16)v;
  }
}

struct Live {
  int64_t step, rows;
  bool live;
};

__device__ __forceinline__ Live live_of(const MoeArgs& a) {
  const int64_t raw = a.stepbuf[0];
  const int64_t step = raw & M32, real = (raw >> 32) & 0x7FFFFFFFll;
  Live l;
  l.step = step;
  l.live = (step % a.nl) == a.idx;
  l.rows = real > 0 ? (real < a.m ? real : a.m) : a.m;
  return l;
}

__device__ __forceinline__ int64_t sample_row(const Live& l, int j, int64_t nl) {
  return ((l.step / nl) * ROW_A + j * ROW_B) % (l.rows > 0 ? l.rows : 1);
}

// The local expert of slot k of a row: -1 for no expert (padding, or an expert the map puts on another GPU), -2 for
// an id outside the router's range or a map entry outside the experts held.  Neither is read: a corrupted id must
// not make the check itself read past the weights.
__device__ __forceinline__ int64_t expert(const MoeArgs& a, int64_t row, int64_t k) {
  int64_t e = a.ids[row * a.K + k];
  if (e == -1) return -1;
  if (e < 0 || e >= (a.emap ? a.maplen : a.E)) return -2;
  if (a.emap) {
    e = a.emap[e];
    if (e == -1) return -1;
    if (e < 0 || e >= a.E) return -2;
  }
  return e;
}

// An id the router cannot have produced (not -1 and outside [0, experts or map entries))
__device__ __forceinline__ bool bad_id(const MoeArgs& a, int64_t id) {
  return id != -1 && (id < 0 || id >= (a.emap ? a.maplen : a.E));
}

__device__ __forceinline__ float wave_sum(float v) { return wave_sum_f32_dpp(v); }
__device__ __forceinline__ float wave_max(float v) { return wave_max_f32_dpp(v); }

// The vector path reads the rows in chunks of NCH 16-byte pieces a lane and row (chunk cb: pieces at values
// cb + 8 lane + 512 u, u < NCH), every load of a chunk issued before any is used.
constexpr int NCH = 4;
using RowChunk = uint4[RPW][NCH];

__device__ __forceinline__ void rows_load(const uint16_t* const (&w)[RPW], int64_t n, int lane, int64_t cb,
                                          RowChunk& q) {
#pragma unroll
  for (int r = 0; r < RPW; ++r)
#pragma unroll
    for (int u = 0; u < NCH; ++u) {
      const int64_t c = cb + lane * 8 + 512 * u;
      q[r][u] = (w[r] && c < n) ? *reinterpret_cast<const uint4*>(w[r] + c) : uint4{0u, 0u, 0u, 0u};
    }
}

// dots of RPW weight rows (n 16-bit values each, rows w[r], null past the matrix) with a float vector v, the rows
// read together so each chunk of v (and of sens) is read once for all of them; each lane takes 8 consecutive values
// at a time when the rows are 16-byte aligned, else one.  With SQ also the sums of squares of the products and the
// largest |w| sens.  With PRE, `pre` holds the vector path's first chunk, already loaded by the caller.
template <int DT, bool SQ, bool PRE = false>
__device__ __forceinline__ void rows_dot(const uint16_t* const (&w)[RPW], const float* v, int64_t n, int lane,
                                         bool vec, const float* sens, float (&acc)[RPW], float (&sq)[RPW],
                                         float (&mx)[RPW], const RowChunk& pre = RowChunk{}) {
#pragma unroll
  for (int r = 0; r < RPW; ++r) acc[r] = sq[r] = mx[r] = 0.f;
  if (vec) {
    for (int64_t cb = 0; cb < n; cb += 512 * NCH) {
      RowChunk qc;
      if (PRE && cb == 0) {
#pragma unroll
        for (int r = 0; r < RPW; ++r)
#pragma unroll
          for (int u = 0; u < NCH; ++u) qc[r][u] = pre[r][u];
      } else {
        rows_load(w, n, lane, cb, qc);
      }
#pragma unroll
      for (int u = 0; u < NCH; ++u) {
        const int64_t c = cb + lane * 8 + 512 * u;
        if (c >= n) break;
        float vv[8], ss[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          vv[e] = v[c + e];
          if constexpr (SQ) ss[e] = sens[c + e];
        }
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
          if (!w[r]) continue;
          const uint4 q = qc[r][u];
          const uint32_t ws[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float w0 = lo_of<DT>(ws[e]), w1 = hi_of<DT>(ws[e]);
            const float p0 = w0 * vv[2 * e], p1 = w1 * vv[2 * e + 1];
            acc[r] += p0;
            acc[r] += p1;
            if constexpr (SQ) {
              sq[r] += p0 * p0;
              sq[r] += p1 * p1;
              mx[r] = fmaxf(mx[r], fmaxf(fabsf(w0) * ss[2 * e], fabsf(w1) * ss[2 * e + 1]));
            }
          }
        }
      }
    }
  } else {
    for (int64_t c = lane; c < n; c += 64) {
      const float vc = v[c];
      const float sc = SQ ? sens[c] : 0.f;
#pragma unroll
      for (int r = 0; r < RPW; ++r) {
        if (!w[r]) continue;
        const float w0 = half_to_f32<DT>(w[r][c]);
        const float p0 = w0 * vc;
        acc[r] += p0;
        if constexpr (SQ) {
          sq[r] += p0 * p0;
          mx[r] = fmaxf(mx[r], fabsf(w0) * sc);
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    acc[r] = wave_sum(acc[r]);
    if constexpr (SQ) {
      sq[r] = wave_sum(sq[r]);
      mx[r] = wave_max(mx[r]);
    }
  }
}

// 1. a = W13_e x (fp32, times g first when the routing weight is applied on the input), rounded
template <int DT>
__global__ __launch_bounds__(256) void moe_up_kernel(MoeArgs a) {
  __shared__ float xs[8192];                     // the sampled row (H <= 8192: checked at the entry point)
  const Live l = live_of(a);
  if (!l.live) return;
  const int jk = blockIdx.x, j = jk / (int)a.K, k = jk % (int)a.K;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int64_t row = sample_row(l, j, a.nl), e = expert(a, row, k);
  const int64_t n2 = 2 * a.I;
  const bool vec = (a.H % 8 == 0) && (a.s13n % 8 == 0) && (a.s13e % 8 == 0) && (((uintptr_t)a.w13 & 15) == 0);
  const int64_t n0 = ((int64_t)blockIdx.y * WPB + w) * RPW;
  const uint16_t* wr[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r)
    wr[r] = (e >= 0 && n0 + r < n2) ? reinterpret_cast<const uint16_t*>(a.w13) + e * a.s13e + (n0 + r) * a.s13n
                                    : nullptr;
  // the rows' first chunk goes out before the sampled row is staged in LDS: both arrive in one round trip
  RowChunk pre = {};
  if (vec) rows_load(wr, a.H, lane, 0, pre);
  for (int64_t h = t; h < a.H; h += 256) xs[h] = ld<DT>(a.x, row * a.sx + h);
  __syncthreads();
  const float g = gweight(a, row * a.K + k);
  float acc[RPW], sq[RPW], mx[RPW];
  rows_dot<DT, false, true>(wr, xs, a.H, lane, vec, nullptr, acc, sq, mx, pre);
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    if (n0 + r >= n2) break;
    float v = e >= 0 ? acc[r] : 0.f;
    if (e >= 0 && a.routed_first) v *= g;
    if (lane == 0) a.A[(int64_t)jk * n2 + n0 + r] = rnd<DT>(v);
  }
}

// 2. h = round(round(act(a1)) a3) and its rounding sensitivity s = 2u (|h| + |act'(a1) a1 a3| + |act(a1) a3|)
template <int DT>
__global__ __launch_bounds__(256) void moe_act_kernel(MoeArgs a) {
  const Live l = live_of(a);
  if (!l.live) return;
  const int jk = blockIdx.x;
  const int64_t n2 = 2 * a.I;
  const float* ar = a.A + (int64_t)jk * n2;
  float* hs = a.Hs + (int64_t)jk * 2 * a.I;
  for (int64_t i = blockIdx.y * 256 + threadIdx.x; i < a.I; i += (int64_t)gridDim.y * 256) {
    const float a1 = ar[i], a3 = ar[a.I + i];
    float s1, d1;
    if (a.act == 0) {
      const float sg = 1.0f / (1.0f + expf(-a1));
      s1 = a1 * sg;
      d1 = sg * (1.0f + a1 * (1.0f - sg));
    } else {
      const float cdf = 0.5f * (1.0f + erff(a1 * 0.7071067811865476f));
      s1 = a1 * cdf;
      d1 = cdf + a1 * expf(-0.5f * a1 * a1) * 0.3989422804014327f;
    }
    s1 = rnd<DT>(s1);
    const float h = rnd<DT>(s1 * a3);
    hs[i] = h;
    hs[a.I + i] = 2.0f * a.u * (fabsf(h) + fabsf(d1 * a1 * a3) + fabsf(s1 * a3));
  }
}

// 3. c = W2_e h (fp32) times g (unless applied first), rounded; sum of squares and worst |w| s, times g^2, |g|
template <int DT>
__global__ __launch_bounds__(256) void moe_down_kernel(MoeArgs a) {
  const Live l = live_of(a);
  if (!l.live) return;
  const int jk = blockIdx.x, j = jk / (int)a.K, k = jk % (int)a.K;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int64_t row = sample_row(l, j, a.nl), e = expert(a, row, k);
  const float* h = a.Hs + (int64_t)jk * 2 * a.I;
  const float* sens = h + a.I;
  const float g = a.routed_first ? 1.0f : gweight(a, row * a.K + k);
  const bool vec = (a.I % 8 == 0) && (a.s2n % 8 == 0) && (a.s2e % 8 == 0) && (((uintptr_t)a.w2 & 15) == 0);
  float* cr = a.C + (int64_t)jk * 3 * a.H;
  const int64_t o0 = ((int64_t)blockIdx.y * WPB + w) * RPW;
  const uint16_t* wr[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r)
    wr[r] = (e >= 0 && o0 + r < a.H) ? reinterpret_cast<const uint16_t*>(a.w2) + e * a.s2e + (o0 + r) * a.s2n
                                     : nullptr;
  float acc[RPW], sq[RPW], mx[RPW];
  rows_dot<DT, true>(wr, h, a.I, lane, vec, sens, acc, sq, mx);
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int64_t o = o0 + r;
    if (o >= a.H) break;
    float c = 0.f, q = 0.f, x = 0.f;
    if (e >= 0) {
      c = rnd<DT>(acc[r] * g);
      q = sq[r] * g * g;
      x = mx[r] * fabsf(g);
    }
    if (lane == 0) {
      cr[o] = c;
      cr[a.H + o] = q;
      cr[2 * a.H + o] = x;
    }
  }
}

__device__ __forceinline__ int64_t fb(float f) { return (int64_t)(uint32_t)__float_as_uint(f); }

// 4. one workgroup per sampled row: the experts summed and every output scored; the worst into the keys; the first
// row over the line kept; workgroup 0 also counts the call.  Workgroups SAMPLES .. SAMPLES + NSCAN - 1 scan every
// known real row's expert ids.
template <int DT>
__global__ __launch_bounds__(256) void moe_compare_kernel(MoeArgs a) {
  __shared__ float rz[4];
  __shared__ int64_t rc[4];
  __shared__ int ru[4];
  __shared__ int rnone[4], rsome[4];
  __shared__ int64_t rlast[4];
  const Live l = live_of(a);
  if (!l.live) return;
  const int j = blockIdx.x, t = threadIdx.x, lane = t & 63, w = t >> 6;
  unsigned long long* s = reinterpret_cast<unsigned long long*>(a.state);
  if (j >= SAMPLES) {
    // the routing's validity: every known real row's expert ids, NSCAN workgroups striding over the rows, four
    // rows a thread at a time (their ids' loads in flight together)
    if (((a.stepbuf[0] >> 32) & 0x7FFFFFFFll) == 0) return;
    int nn = 0, ns = 0;
    int64_t last = 0;
    const int64_t stride = (int64_t)NSCAN * 256;
    for (int64_t r0 = (int64_t)(j - SAMPLES) * 256 + t; r0 < l.rows; r0 += 4 * stride) {
      int neg[4] = {0, 0, 0, 0};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t rr = r0 + q * stride;
        if (rr < l.rows) {
#pragma unroll 8
          for (int64_t k = 0; k < a.K; ++k) {     // slots with no expert, or with an id the router cannot produce
            const int64_t id = a.ids[rr * a.K + k];
            neg[q] += id == -1 || bad_id(a, id);
          }
        }
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t rr = r0 + q * stride;
        const bool none = rr < l.rows && neg[q] >= a.K, some = rr < l.rows && neg[q] > 0 && neg[q] < a.K;
        nn += none;
        ns += some;
        if (none || some) last = rr + 1 > last ? rr + 1 : last;
      }
    }
    nn = wave_sum_i32_dpp(nn);
    ns = wave_sum_i32_dpp(ns);
    last = wave_max_i64_dpp(last);
    if (lane == 0) {
      rnone[w] = nn;
      rsome[w] = ns;
      rlast[w] = last;
    }
    __syncthreads();
    if (t == 0) {
      const int tn = rnone[0] + rnone[1] + rnone[2] + rnone[3];
      const int ts = rsome[0] + rsome[1] + rsome[2] + rsome[3];
      int64_t lr = rlast[0];
      for (int i = 1; i < 4; ++i) lr = rlast[i] > lr ? rlast[i] : lr;
      if (tn > 0) atomicAdd(s + C_UNROUTED, (unsigned long long)tn);
      if (ts > 0) atomicAdd(s + C_PARTIAL, (unsigned long long)ts);
      if (lr > 0) atomicMax(s + C_BADROW, (unsigned long long)((l.step << 32) | lr));
    }
    return;
  }
  const int64_t row = sample_row(l, j, a.nl);
  int nneg = 0;
#pragma unroll 8
  for (int64_t k = 0; k < a.K; ++k) nneg += a.ids[row * a.K + k] == -1;
  const bool routed = nneg < a.K;                // a padding row (no experts) is neither judged nor counted
  float best = 0.f;
  int64_t bcol = 0;
  int unj = 0;
  if (!routed && a.scores)
    for (int64_t o = t; o < a.H; o += 256) a.scores[(int64_t)j * a.H + o] = 0.f;
  if (routed) {
    for (int64_t o = t; o < a.H; o += 256) {
      float r = 0.f, cmax = 0.f, sq = 0.f, mx = 0.f;
      // (unrolled: the loads of eight experts' terms are in flight together)
#pragma unroll 8
      for (int64_t k = 0; k < a.K; ++k) {
        const float* cr = a.C + ((int64_t)j * a.K + k) * 3 * a.H;
        const float cv = cr[o];
        r += cv;
        cmax = fmaxf(cmax, fabsf(cv));
        sq += cr[a.H + o];
        mx = fmaxf(mx, cr[2 * a.H + o]);
      }
      const float y = ld<DT>(a.out, row * a.so + o);
      const float den = a.u * fabsf(r) + 2.0f * 2.0f * a.u * cmax + a.u * sqrtf(sq) + mx + a.spacing;
      float z = fabsf(y - r) / den;
      z = z == z ? z : __builtin_inff();
      const bool ok = (fabsf(r) <= a.fmax) && (den < __builtin_inff());
      z = ok ? z : 0.f;
      unj += !ok;
      if (a.scores) a.scores[(int64_t)j * a.H + o] = z;
      if (z > best) {                            // (first column of the thread's largest)
        best = z;
        bcol = o;
      }
    }
  }
  // the row's worst (ties: the smallest column) as one key, z's bits (non-negative) above the column complemented;
  // the unjudged count
  {
    const int64_t key = wave_max_i64_dpp((fb(best) << 32) | (int64_t)(0xFFFFFFFFu - (uint32_t)bcol));
    best = __uint_as_float((uint32_t)((uint64_t)key >> 32));
    bcol = (int64_t)(0xFFFFFFFFu - (uint32_t)(uint64_t)key);
    unj = wave_sum_i32_dpp(unj);
  }
  if (lane == 0) {
    rz[w] = best;
    rc[w] = bcol;
    ru[w] = unj;
  }
  __syncthreads();
  if (t == 0) {
    for (int i = 1; i < 4; ++i)
      if (rz[i] > best || (rz[i] == best && rc[i] < bcol)) {
        best = rz[i];
        bcol = rc[i];
      }
    unj = ru[0] + ru[1] + ru[2] + ru[3];
    if (best > 0.f) {
      const float y = ld<DT>(a.out, row * a.so + bcol);
      float r = 0.f;
#pragma unroll 8
      for (int64_t k = 0; k < a.K; ++k) r += a.C[((int64_t)j * a.K + k) * 3 * a.H + bcol];
      const int64_t zb = fb(best) << 32;
      const int64_t cur = (int64_t)__atomic_load_n(s + C_ROW, __ATOMIC_RELAXED);
      if (zb >= (cur & ~M32)) {
        atomicMax(s + C_ROW, (unsigned long long)(zb | row));
        atomicMax(s + C_COL, (unsigned long long)(zb | bcol));
        atomicMax(s + C_OUT, (unsigned long long)(zb | fb(y)));
        atomicMax(s + C_REF, (unsigned long long)(zb | fb(r)));
        atomicMax(s + C_STEP, (unsigned long long)(zb | l.step));
      }
    }
    if (j == 0) atomicAdd(s + C_CALLS, 1ull);
    if (routed) atomicAdd(s + C_ROWS, 1ull);
    if (unj > 0) atomicAdd(s + C_UNJ, (unsigned long long)unj);
    if (best > a.line && atomicCAS(a.capm, 0, 1) == 0) {
      a.capm[1] = (int32_t)row;
      a.capm[2] = (int32_t)l.step;
      a.capm[3] = (int32_t)__float_as_uint(best);
      rc[0] = 1;                                 // (this workgroup copies the row below)
    } else {
      rc[0] = 0;
    }
  }
  __syncthreads();
  if (rc[0] == 1) {
    for (int64_t h = t; h < a.H; h += 256) {
      a.capx[h] = ld<DT>(a.x, row * a.sx + h);
      a.capy[h] = ld<DT>(a.out, row * a.so + h);
    }
    for (int64_t k = t; k < a.K; k += 256) {
      a.capi[k] = a.ids[row * a.K + k];
      a.capg[k] = gweight(a, row * a.K + k);
    }
  }
}

template <int DT>
int run(MoeArgs a, hipStream_t stream) {
  const unsigned sk = (unsigned)(SAMPLES * a.K);
  {
    SdcProf prof("moe_up", stream);
    hipLaunchKernelGGL(moe_up_kernel<DT>, dim3(sk, (unsigned)sdc_cdiv(2 * a.I, WPB * RPW)), dim3(256), 0, stream, a);
    SDC_LAUNCH_CHECK();
  }
  {
    SdcProf prof("moe_act", stream);
    hipLaunchKernelGGL(moe_act_kernel<DT>, dim3(sk, (unsigned)sdc_cdiv(a.I, 256)), dim3(256), 0, stream, a);
    SDC_LAUNCH_CHECK();
  }
  {
    SdcProf prof("moe_down", stream);
    hipLaunchKernelGGL(moe_down_kernel<DT>, dim3(sk, (unsigned)sdc_cdiv(a.H, WPB * RPW)), dim3(256), 0, stream, a);
    SDC_LAUNCH_CHECK();
  }
  {
    SdcProf prof("moe_compare", stream);
    hipLaunchKernelGGL(moe_compare_kernel<DT>, dim3(SAMPLES + NSCAN), dim3(256), 0, stream, a);
    SDC_LAUNCH_CHECK();
  }
  return SDC_OK;
}

}  // namespace

extern "C" int64_t sdc_moe_check_workspace(int64_t H, int64_t I, int64_t K) {
  if (H < 1 || I < 1 || K < 1) return 0;
  const int64_t sk = SAMPLES * K;
  return (sk * 2 * I + sk * 2 * I + sk * 3 * H) * 4 + 3 * 256;
}

extern "C" int sdc_moe_check(int dtype, const void* x, int64_t sx, const void* out, int64_t so, const void* gw,
                             int gdtype, const int32_t* ids, const void* w13, int64_t s13e, int64_t s13n,
                             const void* w2, int64_t s2e, int64_t s2n, const int32_t* expert_map,
                             int64_t n_experts, int64_t map_len, int64_t m,
                             int64_t H, int64_t I, int64_t K, int act, int routed_first, const int64_t* stepbuf,
                             int64_t nlayers, int64_t index, float u, float spacing, float fmax, float line,
                             int64_t* state_row, int32_t* cap_meta, float* cap_x, float* cap_y, int64_t* cap_ids,
                             float* cap_g, float* scores_out, void* workspace, int64_t workspace_bytes,
                             hipStream_t stream) {
  SDC_CLEAR_ERRORS();
  if (dtype != SDC_BF16 && dtype != SDC_FP16) return SDC_EUNSUPPORTED;
  if (gdtype != SDC_BF16 && gdtype != SDC_FP16 && gdtype != 4) return SDC_EUNSUPPORTED;
  if (!x || !out || !gw || !ids || !w13 || !w2 || !stepbuf || !state_row || !cap_meta || !cap_x || !cap_y ||
      !cap_ids || !cap_g)
    return SDC_EINVAL;
  if (m < 1 || H < 1 || I < 1 || K < 1 || nlayers < 1 || index < 0 || act < 0 || act > 1) return SDC_EINVAL;
  if (n_experts < 1 || (expert_map && map_len < 1)) return SDC_EINVAL;
  if (H > 8192) return SDC_EUNSUPPORTED;         // the sampled row is staged in LDS
  const int64_t need = sdc_moe_check_workspace(H, I, K);
  if (!workspace || workspace_bytes < need) return SDC_EWORKSPACE;
  uint8_t* ws = (uint8_t*)(((uintptr_t)workspace + 255) & ~(uintptr_t)255);
  const int64_t sk = SAMPLES * K;
  MoeArgs a{};
  a.x = x; a.sx = sx; a.out = out; a.so = so; a.gw = gw; a.gdt = gdtype; a.ids = ids;
  a.w13 = w13; a.s13e = s13e; a.s13n = s13n; a.w2 = w2; a.s2e = s2e; a.s2n = s2n; a.emap = expert_map;
  a.E = n_experts; a.maplen = expert_map ? map_len : 0;
  a.m = m; a.H = H; a.I = I; a.K = K; a.act = act; a.routed_first = routed_first; a.stepbuf = stepbuf;
  a.nl = nlayers; a.idx = index; a.u = u; a.spacing = spacing; a.fmax = fmax; a.line = line;
  a.A = (float*)ws;
  a.Hs = a.A + sk * 2 * I;
  a.C = a.Hs + sk * 2 * I;
  a.state = state_row; a.capm = cap_meta; a.capx = cap_x; a.capy = cap_y; a.capi = cap_ids; a.capg = cap_g;
  a.scores = scores_out;
  return dtype == SDC_BF16 ? run<SDC_BF16>(a, stream) : run<SDC_FP16>(a, stream);
}
