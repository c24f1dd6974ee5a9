// The MoE router check: did a router pick the experts and weights its routing policy gives for the logits?
//
// At the step in stepbuf[0] (low 32 bits) the router whose index is step % nlayers takes SAMPLES real rows of its
// call (row j = ((step / nlayers) * 7919 + j * 104729) % real rows, real rows in rows_buf[0]; none when it is 0)
// and recomputes its policy in fp32 from the row's logits (serve_route.py:83-186 states the policy and tolerances):
//   scores         softmax, or sigmoid, of the logits; the choice score adds the correction bias when there is one
//   groups         (DeepSeek's grouped top-k) a group scores the sum of its two best choice scores with a bias, its
//                  best without; the topk_group best groups are in, and where the next group scores within twice
//                  the choice tolerance of the cut, the groups near it may be in or out
//   experts        each chosen expert's choice score reaches the k-th best of the groups surely in, less the choice
//                  tolerance (1e-6 of the size, at least 1, plus 4 unit roundoffs of 16-bit logits); with groups
//                  also the k-th best of its own group and of the groups that may be in; the k ids distinct and in
//                  range
//   weights        the chosen experts' scores, renormalized over them when the policy does, times the scale, to
//                  2e-5 + (1e-4 + 6 u) |weight|
// One workgroup per sample: the row's choice scores live in LDS; the k-th bests come from k rounds of a
// workgroup (or, within a group, a wave) maximum with the winner taken out, so equal scores count each, as top-k
// does.  The router's state row gets its counts and the packed last finding by atomics, and the first wrong row
// since the last read is kept (logits, ids, weights) behind a compare-and-swap on its flag.  No host
// synchronisation, no memory set: the call can be captured in a graph.
#include <math.h>

#include "common.h"
#include "profile.h"

// The verdicts compare scores with tolerances at float32 rounding, one rounding per operation as numpy and torch
// give them: no fused multiply-adds.
#pragma clang fp contract(off)

namespace {

constexpr int SAMPLES = 2, COLS = 6, CAPC = 6, NT = 256, NW = NT / 64;
constexpr int MAXE = 2048, MAXK = 32, MAXG = 64, EPT = MAXE / NT;   // experts per thread
enum { C_CALLS, C_SET, C_WEIGHT, C_LAST, C_WDIFF, C_ROWS };
constexpr int64_t ROW_A = 7919, ROW_B = 104729, M32 = 0xFFFFFFFFll, S31 = 0x7FFFFFFFll;
constexpr int KIND_SET = 2, KIND_WEIGHT = 1;
constexpr float TIE = 1e-6f, W_ABS = 2e-5f, U_CHOICE = 4.f, U_WEIGHT = 6.f;
constexpr double W_REL = 1e-4;

struct RouteArgs {
  const void* logits;              // (m, E) fp32 / bf16 / fp16 (ldt 0 / 1 / 2), row stride sl
  int64_t sl;
  int ldt;
  const void* w;                   // (m, K) weights, fp32 / bf16 / fp16 (wdt), row stride sw
  int64_t sw;
  int wdt;
  const void* ids;                 // (m, K) expert ids, int32 / int64 (idt 0 / 1), row stride si
  int64_t si;
  int idt;
  const float* bias;               // (E) correction bias, or null
  int64_t m, E, K;
  int scoring, renorm, groups, topk_group;
  float scale, u;
  const int64_t* rows_buf;
  const int64_t* stepbuf;
  int64_t nl, idx;
  int64_t* state;                  // the router's COLS counters
  int64_t* cap_meta;               // the router's kept row: flag, row, step, kind, E, logits dtype
  float* cap_lg;                   // (E)
  int64_t* cap_ids;                // (K)
  float* cap_w;                    // (K)
};

__device__ __forceinline__ float load_val(const void* p, int t, int64_t i) {
  if (t == 0) return reinterpret_cast<const float*>(p)[i];
  const uint16_t h = reinterpret_cast<const uint16_t*>(p)[i];
  return t == 1 ? half_to_f32<SDC_BF16>(h) : half_to_f32<SDC_FP16>(h);
}

__device__ __forceinline__ float tol_of(float v, float u) {
  float a = fabsf(v);
  a = a == __builtin_inff() ? 0.f : a;
  return TIE * fmaxf(a, 1.f) + U_CHOICE * u * a;
}

// the larger of two (value, index) pairs; equal values: the smaller index (the first occurrence)
__device__ __forceinline__ void better(float& v, int& i, float ov, int oi) {
  if (ov > v || (ov == v && oi < i)) {
    v = ov;
    i = oi;
  }
}

__device__ __forceinline__ void wave_best(float& v, int& i) {
#pragma unroll
  for (int msk = 1; msk < 64; msk <<= 1) better(v, i, __shfl_xor(v, msk, 64), __shfl_xor(i, msk, 64));
}

// the smaller (value, index); equal values: the smaller index
__device__ __forceinline__ void wave_least(float& v, int& i) {
#pragma unroll
  for (int msk = 1; msk < 64; msk <<= 1) {
    const float ov = __shfl_xor(v, msk, 64);
    const int oi = __shfl_xor(i, msk, 64);
    if (ov < v || (ov == v && oi < i)) {
      v = ov;
      i = oi;
    }
  }
}

// The k-th largest of the n values vals[base + p * step] (p < n <= 64 * 32) held by one wave, counting equal values
// each: k rounds of the wave maximum, its first occurrence taken out (lane p % 64, bit p / 64 of its mask).
__device__ float wave_kth(const float* vals, int base, int step, int n, int k, int lane) {
  uint32_t gone = 0;
  float last = -__builtin_inff();
  for (int round = 0; round < k; ++round) {
    float v = -__builtin_inff();
    int i = 0x7FFFFFFF;
    for (int q = 0; lane + 64 * q < n; ++q)
      if (!(gone >> q & 1u)) better(v, i, vals[base + (lane + 64 * q) * step], lane + 64 * q);
    wave_best(v, i);
    last = v;
    if (i != 0x7FFFFFFF && i % 64 == lane) gone |= 1u << (i / 64);
  }
  return last;
}

__global__ __launch_bounds__(NT) void route_kernel(RouteArgs a) {
  __shared__ float sc[MAXE], ch[MAXE];          // the row's scores and choice scores
  __shared__ float redv[NW];
  __shared__ int redi[NW];
  __shared__ float gsc[MAXG], kwg[MAXG];        // per group: its score, its k-th best choice score
  __shared__ int gin[MAXG];                     // per group: bit 0 surely in, bit 1 may be in
  __shared__ float s_low, s_kth;
  __shared__ int s_won;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int64_t step = a.stepbuf[0] & M32;
  int64_t real = a.rows_buf[0];
  real = real < 0 ? 0 : (real > a.m ? a.m : real);
  if (!(real > 0 && step % a.nl == a.idx)) return;
  const int j = blockIdx.x;
  const int64_t row = ((step / a.nl) * ROW_A + j * ROW_B) % real;
  const int E = (int)a.E, K = (int)a.K, G = a.groups, TG = a.topk_group;
  const float NEG = -__builtin_inff();

  // ---- scores and choice scores
  float lgv[EPT];
  float mx = NEG;
#pragma unroll
  for (int q = 0; q < EPT; ++q) {
    const int e = t + NT * q;
    lgv[q] = e < E ? load_val(a.logits, a.ldt, row * a.sl + e) : NEG;
    mx = fmaxf(mx, lgv[q]);
  }
  float den = 1.f;
  if (a.scoring == 0) {
#pragma unroll
    for (int msk = 1; msk < 64; msk <<= 1) mx = fmaxf(mx, __shfl_xor(mx, msk, 64));
    if (lane == 0) redv[w] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(redv[0], redv[1]), fmaxf(redv[2], redv[3]));
    float sum = 0.f;
#pragma unroll
    for (int q = 0; q < EPT; ++q)
      if (t + NT * q < E) sum += expf(lgv[q] - mx);
#pragma unroll
    for (int msk = 1; msk < 64; msk <<= 1) sum += __shfl_xor(sum, msk, 64);
    __syncthreads();
    if (lane == 0) redv[w] = sum;
    __syncthreads();
    den = (redv[0] + redv[1]) + (redv[2] + redv[3]);
  }
#pragma unroll
  for (int q = 0; q < EPT; ++q) {
    const int e = t + NT * q;
    if (e < E) {
      const float s = a.scoring == 0 ? expf(lgv[q] - mx) / den : 1.f / (1.f + expf(-lgv[q]));
      sc[e] = s;
      ch[e] = a.bias ? s + a.bias[e] : s;
    }
  }
  __syncthreads();

  // ---- groups: scores, the k-th best within each, which are in
  const int gsz = G ? E / G : E;
  if (G) {
    for (int g = w; g < G; g += NW) {
      float m1 = NEG, m2 = NEG;
      int i1 = 0x7FFFFFFF, i2 = 0x7FFFFFFF;
      for (int p = lane; p < gsz; p += 64) better(m1, i1, ch[g * gsz + p], p);
      wave_best(m1, i1);
      float score = m1;
      if (a.bias) {
        for (int p = lane; p < gsz; p += 64)
          if (p != i1) better(m2, i2, ch[g * gsz + p], p);
        wave_best(m2, i2);
        score = m1 + m2;
      }
      const float kg = gsz >= K ? wave_kth(ch, g * gsz, 1, gsz, K, lane) : NEG;
      if (lane == 0) {
        gsc[g] = score;
        kwg[g] = kg;
      }
    }
    __syncthreads();
    if (w == 0) {
      // the topk_group-th best group score (the cut) and the next one, by rounds of the maximum over the groups
      const float gv = lane < G ? gsc[lane] : NEG;
      uint32_t out = 0;
      float gth = NEG, gnext = NEG;
      for (int round = 0; round <= TG; ++round) {
        float v = out ? NEG : gv;
        int i = lane < G && !out ? lane : 0x7FFFFFFF;
        wave_best(v, i);
        if (round < TG) {
          gth = v;
          if (i == lane) out = 1;
        } else {
          gnext = TG < G ? v : NEG;
        }
      }
      const float tolg = 2.f * tol_of(gth, a.u);
      const bool amb = gnext >= gth - tolg;
      const bool clear = lane < G && gv >= gth;
      const bool sure = amb ? (lane < G && gv > gth + tolg) : clear;
      const bool may = amb ? (lane < G && gv >= gth - tolg) : clear;
      if (lane < G) gin[lane] = (sure ? 1 : 0) | (may ? 2 : 0);
      // the topk_group-th smallest k-th best over the groups that may be in
      float kv = (lane < G && may) ? kwg[lane] : __builtin_inff();
      uint32_t used = 0;
      float low = __builtin_inff();
      for (int round = 0; round < TG; ++round) {
        float v = used ? __builtin_inff() : kv;
        int i = lane < G && !used ? lane : 0x7FFFFFFF;
        wave_least(v, i);
        low = v;
        if (i == lane) used = 1;
      }
      if (lane == 0) s_low = low;
    }
    __syncthreads();
  }

  // ---- the k-th best choice score over the experts of the groups surely in: k workgroup rounds
  {
    float cv[EPT];
#pragma unroll
    for (int q = 0; q < EPT; ++q) {
      const int e = t + NT * q;
      cv[q] = (e < E && (!G || (gin[e / gsz] & 1))) ? ch[e] : NEG;
    }
    float kth = NEG;
    for (int round = 0; round < K; ++round) {
      float v = NEG;
      int i = 0x7FFFFFFF;
#pragma unroll
      for (int q = 0; q < EPT; ++q) better(v, i, cv[q], t + NT * q);
      wave_best(v, i);
      if (lane == 0) {
        redv[w] = v;
        redi[w] = i;
      }
      __syncthreads();
      v = redv[0];
      i = redi[0];
#pragma unroll
      for (int q = 1; q < NW; ++q) better(v, i, redv[q], redi[q]);
      kth = v;
      if (i != 0x7FFFFFFF && i % NT == t) {
#pragma unroll
        for (int q = 0; q < EPT; ++q)
          if (q == i / NT) cv[q] = NEG;
      }
      __syncthreads();
    }
    if (t == 0) s_kth = kth;
  }
  __syncthreads();

  // ---- the router's choices (wave 0, one chosen expert a lane)
  if (w == 0) {
    const bool km = lane < K;
    int64_t id = -1;
    float kw = 0.f;
    if (km) {
      id = a.idt == 0 ? (int64_t)reinterpret_cast<const int32_t*>(a.ids)[row * a.si + lane]
                      : reinterpret_cast<const int64_t*>(a.ids)[row * a.si + lane];
      kw = load_val(a.w, a.wdt, row * a.sw + lane);
    }
    const bool valid = km && id >= 0 && id < E;
    const int kc = (int)(id < 0 ? 0 : (id >= E ? E - 1 : id));
    float bnd = s_kth;
    bool alk = km;
    if (G) {
      const int gk = kc / gsz;
      alk = km && (gin[gk] & 2);
      bnd = fmaxf(fmaxf(bnd, s_low), kwg[gk]);
    }
    const bool ok = valid && alk && ch[kc] >= bnd - tol_of(bnd, a.u);
    // a repeated id among the K
    bool dup = false;
    for (int q = 0; q < MAXK; ++q) {
      const int64_t o = __shfl((long long)id, q, 64);
      if (q < K && q < lane && km && o == id) dup = true;
    }
    const bool set_bad = __any((km && !ok) || dup);
    const bool pad = __all(!km || id == -1);
    const float sk = valid ? sc[kc] : 0.f;
    float ssum = km ? sk : 0.f;
#pragma unroll
    for (int msk = 1; msk < 64; msk <<= 1) ssum += __shfl_xor(ssum, msk, 64);
    float ref = a.renorm ? sk / (ssum + 1e-20f) : sk;
    ref = ref * a.scale;
    const float diff = valid ? fabsf(kw - ref) : 0.f;
    const float wrel = (float)((double)W_REL + (double)U_WEIGHT * (double)a.u);   // (summed in double, as stated)
    const bool wrong_w = valid && !(diff <= W_ABS + wrel * fabsf(ref));
    const bool w_bad = __any(wrong_w) && !set_bad;
    float worst = diff;
#pragma unroll
    for (int msk = 1; msk < 64; msk <<= 1) worst = fmaxf(worst, __shfl_xor(worst, msk, 64));
    unsigned long long* st = reinterpret_cast<unsigned long long*>(a.state);
    int won = 0;
    if (lane == 0) {
      if (j == 0) atomicAdd(st + C_CALLS, 1ull);
      if (!pad) {
        atomicAdd(st + C_ROWS, 1ull);
        const int kind = set_bad ? KIND_SET : (w_bad ? KIND_WEIGHT : 0);
        if (kind) {
          atomicAdd(st + (set_bad ? C_SET : C_WEIGHT), 1ull);
          atomicMax(st + C_LAST, (unsigned long long)(((step & S31) << 32) | ((int64_t)kind << 24) |
                                                      (row & 0xFFFFFF)));
          if (atomicCAS(reinterpret_cast<unsigned long long*>(a.cap_meta), 0ull, 1ull) == 0ull) {
            won = 1;
            a.cap_meta[1] = row;
            a.cap_meta[2] = step;
            a.cap_meta[3] = kind;
            a.cap_meta[4] = E;
            a.cap_meta[5] = a.ldt;
          }
        }
        atomicMax(st + C_WDIFF, (unsigned long long)(uint32_t)__float_as_uint(worst));
      }
      s_won = won;
    }
    if (__shfl(won, 0, 64) && km) {
      a.cap_ids[lane] = id;
      a.cap_w[lane] = kw;
    }
  }
  __syncthreads();
  if (s_won) {
    for (int e = t; e < E; e += NT) a.cap_lg[e] = load_val(a.logits, a.ldt, row * a.sl + e);
  }
}

}  // namespace

extern "C" int sdc_route_check(const void* logits, int64_t sl, int ldt, const void* weights, int64_t sw, int wdt,
                               const void* ids, int64_t si, int idt, const float* bias, int64_t m, int64_t E,
                               int64_t K, int scoring, int renormalize, int groups, int topk_group, float scale,
                               float u, const int64_t* rows_buf, const int64_t* stepbuf, int64_t nlayers,
                               int64_t index, int64_t* state_row, int64_t* cap_meta, float* cap_lg,
                               int64_t* cap_ids, float* cap_w, hipStream_t stream) {
  SDC_CLEAR_ERRORS();
  if (!logits || !weights || !ids || !rows_buf || !stepbuf || !state_row || !cap_meta || !cap_lg || !cap_ids ||
      !cap_w)
    return SDC_EINVAL;
  if (ldt < 0 || ldt > 2 || wdt < 0 || wdt > 2 || idt < 0 || idt > 1 || scoring < 0 || scoring > 1) return SDC_EINVAL;
  if (m < 1 || E < 1 || K < 1 || K > E || nlayers < 1 || index < 0 || sl < E || sw < K || si < K) return SDC_EINVAL;
  if (E > MAXE || K > MAXK) return SDC_EUNSUPPORTED;
  if (groups) {
    if (groups < 0 || groups > MAXG || E % groups || topk_group < 1 || topk_group > groups ||
        (int64_t)topk_group * (E / groups) < K)
      return SDC_EUNSUPPORTED;
    if (E / groups > 64 * 32) return SDC_EUNSUPPORTED;   // (a group's k-th best is taken by one wave)
    if (bias && E / groups < 2) return SDC_EUNSUPPORTED;  // (a biased group scores its two best)
  }
  RouteArgs a{};
  a.logits = logits; a.sl = sl; a.ldt = ldt; a.w = weights; a.sw = sw; a.wdt = wdt; a.ids = ids; a.si = si;
  a.idt = idt; a.bias = bias; a.m = m; a.E = E; a.K = K; a.scoring = scoring; a.renorm = renormalize;
  a.groups = groups; a.topk_group = groups ? topk_group : 0; a.scale = scale; a.u = u; a.rows_buf = rows_buf;
  a.stepbuf = stepbuf; a.nl = nlayers; a.idx = index; a.state = state_row; a.cap_meta = cap_meta;
  a.cap_lg = cap_lg; a.cap_ids = cap_ids; a.cap_w = cap_w;
  SdcProf prof("route_check", stream);
  hipLaunchKernelGGL(route_kernel, dim3(SAMPLES), dim3(NT), 0, stream, a);
  SDC_LAUNCH_CHECK();
  return SDC_OK;
}
