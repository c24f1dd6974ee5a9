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
// One workgroup per sample: the row's choice scores live in LDS, and the k-th bests come from places: an expert's
// place in its group is the number of its group's experts that come before it (larger, or equal at a smaller
// index, as top-k orders them), so the expert at place k - 1 holds the k-th best, equal scores counted each; the
// groups are placed the same way, and the k best of the groups surely in are placed among the k best of each.  The router's state row gets its counts and the packed last finding by atomics, and the first wrong row
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

// Wave reductions on DPP lane moves (quad swaps, then the half-row and row mirrors: every lane of a row of 16 holds
// the row's result) and four lane reads: no LDS round trips.  The whole wave must be active.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float rows_of_wave(float v, bool is_max) {
  const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return is_max ? fmaxf(fmaxf(a, b), fmaxf(c, d)) : (a + b) + (c + d);
}
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  v = fmaxf(v, dpp_f<0x141>(v));
  v = fmaxf(v, dpp_f<0x140>(v));
  return rows_of_wave(v, true);
}
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  v += dpp_f<0x141>(v);
  v += dpp_f<0x140>(v);
  return rows_of_wave(v, false);
}

// Whether value a (at index ia) comes before value b (at index ib) in top-k order: larger first, equal values by
// index, as the reference's sorts and top-k take them.  (Branch-free: a short-circuit form compiles to a branch per
// comparison.)
__device__ __forceinline__ int before(float a, int ia, float b, int ib) {
  return (int)(a > b) | ((int)(a == b) & (int)(ia < ib));
}

// The same order as one unsigned 64-bit key: the float's bits made monotonic (-0 counted as +0) above the index
// complemented, so a key above another comes before it.
__device__ __forceinline__ unsigned long long order_key(float v, int i) {
  const uint32_t u = __float_as_uint(v + 0.f);
  const uint32_t m = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((unsigned long long)m << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)i);
}

__global__ __launch_bounds__(NT) void route_kernel(RouteArgs a) {
  __shared__ __attribute__((aligned(16))) float sc[MAXE], ch[MAXE];   // the row's scores and choice scores
  __shared__ unsigned long long key[MAXE];      // the choice scores' order keys
  __shared__ unsigned short grank[MAXE];        // each expert's place within its group (0: the group's best)
  __shared__ unsigned long long ck[MAXE];       // per group and place < k: that expert's key
  __shared__ float red[NW];
  __shared__ float top1[MAXG], top2[MAXG], gsc[MAXG], kwg[MAXG];   // per group: its two best, score, k-th best
  __shared__ int gin[MAXG];                     // per group: bit 0 surely in, bit 1 may be in
  __shared__ float s_gth, s_gnext, s_low, s_kth, s_w[MAXK], s_d[MAXK];
  __shared__ int s_won;
  __shared__ long long s_id[MAXK];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int64_t step = a.stepbuf[0] & M32;
  int64_t real = a.rows_buf[0];
  real = real < 0 ? 0 : (real > a.m ? a.m : real);
  if (!(real > 0 && step % a.nl == a.idx)) return;
  const int j = blockIdx.x;
  const int64_t row = ((step / a.nl) * ROW_A + j * ROW_B) % real;
  const int E = (int)a.E, K = (int)a.K, G = a.groups, TG = a.topk_group;
  const int gsz = G ? E / G : E, NG = G ? G : 1;
  const float NEG = -__builtin_inff(), POS = __builtin_inff();

  // the router's choice for the row (wave 0, one chosen expert a lane), loaded now: it is judged at the end
  int64_t id = -1;
  float kw = 0.f;
  if (w == 0 && lane < K) {
    id = a.idt == 0 ? (int64_t)reinterpret_cast<const int32_t*>(a.ids)[row * a.si + lane]
                    : reinterpret_cast<const int64_t*>(a.ids)[row * a.si + lane];
    kw = load_val(a.w, a.wdt, row * a.sw + lane);
  }

  // ---- scores and choice scores
  float lgv[EPT];
  float mx = NEG;
#pragma unroll
  for (int q = 0; q < EPT; ++q) {
    const int e = t + NT * q;
    lgv[q] = e < E ? load_val(a.logits, a.ldt, row * a.sl + e) : NEG;
    mx = fmaxf(mx, lgv[q]);
  }
  if (t < MAXG) {
    top1[t] = NEG;
    top2[t] = NEG;
    kwg[t] = NEG;                               // (a group of fewer than k experts has no k-th best)
  }
  if (t == 0) {
    s_gth = NEG;
    s_gnext = NEG;
    s_low = POS;
    s_kth = NEG;
  }
  float den = 1.f;
  if (a.scoring == 0) {
    mx = wave_max(mx);
    if (lane == 0) red[w] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float sum = 0.f;
#pragma unroll
    for (int q = 0; q < EPT; ++q)
      if (t + NT * q < E) sum += expf(lgv[q] - mx);
    sum = wave_sum(sum);
    __syncthreads();
    if (lane == 0) red[w] = sum;
    __syncthreads();
    den = (red[0] + red[1]) + (red[2] + red[3]);
  }
#pragma unroll
  for (int q = 0; q < EPT; ++q) {
    const int e = t + NT * q;
    if (e < E) {
      const float s = a.scoring == 0 ? expf(lgv[q] - mx) / den : 1.f / (1.f + expf(-lgv[q]));
      sc[e] = s;
      const float c = a.bias ? s + a.bias[e] : s;
      ch[e] = c;
      key[e] = order_key(c, e);
    }
  }
  __syncthreads();

  // ---- each expert's place within its group (the whole row without groups): the experts of its group that come
  //      before it.  Its group's best, second best and k-th best are the experts at places 0, 1 and k - 1.
#pragma unroll
  for (int q = 0; q < EPT; ++q) {
    const int e = t + NT * q;
    if (e < E) {
      const float v = ch[e];
      const unsigned long long kv = key[e];
      const int g = e / gsz, b0 = g * gsz;
      int place = 0;
#pragma unroll 8
      for (int p = 0; p < gsz; ++p) place += (int)(key[b0 + p] > kv);
      grank[e] = (unsigned short)place;
      if (place == 0) top1[g] = v;
      if (place == 1) top2[g] = v;
      if (place == K - 1) kwg[g] = v;
      if (G && place < K) ck[g * K + place] = kv;
    }
  }
  __syncthreads();

  if (G) {
    // ---- groups: a group's score (its two best with a bias, its best without); the cut (the topk_group-th best
    //      score) and the next; which groups are surely in and which may be
    if (t < G) gsc[t] = a.bias ? top1[t] + top2[t] : top1[t];
    __syncthreads();
    if (t < G) {
      const float v = gsc[t];
      int place = 0;
      for (int h = 0; h < G; ++h) place += before(gsc[h], h, v, t);
      if (place == TG - 1) s_gth = v;
      if (place == TG) s_gnext = v;
    }
    __syncthreads();
    if (t < G) {
      const float gth = s_gth, v = gsc[t];
      const float tolg = 2.f * tol_of(gth, a.u);
      const bool amb = s_gnext >= gth - tolg;
      const bool clear = v >= gth;
      const bool sure = amb ? v > gth + tolg : clear;
      const bool may = amb ? v >= gth - tolg : clear;
      gin[t] = (sure ? 1 : 0) | (may ? 2 : 0);
    }
    __syncthreads();
    // the topk_group-th smallest k-th best over the groups that may be in
    if (t < G && (gin[t] & 2)) {
      const float v = kwg[t];
      int place = 0;
      for (int h = 0; h < G; ++h)
        if (gin[h] & 2) place += (int)(kwg[h] < v) | ((int)(kwg[h] == v) & (int)(h < t));
      if (place == TG - 1) s_low = v;
    }
  }

  // ---- the k-th best choice score over the experts of the groups surely in: only an expert among the k best of
  //      its group can be among the k best of several groups, so those candidates (held by group and place) are
  //      placed among themselves
  if (!G) {
    if (t == 0) s_kth = kwg[0];
  } else {
    const int per = gsz < K ? gsz : K;
    for (int c = t; c < G * K; c += NT) {
      const int g = c / K;
      if ((c % K) < per && (gin[g] & 1)) {
        const unsigned long long kv = ck[c];
        int place = 0;
        for (int h = 0; h < G; ++h)
          if (gin[h] & 1)
            for (int q = 0; q < per; ++q) place += (int)(ck[h * K + q] > kv);
        if (place == K - 1) s_kth = ch[0xFFFFFFFFu - (uint32_t)kv];
      }
    }
  }
  __syncthreads();

  // ---- the router's choices (wave 0, one chosen expert a lane)
  if (w == 0) {
    const bool km = lane < K;
    if (km) s_id[lane] = (long long)id;
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
    const float sk = valid ? sc[kc] : 0.f;
    if (km) s_w[lane] = sk;
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    // a repeated id among the k, and the chosen experts' scores added in order
    bool dup = false;
    float ssum = 0.f;
    for (int q = 0; q < K; ++q) {
      dup = dup || (km && q < lane && s_id[q] == (long long)id);
      ssum += s_w[q];
    }
    const bool set_bad = __any((km && !ok) || dup);
    const bool pad = __all(!km || id == -1);
    float ref = a.renorm ? sk / (ssum + 1e-20f) : sk;
    ref = ref * a.scale;
    const float diff = valid ? fabsf(kw - ref) : 0.f;
    const float wrel = (float)((double)W_REL + (double)U_WEIGHT * (double)a.u);   // (summed in double, as stated)
    const bool wrong_w = valid && !(diff <= W_ABS + wrel * fabsf(ref));
    const bool w_bad = __any(wrong_w) && !set_bad;
    if (km) s_d[lane] = diff;
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    unsigned long long* st = reinterpret_cast<unsigned long long*>(a.state);
    int won = 0;
    if (lane == 0) {
      float worst = 0.f;
      for (int q = 0; q < K; ++q) worst = fmaxf(worst, s_d[q]);
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
    if (__builtin_amdgcn_readfirstlane(won) && km) {
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
