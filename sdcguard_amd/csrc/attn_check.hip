// Sampled attention recompute from a paged KV cache, and the check of the sampled tokens' own KV writes.
//
// Reference: serve_attn.py:165-280 (`attn_check_torch`, the arithmetic), :292-327 (`_lower_bound`,
// `_attn_sample`: which (token, head) a sample takes), :335-407 (`_attn_part`), :414-571 (`_attn_judge`: the
// combine, the bound, the score, the 18-column state row, the capture, the KV-write check), :574-602
// (`attn_check_triton`, the boundary this replaces).
//
// One launch.  Sample j's keys lo..pos are split evenly over `nsplit` workgroups.  Inside a workgroup each wave
// walks tiles of keys: D/8 lanes share a key, each holding 8 of its dimensions, and read the key's K and V rows
// with one 16-byte load each through the block table (block bt[r, t / N], slot t % N); the q.k products and the
// |q|.|k| sums are added over those lanes with DPP steps.  Each lane group keeps an online softmax (running max,
// rescaled sums): sum p, sum p e, and per dimension sum p v, sum p |v|, sum p e |v|, sum |v|.  The groups and
// waves are combined in registers and LDS, then one record per workgroup goes to the workspace; the last
// workgroup of a sample to finish (an atomic counter, which it sets back to zero) combines the records with the
// log-sum-exp rescale, scores the sample against the first-order rounding bound and updates the layer's state row
// with atomics.  With one split per sample the workgroup judges directly.
#include <algorithm>
#include <atomic>
#include <mutex>

#include "common.h"
#include "profile.h"

namespace {

constexpr int NCOLS = 18;
constexpr int NCAPM = 12;
enum {
  C_ZT, C_ZH, C_ZD, C_ZO, C_ZR, C_ZS, C_ZP, C_CALLS, C_SAMPLES, C_SKIP, C_UNJ, C_BADBLK, C_KEYS, C_WN, C_WBAD,
  C_WSLOT, C_WLAST, C_WWHERE
};
enum { CM_CLAIM, CM_ROW, CM_HEAD, CM_REQ, CM_POS, CM_SL, CM_LO, CM_STEP, CM_Z, CM_KEPT, CM_DIM, CM_HK };

constexpr float TWO22 = 2.384185791015625e-07f;   // 2^-22
constexpr float TWO21 = 4.76837158203125e-07f;    // 2^-21
constexpr float NEG_INF = -__builtin_inff();
constexpr int BTCAP = 256;                        // block-table entries a workgroup holds in LDS
constexpr int QCAP = 1025;                        // query start locations a workgroup holds in LDS (1024 requests)

struct AttnArgs {
  const uint16_t* q; const uint16_t* o; const uint16_t* kv; const uint16_t* key; const uint16_t* val;
  const int32_t* qsl; const int32_t* seqlens; const int32_t* bt; const int64_t* slots; const int64_t* ctrl;
  float* ws; int32_t* cnt; int64_t* state; int32_t* capm; float* capq; float* capo; uint16_t* capkv;
  int32_t* capkvm;
  float* zdump;        // optional: every judged sample's per-dimension scores, (samples, D) fp32 (tests)
  int64_t T, R, W, NB, N, Hq, GQ, Hkv, D, SN;
  int64_t sqt, sqh, sot, soh, skb, skh, skn, skd, sbt, skt, skh2, svt, svh;
  int64_t slot, nl, idx, left, caprows, capw;
  float scale, g_qk, u, sig_o, hsig_p, line;
  int nsplit, has_write, keep_kv, nshift;     // nshift: log2(N) when N is a power of two, else -1
  int nsamp;                                  // samples (workgroups past nsamp * nsplit check the KV writes)
};

struct Sample {
  bool valid;
  int64_t i, r, pos, sl, hq;
};

// The smallest k in [0, n] with arr[k] >= x (arr non-decreasing with n + 1 entries; n when none of arr[0..n-1]
// is): serve_attn.py:292-304.
__device__ __forceinline__ int64_t lower_bound(const int32_t* arr, int64_t n, int64_t x) {
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if ((int64_t)arr[mid] >= x) hi = mid; else lo = mid + 1;
  }
  return lo;
}

// Sample j of the layer at a step: serve_attn.py:306-327 (even j: a token of the step; odd j: the newest token
// of a request; one number picks the token or request and the head together).
// qsl: the query start locations (R + 1 entries), read from LDS when the workgroup holds them.
__device__ __forceinline__ Sample pick_sample(const AttnArgs& a, int64_t step, int64_t j, const int32_t* qsl) {
  Sample s;
  const int64_t ntok = min((int64_t)qsl[a.R], a.T);
  const int64_t h = (step / a.nl) * 1000003ll + j * 7919ll + a.idx * 104729ll;
  const bool odd = (j & 1) != 0;
  int64_t i, pk;
  bool have;
  if (!odd) {
    pk = h % max(ntok * a.Hq, (int64_t)1);
    i = pk / a.Hq;
    have = ntok > 0;
  } else {
    const int64_t rreal = lower_bound(qsl, a.R, ntok);
    pk = h % max(rreal * a.Hq, (int64_t)1);
    const int64_t rq = min(pk / a.Hq, a.R - 1);
    i = (int64_t)qsl[rq + 1] - 1;
    have = ntok > 0 && rreal > 0;
  }
  i = min(max(i, (int64_t)0), a.T - 1);
  const int64_t r = min(max(lower_bound(qsl, a.R, i + 1) - 1, (int64_t)0), a.R - 1);
  const int64_t q0 = qsl[r], q1 = qsl[r + 1], sl = a.seqlens[r];
  const int64_t qlen = q1 - q0, pos = sl - qlen + (i - q0);
  s.valid = have && qlen > 0 && sl > 0 && pos >= 0 && pos < sl && sl <= a.W * a.N;
  s.i = i;
  s.r = r;
  s.pos = pos;
  s.sl = sl;
  s.hq = pk % a.Hq;
  return s;
}

// Sum over the LPT lanes that share a key (aligned groups of 2..32 lanes): DPP inside a row of 16, a swizzle
// across rows.
template <int LPT>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (LPT >= 2) v += dpp_xor1(v);
  if constexpr (LPT >= 4) v += dpp_xor2(v);
  if constexpr (LPT >= 8)
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));  // half mirror
  if constexpr (LPT >= 16)
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));  // row mirror
  if constexpr (LPT >= 32) v += __shfl_xor(v, 16, 64);
  return v;
}

// Eight 16-bit elements of one row (dims d0..d0+7) as floats; dims >= D read as 0.
template <int DT, bool VEC>
__device__ __forceinline__ void load8(const uint16_t* p, int64_t stride, int d0, int D, float* out) {
  if constexpr (VEC) {
    u32x4 w = {0u, 0u, 0u, 0u};
    if (d0 < D) w = *reinterpret_cast<const u32x4*>(p + d0);
    const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      out[2 * e] = lo_of<DT>(ww[e]);
      out[2 * e + 1] = hi_of<DT>(ww[e]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = (d0 + e < D) ? half_to_f32<DT>(p[(int64_t)(d0 + e) * stride]) : 0.f;
  }
}

template <int DT, bool VEC>
__device__ __forceinline__ u32x4 raw8(const uint16_t* p, int64_t stride, int d0, int D) {
  u32x4 w = {0u, 0u, 0u, 0u};
  if constexpr (VEC) {
    if (d0 < D) w = *reinterpret_cast<const u32x4*>(p + d0);
  } else {
    uint16_t h[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e] = (d0 + e < D) ? p[(int64_t)(d0 + e) * stride] : (uint16_t)0;
    w.x = h[0] | ((uint32_t)h[1] << 16);
    w.y = h[2] | ((uint32_t)h[3] << 16);
    w.z = h[4] | ((uint32_t)h[5] << 16);
    w.w = h[6] | ((uint32_t)h[7] << 16);
  }
  return w;
}

__device__ __forceinline__ void unpack8(u32x4 w, int dt, float* out) {
  const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    out[2 * e] = dt == SDC_BF16 ? bf16_lo(ww[e]) : f16_lo(ww[e]);
    out[2 * e + 1] = dt == SDC_BF16 ? bf16_hi(ww[e]) : f16_hi(ww[e]);
  }
}

__device__ __forceinline__ int64_t key_of(float z, int64_t low) {
  return ((int64_t)(uint32_t)__float_as_uint(z) << 32) | (low & 0xFFFFFFFFll);
}

// A split record's value stored, and read back, at the device's coherence point (agent-scope atomics).
__device__ __forceinline__ void publish(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float coherent_load(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The scalars of one record (workgroup partial): max score, sum p, sum p e, out-of-cache keys; then D values
// each of sum p v, sum p |v|, sum p e |v|, sum |v|.
template <int DP>
struct Lds {
  float m[4], l[4], le[4];
  int bad[4];
  float vec[4][4][DP];        // [wave][acc, A, acc_e, |v|][dim]
  float zmax[4];
  int zarg[4], nonfin[4];
  int mk[4], mv[4], fk[4], fv[4];
  float py, pr;
  int last, claim, keep;
  int bt[BTCAP];              // the block-table entries of the workgroup's keys, when they fit
  int qs[QCAP];               // the query start locations, when they fit
  float cw[64];               // (the combine) each split record's weight exp(m_c - M)
};

// The sampled token's own KV write (serve_attn.py:533-569): the cache slot its K and V went to, against the slot
// its position maps to, and their values against the step's keys and values.  Run by one workgroup of the sample
// (the last split's), before its keys, so it overlaps the other splits' work.
template <int DT, int DP>
__device__ void check_write(const AttnArgs& a, const Sample& s, Lds<DP>& sh, int64_t* sb, int64_t step, int D,
                            const int32_t* btr) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  if (a.has_write && s.i < a.SN) {
    const int64_t si = a.slots[s.i];
    if (si >= 0 && si < a.NB * a.N) {
      const int64_t want = (int64_t)btr[s.pos / a.N] * a.N + s.pos % a.N;
      const int64_t cblk = si / a.N, coff = si % a.N;
      const int64_t total = a.Hkv * D;
      int nbk = 0, nbv = 0, fk = 0x7FFFFFFF, fv = 0x7FFFFFFF;
#pragma unroll 4
      for (int64_t e = tid; e < total; e += 256) {       // (unrolled: several elements' loads in flight)
        const int64_t hh = e / D, dd = e % D;
        const uint16_t* cp = a.kv + cblk * a.skb + hh * a.skh + coff * a.skn;
        const bool bk = cp[dd * a.skd] != a.key[s.i * a.skt + hh * a.skh2 + dd];
        const bool bv = cp[(D + dd) * a.skd] != a.val[s.i * a.svt + hh * a.svh + dd];
        nbk += bk;
        nbv += bv;
        if (bk && e < fk) fk = (int)e;
        if (bv && e < fv) fv = (int)e;
      }
      nbk = wave_sum_i32_dpp(nbk);
      nbv = wave_sum_i32_dpp(nbv);
      fk = (int)(0x7FFFFFFFu - wave_max_u32_dpp(0x7FFFFFFFu - (uint32_t)fk));   // the first (smallest) element
      fv = (int)(0x7FFFFFFFu - wave_max_u32_dpp(0x7FFFFFFFu - (uint32_t)fv));
      if (lane == 0) {
        sh.mk[w] = nbk;
        sh.mv[w] = nbv;
        sh.fk[w] = fk;
        sh.fv[w] = fv;
      }
      __syncthreads();
      if (tid == 0) {
        int tk = 0, tv = 0, FK = 0x7FFFFFFF, FV = 0x7FFFFFFF;
        for (int ww = 0; ww < 4; ++ww) {
          tk += sh.mk[ww];
          tv += sh.mv[ww];
          FK = min(FK, sh.fk[ww]);
          FV = min(FV, sh.fv[ww]);
        }
        atomicAdd((unsigned long long*)(sb + C_WN), 1ull);
        const bool badc = tk + tv > 0, bads = si != want;
        if (badc || bads) {
          const int64_t big = total;
          const int64_t fk64 = FK == 0x7FFFFFFF ? big : FK, fv64 = FV == 0x7FFFFFFF ? big : FV;
          const bool isv = fk64 >= big;
          const int64_t first = isv ? fv64 : fk64;
          int64_t wh = ((first / D) << 12) | ((first % D) << 1) | (isv ? 1 : 0);
          const int64_t kind = (badc ? 1 : 0) | (bads ? 2 : 0);
          wh = badc ? wh : 0;
          if (badc) atomicAdd((unsigned long long*)(sb + C_WBAD), 1ull);
          if (bads) atomicAdd((unsigned long long*)(sb + C_WSLOT), 1ull);
          const int64_t s31 = (step & 0x7FFFFFFFll) << 32;
          atomicMax((unsigned long long*)(sb + C_WLAST), (unsigned long long)(s31 | s.i));
          atomicMax((unsigned long long*)(sb + C_WWHERE), (unsigned long long)(s31 | (kind << 28) | wh));
        }
      }
    }
  }
}

template <int DT, int DP, bool VEC>
__global__ __launch_bounds__(256) void attn_check_kernel(AttnArgs a) {
  constexpr int LPT = DP / 8;               // lanes per key
  constexpr int G = 64 / LPT;               // keys per wave-wide load
  constexpr int U = 4;                      // keys per lane group per tile
  constexpr int TOK = G * U;                // keys per wave per tile
  __shared__ Lds<DP> sh;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  // the query start locations into LDS with one round trip (the sample's binary searches then read LDS); their
  // loads go out beside the control word's
  const bool qs_lds = a.R + 1 <= QCAP;
  int32_t qv[(QCAP + 255) / 256];
#pragma unroll
  for (int u = 0; u < (QCAP + 255) / 256; ++u) {
    const int64_t i = tid + 256 * u;
    qv[u] = (qs_lds && i <= a.R) ? a.qsl[i] : 0;
  }
  const int64_t step = a.ctrl[0] & 0xFFFFFFFFll;
  const bool live = a.ctrl[1] != 0 && (step % a.nl) == a.idx;
  if (!live) return;
#pragma unroll
  for (int u = 0; u < (QCAP + 255) / 256; ++u) {
    const int64_t i = tid + 256 * u;
    if (qs_lds && i <= a.R) sh.qs[i] = qv[u];
  }
  __syncthreads();
  auto pick = [&](int64_t j) { return qs_lds ? pick_sample(a, step, j, sh.qs) : pick_sample(a, step, j, a.qsl); };
  int64_t* sb = a.state + a.slot * NCOLS;
  if ((int64_t)blockIdx.x >= (int64_t)a.nsamp * a.nsplit) {
    // a workgroup of its own per sample checks the sampled token's KV write, beside the splits' keys
    const int64_t sw = (int64_t)blockIdx.x - (int64_t)a.nsamp * a.nsplit;
    const Sample s = pick(sw);
    if (s.valid) check_write<DT, DP>(a, s, sh, sb, step, (int)a.D, a.bt + s.r * a.sbt);
    return;
  }
  const int64_t sj = blockIdx.x / a.nsplit, c = blockIdx.x - sj * a.nsplit;
  if (blockIdx.x == 0 && tid == 0) atomicAdd((unsigned long long*)(sb + C_CALLS), 1ull);
  const Sample s = pick(sj);
  if (!s.valid) {
    if (c == 0 && tid == 0) atomicAdd((unsigned long long*)(sb + C_SKIP), 1ull);
    return;
  }
  const int D = (int)a.D;
  const int64_t hk = s.hq / a.GQ;
  const int64_t lo = a.left >= 0 ? max(s.pos - a.left, (int64_t)0) : (int64_t)0;
  const int64_t nkeys = s.pos - lo + 1;
  const int64_t chunk = (nkeys + a.nsplit - 1) / a.nsplit;
  const int64_t t0 = lo + c * chunk;
  const int64_t t1 = min(t0 + chunk, s.pos + 1);
  const int cl = lane % LPT, g = lane / LPT, d0 = 8 * cl;
  const int32_t* btr = a.bt + s.r * a.sbt;
  const uint16_t* kvh = a.kv + hk * a.skh;
  auto block_of = [&](int64_t t) { return a.nshift >= 0 ? (t >> a.nshift) : t / a.N; };
  // the sampled row's output (what the judging workgroup compares) and q, loaded beside the block-table entries
  const float ov = tid < D ? half_to_f32<DT>(a.o[s.i * a.sot + s.hq * a.soh + tid]) : 0.f;
  float q8[8], qa8[8];
  load8<DT, false>(a.q + s.i * a.sqt + s.hq * a.sqh, 1, d0, D, q8);
  // the block-table entries of keys t0 .. t1 - 1 into LDS with one round trip (when they fit)
  const int64_t b_first = t1 > t0 ? block_of(t0) : 0;
  const int64_t nbt = t1 > t0 ? block_of(t1 - 1) - b_first + 1 : 0;
  const bool bt_lds = nbt <= BTCAP;
  if (bt_lds)
    for (int64_t i = tid; i < nbt; i += 256) sh.bt[i] = btr[b_first + i];

#pragma unroll
  for (int e = 0; e < 8; ++e) qa8[e] = fabsf(q8[e]);
  const float sc = a.scale, gq = a.g_qk * a.scale;
  __syncthreads();

  float m = NEG_INF, lsum = 0.f, le = 0.f;
  float acc[8], aa[8], ae[8], v1[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = aa[e] = ae[e] = v1[e] = 0.f;
  int bad = 0;

  // a tile: U keys of each lane group (G groups a wave): their K and V rows through the block table
  auto fetch = [&](int64_t tb, u32x4* kw, u32x4* vw, bool* in) {
#pragma unroll
    for (int uu = 0; uu < U; ++uu) {
      const int64_t t = tb + uu * G + g;
      in[uu] = t < t1;
      int64_t blk = 0, off = 0;
      if (in[uu]) {
        const int64_t bi = block_of(t);
        off = t - bi * a.N;
        blk = bt_lds ? sh.bt[bi - b_first] : btr[bi];
        const bool ok = blk >= 0 && blk < a.NB;
        bad |= !ok;
        blk = ok ? blk : 0;
      }
      const uint16_t* p = kvh + blk * a.skb + off * a.skn;
      kw[uu] = in[uu] ? raw8<DT, VEC>(p, a.skd, d0, D) : u32x4{0u, 0u, 0u, 0u};
      vw[uu] = in[uu] ? raw8<DT, VEC>(p + (int64_t)D * a.skd, a.skd, d0, D) : u32x4{0u, 0u, 0u, 0u};
    }
  };
  // the online softmax over a fetched tile
  auto consume = [&](const u32x4* kw, const u32x4* vw, const bool* in) {
    float s_[U], sa_[U];
    float mt = NEG_INF;
#pragma unroll
    for (int uu = 0; uu < U; ++uu) {
      float k8[8];
      unpack8(kw[uu], DT, k8);
      float dt = 0.f, da = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        dt = fmaf(q8[e], k8[e], dt);
        da = fmaf(qa8[e], fabsf(k8[e]), da);
      }
      dt = group_sum<LPT>(dt);
      da = group_sum<LPT>(da);
      s_[uu] = in[uu] ? dt * sc : NEG_INF;
      sa_[uu] = da;
      mt = fmaxf(mt, s_[uu]);
    }
    const float mn = fmaxf(m, mt);
    if (mn != NEG_INF) {
      const float corr = __expf(m - mn);
      lsum *= corr;
      le *= corr;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        acc[e] *= corr;
        aa[e] *= corr;
        ae[e] *= corr;
      }
      m = mn;
    }
#pragma unroll
    for (int uu = 0; uu < U; ++uu) {
      if (!in[uu]) continue;
      const float p = __expf(s_[uu] - m);
      const float ee = fmaf(gq, sa_[uu], fmaf(TWO22, fabsf(s_[uu]), TWO21));
      const float pe = p * ee;
      lsum += p;
      le += pe;
      float v8[8];
      unpack8(vw[uu], DT, v8);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float va = fabsf(v8[e]);
        acc[e] = fmaf(p, v8[e], acc[e]);
        aa[e] = fmaf(p, va, aa[e]);
        ae[e] = fmaf(pe, va, ae[e]);
        v1[e] += va;
      }
    }
  };
  // two tiles' buffers: the next tile's loads are in flight while this one is consumed
  {
    u32x4 ka[U], va[U], kb[U], vb[U];
    bool ia[U], ib[U];
    int64_t tb = t0 + (int64_t)w * TOK;
    const int64_t stride = 4 * TOK;
    if (tb < t1) fetch(tb, ka, va, ia);
    while (tb < t1) {
      if (tb + stride < t1) fetch(tb + stride, kb, vb, ib);
      consume(ka, va, ia);
      tb += stride;
      if (tb >= t1) break;
      if (tb + stride < t1) fetch(tb + stride, ka, va, ia);
      consume(kb, vb, ib);
      tb += stride;
    }
  }
  // the lane groups of the wave into group 0
#pragma unroll
  for (int off = LPT; off < 64; off <<= 1) {
    const float m2 = __shfl_xor(m, off, 64);
    const float mm = fmaxf(m, m2);
    const float c1 = mm == NEG_INF ? 1.f : __expf(m - mm), c2 = mm == NEG_INF ? 1.f : __expf(m2 - mm);
    lsum = lsum * c1 + __shfl_xor(lsum, off, 64) * c2;
    le = le * c1 + __shfl_xor(le, off, 64) * c2;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      acc[e] = acc[e] * c1 + __shfl_xor(acc[e], off, 64) * c2;
      aa[e] = aa[e] * c1 + __shfl_xor(aa[e], off, 64) * c2;
      ae[e] = ae[e] * c1 + __shfl_xor(ae[e], off, 64) * c2;
      v1[e] += __shfl_xor(v1[e], off, 64);
    }
    m = mm;
  }
  bad = __any(bad) ? 1 : 0;
  if (lane < LPT) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      sh.vec[w][0][d0 + e] = acc[e];
      sh.vec[w][1][d0 + e] = aa[e];
      sh.vec[w][2][d0 + e] = ae[e];
      sh.vec[w][3][d0 + e] = v1[e];
    }
  }
  if (lane == 0) {
    sh.m[w] = m;
    sh.l[w] = lsum;
    sh.le[w] = le;
    sh.bad[w] = bad;
  }
  __syncthreads();
  // the workgroup's record: thread d holds dimension d
  float M = sh.m[0];
  for (int ww = 1; ww < 4; ++ww) M = fmaxf(M, sh.m[ww]);
  float L = 0.f, LE = 0.f, RA = 0.f, RAA = 0.f, RAE = 0.f, RV = 0.f;
  int BAD = 0;
  const int d = tid;
  for (int ww = 0; ww < 4; ++ww) {
    const float cw = M == NEG_INF ? 1.f : __expf(sh.m[ww] - M);
    L += cw * sh.l[ww];
    LE += cw * sh.le[ww];
    BAD += sh.bad[ww];
    if (d < DP) {
      RA += cw * sh.vec[ww][0][d];
      RAA += cw * sh.vec[ww][1][d];
      RAE += cw * sh.vec[ww][2][d];
      RV += sh.vec[ww][3][d];
    }
  }
  if (a.nsplit > 1) {
    // Publish the record at the device's coherence point (agent-scope stores go past this XCD's L2), wait until
    // every store of the workgroup has completed, then count the split in.  The last split to count reads the
    // records back from the coherence point.  No L2 write-back or invalidation is needed: nothing here goes
    // through the non-coherent L2 lines another XCD may hold.
    const int64_t PW = 4 + 4 * (int64_t)DP;
    float* rec = a.ws + (sj * a.nsplit + c) * PW;
    if (d < DP) {
      publish(rec + 4 + d, RA);
      publish(rec + 4 + DP + d, RAA);
      publish(rec + 4 + 2 * DP + d, RAE);
      publish(rec + 4 + 3 * DP + d, RV);
    }
    if (tid == 0) {
      publish(rec, M);
      publish(rec + 1, L);
      publish(rec + 2, LE);
      publish(rec + 3, (float)BAD);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
      const int prev = __hip_atomic_fetch_add(a.cnt + sj, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      sh.last = prev == a.nsplit - 1;
      if (sh.last) __hip_atomic_store(a.cnt + sj, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);   // next call
    }
    __syncthreads();
    if (!sh.last) return;
    const float* base = a.ws + sj * a.nsplit * PW;
    // Every record's values in flight at once: thread t < nsplit reads record t's scalars; the 256 / DP threads
    // of dimension d (t % DP == d) read its four values of their share of the records, 32 records' loads at a
    // time.  Then the maximum, the weights exp(m_c - M) and the sums, records added in order.
    constexpr int TPD = 256 / DP;                               // threads per dimension (1, 2 or 4)
    constexpr int CH = 32;                                      // records a thread has in flight
    float sm = NEG_INF, sl = 0.f, sle = 0.f, sbad = 0.f;
    if (tid < a.nsplit) {
      const float* r = base + tid * PW;
      sm = coherent_load(r);
      sl = coherent_load(r + 1);
      sle = coherent_load(r + 2);
      sbad = coherent_load(r + 3);
    }
    const int dd = tid % DP, part = tid / DP;
    const int per = (a.nsplit + TPD - 1) / TPD;
    const int c_lo = part * per, c_hi = min(a.nsplit, c_lo + per);
    float va[CH][4];
    auto load_chunk = [&](int cb) {
#pragma unroll
      for (int u = 0; u < CH; ++u) {
        const bool in = cb + u < c_hi;
        const float* r = base + (in ? cb + u : 0) * PW + 4 + dd;
#pragma unroll
        for (int q = 0; q < 4; ++q) va[u][q] = in ? coherent_load(r + q * DP) : 0.f;
      }
    };
    load_chunk(c_lo);
    if (tid < a.nsplit) {
      sh.cw[tid] = sm;
      sh.vec[0][0][tid] = sl;
      sh.vec[0][1][tid] = sle;
      sh.vec[0][2][tid] = sbad;
    }
    __syncthreads();
    M = NEG_INF;
    for (int cc = 0; cc < a.nsplit; ++cc) M = fmaxf(M, sh.cw[cc]);
    L = LE = 0.f;
    BAD = 0;
    for (int cc = 0; cc < a.nsplit; ++cc) {
      const float mc = sh.cw[cc];
      const float cw = mc > NEG_INF ? __expf(mc - M) : 0.f;
      L += cw * sh.vec[0][0][cc];
      LE += cw * sh.vec[0][1][cc];
      BAD += sh.vec[0][2][cc] > 0.f ? 1 : 0;
    }
    float pa = 0.f, paa = 0.f, pae = 0.f, pv = 0.f;
    for (int cb = c_lo; cb < c_hi; cb += CH) {
      if (cb > c_lo) load_chunk(cb);
#pragma unroll
      for (int u = 0; u < CH; ++u) {
        if (cb + u >= c_hi) break;
        const float mc = sh.cw[cb + u];
        const float cw = mc > NEG_INF ? __expf(mc - M) : 0.f;
        pa += cw * va[u][0];
        paa += cw * va[u][1];
        pae += cw * va[u][2];
        pv += va[u][3];
      }
    }
    __syncthreads();                                            // (sh.vec is reused for the parts' sums)
    sh.vec[part][0][dd] = pa;
    sh.vec[part][1][dd] = paa;
    sh.vec[part][2][dd] = pae;
    sh.vec[part][3][dd] = pv;
    __syncthreads();
    RA = RAA = RAE = RV = 0.f;
    if (d < DP) {
#pragma unroll
      for (int pp = 0; pp < TPD; ++pp) {
        RA += sh.vec[pp][0][d];
        RAA += sh.vec[pp][1][d];
        RAE += sh.vec[pp][2][d];
        RV += sh.vec[pp][3][d];
      }
    }
  }

  // ---- judge (serve_attn.py:438-470): ref = acc / sum p, the bound, the score of every dimension
  const float inf = __builtin_inff();
  const float ref = RA / L, ra = fabsf(ref);
  const float gam = ((float)nkeys / 16.0f + 32.0f) * TWO22 + TWO22 * fabsf(M);
  const float bound = (2.0f * a.u + gam) * (RAA / L + ra) + (RAE + ra * LE) / L + a.hsig_p * RV / L + a.sig_o;
  float z = fabsf(ov - ref) / bound;
  z = z == z ? z : inf;
  z = d < D ? z : 0.f;
  const int nonfin = d < D && (ra != ra || ra == inf || bound != bound || bound == inf);
  if (a.zdump && d < D) a.zdump[sj * D + d] = z;
  // worst dimension (the first of equal scores) and any non-finite value, over the workgroup
  float bz = z;
  int bd = d < D ? d : 0x7FFFFFFF;
  for (int off = 32; off > 0; off >>= 1) {
    const float z2 = __shfl_xor(bz, off, 64);
    const int d2 = __shfl_xor(bd, off, 64);
    if (z2 > bz || (z2 == bz && d2 < bd)) { bz = z2; bd = d2; }
  }
  const int nf = __any(nonfin) ? 1 : 0;
  if (lane == 0) {
    sh.zmax[w] = bz;
    sh.zarg[w] = bd;
    sh.nonfin[w] = nf;
  }
  __syncthreads();
  float pz = sh.zmax[0];
  int pd = sh.zarg[0], anynf = sh.nonfin[0];
  for (int ww = 1; ww < 4; ++ww) {
    if (sh.zmax[ww] > pz || (sh.zmax[ww] == pz && sh.zarg[ww] < pd)) { pz = sh.zmax[ww]; pd = sh.zarg[ww]; }
    anynf |= sh.nonfin[ww];
  }
  if (d == pd) {
    sh.py = ov;
    sh.pr = ref;
  }
  const bool notfin = anynf || L != L || L <= 0.f || L == inf;
  if (tid == 0) sh.claim = 0;
  __syncthreads();
  if (BAD > 0) {
    if (tid == 0) atomicAdd((unsigned long long*)(sb + C_BADBLK), 1ull);
  } else if (notfin) {
    if (tid == 0) atomicAdd((unsigned long long*)(sb + C_UNJ), 1ull);
  } else {
    if (tid == 0) {
      atomicAdd((unsigned long long*)(sb + C_SAMPLES), 1ull);
      atomicAdd((unsigned long long*)(sb + C_KEYS), (unsigned long long)nkeys);
      if (pz > 0.f) {
        // (each column keeps the key of the largest score; no read of the row first, so no round trip)
        atomicMax((unsigned long long*)(sb + C_ZT), (unsigned long long)key_of(pz, s.i));
        atomicMax((unsigned long long*)(sb + C_ZH), (unsigned long long)key_of(pz, s.hq));
        atomicMax((unsigned long long*)(sb + C_ZD), (unsigned long long)key_of(pz, pd));
        atomicMax((unsigned long long*)(sb + C_ZO), (unsigned long long)key_of(pz, __float_as_uint(sh.py)));
        atomicMax((unsigned long long*)(sb + C_ZR), (unsigned long long)key_of(pz, __float_as_uint(sh.pr)));
        atomicMax((unsigned long long*)(sb + C_ZS), (unsigned long long)key_of(pz, step));
        atomicMax((unsigned long long*)(sb + C_ZP), (unsigned long long)key_of(pz, s.pos));
      }
      if (pz > a.line && a.capm) {
        int32_t* cb = a.capm + a.slot * NCAPM;
        if (atomicCAS(cb + CM_CLAIM, 0, 1) == 0) {
          cb[CM_ROW] = (int32_t)s.i;
          cb[CM_HEAD] = (int32_t)s.hq;
          cb[CM_REQ] = (int32_t)s.r;
          cb[CM_POS] = (int32_t)s.pos;
          cb[CM_SL] = (int32_t)s.sl;
          cb[CM_LO] = (int32_t)lo;
          cb[CM_STEP] = (int32_t)step;
          cb[CM_Z] = (int32_t)__float_as_uint(pz);
          cb[CM_DIM] = pd;
          cb[CM_HK] = (int32_t)hk;
          sh.claim = 1;
          sh.keep = 0;
          if (a.keep_kv && a.capkv && a.capkvm && nkeys <= a.caprows)
            sh.keep = atomicCAS(a.capkvm, 0, 1) == 0;
        }
      }
    }
    __syncthreads();
    if (sh.claim) {
      if (d < D) {
        a.capq[a.slot * a.capw + d] = half_to_f32<DT>(a.q[s.i * a.sqt + s.hq * a.sqh + d]);
        a.capo[a.slot * a.capw + d] = ov;
      }
      if (sh.keep) {                        // the keys and values it attended, exact, for the CPU recheck
        for (int64_t e = tid; e < nkeys * D; e += 256) {
          const int64_t t = lo + e / D, dd = e % D;
          int64_t blk = btr[t / a.N];
          blk = (blk >= 0 && blk < a.NB) ? blk : 0;
          const uint16_t* p = kvh + blk * a.skb + (t % a.N) * a.skn;
          uint16_t* dst = a.capkv + ((t - lo) * 2) * a.capw + dd;
          dst[0] = p[dd * a.skd];
          dst[a.capw] = p[(D + dd) * a.skd];
        }
        __threadfence();
        __syncthreads();
        if (tid == 0) {
          a.capkvm[1] = (int32_t)a.slot;
          a.capkvm[2] = (int32_t)nkeys;
          a.capkvm[3] = (int32_t)step;
          a.capm[a.slot * NCAPM + CM_KEPT] = 1;
        }
      }
    }
  }
}

template <int DT, int DP>
int launch_dp(const AttnArgs& a, int vec, unsigned grid, hipStream_t stream) {
  if (vec)
    hipLaunchKernelGGL((attn_check_kernel<DT, DP, true>), dim3(grid), dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((attn_check_kernel<DT, DP, false>), dim3(grid), dim3(256), 0, stream, a);
  return SDC_OK;
}

template <int DT>
int launch_dt(const AttnArgs& a, int dp, int vec, unsigned grid, hipStream_t stream) {
  if (dp == 64) return launch_dp<DT, 64>(a, vec, grid, stream);
  if (dp == 128) return launch_dp<DT, 128>(a, vec, grid, stream);
  return launch_dp<DT, 256>(a, vec, grid, stream);
}

int64_t pad_dim(int64_t D) { return D <= 64 ? 64 : D <= 128 ? 128 : 256; }

}  // namespace

// Workspace layout: per-sample counters first, at a fixed place (COUNTER_BYTES: up to MAX_SAMPLES samples), so a
// buffer reused with another sample or split count still finds them at zero; then one record per workgroup.
constexpr int64_t MAX_SAMPLES = 1024;
constexpr int64_t COUNTER_BYTES = MAX_SAMPLES * (int64_t)sizeof(int32_t);

// Workgroups per sample: enough that a long context spreads over the chip (about 64 keys each: one tile a wave),
// at most 64, and at most 1024 workgroups in all.
extern "C" int64_t sdc_attn_splits(int64_t samples, int64_t max_keys) {
  if (samples <= 0 || max_keys <= 0) return 1;
  const int64_t cap = std::max<int64_t>(1, 1024 / samples);
  const int64_t s = std::min<int64_t>(sdc_cdiv(max_keys, 64), cap);
  return std::max<int64_t>(1, std::min<int64_t>(s, 64));
}

extern "C" int64_t sdc_attn_check_workspace(int64_t samples, int64_t max_keys, int64_t head_size) {
  if (samples <= 0 || head_size <= 0) return 0;
  const int64_t nsplit = sdc_attn_splits(samples, max_keys);
  const int64_t dp = pad_dim(head_size);
  return 256 + COUNTER_BYTES + samples * nsplit * (4 + 4 * dp) * (int64_t)sizeof(float);
}

#define SDC_ATTN_PARAMS                                                                                          \
  int dtype, const void *q, int64_t sqt, int64_t sqh, const void *o, int64_t sot, int64_t soh, int64_t T,          \
      int64_t Hq, int64_t D, const void *kv, int64_t skb, int64_t skh, int64_t skn, int64_t skd, int64_t NB,       \
      int64_t Hkv, int64_t N, const void *key, int64_t skt, int64_t skh2, const void *val, int64_t svt,            \
      int64_t svh, const int32_t *qsl, const int32_t *seq_lens, int64_t R, const int32_t *bt, int64_t sbt,         \
      int64_t W, const int64_t *slots, int64_t SN, int64_t *state, int64_t slot, const int64_t *ctrl, int64_t nl,  \
      int64_t idx, float scale, int64_t left, float line, int32_t *capm, float *capq, float *capo, int64_t capw,   \
      void *capkv, int32_t *capkvm, int64_t caprows, int samples
#define SDC_ATTN_ARGS                                                                                            \
  dtype, q, sqt, sqh, o, sot, soh, T, Hq, D, kv, skb, skh, skn, skd, NB, Hkv, N, key, skt, skh2, val, svt, svh,    \
      qsl, seq_lens, R, bt, sbt, W, slots, SN, state, slot, ctrl, nl, idx, scale, left, line, capm, capq, capo,    \
      capw, capkv, capkvm, caprows, samples

static int attn_check_impl(SDC_ATTN_PARAMS, void* workspace, int64_t workspace_bytes, int has_write, int keep_kv,
                           float* scores_out, hipStream_t stream) {
  if (dtype != SDC_BF16 && dtype != SDC_FP16) return SDC_EINVAL;
  if (T <= 0 || Hq <= 0 || Hkv <= 0 || D <= 0 || N <= 0 || R <= 0 || W <= 0 || NB <= 0) return SDC_EINVAL;
  if (Hq % Hkv != 0) return SDC_EINVAL;
  if (D > 256) return SDC_EUNSUPPORTED;                       // serve_attn.why_not: head sizes up to 256
  if (R > 65535) return SDC_EUNSUPPORTED;                     // MAX_REQUESTS (serve_attn.py:80)
  if (samples < 1 || samples > MAX_SAMPLES || nl < 1 || idx < 0) return SDC_EINVAL;
  if (!q || !o || !kv || !qsl || !seq_lens || !bt || !state || !ctrl) return SDC_EINVAL;
  if (has_write && (!key || !val || !slots || SN < 0)) return SDC_EINVAL;
  if (capm && (!capq || !capo || capw < D)) return SDC_EINVAL;
  if (keep_kv && capkv && (!capkvm || caprows < 0 || capw < D)) return SDC_EINVAL;
  const int64_t dp = pad_dim(D);
  const int64_t nsplit = sdc_attn_splits(samples, W * N);
  if (nsplit > 1 && (!workspace || workspace_bytes < sdc_attn_check_workspace(samples, W * N, D)))
    return SDC_EWORKSPACE;
  AttnArgs a;
  a.q = (const uint16_t*)q; a.o = (const uint16_t*)o; a.kv = (const uint16_t*)kv;
  a.key = (const uint16_t*)key; a.val = (const uint16_t*)val;
  a.qsl = qsl; a.seqlens = seq_lens; a.bt = bt; a.slots = slots; a.ctrl = ctrl;
  char* wsb = (char*)(((uintptr_t)workspace + 255) & ~(uintptr_t)255);
  a.cnt = workspace ? (int32_t*)wsb : nullptr;
  a.ws = workspace ? (float*)(wsb + COUNTER_BYTES) : nullptr;
  a.zdump = scores_out;
  a.state = state; a.capm = capm; a.capq = capq; a.capo = capo; a.capkv = (uint16_t*)capkv; a.capkvm = capkvm;
  a.T = T; a.R = R; a.W = W; a.NB = NB; a.N = N; a.Hq = Hq; a.GQ = Hq / Hkv; a.Hkv = Hkv; a.D = D;
  a.SN = has_write ? SN : 0;
  a.sqt = sqt; a.sqh = sqh; a.sot = sot; a.soh = soh; a.skb = skb; a.skh = skh; a.skn = skn; a.skd = skd;
  a.sbt = sbt; a.skt = skt; a.skh2 = skh2; a.svt = svt; a.svh = svh;
  a.slot = slot; a.nl = nl; a.idx = idx; a.left = left; a.caprows = caprows; a.capw = capw;
  const double u = dtype == SDC_BF16 ? 1.0 / 256.0 : 1.0 / 2048.0;            // serve_norm.dtype_consts
  a.scale = scale;
  a.g_qk = (float)((double)(D + 8) * 1.1920928955078125e-07);                  // (D + 8) 2^-23
  a.u = (float)u;
  a.sig_o = dtype == SDC_BF16 ? 1e-37f : 5.9604644775390625e-08f;             // output spacing
  a.hsig_p = dtype == SDC_BF16 ? 1.1754943508222875e-38f : 2.9802322387695312e-08f;   // p_spacing
  a.line = line;
  a.nsplit = (int)nsplit;
  a.has_write = has_write != 0;
  a.keep_kv = keep_kv != 0 && capkv != nullptr;
  a.nshift = (N & (N - 1)) == 0 ? __builtin_ctzll((unsigned long long)N) : -1;
  const int vec = skd == 1 && D % 8 == 0 && skb % 8 == 0 && skh % 8 == 0 && skn % 8 == 0 &&
                  ((uintptr_t)kv % 16) == 0;
  a.nsamp = samples;
  const unsigned grid = (unsigned)(samples * nsplit + (has_write ? samples : 0));
  SdcProf prof("attn_check", stream);
  if (dtype == SDC_BF16)
    launch_dt<SDC_BF16>(a, (int)dp, vec, grid, stream);
  else
    launch_dt<SDC_FP16>(a, (int)dp, vec, grid, stream);
  SDC_LAUNCH_CHECK();
  return SDC_OK;
}

extern "C" int sdc_attn_check(SDC_ATTN_PARAMS, void* workspace, int64_t workspace_bytes, int has_write, int keep_kv,
                              float* scores_out, hipStream_t stream) {
  SDC_CLEAR_ERRORS();
  return attn_check_impl(SDC_ATTN_ARGS, workspace, workspace_bytes, has_write, keep_kv, scores_out, stream);
}

// ---- the same check without a workspace argument, for callers that cannot allocate -------------------------------
// The workspace lives in `scratch`, a static device array: each GPU the library runs on holds its own copy until the
// process ends.  SCRATCH_BYTES covers every call the check accepts (at most 1024 sample x split records of a head
// size up to 256, plus the counters).  Its counters are cleared once per device, at the first call there, by a fill
// kernel on the caller's stream (no memset node, so the call can be captured in a graph); every call leaves them at
// zero again.  Calls on one GPU share the array: calls that overlap in time (other streams, other host threads)
// race and must not be made.
constexpr int64_t SCRATCH_BYTES = 4456448;        // 4.25 MiB
static __device__ __align__(256) unsigned char scratch[SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::atomic<void*> g_scratch[MAX_DEVICES];
std::mutex g_scratch_mu;

__global__ void clear_counters_kernel(int32_t* cnt, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    cnt[i] = 0;
}

// The device address of this device's scratch array (set up at the first call on the device, which must be the
// current device), or an error status.
static int scratch_of_current_device(void** out, hipStream_t stream) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    sdc_note_error(e);
    return SDC_ELAUNCH;
  }
  if (dev < 0 || dev >= MAX_DEVICES) return SDC_EUNSUPPORTED;
  void* p = g_scratch[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (!p) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !p) {
        sdc_note_error(e != hipSuccess ? e : hipErrorInvalidSymbol);
        return SDC_ELAUNCH;
      }
      hipLaunchKernelGGL(clear_counters_kernel, dim3(4), dim3(256), 0, stream, (int32_t*)p,
                         COUNTER_BYTES / (int64_t)sizeof(int32_t));
      e = hipGetLastError();
      if (e != hipSuccess) {
        sdc_note_error(e);
        return SDC_ELAUNCH;
      }
      g_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return SDC_OK;
}

extern "C" int sdc_attn_check_noalloc(SDC_ATTN_PARAMS, int has_write, int keep_kv, float* scores_out,
                                      hipStream_t stream) {
  SDC_CLEAR_ERRORS();
  if (samples < 1 || samples > MAX_SAMPLES || D <= 0 || W <= 0 || N <= 0) return SDC_EINVAL;
  if (sdc_attn_check_workspace(samples, W * N, D) > SCRATCH_BYTES) return SDC_EWORKSPACE;
  void* ws = nullptr;
  const int rc = scratch_of_current_device(&ws, stream);
  if (rc != SDC_OK) return rc;
  return attn_check_impl(SDC_ATTN_ARGS, ws, SCRATCH_BYTES, has_write, keep_kv, scores_out, stream);
}
