// Integer fingerprints of raw tensor bits: bit-exact, order-independent (sums mod 2^64).
//
//   fp3 (recompute.fingerprint; recompute.py:59-116, _fingerprint.py:51-65): words b = signed int16 (int8 for
//       1-byte tensors), weights w1 = z | 1, w2 = (z ^ z>>>32) | 1 with z = splitmix64's mix of (p + SEED);
//       sums (b, b*w1, b*w2).
//   fp2 (serve_weights.fingerprint; serve_weights.py:73-86, :151-185): words x = int16 / int32 / uint8, key
//       k(i) = fmix64(i ^ KEY_SEED); sums (x, x*k).
//
// One pass, 16 bytes per lane per load, grid-stride; each thread keeps its sums in registers, a wave adds
// them with shuffles and one lane per wave adds them into the output with 64-bit atomics (wrapping addition,
// so the result is exact whatever the order).
#include <atomic>
#include <mutex>
#include <type_traits>

#include "common.h"
#include "profile.h"

namespace {

constexpr uint64_t FP_SEED = 0x9E3779B97F4A7C15ull;
constexpr uint64_t FP_M1 = 0xBF58476D1CE4E5B9ull;
constexpr uint64_t FP_M2 = 0x94D049BB133111EBull;
constexpr uint64_t KEY_SEED = 0x2545F4914F6CDD1Dull;
constexpr uint64_t MIX1 = 0xFF51AFD7ED558CCDull;
constexpr uint64_t MIX2 = 0xC4CEB9FE1A85EC53ull;

__device__ __forceinline__ uint64_t fp3_z(uint64_t p) {
  uint64_t z = p + FP_SEED;
  z = (z ^ (z >> 30)) * FP_M1;
  z = (z ^ (z >> 27)) * FP_M2;
  return z ^ (z >> 31);
}

__device__ __forceinline__ uint64_t fmix_key(uint64_t i) {
  uint64_t h = i ^ KEY_SEED;
  h = (h ^ (h >> 33)) * MIX1;
  h = (h ^ (h >> 33)) * MIX2;
  return h ^ (h >> 33);
}

struct Acc3 { uint64_t s0, s1, s2; };

__device__ __forceinline__ void fp3_word(Acc3& a, int64_t b, uint64_t p) {
  const uint64_t z = fp3_z(p);
  const uint64_t ub = (uint64_t)b;
  a.s0 += ub;
  a.s1 += ub * (z | 1ull);
  a.s2 += ub * ((z ^ (z >> 32)) | 1ull);
}

__device__ __forceinline__ void flush3(Acc3 a, int64_t* out) {
  int64_t s0 = wave_sum_i64((int64_t)a.s0), s1 = wave_sum_i64((int64_t)a.s1), s2 = wave_sum_i64((int64_t)a.s2);
  if ((threadIdx.x & 63) == 0) {
    atomicAdd((unsigned long long*)out, (unsigned long long)s0);
    atomicAdd((unsigned long long*)(out + 1), (unsigned long long)s1);
    atomicAdd((unsigned long long*)(out + 2), (unsigned long long)s2);
  }
}

// WB: word bytes (2: int16, 1: int8).  `n` words from `X` (16-byte aligned), positions from `start`.
template <int WB>
__global__ __launch_bounds__(256) void fp3_kernel(const uint8_t* __restrict__ X, int64_t n, int64_t start,
                                                  int64_t* __restrict__ out) {
  constexpr int PER = 16 / WB;                       // words per 16-byte load
  Acc3 acc = {0, 0, 0};
  const int64_t nvec = n / PER;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nvec; i += stride) {
    u32x4 v = *reinterpret_cast<const u32x4*>(X + i * 16);
    uint32_t wv[4] = {v.x, v.y, v.z, v.w};
    const uint64_t p0 = (uint64_t)(start + i * PER);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (WB == 2) {
        fp3_word(acc, (int64_t)(int16_t)(wv[j] & 0xFFFFu), p0 + 2 * j);
        fp3_word(acc, (int64_t)(int16_t)(wv[j] >> 16), p0 + 2 * j + 1);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) fp3_word(acc, (int64_t)(int8_t)((wv[j] >> (8 * e)) & 0xFFu), p0 + 4 * j + e);
      }
    }
  }
  // tail words (fewer than one load)
  const int64_t tail0 = nvec * PER;
  if (blockIdx.x == 0 && threadIdx.x < n - tail0) {
    const int64_t i = tail0 + threadIdx.x;
    int64_t b = WB == 2 ? (int64_t)((const int16_t*)X)[i] : (int64_t)((const int8_t*)X)[i];
    fp3_word(acc, b, (uint64_t)(start + i));
  }
  flush3(acc, out);
}

// element-wise variant for unaligned data
template <int WB>
__global__ __launch_bounds__(256) void fp3_scalar_kernel(const uint8_t* __restrict__ X, int64_t n, int64_t start,
                                                         int64_t* __restrict__ out) {
  Acc3 acc = {0, 0, 0};
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    int64_t b = WB == 2 ? (int64_t)((const int16_t*)X)[i] : (int64_t)((const int8_t*)X)[i];
    fp3_word(acc, b, (uint64_t)(start + i));
  }
  flush3(acc, out);
}

// fp2: KIND 0 = int16, 1 = int32, 2 = uint8
template <int KIND>
__global__ __launch_bounds__(256) void fp2_kernel(const uint8_t* __restrict__ X, int64_t n, int64_t* __restrict__ out) {
  uint64_t s0 = 0, s1 = 0;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  constexpr int WB = KIND == 0 ? 2 : KIND == 1 ? 4 : 1;
  constexpr int PER = 16 / WB;
  const bool aligned = ((uintptr_t)X % 16) == 0;
  const int64_t nvec = aligned ? n / PER : 0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nvec; i += stride) {
    u32x4 v = *reinterpret_cast<const u32x4*>(X + i * 16);
    uint32_t wv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int e = 0; e < 4 / WB; ++e) {
        int64_t xv;
        if constexpr (KIND == 0) xv = (int16_t)((wv[j] >> (16 * e)) & 0xFFFFu);
        else if constexpr (KIND == 1) xv = (int32_t)wv[j];
        else xv = (int64_t)((wv[j] >> (8 * e)) & 0xFFu);
        const uint64_t pos = (uint64_t)(i * PER + j * (4 / WB) + e);
        s0 += (uint64_t)xv;
        s1 += (uint64_t)xv * fmix_key(pos);
      }
    }
  }
  for (int64_t i = nvec * PER + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    int64_t xv;
    if constexpr (KIND == 0) xv = ((const int16_t*)X)[i];
    else if constexpr (KIND == 1) xv = ((const int32_t*)X)[i];
    else xv = ((const uint8_t*)X)[i];
    s0 += (uint64_t)xv;
    s1 += (uint64_t)xv * fmix_key((uint64_t)i);
  }
  int64_t a = wave_sum_i64((int64_t)s0), b = wave_sum_i64((int64_t)s1);
  if ((threadIdx.x & 63) == 0) {
    atomicAdd((unsigned long long*)out, (unsigned long long)a);
    atomicAdd((unsigned long long*)(out + 1), (unsigned long long)b);
  }
}

unsigned grid_for(int64_t work_items) {
  int64_t g = sdc_cdiv(work_items, 256);
  if (g > 4096) g = 4096;
  if (g < 1) g = 1;
  return (unsigned)g;
}


// Paged-KV block fingerprints: fp3 of every block of a paged cache, each block's words numbered from 0 (what
// recompute.fingerprint gives the block as a tensor of its own).  The weights depend only on the position in the
// block, so a wave owns one slice of KV_SLICE positions (16 words per lane) of every block it visits and keeps its
// weights in registers while it streams blocks.  The products run on packed 16-bit dot products
// (v_dot2c_i32_i16, two words per instruction): with w = lo + 2^32 hi (lo the signed low half, hi the high half
// plus lo's sign bit), b w mod 2^64 = b lo + 2^32 (b hi mod 2^32), where lo is taken as three balanced 12-bit
// digits (b times a digit summed over 16 words stays exact in 32 bits) and hi as two balanced 16-bit digits whose
// sums may wrap (only hi's value mod 2^32 counts).  Each wave adds its lanes' sums (DPP steps, then two shuffles)
// and three of its lanes add them into the block's three outputs with 64-bit atomics (wrapping, so the result does
// not depend on the order).  Four blocks are in flight per wave.
// A cache of 1-byte elements has int8 words (recompute.py:86-87): a lane's 16 words are one 16-byte load; each
// byte is taken as u = v + 128 (its sign bit flipped), zero-extended into a 16-bit lane of the same dot products,
// and the lane subtracts 128 times the sum of its positions' weights (made once, mod 2^64) from its sums.
constexpr int KV_WPT = 16;                       // words per lane
constexpr int KV_SLICE = 64 * KV_WPT;            // positions per wave slice
constexpr int KV_UNROLL = 4;                     // (grid sizing) blocks per wave and round
constexpr int KV_BUF = 3;                        // blocks per register buffer (two buffers in flight)

struct KvArgs {
  const uint8_t* cache;
  int64_t block_bytes, words, nblocks;           // nblocks: valid block ids are 0 .. nblocks - 1
  const int64_t* ids;                            // block of entry i (null: entry i is block i); < 0: no block
  int64_t n;
  int64_t* out;                                  // [n][3]
  int vec;
};

typedef short short2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ int dot16(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot2(__builtin_bit_cast(short2_t, a), __builtin_bit_cast(short2_t, b), c, false);
}

// the balanced digit of v in base 2^bits (in [-2^(bits-1), 2^(bits-1))), as the low 16 bits of a word
__device__ __forceinline__ int32_t bdigit(int64_t v, int bits) {
  const int64_t h = 1ll << (bits - 1);
  return (int32_t)(((v + h) & ((1ll << bits) - 1)) - h);
}

// a weight's five digits at position p: three of lo (12 bits each), two of hi (16 bits)
__device__ __forceinline__ void weight_digits(uint64_t w, int32_t* d) {
  const int64_t lo = (int32_t)(uint32_t)w;
  const uint32_t hi = (uint32_t)(w >> 32) + ((uint32_t)w >> 31);
  d[0] = bdigit(lo, 12);
  const int64_t r1 = (lo - d[0]) >> 12;
  d[1] = bdigit(r1, 12);
  d[2] = (int32_t)((r1 - d[1]) >> 12);
  d[3] = bdigit((int64_t)hi, 16);
  d[4] = (int16_t)(uint16_t)(((uint32_t)hi - (uint32_t)d[3]) >> 16);
}

__device__ __forceinline__ uint32_t pack16(int32_t a, int32_t b) {
  return ((uint32_t)a & 0xFFFFu) | ((uint32_t)b << 16);
}

// v plus its DPP partner's value (64-bit wrapping)
template <int CTL>
__device__ __forceinline__ uint64_t dpp_add_u64(uint64_t v) {
  const uint32_t lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTL, 0xF, 0xF, false);
  const uint32_t hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), CTL, 0xF, 0xF, false);
  return v + (((uint64_t)hi << 32) | lo);
}

// sum over the wave, 64-bit wrapping: four DPP steps inside each row of 16 lanes (quad xor 1, quad xor 2, half-row
// mirror, row mirror; no LDS), then two shuffles across rows
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
  v = dpp_add_u64<0xB1>(v);
  v = dpp_add_u64<0x4E>(v);
  v = dpp_add_u64<0x141>(v);
  v = dpp_add_u64<0x140>(v);
  v += (uint64_t)shfl_xor_i64((int64_t)v, 16);
  v += (uint64_t)shfl_xor_i64((int64_t)v, 32);
  return v;
}

constexpr int KV_WAVES = 4;                      // waves per workgroup: KV_WAVES slices of one block range

template <int WB>
__global__ __launch_bounds__(64 * KV_WAVES) void kv_fp3_kernel(KvArgs a, const int64_t* ids) {
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  // the lane's words: two runs of KV_WPT / 2 at p0 and p0 + KV_SLICE / 2, so that each of a wave's two loads per
  // block reads one contiguous run (2-byte words: 1 KB; whole lines per instruction)
  const int64_t p0 = ((int64_t)blockIdx.x * KV_WAVES + w) * KV_SLICE + (int64_t)lane * (KV_WPT / 2);
  auto pos_of = [&](int q) -> int64_t {                         // position of the lane's word q (0 .. KV_WPT - 1)
    return p0 + (q < KV_WPT / 2 ? q : KV_SLICE / 2 + q - KV_WPT / 2);
  };
  // dg[j][c][d]: word pair j (the lane's words 2j, 2j + 1), weight c, digit d, packed for the dot products
  uint32_t dg[KV_WPT / 2][2][5];
#pragma unroll
  for (int j = 0; j < KV_WPT / 2; ++j) {
    int32_t e0[2][5], e1[2][5];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint64_t z = fp3_z((uint64_t)pos_of(2 * j + h));
      weight_digits(z | 1ull, h ? e1[0] : e0[0]);
      weight_digits((z ^ (z >> 32)) | 1ull, h ? e1[1] : e0[1]);
    }
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int d = 0; d < 5; ++d) dg[j][c][d] = pack16(e0[c][d], e1[c][d]);
  }
  // the lane's words that fall inside the block (bit q: word q)
  uint32_t valid = 0;
#pragma unroll
  for (int q = 0; q < KV_WPT; ++q) valid |= (pos_of(q) < a.words ? 1u : 0u) << q;
  const int nw = __builtin_popcount(valid);
  const bool full = a.vec && nw == KV_WPT;
  // 1-byte words: 128 x the sums of this lane's weights over its positions (the offset of u = v + 128)
  uint64_t corr[2] = {0ull, 0ull};
  if constexpr (WB == 1) {
    for (int q = 0; q < KV_WPT; ++q) {
      if (pos_of(q) >= a.words) continue;
      const uint64_t z = fp3_z((uint64_t)pos_of(q));
      corr[0] += (z | 1ull) << 7;
      corr[1] += ((z ^ (z >> 32)) | 1ull) << 7;
    }
  }
  const int64_t off1 = (int64_t)(KV_SLICE / 2) * WB;            // bytes from the lane's first run to its second
  // fingerprint of block entry i from this lane's 8 word pairs b[0 .. 7]: the dot products, the wave's sums and
  // three lanes' atomic additions
  auto finish = [&](const uint32_t* bw, int64_t i, bool live_i) {
    int s0 = 0, A[2][3] = {{0, 0, 0}, {0, 0, 0}}, H[2][2] = {{0, 0}, {0, 0}};
#pragma unroll
    for (int j = 0; j < KV_WPT / 2; ++j) {
      s0 = dot16(bw[j], 0x00010001u, s0);
#pragma unroll
      for (int c = 0; c < 2; ++c) {
#pragma unroll
        for (int d = 0; d < 3; ++d) A[c][d] = dot16(bw[j], dg[j][c][d], A[c][d]);
#pragma unroll
        for (int d = 0; d < 2; ++d) H[c][d] = dot16(bw[j], dg[j][c][3 + d], H[c][d]);
      }
    }
    uint64_t v[3];
    if constexpr (WB == 1) s0 -= 128 * nw;
    v[0] = (uint64_t)(int64_t)wave_sum_i32(s0);
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int64_t low = (int64_t)A[c][0] + ((int64_t)A[c][1] << 12) + ((int64_t)A[c][2] << 24);
      const uint32_t high = (uint32_t)H[c][0] + ((uint32_t)H[c][1] << 16);
      v[1 + c] = wave_sum_u64((uint64_t)low + ((uint64_t)high << 32) - corr[c]);
    }
    if (lane < 3 && live_i)
      atomicAdd((unsigned long long*)(a.out + 3 * i + lane), (unsigned long long)v[lane == 0 ? 0 : (lane == 1 ? 1 : 2)]);
  };
  // the block of entry i (or -1) and the address of this lane's first run in it
  auto entry = [&](int64_t i, bool& live_i) {
    int64_t blk = -1;
    if (i < a.n) {
      if (ids) {
        // a scalar load (i is the same for the whole wave): counted by lgkmcnt, it does not wait behind the blocks'
        // vector loads in flight
        const int64_t* ip = ids + i;
        asm volatile("s_load_dwordx2 %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(blk) : "s"(ip) : "memory");
      } else {
        blk = i;
      }
    }
    live_i = blk >= 0 && blk < a.nblocks;
    return a.cache + (live_i ? blk : 0) * a.block_bytes + (nw ? p0 : 0) * WB;
  };
  const int64_t G = gridDim.y;
  // a wave whose every lane is full (the common case: blocks a multiple of the slice) streams blocks with two
  // register buffers of KV_BUF entries: the next buffer's loads are issued before the current one's dot products
  const bool wave_full = __builtin_amdgcn_ballot_w64(!full) == 0;
  if (wave_full) {
    using Raw = typename std::conditional<WB == 2, u32x4, u32x2>::type;
    auto load = [&](int64_t i, Raw& r0, Raw& r1, bool& live_i) {
      const uint8_t* src = entry(i, live_i);
      r0 = __builtin_nontemporal_load(reinterpret_cast<const Raw*>(src));
      r1 = __builtin_nontemporal_load(reinterpret_cast<const Raw*>(src + off1));
    };
    auto words_of = [&](const Raw& r0, const Raw& r1, uint32_t* bw) {
      if constexpr (WB == 2) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          bw[q] = r0[q];
          bw[4 + q] = r1[q];
        }
      } else {
        const uint32_t xs[4] = {r0[0] ^ 0x80808080u, r0[1] ^ 0x80808080u,    // u = v + 128 in every byte
                                r1[0] ^ 0x80808080u, r1[1] ^ 0x80808080u};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          bw[2 * q] = __builtin_amdgcn_perm(0u, xs[q], 0x0C010C00u);         // bytes 0, 1 -> two 16-bit lanes
          bw[2 * q + 1] = __builtin_amdgcn_perm(0u, xs[q], 0x0C030C02u);     // bytes 2, 3
        }
      }
    };
    Raw xa0[KV_BUF], xa1[KV_BUF], xb0[KV_BUF], xb1[KV_BUF];
    bool la[KV_BUF], lb[KV_BUF];
    // entries i0 + u G (u < KV_BUF) per buffer; entries past n load entry 0's block again (live false)
#pragma unroll
    for (int u = 0; u < KV_BUF; ++u) load((int64_t)blockIdx.y + u * G, xa0[u], xa1[u], la[u]);
    for (int64_t i0 = blockIdx.y; i0 < a.n; i0 += 2 * KV_BUF * G) {
      const int64_t i1 = i0 + KV_BUF * G;
#pragma unroll
      for (int u = 0; u < KV_BUF; ++u) load(i1 + u * G, xb0[u], xb1[u], lb[u]);
#pragma unroll
      for (int u = 0; u < KV_BUF; ++u) {
        uint32_t bw[KV_WPT / 2];
        words_of(xa0[u], xa1[u], bw);
        finish(bw, i0 + u * G, la[u]);
      }
      if (i1 >= a.n) break;
#pragma unroll
      for (int u = 0; u < KV_BUF; ++u) load(i1 + KV_BUF * G + u * G, xa0[u], xa1[u], la[u]);
#pragma unroll
      for (int u = 0; u < KV_BUF; ++u) {
        uint32_t bw[KV_WPT / 2];
        words_of(xb0[u], xb1[u], bw);
        finish(bw, i1 + u * G, lb[u]);
      }
    }
    return;
  }
  // otherwise (some of the wave's words fall past the block's end, or unaligned blocks): guarded loads
  for (int64_t i0 = blockIdx.y; i0 < a.n; i0 += G) {
    bool live_i;
    const uint8_t* src = entry(i0, live_i);
    uint32_t bw[KV_WPT / 2];
#pragma unroll
    for (int j = 0; j < KV_WPT / 2; ++j) {
      uint32_t hv[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int q = 2 * j + e;
        if constexpr (WB == 2) {
          const uint8_t* wp = src + (q < KV_WPT / 2 ? 2 * q : off1 + 2 * (q - KV_WPT / 2));
          hv[e] = (valid >> q) & 1u ? (uint32_t)(wp[0] | (wp[1] << 8)) : 0u;
        } else {
          const uint8_t* wp = src + (q < KV_WPT / 2 ? q : off1 + q - KV_WPT / 2);
          hv[e] = (valid >> q) & 1u ? (uint32_t)(wp[0] ^ 0x80u) : 0u;
        }
      }
      bw[j] = hv[0] | (hv[1] << 16);
    }
    finish(bw, i0, live_i);
  }
}

// ------------------------------------------------------------------------------------------- MFMA fingerprints
// The weighted sums of a block's words as int8 matrix products: C[r][b] = sum over the bytes q of block b of
// T[r][q] * D[q][b], on v_mfma_i32_32x32x32_i8.  T (the weight table) holds, for weight c (w1, w2) and digit d
// (each weight as eight balanced base-256 digits, sum dig_d 256^d = w mod 2^64), row 8 c + d.
//   2-byte words: D is the block's bytes, low bytes with their top bit flipped (lo - 128, exact as int8), high
//   bytes the word's signed high half; row 8 c + d holds dig_d(w_c(p)) at the low byte of word p and
//   dig_{d-1}(w_c(p)) at its high byte, so that
//     sum_p word_p w_c(p) = sum_d 256^d C[8 c + d] + 128 sum_p w_c(p)          (mod 2^64; 256^8 = 0)
//   and rows 16 / 17 (ones at the low / high bytes) give sum_p word_p = C[16] + 256 C[17] + 128 (words).
//   1-byte words (int8, recompute.py:86-87): every byte is a word and D is the bytes as they are (signed int8);
//   row 8 c + d holds dig_d(w_c(p)) at byte p and row 16 ones, so sum_p word_p w_c(p) = sum_d 256^d C[8 c + d]
//   and sum_p word_p = C[16], with no offset.
// Every product is at most 2^14 in magnitude and a wave adds at most 2^15 of them per row: exact in int32.
// T is the same for every block: a table in the MFMA's operand order per word size, made once per device, with
// (2-byte words) the prefix sums of 128 w_c(p) (the low bytes' offset) per 32-byte step.
constexpr int KVM_BYTES = 65536;                 // bytes per block the tables cover (32768 2-byte words)
constexpr int KVM_STEPS = KVM_BYTES / 32;        // 32-byte steps of a block (one MFMA each)
constexpr int KVM_ENT = 64;                      // block entries per workgroup: two 32-column tiles per wave
__device__ __attribute__((aligned(256))) uint8_t kvm_tab[2][KVM_STEPS * 1024];            // [word bytes - 1]
__device__ __attribute__((aligned(256))) uint64_t kvm_corr[2][2 * (KVM_STEPS + 1)];

// balanced base-256 digit d of w (in [-128, 128))
__device__ __forceinline__ int bdig8(uint64_t w, int d) {
  uint64_t v = w;
  int dig = 0;
  for (int i = 0; i <= d; ++i) {
    const int b = (int)(v & 0xFFu);
    dig = b >= 128 ? b - 256 : b;
    v = (v - (uint64_t)(int64_t)dig) >> 8;
  }
  return dig;
}

__device__ __forceinline__ uint64_t kvm_weight(uint64_t p, int c) {
  const uint64_t z = fp3_z(p);
  return c ? ((z ^ (z >> 32)) | 1ull) : (z | 1ull);
}

// table step s (bytes 32 s .. 32 s + 31), lane l: row l % 32, bytes 16 (l / 32) .. + 15 of the step: the A operand
// of the step's MFMA, 1 KB per step with lane l's 16 bytes at 16 l
template <int WB>
__global__ __launch_bounds__(64) void kvm_fill_kernel(uint8_t* tab) {
  const int s = blockIdx.x, l = threadIdx.x, r = l & 31, h = l >> 5;
  uint32_t out[4] = {0u, 0u, 0u, 0u};
  for (int j = 0; j < 16; ++j) {
    const int64_t q = 32 * (int64_t)s + 16 * h + j;
    const uint64_t p = (uint64_t)(WB == 2 ? q >> 1 : q);
    const int hb = WB == 2 ? (int)(q & 1) : 0;
    int v = 0;
    if (r < 16) {
      const int c = r >> 3, d = r & 7;
      const uint64_t wt = kvm_weight(p, c);
      v = hb == 0 ? bdig8(wt, d) : (d > 0 ? bdig8(wt, d - 1) : 0);
    } else if (r == 16) {
      v = hb == 0 ? 1 : 0;
    } else if (r == 17) {
      v = hb == 1 ? 1 : 0;
    }
    out[j >> 2] |= ((uint32_t)v & 0xFFu) << (8 * (j & 3));
  }
  *reinterpret_cast<u32x4*>(tab + (int64_t)s * 1024 + 16 * l) = u32x4{out[0], out[1], out[2], out[3]};
}

// (2-byte words) corr[c (KVM_STEPS + 1) + s] = sum over words p < 16 s of 128 w_c(p) (mod 2^64): one workgroup,
// thread t the steps 8 t .. 8 t + 7, a serial scan of the 256 threads' totals
__global__ __launch_bounds__(256) void kvm_corr_kernel(uint64_t* corr) {
  constexpr int PPS = 16;                        // words per step
  __shared__ uint64_t tot[2][256];
  const int t = threadIdx.x;
  uint64_t st[2][8];
  for (int c = 0; c < 2; ++c) {
    uint64_t sum = 0;
    for (int k = 0; k < 8; ++k) {
      uint64_t v = 0;
      for (int j = 0; j < PPS; ++j) v += kvm_weight((uint64_t)(PPS * (8 * t + k) + j), c);
      st[c][k] = v << 7;
      sum += st[c][k];
    }
    tot[c][t] = sum;
  }
  __syncthreads();
  if (t < 2) {
    uint64_t run = 0;
    for (int i = 0; i < 256; ++i) {
      const uint64_t v = tot[t][i];
      tot[t][i] = run;
      run += v;
    }
  }
  __syncthreads();
  for (int c = 0; c < 2; ++c) {
    uint64_t run = tot[c][t];
    for (int k = 0; k < 8; ++k) {
      corr[c * (KVM_STEPS + 1) + 8 * t + k] = run;
      run += st[c][k];
    }
    if (t == 255) corr[c * (KVM_STEPS + 1) + KVM_STEPS] = run;
  }
}

// Workgroup: entries e0 .. e0 + 63; wave w: the w-th quarter of each block's 128-byte chunks.  Per chunk, each lane
// loads 8 pieces of 16 bytes (load i: entry 8 i + lane / 8, piece lane % 8: whole lines), flips the low bytes' top
// bits and stores them to the wave's LDS tile (entry row of 128 bytes, piece j at slot j ^ (row % 8)); then per
// 32-byte step s and column tile u, lane l reads row 32 u + l % 32, piece 2 s + l / 32 (the B operand) and the
// MFMA takes the table's step (the A operand) against it.  Chunks alternate between two register sets, the next
// one's loads issued before the current one is stored.
template <int WB>
__global__ __launch_bounds__(256) void kv_mfma_kernel(KvArgs a, const int64_t* ids, const uint8_t* tab,
                                                      const uint64_t* corr) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[4][KVM_ENT * 128];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int64_t e0 = (int64_t)blockIdx.x * KVM_ENT;
  const int64_t chunks = a.words * WB / 128;
  const int64_t per = (chunks + 3) / 4;
  const int64_t c0 = w * per < chunks ? w * per : chunks;
  const int64_t c1 = c0 + per < chunks ? c0 + per : chunks;
  const uint8_t* src[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int64_t ent = e0 + 8 * i + (lane >> 3);
    int64_t blk = -1;
    if (ent < a.n) blk = ids ? ids[ent] : ent;
    const bool live = blk >= 0 && blk < a.nblocks;
    src[i] = a.cache + (live ? blk : 0) * a.block_bytes + 16 * (lane & 7);
  }
  uint8_t* const L = lds[w];
  i32x16 acc[2];
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[u][e] = 0;
  auto load = [&](int64_t c, u32x4* d, i32x4* tf) {
#pragma unroll
    for (int i = 0; i < 8; ++i) d[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src[i] + 128 * c));
#pragma unroll
    for (int s = 0; s < 4; ++s) tf[s] = *reinterpret_cast<const i32x4*>(tab + (4 * c + s) * 1024 + 16 * lane);
  };
  const int wslot = (lane & 7) ^ (lane >> 3);                  // load i's piece lane % 8 of row 8 i + lane / 8
  auto process = [&](const u32x4* d, const i32x4* tf) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      // 2-byte words: the low bytes' top bits flipped (lo - 128); 1-byte words as they are
      const u32x4 x = WB == 2 ? d[i] ^ u32x4{0x00800080u, 0x00800080u, 0x00800080u, 0x00800080u} : d[i];
      *reinterpret_cast<u32x4*>(L + (8 * i + (lane >> 3)) * 128 + 16 * wslot) = x;
    }
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int row = 32 * u + (lane & 31), piece = 2 * s + (lane >> 5);
        const i32x4 b = *reinterpret_cast<const i32x4*>(L + row * 128 + 16 * (piece ^ (row & 7)));
        acc[u] = __builtin_amdgcn_mfma_i32_32x32x32_i8(tf[s], b, acc[u], 0, 0, 0);
      }
  };
  if (c0 < c1) {
    u32x4 da[8], db[8];
    i32x4 ta[4], tb[4];
    load(c0, da, ta);
    for (int64_t c = c0; c < c1; c += 2) {
      if (c + 1 < c1) load(c + 1, db, tb);
      process(da, ta);
      if (c + 1 >= c1) break;
      if (c + 2 < c1) load(c + 2, da, ta);
      process(db, tb);
    }
  }
  // lane l holds column (entry) 32 u + l % 32 of tile u, rows 8 (e / 4) + 4 (l / 32) + e % 4 of its 16 values
  const int h = lane >> 5;
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    uint64_t v1 = 0, v2 = 0, v0 = 0;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int r = 8 * (e >> 2) + 4 * h + (e & 3);
      const uint64_t x = (uint64_t)(int64_t)acc[u][e];
      if (r < 8) v1 += x << (8 * r);
      else if (r < 16) v2 += x << (8 * (r - 8));
      else if (r == 16) v0 += x;
      else if (r == 17) v0 += x << 8;
    }
    if (WB == 2 && h == 0) {
      v0 += (uint64_t)(128 * 64) * (uint64_t)(c1 - c0);
      v1 += corr[4 * c1] - corr[4 * c0];
      v2 += corr[(KVM_STEPS + 1) + 4 * c1] - corr[(KVM_STEPS + 1) + 4 * c0];
    }
    const int64_t ent = e0 + 32 * u + (lane & 31);
    int64_t blk = -1;
    if (ent < a.n) blk = ids ? ids[ent] : ent;
    if (blk >= 0 && blk < a.nblocks && c0 < c1) {
      int64_t* o = a.out + 3 * ent;
      if (h == 0) atomicAdd((unsigned long long*)o, (unsigned long long)v0);
      atomicAdd((unsigned long long*)(o + 1), (unsigned long long)v1);
      atomicAdd((unsigned long long*)(o + 2), (unsigned long long)v2);
    }
  }
}

constexpr int KVM_MAXDEV = 64;
std::atomic<const uint8_t*> g_kvm_tab[KVM_MAXDEV][2];
std::atomic<const uint64_t*> g_kvm_corr[KVM_MAXDEV][2];
std::mutex g_kvm_mu;

// This device's weight table and corrections for words of wb bytes, made at the first such call on the device
// (which waits for them); false when they are not there and cannot be made now (the stream is being captured, or a
// HIP error)
bool kvm_tables(hipStream_t stream, int wb, const uint8_t** tab, const uint64_t** corr) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= KVM_MAXDEV || (wb != 1 && wb != 2)) return false;
  const uint8_t* tp = g_kvm_tab[dev][wb - 1].load(std::memory_order_acquire);
  if (!tp) {
    std::lock_guard<std::mutex> lk(g_kvm_mu);
    tp = g_kvm_tab[dev][wb - 1].load(std::memory_order_relaxed);
    if (!tp) {
      hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
      if (hipStreamIsCapturing(stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return false;
      void *pt = nullptr, *pc = nullptr;
      if (hipGetSymbolAddress(&pt, HIP_SYMBOL(kvm_tab)) != hipSuccess || !pt) return false;
      if (hipGetSymbolAddress(&pc, HIP_SYMBOL(kvm_corr)) != hipSuccess || !pc) return false;
      uint8_t* t = (uint8_t*)pt + (int64_t)(wb - 1) * KVM_STEPS * 1024;
      uint64_t* c = (uint64_t*)pc + (int64_t)(wb - 1) * 2 * (KVM_STEPS + 1);
      if (wb == 2) {
        hipLaunchKernelGGL(kvm_fill_kernel<2>, dim3(KVM_STEPS), dim3(64), 0, stream, t);
        hipLaunchKernelGGL(kvm_corr_kernel, dim3(1), dim3(256), 0, stream, c);
      } else {
        hipLaunchKernelGGL(kvm_fill_kernel<1>, dim3(KVM_STEPS), dim3(64), 0, stream, t);   // (no offset to undo)
      }
      if (hipGetLastError() != hipSuccess || hipStreamSynchronize(stream) != hipSuccess) return false;
      g_kvm_corr[dev][wb - 1].store(c, std::memory_order_relaxed);
      g_kvm_tab[dev][wb - 1].store(t, std::memory_order_release);
      tp = t;
    }
  }
  *tab = tp;
  *corr = g_kvm_corr[dev][wb - 1].load(std::memory_order_relaxed);
  return true;
}

}  // namespace

// out[3] (int64, zeroed by the caller) += fp3 of n words of word_bytes (2 or 1) bytes at bits, positions from start
extern "C" int sdc_fingerprint3(const void* bits, int64_t n, int word_bytes, int64_t start, int64_t* out,
                                hipStream_t stream) {
  SDC_CLEAR_ERRORS();
  if (n < 0 || !out || (word_bytes != 1 && word_bytes != 2)) return SDC_EINVAL;
  if (n == 0) return SDC_OK;
  if (!bits) return SDC_EINVAL;
  const uint8_t* X = (const uint8_t*)bits;
  const bool aligned = ((uintptr_t)X % 16) == 0;
  const int per = 16 / word_bytes;
  SdcProf prof("fingerprint3", stream);
  if (aligned) {
    const unsigned g = grid_for(n / per);
    if (word_bytes == 2) hipLaunchKernelGGL(fp3_kernel<2>, dim3(g), dim3(256), 0, stream, X, n, start, out);
    else hipLaunchKernelGGL(fp3_kernel<1>, dim3(g), dim3(256), 0, stream, X, n, start, out);
  } else {
    const unsigned g = grid_for(n);
    if (word_bytes == 2) hipLaunchKernelGGL(fp3_scalar_kernel<2>, dim3(g), dim3(256), 0, stream, X, n, start, out);
    else hipLaunchKernelGGL(fp3_scalar_kernel<1>, dim3(g), dim3(256), 0, stream, X, n, start, out);
  }
  SDC_LAUNCH_CHECK();
  return SDC_OK;
}

// out[2] (int64, zeroed by the caller) += fp2 of n words; kind 0 = int16, 1 = int32, 2 = uint8
extern "C" int sdc_fingerprint2(const void* bits, int64_t n, int kind, int64_t* out, hipStream_t stream) {
  SDC_CLEAR_ERRORS();
  if (n < 0 || !out || kind < 0 || kind > 2) return SDC_EINVAL;
  if (n == 0) return SDC_OK;
  if (!bits) return SDC_EINVAL;
  const uint8_t* X = (const uint8_t*)bits;
  const int per = kind == 0 ? 8 : kind == 1 ? 4 : 16;
  SdcProf prof("fingerprint2", stream);
  const unsigned g = grid_for(sdc_cdiv(n, per));
  if (kind == 0) hipLaunchKernelGGL(fp2_kernel<0>, dim3(g), dim3(256), 0, stream, X, n, out);
  else if (kind == 1) hipLaunchKernelGGL(fp2_kernel<1>, dim3(g), dim3(256), 0, stream, X, n, out);
  else hipLaunchKernelGGL(fp2_kernel<2>, dim3(g), dim3(256), 0, stream, X, n, out);
  SDC_LAUNCH_CHECK();
  return SDC_OK;
}

// out[i][0..2] (int64, zeroed by the caller) += fp3 of block ids[i] (or block i) of a paged cache of int16 words
// (word_bytes 2) or int8 words (1): block b holds `words` words at cache + b * block_bytes, its positions numbered
// from 0.  Entries whose id is negative or >= nblocks are left as they are.
extern "C" int sdc_kv_fingerprint(const void* cache, int64_t nblocks, int64_t block_bytes, int64_t words,
                                  int word_bytes, const int64_t* ids, int64_t n, int64_t* out, hipStream_t stream) {
  SDC_CLEAR_ERRORS();
  if (word_bytes != 1 && word_bytes != 2) return SDC_EINVAL;
  if (!cache || !out || nblocks < 1 || words < 1 || n < 0 || block_bytes < words * word_bytes) return SDC_EINVAL;
  if (n == 0) return SDC_OK;
  KvArgs a{(const uint8_t*)cache, block_bytes, words, nblocks, ids, n, out,
           (block_bytes % 16 == 0) && ((uintptr_t)cache % 16 == 0)};
  const int64_t gx = sdc_cdiv(sdc_cdiv(words, KV_SLICE), KV_WAVES);      // workgroups of KV_WAVES wave slices
  int64_t gy = sdc_cdiv(2048, gx);
  if (gy > sdc_cdiv(n, KV_UNROLL)) gy = sdc_cdiv(n, KV_UNROLL);
  if (gy > 65535) gy = 65535;
  // words in whole 128-byte chunks, aligned, within the tables: the MFMA kernel
  const uint8_t* tab = nullptr;
  const uint64_t* corr = nullptr;
  const int64_t wbytes = words * word_bytes;
  if (a.vec && wbytes % 128 == 0 && wbytes <= KVM_BYTES && kvm_tables(stream, word_bytes, &tab, &corr)) {
    SdcProf prof("kv_fingerprint", stream);
    const dim3 grid((unsigned)sdc_cdiv(n, KVM_ENT));
    if (word_bytes == 2) hipLaunchKernelGGL(kv_mfma_kernel<2>, grid, dim3(256), 0, stream, a, ids, tab, corr);
    else hipLaunchKernelGGL(kv_mfma_kernel<1>, grid, dim3(256), 0, stream, a, ids, tab, corr);
    SDC_LAUNCH_CHECK();
    return SDC_OK;
  }
  SdcProf prof("kv_fingerprint", stream);
  if (word_bytes == 2)
    hipLaunchKernelGGL(kv_fp3_kernel<2>, dim3((unsigned)gx, (unsigned)gy), dim3(64 * KV_WAVES), 0, stream, a, ids);
  else
    hipLaunchKernelGGL(kv_fp3_kernel<1>, dim3((unsigned)gx, (unsigned)gy), dim3(64 * KV_WAVES), 0, stream, a, ids);
  SDC_LAUNCH_CHECK();
  return SDC_OK;
}
