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
// block, so a workgroup owns one slice of KV_SLICE positions of every block it visits (16 words per thread) and
// keeps their weights in registers while it streams blocks; per block the three sums use one 64-bit and one
// 32-bit multiply-add per weight (b w = b lo_s + 2^32 b hi' mod 2^64, with lo_s the signed low half of w and
// hi' its high half plus the low half's sign bit), then a wave and workgroup reduction and three 64-bit atomics.
constexpr int KV_WPT = 16;                       // words per thread
constexpr int KV_SLICE = 256 * KV_WPT;           // positions per workgroup slice

struct KvArgs {
  const uint8_t* cache;
  int64_t block_bytes, words, nblocks;           // nblocks: valid block ids are 0 .. nblocks - 1
  const int64_t* ids;                            // block of entry i (null: entry i is block i); < 0: no block
  int64_t n;
  int64_t* out;                                  // [n][3]
  int vec;
};

__global__ __launch_bounds__(256) void kv_fp3_kernel(KvArgs a) {
  __shared__ int64_t red[4][3];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int64_t p0 = (int64_t)blockIdx.x * KV_SLICE + (int64_t)t * KV_WPT;
  int32_t w1l[KV_WPT], w2l[KV_WPT];
  uint32_t w1h[KV_WPT], w2h[KV_WPT];
#pragma unroll
  for (int e = 0; e < KV_WPT; ++e) {
    const uint64_t z = fp3_z((uint64_t)(p0 + e));
    const uint64_t q1 = z | 1ull, q2 = (z ^ (z >> 32)) | 1ull;
    w1l[e] = (int32_t)(uint32_t)q1;
    w2l[e] = (int32_t)(uint32_t)q2;
    w1h[e] = (uint32_t)(q1 >> 32) + ((uint32_t)q1 >> 31);
    w2h[e] = (uint32_t)(q2 >> 32) + ((uint32_t)q2 >> 31);
  }
  const int nw = p0 >= a.words ? 0 : (a.words - p0 < KV_WPT ? (int)(a.words - p0) : KV_WPT);
  for (int64_t i = blockIdx.y; i < a.n; i += gridDim.y) {
    const int64_t blk = a.ids ? a.ids[i] : i;
    if (blk < 0 || blk >= a.nblocks) continue;                  // (uniform over the workgroup)
    const uint8_t* src = a.cache + blk * a.block_bytes + p0 * 2;
    int32_t b[KV_WPT];
    if (a.vec && nw == KV_WPT) {
      const u32x4 v0 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src));
      const u32x4 v1 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + 16));
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        b[2 * j] = (int16_t)(v0[j] & 0xFFFFu);
        b[2 * j + 1] = (int16_t)(v0[j] >> 16);
        b[8 + 2 * j] = (int16_t)(v1[j] & 0xFFFFu);
        b[8 + 2 * j + 1] = (int16_t)(v1[j] >> 16);
      }
    } else {
#pragma unroll
      for (int e = 0; e < KV_WPT; ++e) b[e] = e < nw ? (int16_t)(src[2 * e] | (src[2 * e + 1] << 8)) : 0;
    }
    int64_t s0 = 0, l1 = 0, l2 = 0;
    uint32_t h1 = 0, h2 = 0;
#pragma unroll
    for (int e = 0; e < KV_WPT; ++e) {
      s0 += b[e];
      l1 += (int64_t)b[e] * (int64_t)w1l[e];
      l2 += (int64_t)b[e] * (int64_t)w2l[e];
      h1 += (uint32_t)b[e] * w1h[e];
      h2 += (uint32_t)b[e] * w2h[e];
    }
    int64_t v[3] = {s0, (int64_t)((uint64_t)l1 + ((uint64_t)h1 << 32)), (int64_t)((uint64_t)l2 + ((uint64_t)h2 << 32))};
#pragma unroll
    for (int c = 0; c < 3; ++c) v[c] = wave_sum_i64(v[c]);
    if (lane == 0) {
      red[w][0] = v[0];
      red[w][1] = v[1];
      red[w][2] = v[2];
    }
    __syncthreads();
    if (t < 3) {
      const uint64_t sum = (uint64_t)red[0][t] + (uint64_t)red[1][t] + (uint64_t)red[2][t] + (uint64_t)red[3][t];
      atomicAdd((unsigned long long*)(a.out + 3 * i + t), (unsigned long long)sum);
    }
    __syncthreads();
  }
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

// out[i][0..2] (int64, zeroed by the caller) += fp3 of block ids[i] (or block i) of a paged cache of int16 words:
// block b holds `words` words at cache + b * block_bytes, its positions numbered from 0.  Entries whose id is
// negative or >= nblocks are left as they are.
extern "C" int sdc_kv_fingerprint(const void* cache, int64_t nblocks, int64_t block_bytes, int64_t words,
                                  const int64_t* ids, int64_t n, int64_t* out, hipStream_t stream) {
  SDC_CLEAR_ERRORS();
  if (!cache || !out || nblocks < 1 || words < 1 || n < 0 || block_bytes < words * 2) return SDC_EINVAL;
  if (n == 0) return SDC_OK;
  KvArgs a{(const uint8_t*)cache, block_bytes, words, nblocks, ids, n, out,
           (block_bytes % 16 == 0) && ((uintptr_t)cache % 16 == 0)};
  const int64_t slices = sdc_cdiv(words, KV_SLICE);
  int64_t gy = sdc_cdiv(2048, slices);
  if (gy > n) gy = n;
  if (gy > 65535) gy = 65535;
  SdcProf prof("kv_fingerprint", stream);
  hipLaunchKernelGGL(kv_fp3_kernel, dim3((unsigned)slices, (unsigned)gy), dim3(256), 0, stream, a);
  SDC_LAUNCH_CHECK();
  return SDC_OK;
}
