// Block sums of a matrix of bf16/fp16 outputs, shared by the serving and training checks.
//
// A (row, block) pair is `bs` consecutive outputs of one row (the last block of a row may be narrower, `rem`).
// For each pair the check needs four fp32 sums: plain, signed with the block width's +-1 pattern, of squares and
// of |values| (serve.py:247-254, checksum.py:481-509).  A wave reads 64 consecutive pairs; four lanes share a pair
// in each of four rounds (each reads 4 x 16 bytes of the 256-byte block, in runs of 64 bytes), all sixteen
// loads in flight before any is used, and adds the sums with packed dot products (two elements per instruction)
// and two DPP steps; lane l ends up with pair base + (l & 3) * 16 + (l >> 2).
#pragma once
#include "common.h"

// Where the outputs are: element (batch b, row r, column c) at y[b * sb + r * sm + c * sn].
struct YView {
  const uint16_t* y;
  int64_t sb, sm, sn;
  int64_t m, nb, bs, rem, npairs;      // npairs = batches * m * nb (flat pair index p = (b * m + r) * nb + jb)
  int vec;                             // 16-byte loads allowed (sn == 1, aligned rows, bs % 8 == 0)
  const float* s_full;                 // +-1 pattern of width bs (a 128-entry row of the sign table)
  const float* s_last;                 // +-1 pattern of width rem
};

__device__ __forceinline__ void pair_index(const YView& v, int64_t p, int64_t& b, int64_t& r, int64_t& jb) {
  const uint32_t rr = (uint32_t)p / (uint32_t)v.nb;
  jb = (uint32_t)p - rr * (uint32_t)v.nb;
  b = rr / (uint32_t)v.m;
  r = rr - (uint32_t)b * (uint32_t)v.m;
}

// Division and square root by the hardware's reciprocal and square-root approximations (about 1 ulp): the scores
// only need to agree with the reference's to 1e-3 of the noise, and the special cases keep their IEEE results
// (x / 0 = inf, 0 / 0 = NaN, inf / inf = NaN, sqrt(inf) = inf, sqrt(NaN) = NaN).
__device__ __forceinline__ float fdiv(float a, float b) { return a * __builtin_amdgcn_rcpf(b); }
__device__ __forceinline__ float fsqrt(float a) { return __builtin_amdgcn_sqrtf(a); }

// Four sums of 8 elements (one 16-byte load) with packed dot products: v_dot2_f32_{bf16,f16} adds two products
// to an fp32 accumulator, so each instruction takes two elements: plain sum (x . 1), signed sum (x . s), sum of
// squares (x . x) and sum of |x| (|x| . 1).  `sg2` holds the four sign pairs of these eight columns.
template <int DT>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  if constexpr (DT == SDC_BF16) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
  } else {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c, false);
  }
}

// a . b + 0, the first term of a sum: the three-operand form takes the zero as an inline constant, where the
// accumulating form (what the compiler picks for dot2(a, b, 0)) needs a register cleared first
template <int DT>
__device__ __forceinline__ float dot2_first(uint32_t a, uint32_t b) {
  float r;
  if constexpr (DT == SDC_BF16) asm("v_dot2_f32_bf16 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
  else asm("v_dot2_f32_f16 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

template <int DT>
__device__ __forceinline__ void acc8(u32x4 v, const uint32_t* sg2, float& pl, float& sg, float& sq, float& ab) {
  constexpr uint32_t ONES = DT == SDC_BF16 ? 0x3F803F80u : 0x3C003C00u;
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    pl = dot2<DT>(w[i], ONES, pl);
    sg = dot2<DT>(w[i], sg2[i], sg);
    sq = dot2<DT>(w[i], w[i], sq);
    ab = dot2<DT>(w[i] & 0x7FFF7FFFu, ONES, ab);
  }
}

// The four sums of the (row, block) pair each lane keeps: a wave reads 64 consecutive pairs starting at `base`;
// lane l ends up with pair base + (l & 3) * 16 + (l >> 2).  Four lanes share a pair in each of four rounds; all
// sixteen 16-byte loads are issued before any is used (256 bytes per lane in flight).  Pairs that are not full
// 128-wide vector-loadable blocks (a narrower last block, strided y) take an element-wise path.
template <int DT>
__device__ __forceinline__ void pair_sums(const YView& a, int64_t base, int lane, const uint32_t* sg2, float& my_pl,
                                          float& my_sg, float& my_sq, float& my_ab) {
  const int q = lane & 3;
  bool full[4];
  u32x4 v[4][4];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int64_t p = base + g * 16 + (lane >> 2);
    full[g] = false;
    if (p < a.npairs && a.vec) {
      int64_t b, r, jb;
      pair_index(a, p, b, r, jb);
      const bool last = (jb == a.nb - 1) && (a.rem > 0);
      if (!last && a.bs == 128) {
        full[g] = true;
        const uint16_t* yr = a.y + b * a.sb + r * a.sm + jb * 128;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          v[g][j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(yr + 8 * (q + 4 * j)));
      }
    }
  }
  my_pl = my_sg = my_sq = my_ab = 0.f;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int64_t p = base + g * 16 + (lane >> 2);
    float pl = 0.f, sg = 0.f, sq = 0.f, ab = 0.f;
    if (full[g]) {
#pragma unroll
      for (int j = 0; j < 4; ++j) acc8<DT>(v[g][j], &sg2[j * 4], pl, sg, sq, ab);
    } else if (p < a.npairs) {
      int64_t b, r, jb;
      pair_index(a, p, b, r, jb);
      const bool last = (jb == a.nb - 1) && (a.rem > 0);
      const int64_t wid = last ? a.rem : a.bs;
      const uint16_t* yr = a.y + b * a.sb + r * a.sm + jb * a.bs * a.sn;
      const float* sp = last ? a.s_last : a.s_full;
#pragma unroll 1
      for (int j = 0; j < 4; ++j)
#pragma unroll 1
        for (int e = 0; e < 8; ++e) {
          const int c = 8 * (q + 4 * j) + e;
          if (c < wid) {
            float x = half_to_f32<DT>(yr[c * a.sn]);
            pl += x;
            sg = fmaf(x, sp[c], sg);
            sq = fmaf(x, x, sq);
            ab += fabsf(x);
          }
        }
    }
    pl = quad_sum(pl); sg = quad_sum(sg); sq = quad_sum(sq); ab = quad_sum(ab);
    if (q == g) { my_pl = pl; my_sg = sg; my_sq = sq; my_ab = ab; }
  }
}

// The signs of this lane's 32 columns of a full block (chunks q, q+4, q+8, q+12 of 8 columns) as packed pairs; a
// table row holds 128 entries (zeros past its width), so these loads need no bounds test.
template <int DT>
__device__ __forceinline__ void lane_signs(const YView& a, int q, uint32_t* sg2) {
  constexpr uint32_t POS = DT == SDC_BF16 ? 0x3F80u : 0x3C00u, NEG = DT == SDC_BF16 ? 0xBF80u : 0xBC00u;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const f32x4 s0 = *reinterpret_cast<const f32x4*>(a.s_full + 8 * (q + 4 * j));
    const f32x4 s1 = *reinterpret_cast<const f32x4*>(a.s_full + 8 * (q + 4 * j) + 4);
    sg2[j * 4 + 0] = (s0.x < 0.f ? NEG : POS) | ((s0.y < 0.f ? NEG : POS) << 16);
    sg2[j * 4 + 1] = (s0.z < 0.f ? NEG : POS) | ((s0.w < 0.f ? NEG : POS) << 16);
    sg2[j * 4 + 2] = (s1.x < 0.f ? NEG : POS) | ((s1.y < 0.f ? NEG : POS) << 16);
    sg2[j * 4 + 3] = (s1.z < 0.f ? NEG : POS) | ((s1.w < 0.f ? NEG : POS) << 16);
  }
}

