// Expected side of the column-block checksum: E = A @ (block sums of B), on MFMA.
//
// The block sums B2 (k x 2nb fp32 per batch) multiply A as three low-precision parts (hi + mid + lo, whose sum is
// B2 to ~2^-27; checksum.py:160-166, :313-343, serve.py:185-186), so A (bf16/fp16) is never widened and the
// tensor-core products stay exact; every part accumulates into one fp32 accumulator, so E comes out summed over
// parts.  The parts are a (3 x ncols) x k matrix stored k-contiguous per column: precomputed per layer for the
// serving check (LayerChecksums.parts), made per call by split_kernel for the training check (from the B-side
// stage's fp32 sums, after division by a per-column power of two that keeps fp16 parts in range, as
// checksum._matmul_fp32 scales).  The same pass over A adds |a_row|_2^2 and |a_row|_1 (the noise model's row
// norms), in the workgroups of the first column tile.  Depth is split over workgroups when the tiles alone cannot
// fill the 256 CUs: each split writes its own plane of E and the scoring kernels add the planes.
#include <type_traits>

#include "common.h"
#include "gemm.h"
#include "mfma_pipe.h"
#include "profile.h"

namespace {

using sdc_pipe::mfma32;

__device__ __forceinline__ f32x16 mfma32_i8(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_bit_cast(f32x16, __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, a),
                                                                          __builtin_bit_cast(i32x4, b),
                                                                          __builtin_bit_cast(i32x16, c), 0, 0, 0));
}

// fp8 e4m3 (OCP: bias 7, no infinities, S.1111.111 NaN) -> bf16 bits, exactly: normals move their exponent
// (e + 120) and keep 3 mantissa bits; subnormals m * 2^-9 are normal in bf16.
__device__ __forceinline__ uint32_t e4m3_to_bf16(uint32_t b) {
  const uint32_t s = (b & 0x80u) << 8, e = (b >> 3) & 15u, m = b & 7u;
  if (e == 15u && m == 7u) return s | 0x7FC0u;
  if (e != 0u) return s | ((e + 120u) << 7) | (m << 4);
  if (m == 0u) return s;
  const uint32_t f = __float_as_uint((float)m * 0.001953125f);         // m * 2^-9, exact
  return s | (f >> 16);
}

// 8 fp8 values (one 8-byte word pair) -> 8 bf16 (16 bytes): gfx950's scaled pair conversion with scale 1, which is
// exact (every e4m3 value is a bf16 value; 0x7F / 0xFF become NaN), two bytes of a word per instruction
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ u32x4 fp8x8_to_bf16(u32x2 v) {
  u32x4 o;
#pragma unroll
  for (int w = 0; w < 2; ++w) {
    o[2 * w] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v[w], 1.0f, false));
    o[2 * w + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v[w], 1.0f, true));
  }
  return o;
}

// a . b + c over the two 16-bit halves of a and b (fp32 accumulation)
template <int DT>
__device__ __forceinline__ float pk_dot2(uint32_t a, uint32_t b, float c) {
  if constexpr (DT == SDC_BF16)
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
  else
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c, false);
}

// 8 consecutive (in depth) 16-bit elements at p[kk * sk], or zeros past `lim`
template <bool VEC>
__device__ __forceinline__ u32x4 load8(const uint16_t* p, int64_t sk, int64_t kk, int64_t lim, bool ok) {
  u32x4 v = {0u, 0u, 0u, 0u};
  if (!ok || kk >= lim) return v;
  if constexpr (VEC) {
    return *reinterpret_cast<const u32x4*>(p + kk);
  } else {
    uint16_t e[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) e[i] = (kk + i < lim) ? p[(kk + i) * sk] : (uint16_t)0;
    v.x = e[0] | ((uint32_t)e[1] << 16);
    v.y = e[2] | ((uint32_t)e[3] << 16);
    v.z = e[4] | ((uint32_t)e[5] << 16);
    v.w = e[6] | ((uint32_t)e[7] << 16);
    return v;
  }
}

// 8 fp8 values at p[kk * sk ...] (bounds-checked, zero past `lim`) as bf16
__device__ __forceinline__ u32x4 load8_fp8(const uint8_t* p, int64_t sk, int64_t kk, int64_t lim, bool ok) {
  u32x4 v = {0u, 0u, 0u, 0u};
  if (!ok) return v;
  uint32_t* pv = reinterpret_cast<uint32_t*>(&v);
#pragma unroll
  for (int i = 0; i < 8; i += 2) {
    const uint32_t lo = kk + i < lim ? e4m3_to_bf16(p[(kk + i) * sk]) : 0u;
    const uint32_t hi = kk + i + 1 < lim ? e4m3_to_bf16(p[(kk + i + 1) * sk]) : 0u;
    pv[i / 2] = lo | (hi << 16);
  }
  return v;
}

__device__ __forceinline__ uint32_t to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 16) | 0x40u;       // NaN stays NaN (quiet)
  u += 0x7FFFu + ((u >> 16) & 1u);                                    // round to nearest even
  return u >> 16;
}

template <int DT>
__device__ __forceinline__ uint32_t round_bits(float f) {
  if constexpr (DT == SDC_BF16) return to_bf16_bits(f);
  else return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}

template <int DT>
__device__ __forceinline__ float bits_value(uint32_t b) {
  return half_to_f32<DT>((uint16_t)b);
}

// fp32 -> hi, mid, lo parts of 8 values (checksum._split3), packed as three u32x4
template <int DT>
__device__ __forceinline__ void split8(const float* v, u32x4* parts) {
  uint32_t h[8], md[8], lo[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    h[i] = round_bits<DT>(v[i]);
    const float r = v[i] - bits_value<DT>(h[i]);
    md[i] = round_bits<DT>(r);
    lo[i] = round_bits<DT>(r - bits_value<DT>(md[i]));
  }
  uint32_t* o0 = reinterpret_cast<uint32_t*>(&parts[0]);
  uint32_t* o1 = reinterpret_cast<uint32_t*>(&parts[1]);
  uint32_t* o2 = reinterpret_cast<uint32_t*>(&parts[2]);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o0[i] = h[2 * i] | (h[2 * i + 1] << 16);
    o1[i] = md[2 * i] | (md[2 * i + 1] << 16);
    o2[i] = lo[2 * i] | (lo[2 * i + 1] << 16);
  }
}

template <int DT>
__device__ __forceinline__ void norm_acc(u32x4 v, float& sq, float& ab) {
  uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float a = lo_of<DT>(w[i]), b = hi_of<DT>(w[i]);
    sq = fmaf(a, a, sq);
    sq = fmaf(b, b, sq);
    ab += fabsf(a);
    ab += fabsf(b);
  }
}

// One workgroup of 8 waves (two per SIMD, one workgroup per CU) owns a TM x TN tile of E and one depth slice.
// WGN = 2: waves 4 x 2, tile 256 x 128 (wide checksum sets); WGN = 1: waves 8 x 1, tile 512 x 64 (narrow ones, such
// as the 64 columns of a row-block check).  Each wave computes 64 x 64 with 2 x 2 fragments of v_mfma_f32_32x32x16
// and, per fragment pair, the three parts of B into the same accumulator.
//
// Depth advances in stages of 32 (two MFMA steps of 16) through three LDS buffers.  In stage s a wave reads the
// fragments of step s.1 while the MFMAs of step s.0 run, then those of step (s + 1).0 while the MFMAs of s.1 run, so
// LDS reads overlap the matrix cores inside every wave; it then stores stage s + 2 (loaded from global memory one
// stage earlier) into the third buffer, issues the loads of stage s + 3, and one barrier ends the stage.  A buffer
// is rewritten only after the barrier that follows every wave's last read of it.  Loads and stores are
// unconditional (a guarded load makes the compiler wait for it at the end of the guarded block): past the last stage
// they repeat the last stage's data into a buffer nobody reads again.
// LDS rows hold 32 elements (64 bytes, four 16-byte chunks); chunk q of row r sits at position q ^ ((r / 2) % 4),
// so the eight lanes of each ds_read_b128 phase (eight consecutive rows, one chunk) and of each ds_write_b128 phase
// (two rows, four chunks each) hit 32 distinct banks.
// Workgroups are numbered so that each XCD (dispatch is round-robin over the eight) takes a contiguous range of
// tiles: column tiles of one row tile, and row tiles of one depth slice, share an XCD's L2.
using sdc_pipe::KS;                    // depth per stage
using sdc_pipe::lds_at;
using sdc_pipe::lds_load16;
using sdc_pipe::lgkmcnt0_imm;
using sdc_pipe::vmcnt_imm;
constexpr int NT = 512;                // threads per workgroup
constexpr int NBUF = 3;                // LDS buffers

template <int WGN, int NP>
struct Tile {
  static constexpr int WGM = 8 / WGN;
  static constexpr int TM = 64 * WGM;
  static constexpr int TN = 64 * WGN;
  static constexpr int ACH = TM * (KS / 8);                   // 16-byte chunks of A per stage
  static constexpr int BCH = NP * TN * (KS / 8);              // ... of the NP parts of B
  static constexpr int NA = (ACH + NT - 1) / NT;              // per thread
  static constexpr int NB = (BCH + NT - 1) / NT;
  static constexpr int ROWS = TM + NP * TN;                   // LDS rows per buffer
};

// MODE: SDC_BF16 / SDC_FP16 (A and 3 parts of that type), SDC_FP8 (A fp8 converted to bf16 on load, 3 bf16
// parts), SDC_I8 (A int8 and 2 int8 parts: the block sums' base-128 digits, each into its own int32
// accumulator; depth and strides are in pairs of int8 so that a 16-byte chunk is 8 "elements" as for 16-bit data,
// and the 32x32x32 int8 MFMA takes a k-step of 16 pairs).
template <int MODE, int WGN, bool VEC, bool DIRECT>
__global__ __launch_bounds__(NT) void expected_gemm_kernel(GemmArgs g) {
  constexpr int NP = MODE == SDC_I8 ? 2 : 3;                  // parts
  constexpr int NACC = MODE == SDC_I8 ? 2 : 1;                // accumulator sets
  constexpr int DT = MODE == SDC_FP16 ? SDC_FP16 : SDC_BF16;  // element type of the LDS tiles (16-bit modes)
  constexpr int ESA = MODE == SDC_FP8 ? 1 : 2;                // bytes per A element in memory
  using T = Tile<WGN, NP>;
  __shared__ __attribute__((aligned(16))) uint16_t lds[NBUF][T::ROWS * KS];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int wm = w / WGN, wn = w % WGN;
  const int64_t nrt = sdc_cdiv(g.m, T::TM) + (g.goffs ? g.ngroups : 0), nct = sdc_cdiv(g.N, T::TN);
  // XCD-aware order: block b runs on XCD b % 8; give XCD x the x-th eighth of the tiles (column tile fastest)
  const int64_t G = (int64_t)gridDim.x, b = blockIdx.x;
  const int64_t wid = (G % 8 == 0) ? (b % 8) * (G / 8) + b / 8 : b;
  int64_t ct, rt, split, batch;
  if (g.rows_per_xcd) {
    split = wid % g.splits;
    ct = (wid / g.splits) % nct;
    rt = (wid / (g.splits * nct)) % nrt;
    batch = wid / (g.splits * nct * nrt);
  } else {
    ct = wid % nct;
    rt = (wid / nct) % nrt;
    const int64_t rest = wid / (nct * nrt);
    split = rest % g.splits;
    batch = rest / g.splits;
  }
  int64_t r0 = rt * T::TM, m = g.m;
  if (g.goffs) {
    // grouped rows: find the group whose row tiles contain tile rt (every thread walks the same offsets)
    int64_t start = 0, acc = 0, grp = -1;
    for (int64_t q = 0; q < g.ngroups; ++q) {
      const int64_t end = g.goffs[q] < g.m ? g.goffs[q] : g.m;   // offsets past the rows are clamped
      const int64_t nt = end > start ? sdc_cdiv(end - start, T::TM) : 0;
      if (rt < acc + nt) {
        grp = q;
        r0 = start + (rt - acc) * T::TM;
        m = end;                        // rows of this tile stop at the group's end
        break;
      }
      acc += nt;
      start = end > start ? end : start;
    }
    if (grp < 0) return;                // past the last tile: the whole workgroup leaves before any barrier
    batch = grp;
  }
  const int64_t c0 = ct * T::TN;
  const int64_t kbeg = split * g.kchunk;
  const int64_t kend = kbeg + g.kchunk < g.k ? kbeg + g.kchunk : g.k;
  const int nst = kbeg < kend ? (int)sdc_cdiv(kend - kbeg, KS) : 0;
  const bool norms = ct == 0 && g.XN != nullptr;      // (a caller with the row norms already passes no XN)
  const int64_t N = g.N, me = g.m;      // me: rows of E and XN (the global row count)
  const uint8_t* Ab = (const uint8_t*)g.A + (g.goffs ? 0 : batch * g.sab * ESA);
  const uint16_t* Pb = (const uint16_t*)g.B + batch * g.sbb;
  const int64_t eb = g.goffs ? 0 : batch;           // E / XN plane set

  // this thread's chunks: A chunk c is (row c / 4, depth 8 (c % 4)); B chunk c is (LDS row c / 4: part, column);
  // indexes past the end repeat the last chunk (the same value is stored twice)
  const uint8_t* asrc[T::NA];
  int alds[T::NA], ak[T::NA];
  bool aok[T::NA];
#pragma unroll
  for (int j = 0; j < T::NA; ++j) {
    const int c = (t + NT * j) < T::ACH ? t + NT * j : T::ACH - 1;
    const int64_t row = r0 + c / 4;
    aok[j] = row < m;
    asrc[j] = Ab + (aok[j] ? row : 0) * g.sam * ESA;
    alds[j] = lds_at(c / 4, c % 4);
    ak[j] = 8 * (c % 4);
  }
  const uint16_t* bsrc[T::NB];
  int blds[T::NB], bk[T::NB];
  bool bok[T::NB];
#pragma unroll
  for (int j = 0; j < T::NB; ++j) {
    const int c = (t + NT * j) < T::BCH ? t + NT * j : T::BCH - 1;
    const int cr = c / 4;                                     // 0 .. 3 TN - 1: part cr / TN, column cr % TN
    const int64_t col = c0 + cr % T::TN;
    bok[j] = col < N;
    bsrc[j] = Pb + ((int64_t)(cr / T::TN) * N + (bok[j] ? col : 0)) * g.sbc;
    blds[j] = lds_at(T::TM + cr, c % 4);
    bk[j] = 8 * (c % 4);
  }

  // VEC (k-contiguous operands, depth a multiple of KS): loads are unconditional and unmasked.  Rows of A past m
  // read row 0 and columns past N read column 0; they only feed rows / columns of E that are never stored.
  // Otherwise every element is loaded with its own bounds check and zero-filled.
  u32x4 ra[T::NA], rb[T::NB];
  auto load = [&](int st) {
    const int64_t k0 = kbeg + (int64_t)st * KS;
    if constexpr (VEC) {
#pragma unroll
      for (int j = 0; j < T::NA; ++j) {
        if constexpr (MODE == SDC_FP8)
          ra[j] = fp8x8_to_bf16(*reinterpret_cast<const u32x2*>(asrc[j] + (k0 + ak[j])));
        else
          ra[j] = *reinterpret_cast<const u32x4*>(asrc[j] + (k0 + ak[j]) * 2);
      }
#pragma unroll
      for (int j = 0; j < T::NB; ++j) rb[j] = *reinterpret_cast<const u32x4*>(bsrc[j] + (k0 + bk[j]));
    } else {
#pragma unroll
      for (int j = 0; j < T::NA; ++j) {
        if constexpr (MODE == SDC_FP8) ra[j] = load8_fp8(asrc[j], g.sak, k0 + ak[j], kend, aok[j]);
        else ra[j] = load8<false>((const uint16_t*)asrc[j], g.sak, k0 + ak[j], kend, aok[j]);
      }
#pragma unroll
      for (int j = 0; j < T::NB; ++j) rb[j] = load8<false>(bsrc[j], 1, k0 + bk[j], kend, bok[j]);
    }
  };
  float sq[T::NA], ab[T::NA];
#pragma unroll
  for (int j = 0; j < T::NA; ++j) sq[j] = ab[j] = 0.f;
  // counted: this store holds a stage of the slice (not a repeat past the last one), so its A rows add to the norms
  auto store = [&](int buf, bool counted) {
    uint16_t* L = lds[buf];
#pragma unroll
    for (int j = 0; j < T::NA; ++j) {
      *reinterpret_cast<u32x4*>(&L[alds[j]]) = ra[j];
      if constexpr (MODE != SDC_I8)
        if (norms && counted && t + NT * j < T::ACH) norm_acc<DT>(ra[j], sq[j], ab[j]);
    }
#pragma unroll
    for (int j = 0; j < T::NB; ++j) *reinterpret_cast<u32x4*>(&L[blds[j]]) = rb[j];
  };

  f32x16 acc[NACC][2][2];
#pragma unroll
  for (int q = 0; q < NACC; ++q)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int n = 0; n < 2; ++n)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[q][i][n][r] = 0.f;         // (int8: the bits of integer 0)

  // the fragments of one MFMA step (16 deep): A rows of this wave, B columns of the NP parts
  struct Frag {
    u32x4 a[2], b[NP][2];
  };
  auto read = [&](Frag& f, int buf, int step) {
    const uint16_t* L = lds[buf];
    const int q = 2 * step + (lane >> 5);
#pragma unroll
    for (int i = 0; i < 2; ++i) f.a[i] = *reinterpret_cast<const u32x4*>(&L[lds_at(wm * 64 + 32 * i + (lane & 31), q)]);
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int n = 0; n < 2; ++n)
        f.b[p][n] = *reinterpret_cast<const u32x4*>(&L[lds_at(T::TM + p * T::TN + wn * 64 + 32 * n + (lane & 31), q)]);
  };
  auto mma = [&](const Frag& f) {
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int n = 0; n < 2; ++n) {
        if constexpr (MODE == SDC_I8) {
          acc[p][0][n] = mfma32_i8(f.a[0], f.b[p][n], acc[p][0][n]);
          acc[p][1][n] = mfma32_i8(f.a[1], f.b[p][n], acc[p][1][n]);
        } else {
          acc[0][0][n] = mfma32<DT>(f.a[0], f.b[p][n], acc[0][0][n]);
          acc[0][1][n] = mfma32<DT>(f.a[1], f.b[p][n], acc[0][1][n]);
        }
      }
  };

  if constexpr (DIRECT) {
    // Global memory straight into LDS (global_load_lds_dwordx4): one instruction of a wave fills 16 consecutive
    // tile rows, lane L the 16 bytes at position L % 4 of row L / 4, i.e. the chunk that the swizzle puts there.
    // The tile's ROWS / 16 instructions per stage are dealt round-robin to the 8 waves (indexes past the end repeat
    // the last one: the same bytes written twice).  Stage s + 3 is loaded during stage s into the buffer of stage
    // s, after the barrier in the middle of stage s that follows every wave's last read of it; the wait before that
    // barrier leaves only stage s + 2 in flight, so stage s + 1 is complete when its first fragments are read.
    constexpr int NI = T::ROWS / 16;                           // load instructions per stage
    constexpr int NIW = (NI + 7) / 8;                           // per wave
    const uint8_t* src[NIW];
    int dst[NIW];
#pragma unroll
    for (int j = 0; j < NIW; ++j) {
      const int I = (w + 8 * j) < NI ? w + 8 * j : NI - 1;
      const int R = 16 * I + lane / 4, P = lane % 4;
      const int q = P ^ ((R >> 1) & 3);
      dst[j] = 16 * I * KS;
      if (R < T::TM) {
        const int64_t row = r0 + R;
        src[j] = Ab + (row < m ? row : 0) * g.sam * 2 + 16 * q;
      } else {
        const int cr = R - T::TM;
        const int64_t col = c0 + cr % T::TN;
        src[j] = reinterpret_cast<const uint8_t*>(Pb + ((int64_t)(cr / T::TN) * N + (col < N ? col : 0)) * g.sbc) + 16 * q;
      }
    }
    auto issue = [&](int st, int buf) {
      const int64_t off = (kbeg + (int64_t)st * KS) * 2;
#pragma unroll
      for (int j = 0; j < NIW; ++j)
        lds_load16(src[j] + off, &lds[buf][dst[j]]);
    };
    if (nst > 0) {
      const int last = nst - 1;
      issue(0, 0);
      issue(1 < last ? 1 : last, 1);
      issue(2 < last ? 2 : last, 2);
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * NIW));        // stage 0 in LDS (stages 1, 2 may be in flight)
      __syncthreads();
      Frag fx, fy;
      read(fx, 0, 0);
      // (the reads of fx complete under the MFMAs that follow them; waiting for them at the end of a stage, where
      // it costs nothing, keeps the compiler from waiting for the next fragments too at the top of the loop)
      __builtin_amdgcn_s_waitcnt(lgkmcnt0_imm());
      int b0 = 0, b1 = 1;                                      // buffers of stages s, s + 1
      for (int s = 0; s < nst; ++s) {
        read(fy, b0, 1);
        __builtin_amdgcn_sched_barrier(0);
        mma(fx);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(NIW));          // stage s + 1 in LDS (stage s + 2 may be in flight)
        __syncthreads();
        issue(s + 3 < last ? s + 3 : last, b0);
        read(fx, b1, 0);
        __builtin_amdgcn_sched_barrier(0);
        mma(fy);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(lgkmcnt0_imm());
        b0 = b1;
        b1 = b1 == NBUF - 1 ? 0 : b1 + 1;
      }
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));              // no load into LDS outlives the workgroup
    }
  } else {
    if (nst > 0) {
      const int last = nst - 1;
      load(0);
      store(0, true);
      load(1 < last ? 1 : last);
      store(1, nst > 1);
      __syncthreads();
      Frag fx, fy;
      read(fx, 0, 0);
      load(2 < last ? 2 : last);
      int b0 = 0, b1 = 1, b2 = 2;                       // buffers of stages s, s + 1, s + 2
      for (int s = 0; s < nst; ++s) {
        // (the scheduling barriers keep each group of reads ahead of the MFMAs it overlaps)
        read(fy, b0, 1);
        __builtin_amdgcn_sched_barrier(0);
        mma(fx);
        __builtin_amdgcn_sched_barrier(0);
        read(fx, b1, 0);
        __builtin_amdgcn_sched_barrier(0);
        mma(fy);
        __builtin_amdgcn_sched_barrier(0);
        store(b2, s + 2 < nst);
        load(s + 3 < last ? s + 3 : last);
        __syncthreads();
        const int bt = b0;
        b0 = b1;
        b1 = b2;
        b2 = bt;
      }
    }
  }

  // C[i][j] of a 32x32 MFMA tile sits in lane j + 32 * ((i / 4) % 2), register (i / 8) * 4 + i % 4
  // (transposed planes: each lane's 4 consecutive registers are 4 consecutive rows, one 16-byte store).  int8: the
  // two digit planes of a split are adjacent planes, their values the int32 bits.
#pragma unroll
  for (int pa = 0; pa < NACC; ++pa) {
    float* Es = g.E + ((eb * g.splits + split) * NACC + pa) * me * N;
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      const int64_t col = c0 + wn * 64 + 32 * n + (lane & 31);
      if (col < N) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4) {
            const int64_t row = r0 + wm * 64 + i * 32 + 8 * r4 + 4 * (lane >> 5);
            const f32x16& av = acc[pa][i][n];
            if (g.et && row + 4 <= m && (me % 4) == 0 && (row % 4) == 0) {
              f32x4 v = {av[4 * r4], av[4 * r4 + 1], av[4 * r4 + 2], av[4 * r4 + 3]};
              *reinterpret_cast<f32x4*>(&Es[col * me + row]) = v;
            } else {
#pragma unroll
              for (int q = 0; q < 4; ++q)
                if (row + q < m) Es[g.et ? col * me + row + q : (row + q) * N + col] = av[4 * r4 + q];
            }
          }
      }
    }
  }
  if (norms && MODE != SDC_I8) {
    float* xs = g.XN + (eb * g.splits + split) * 2 * me;
#pragma unroll
    for (int j = 0; j < T::NA; ++j) {
      float q = sq[j], a1 = ab[j];
      q += __shfl_xor(q, 1, 64);
      a1 += __shfl_xor(a1, 1, 64);
      q += __shfl_xor(q, 2, 64);
      a1 += __shfl_xor(a1, 2, 64);
      const int c = t + NT * j;
      const int64_t row = r0 + c / 4;
      if ((c & 3) == 0 && c < T::ACH && row < m) {
        xs[row] = q;
        xs[me + row] = a1;
      }
    }
  }
}

template <int MODE, int WGN>
int launch_dt(GemmArgs g, bool vec, int64_t blocks, hipStream_t stream) {
  // straight-to-LDS loads for k-contiguous 16-bit (or int8 pair) operands when no row norms are asked for
  bool direct = false;
  if constexpr (MODE != SDC_FP8) {
    if (vec && g.XN == nullptr) {
      hipLaunchKernelGGL((expected_gemm_kernel<MODE, WGN, true, true>), dim3((unsigned)blocks), dim3(NT), 0, stream, g);
      direct = true;
    }
  }
  if (direct) {
  } else if (vec)
    hipLaunchKernelGGL((expected_gemm_kernel<MODE, WGN, true, false>), dim3((unsigned)blocks), dim3(NT), 0, stream, g);
  else hipLaunchKernelGGL((expected_gemm_kernel<MODE, WGN, false, false>), dim3((unsigned)blocks), dim3(NT), 0, stream, g);
  SDC_LAUNCH_CHECK();
  return SDC_OK;
}

template <int MODE>
int launch_mode(GemmArgs g, bool vec, int wgn, int64_t blocks, hipStream_t stream) {
  return wgn == 2 ? launch_dt<MODE, 2>(g, vec, blocks, stream) : launch_dt<MODE, 1>(g, vec, blocks, stream);
}

// fp32 B2^T columns -> three parts (dtype), each column divided by its power of two first (exact)
struct SplitArgs {
  const float* B2T;                 // [batch][ncols][k]
  const float* scale;               // scale[batch * sscb + col * scale_stride], or null (1)
  int64_t sscb, scale_stride;
  int64_t ncols, k, kp, batches;
  uint16_t* parts;                  // [batch][3 * ncols][kp]
};

template <int DT>
__global__ __launch_bounds__(256) void split_kernel(SplitArgs a) {
  const int64_t nch = sdc_cdiv(a.kp, 8);
  const int64_t total = a.batches * a.ncols * nch;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t ch = i % nch, cb = i / nch, col = cb % a.ncols, bb = cb / a.ncols;
    const float inv = a.scale ? 1.f / a.scale[bb * a.sscb + col * a.scale_stride] : 1.f;
    const float* src = a.B2T + cb * a.k;
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int64_t kk = 8 * ch + e;
      v[e] = kk < a.k ? src[kk] * inv : 0.f;
    }
    u32x4 pr[3];
    split8<DT>(v, pr);
#pragma unroll
    for (int p = 0; p < 3; ++p)
      *reinterpret_cast<u32x4*>(a.parts + ((bb * 3 + p) * a.ncols + col) * a.kp + 8 * ch) = pr[p];
  }
}

// ---------------------------------------------------------------------------------- register-streamed GEMM
// E = A @ (three parts of the block sums) with no depth split across workgroups.  A workgroup of 4 waves owns a
// 64 x 64 tile of E (64 rows of A, 64 checksum columns) over the whole depth; wave q takes the q-th quarter of the
// 64-deep segments, and the waves never wait for each other until the end.
//
// Depth order inside a segment: lane l (row or column l % 32, half h = l / 32) takes the 16-byte pieces 4 h + j
// (j = 0 .. 3) of its 128-byte row segment, and step j multiplies depths {8 j .. 8 j + 7} u {32 + 8 j .. 32 + 8 j
// + 7} -- the same ones in A and B -- so the four steps cover the segment.
// A (the operand read once from HBM) goes through a ring of LDS buffers private to the wave, filled by
// global_load_lds two segments ahead: each of the 8 instructions of a segment reads 8 rows x 128 bytes (whole
// lines: HBM streams those at twice the rate of the MFMA lane order's 32-byte pieces), lane L the piece
// (L % 8) ^ (L / 8) of row L / 8, landing at 16 L; so the fragment reads (8 lanes of a phase: 8 rows, one piece)
// hit 8 different 16-byte bank groups.  B comes in fragment order (sdc_parts_fragments): the fragment of (step,
// part, 32 columns) is 1024 contiguous bytes, lane l's 16 at 16 l; loaded straight into registers RB steps ahead.
// (Measured on MI355X: the loop is bound by the vector memory path mixing A's HBM misses with B's cache hits, not
// by the matrix cores; more waves, a deeper B ring or staggered depth orders did not speed it up.)
// Every wave has the same number of segments (the depth is a multiple of 256).  The four waves' accumulators meet
// in LDS and are added in wave (depth) order, so E is the same on every run; one plane, stored transposed
// (E[col][row]).
constexpr int RS_WAVES = 4;
constexpr int RS_KMULT = 64 * RS_WAVES;       // depth granularity of the register-streamed GEMM
constexpr int RS_RB = 4;                      // B's ring (steps); 8 measured no faster
constexpr int RS_SEGB = 64 * 128;             // bytes of A per wave and segment (64 rows x 128 bytes)

// ROLE only names the kernel apart (0: the column check's GEMM, 1: the row check's), for per-kernel profiles.
template <int DT, int RB, int ROLE>
__global__ __launch_bounds__(64 * RS_WAVES, 1) void rs_gemm_kernel(GemmArgs g) {
  constexpr int TRF = 2, TCF = 2, TR = 64, TC = 64, NG = TRF * TCF * 4;   // f32x4 groups of a wave's accumulators
  constexpr int SPB = RB / 4;                                   // segments per loop iteration (B's ring: RB steps)
  constexpr int ABUF = SPB + 2;                                 // A's ring: ABUF - 1 segments ahead
  __shared__ __attribute__((aligned(16))) uint8_t smem[RS_WAVES * ABUF * RS_SEGB];
  const int t = threadIdx.x, lane = t & 63;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);
  const int r = lane & 31, h = lane >> 5;
  const int64_t N = g.N, m = g.m;
  const int64_t nct = sdc_cdiv(N, TC), ncf = sdc_cdiv(N, 32);
  // XCD-aware order: block b runs on XCD b % 8; XCD x takes the x-th eighth of the tiles, column tiles fastest (the
  // column tiles of one row tile share their rows of A in that XCD's L2)
  const int64_t G = (int64_t)gridDim.x, b = blockIdx.x;
  const int64_t wid = (G % 8 == 0) ? (b % 8) * (G / 8) + b / 8 : b;
  const int64_t ct = wid % nct, rt = wid / nct;
  const int64_t r0 = rt * TR, c0 = ct * TC;
  const int per = (int)(g.k / 64) / RS_WAVES;                   // segments per wave (the depth is a multiple of 256)
  const int seg0 = w * per;
  uint8_t* const abuf = smem + w * ABUF * RS_SEGB;
  // fragment reads: frag i, step j -> row R = 32 i + r, piece 4 h + j -> slot 8 (R % 8) + ((4 h + j) ^ (R % 8)) of
  // block R / 8
  int ard[TRF][4];
#pragma unroll
  for (int i = 0; i < TRF; ++i)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int R = 32 * i + r, rr = R & 7;
      ard[i][jj] = (R >> 3) * 1024 + 16 * (8 * rr + ((4 * h + jj) ^ rr));
    }
  // fragment (step s, part p, column fragment f) at B + ((s * 3 + p) * ncf + f) * 512 elements; column fragments
  // past the last are replaced by the last one (their columns of E are never stored)
  const uint16_t* bq = (const uint16_t*)g.B + (int64_t)(4 * seg0) * 3 * ncf * 512 + 8 * lane;
  int bf[TCF];
#pragma unroll
  for (int n = 0; n < TCF; ++n) {
    const int64_t f = c0 / 32 + n;
    bf[n] = (int)((f < ncf ? f : ncf - 1) * 512);
  }
  const int64_t bstep = 3 * ncf * 512;                          // elements per step of B
  const int lastseg = per - 1;
  const int last = 4 * per - 1;
  // A's loads: instruction I (0 .. 7) of a segment, lane L: row 8 I + L / 8 (rows past m read row m - 1; they only
  // feed rows of E that are never stored), piece (L % 8) ^ (L / 8)
  const uint8_t* aptr[8];
#pragma unroll
  for (int I = 0; I < 8; ++I) {
    const int64_t row = r0 + 8 * I + (lane >> 3);
    const int pc = (lane & 7) ^ (lane >> 3);
    aptr[I] = (const uint8_t*)g.A + ((row < m ? row : m - 1) * g.sam + 64 * (int64_t)seg0) * 2 + 16 * pc;
  }

  u32x4 rb[RB][3][TCF];
  // two of the 8 instructions of segment sg of A (into its ring buffer)
  auto issue_a2 = [&](int sg, int I0) {
    const int s2 = sg < lastseg ? sg : lastseg;
    uint8_t* dst = abuf + (sg % ABUF) * RS_SEGB;
#pragma unroll
    for (int I = I0; I < I0 + 2; ++I) sdc_pipe::lds_load16(aptr[I] + 128 * (int64_t)s2, (uint16_t*)(dst + 1024 * I));
  };
  // B's loads and A's fragment reads are written out (global_load_dwordx4, ds_read_b128) and every wait is explicit:
  // left to the compiler, a read of the LDS ring waits for all loads into LDS (it cannot tell the buffers apart) and
  // the loop head waits for every load in flight.  Each B register is loaded in place ("+v": the register keeps its
  // value's place across the loop) and passes through the s_waitcnt that covers its load ("+v" again) before an
  // MFMA reads it.  smem is the kernel's only LDS object, so its LDS address is the low 32 bits of its generic
  // address.
  auto issue_b = [&](int slot, int st) {
    const uint16_t* q = bq + (int64_t)(st < last ? st : last) * bstep;
#pragma unroll
    for (int p = 0; p < 3; ++p)
#pragma unroll
      for (int n = 0; n < TCF; ++n)
        asm volatile("global_load_dwordx4 %0, %1, off" : "+v"(rb[slot][p][n]) : "v"(q + p * ncf * 512 + bf[n]));
  };
  const uint32_t lds0 = (uint32_t)(uintptr_t)abuf;
  f32x16 acc[TRF][TCF];
#pragma unroll
  for (int i = 0; i < TRF; ++i)
#pragma unroll
    for (int n = 0; n < TCF; ++n)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][n][e] = 0.f;
#pragma unroll
  for (int q = 0; q < RB; ++q)
#pragma unroll
    for (int p = 0; p < 3; ++p)
#pragma unroll
      for (int n = 0; n < TCF; ++n) rb[q][p][n] = u32x4{0u, 0u, 0u, 0u};
  if (per > 0) {
    // every step issues 3 TCF loads of B (RB steps ahead), then two of the 8 instructions of the segment ABUF - 1
    // ahead of A; the prologue issues them as the steps before the first would.  So when step st begins, the loads
    // issued after B(st) are the two of A in its step and the 3 TCF + 2 of each of the RB - 1 steps between: a
    // constant, 8 RB - 6; the last loads of the step's segment of A were issued more than RB steps earlier.
    for (int sgv = 0; sgv < ABUF - 1 - SPB; ++sgv)
#pragma unroll
      for (int I = 0; I < 8; I += 2) issue_a2(sgv, I);
#pragma unroll
    for (int q = 0; q < RB; ++q) {
      issue_b(q, q);
      issue_a2(q / 4 + ABUF - 1 - SPB, 2 * (q % 4));
    }
    for (int sg = 0; sg < per; sg += SPB) {
#pragma unroll
      for (int u = 0; u < SPB; ++u) {
        const uint32_t L = lds0 + (uint32_t)(((sg + u) % ABUF) * RS_SEGB);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int q = 4 * u + jj;                            // B's slot of this step
          static_assert(TCF == 2 && 8 * RB - 6 <= 63, "6 + 2 loads per step, at most 63 in flight");
          asm volatile("s_waitcnt vmcnt(%6)"
                       : "+v"(rb[q][0][0]), "+v"(rb[q][0][1]), "+v"(rb[q][1][0]), "+v"(rb[q][1][1]),
                         "+v"(rb[q][2][0]), "+v"(rb[q][2][1])
                       : "n"(8 * RB - 6));
          u32x4 a0, a1;
          asm volatile("ds_read_b128 %0, %1" : "=v"(a0) : "v"(L + (uint32_t)ard[0][jj]));
          asm volatile("ds_read_b128 %0, %1" : "=v"(a1) : "v"(L + (uint32_t)ard[1][jj]));
          asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a0), "+v"(a1));
          const u32x4 a[TRF] = {a0, a1};
#pragma unroll
          for (int p = 0; p < 3; ++p)
#pragma unroll
            for (int i = 0; i < TRF; ++i)
#pragma unroll
              for (int n = 0; n < TCF; ++n) acc[i][n] = sdc_pipe::mfma32<DT>(a[i], rb[q][p][n], acc[i][n]);
          __builtin_amdgcn_sched_barrier(0);
          issue_b(q, 4 * (sg + u) + jj + RB);
          issue_a2(sg + u + ABUF - 1, 2 * jj);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
    // every load done before the loop's registers are reused (the last steps' B loads land in registers nothing
    // reads again) and before the workgroup's LDS is
    asm volatile("s_waitcnt vmcnt(0)"
                 : "+v"(rb[0][0][0]), "+v"(rb[0][0][1]), "+v"(rb[0][1][0]), "+v"(rb[0][1][1]), "+v"(rb[0][2][0]),
                   "+v"(rb[0][2][1]));
#pragma unroll
    for (int q = 1; q < RB; ++q)
      asm volatile("" : "+v"(rb[q][0][0]), "+v"(rb[q][0][1]), "+v"(rb[q][1][0]), "+v"(rb[q][1][1]), "+v"(rb[q][2][0]),
                   "+v"(rb[q][2][1]));
    __builtin_amdgcn_sched_barrier(0);
  }
  __syncthreads();                                             // (the epilogue's LDS overlaps other waves' A)
  // the waves' accumulators, added in wave order; group (i, n, r4) of a lane holds rows 8 r4 + 4 h .. + 3 of
  // fragment row i, column l % 32 of fragment column n
  f32x4* red = reinterpret_cast<f32x4*>(smem);                  // [RS_WAVES][NG][64]
#pragma unroll
  for (int i = 0; i < TRF; ++i)
#pragma unroll
    for (int n = 0; n < TCF; ++n)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4)
        red[(w * NG + (i * TCF + n) * 4 + r4) * 64 + lane] =
            f32x4{acc[i][n][4 * r4], acc[i][n][4 * r4 + 1], acc[i][n][4 * r4 + 2], acc[i][n][4 * r4 + 3]};
  __syncthreads();
  const int64_t me = g.m;
#pragma unroll
  for (int gq = 0; gq < NG / RS_WAVES; ++gq) {
    const int gi = w * (NG / RS_WAVES) + gq;
    f32x4 v = red[gi * 64 + lane];
#pragma unroll
    for (int q = 1; q < RS_WAVES; ++q) v += red[(q * NG + gi) * 64 + lane];
    const int i = gi / (4 * TCF), n = (gi / 4) % TCF, r4 = gi % 4;
    const int64_t row = r0 + 32 * i + 8 * r4 + 4 * h;
    const int64_t col = c0 + 32 * n + r;
    if (col < N) {
      float* Ec = g.E + col * me;
      if (row + 4 <= m && (me % 4) == 0) {
        *reinterpret_cast<f32x4*>(Ec + row) = v;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (row + e < m) Ec[row + e] = v[e];
      }
    }
  }
}

// ------------------------------------------------------------------------- register-streamed GEMM, tall tiles
// The same loop with 128 rows of A per wave: each B fragment loaded from L2 meets twice the rows, so a workgroup
// moves 36% fewer bytes through the vector memory path per MFMA (1.25 MB instead of 2 MB for the same 64 x 64 x
// 4096 worth of products).  The workgroup tile is 128 x 64 over half the depth; the two halves are separate
// workgroups, each writing its own plane of E (plane h = depth half h), which the scoring pass adds in half order.
// A's ring per wave is two 16 KB segments (128 rows x 128 bytes; 128 KB for the 4 waves), the next segment loading
// while the current one is read.  A segment is 64 depths of a 16-bit A, or 128 of an fp8 A (AT = 1: one byte per
// element, widened exactly to bf16 after the LDS read; the MFMAs are bf16), so 4 or 8 steps of 16 depths.  Per step
// a wave issues its share of the next segment's 16 A instructions (APS = 16 / steps), then the B fragments RB
// steps ahead.  So at a step's wait, the loads issued after B(st) are (RB - 1) (APS + 6) and, at the first step of
// a segment, those after the segment's last A piece are the 6 B loads of one step: the wait is
// vmcnt((RB - 1) (APS + 6)) inside a segment and vmcnt(6) at its first step.
// XN: the workgroups of the first column tile also add up |a_row|_2^2 and |a_row|_1 of their rows (from the A
// fragments, over their depth half) into plane `half` of g.XN ([half][2][m]).
// XCD order: XCDs 0-3 take depth half 0 and 4-7 half 1 (each XCD's L2 holds its half of B), row tiles in order.
#ifndef SDC_TALL_TRF
#define SDC_TALL_TRF 4
#endif

constexpr int GSCAN = 1024;                       // groups the grouped tall GEMM takes

// TCF: 32-column fragments a tile (2; 1 for outputs of at most 32 columns, whose second fragment would be empty)
template <int DT, int ROLE, int TRF, int AT, bool XNORM, bool GROUPED = false, int TCF = 2>
__global__ __launch_bounds__(64 * RS_WAVES, TRF == 4 ? 1 : 2) void rs_gemm_tall_kernel(GemmArgs g) {
  constexpr int MDT = AT ? SDC_BF16 : DT;       // the MFMAs' type (AT 2: int8)
  constexpr int SPS = AT ? 8 : 4;               // steps per segment
  constexpr int SD = 16 * SPS;                  // depths per segment
  constexpr int ES = AT ? 1 : 2;                // bytes per A element
  constexpr int NP = AT == 2 ? 2 : 3;           // B parts (int8: the block sums' two base-128 digits)
  constexpr int NACC = AT == 2 ? 2 : 1;         // accumulator sets (int8: one per digit, exact int32)
  constexpr int FRAG = AT == 2 ? 256 : 512;     // 16-bit units per B fragment (int8: 8 bytes a lane)
  static_assert(AT != 2 || (TRF == 2 && !XNORM && !GROUPED), "int8: 64-row tiles, no row norms");
  static_assert(TCF == 1 || TCF == 2, "one or two column fragments a tile");
  constexpr int TR = 32 * TRF, TC = 32 * TCF, RB = 4, NAI = TR / 8, APS = NAI / SPS;
  constexpr int RT_SEGB = TR * 128;             // bytes of A per wave and segment (TR rows x 128 bytes)
  constexpr int RED_BYTES = RS_WAVES * TC * (TR + 4) * 4;       // the epilogue's reduction (below)
  __shared__ __attribute__((aligned(16)))
  uint8_t smem[RS_WAVES * 2 * RT_SEGB > RED_BYTES ? RS_WAVES * 2 * RT_SEGB : RED_BYTES];
  __shared__ float xred[XNORM ? RS_WAVES : 1][XNORM ? TR : 1][2];
  const int t = threadIdx.x, lane = t & 63;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);
  const int r = lane & 31, h = lane >> 5;
  const int64_t N = g.N, m = g.m;
  // (tile indices in 32 bits, their divisions by run-time divisors the short unsigned ones: the launcher keeps the
  // grid, and so every tile count, below 2^31)
  const uint32_t nct = ((uint32_t)N + TC - 1) / TC, ncf = ((uint32_t)N + 31) / 32;
  const uint32_t G = gridDim.x - (uint32_t)g.xf_blocks, b = blockIdx.x;
  if (b >= G) {
    xfinish_block(g.xf, (int64_t)(b - G), t);     // (a spare workgroup: the x pass's finishing step)
    return;
  }
  const uint32_t wid = (G % 8 == 0) ? (b % 8) * (G / 8) + b / 8 : b;
  uint32_t tile, half;
  int64_t r0, rend, grp = 0;
  if constexpr (GROUPED) {
    // grouped rows (g.goffs: the groups' cumulative ends): a row tile never crosses a group, so group q has
    // ceil(rows_q / TR) row tiles; their running count comes from the ends in LDS (a scan over the groups), and
    // the grid covers (ceil(m / TR) + groups) row tiles per column tile and half -- workgroups past the last exit
    __shared__ int64_t gend[GSCAN], gtile[GSCAN];
    const int ng = (int)g.ngroups;
    for (int q = t; q < ng; q += 64 * RS_WAVES) {
      const int64_t e = min(max(g.goffs[q], (int64_t)0), m), s0 = q ? min(max(g.goffs[q - 1], (int64_t)0), m) : 0;
      gend[q] = e;
      gtile[q] = e > s0 ? sdc_cdiv(e - s0, TR) : 0;
    }
    __syncthreads();
    if (w == 0) {
      // the inclusive running count (1024 groups at most), 64 groups at a time: a shuffle scan across the wave,
      // plus the running total of the chunks before
      int64_t carry = 0;
      for (int q0 = 0; q0 < ng; q0 += 64) {
        const int q = q0 + lane;
        int64_t c = q < ng ? gtile[q] : 0;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
          const int64_t u = __shfl_up(c, d, 64);
          c += lane >= d ? u : 0;
        }
        c += carry;
        if (q < ng) gtile[q] = c;
        carry = __shfl(c, 63, 64);
      }
    }
    __syncthreads();
    const uint32_t tiles = ((uint32_t)((m + TR - 1) / TR) + (uint32_t)ng) * nct;
    half = wid / tiles;
    tile = wid - half * tiles;
    const int64_t rt = tile / nct;
    if (rt >= gtile[ng - 1] || (int64_t)half >= g.splits) return;
    int lo = 0, hi = ng - 1;                                     // first group whose running count exceeds rt
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (gtile[mid] > rt) hi = mid;
      else lo = mid + 1;
    }
    grp = lo;
    const int64_t gs = grp ? gend[grp - 1] : 0, lt = rt - (grp ? gtile[grp - 1] : 0);
    r0 = gs + lt * TR;
    rend = gend[grp];
  } else {
    const uint32_t tiles = (uint32_t)((m + TR - 1) / TR) * nct;
    half = wid / tiles;
    tile = wid - half * tiles;
    r0 = (int64_t)(tile / nct) * TR;
    rend = m;
  }
  const uint32_t ct = tile % nct;
  const int64_t c0 = (int64_t)ct * TC;
  const bool do_xn = XNORM && ct == 0;
  const int per = (int)((uint32_t)(g.k / SD) / (uint32_t)(RS_WAVES * g.splits));   // segments per wave
  const int seg0 = (int)half * per * RS_WAVES + w * per;
  uint8_t* const abuf = smem + w * 2 * RT_SEGB;
  // LDS address of fragment i (rows 32 i + r) at step jj of a segment: the 16-bit depth piece 4 h + jj, or the
  // fp8 byte offset 64 (jj / 4) + 32 h + 8 (jj % 4) (its 16-byte chunk c, swizzled by the row, and half of it)
  int ard[TRF][SPS];
#pragma unroll
  for (int i = 0; i < TRF; ++i)
#pragma unroll
    for (int jj = 0; jj < SPS; ++jj) {
      const int R = 32 * i + r, rr = R & 7;
      if constexpr (AT) {
        const int o = 64 * (jj / 4) + 32 * h + 8 * (jj % 4);
        ard[i][jj] = (R >> 3) * 1024 + 16 * (8 * rr + ((o >> 4) ^ rr)) + (o & 15);
      } else {
        ard[i][jj] = (R >> 3) * 1024 + 16 * (8 * rr + ((4 * h + jj) ^ rr));
      }
    }
  const uint16_t* bq =
      (const uint16_t*)g.B + grp * g.sbb + (int64_t)(SPS * seg0) * NP * (int64_t)ncf * FRAG + (FRAG / 64) * lane;
  int bf[TCF];
#pragma unroll
  for (int n = 0; n < TCF; ++n) {
    const uint32_t f = (uint32_t)(c0 / 32) + n;
    bf[n] = (int)((f < ncf ? f : ncf - 1) * FRAG);
  }
  const int64_t bstep = NP * (int64_t)ncf * FRAG;
  const int lastseg = per - 1;
  const int last = SPS * per - 1;
  // A's instruction I (0 .. 15) of a segment, lane L: row 8 I + L / 8 (clamped to m - 1), 16-byte piece
  // (L % 8) ^ (L / 8) of the row's 128 bytes
  const uint8_t* abase = (const uint8_t*)g.A + (SD * (int64_t)seg0) * ES + 16 * ((lane & 7) ^ (lane >> 3));
  int64_t arow[NAI];
#pragma unroll
  for (int I = 0; I < NAI; ++I) {
    const int64_t row = r0 + 8 * I + (lane >> 3);
    arow[I] = (row < rend ? row : rend - 1) * g.sam * ES;
  }
  using BT = typename std::conditional<AT == 2, u32x2, u32x4>::type;
  BT rb[RB][NP][TCF];
  // A instruction I of segment sg into its half of the ring (past the last segment: the last again)
  auto issue_a1 = [&](int sg, int I) {
    const int s2 = sg < lastseg ? sg : lastseg;
    uint8_t* dst = abuf + (sg & 1) * RT_SEGB;
    sdc_pipe::lds_load16(abase + arow[I] + 128 * (int64_t)s2, (uint16_t*)(dst + 1024 * I));
  };
  auto issue_a4 = [&](int sg, int I0) {
#pragma unroll
    for (int I = I0; I < I0 + APS; ++I) issue_a1(sg, I);
  };
  // column fragment n of part p of B(st) into slot `slot`
  auto issue_b1 = [&](int slot, int st, int p, int n) {
    const uint16_t* q = bq + (int64_t)(st < last ? st : last) * bstep + p * ncf * FRAG;
    if constexpr (AT == 2) asm volatile("global_load_dwordx2 %0, %1, off" : "+v"(rb[slot][p][n]) : "v"(q + bf[n]));
    else asm volatile("global_load_dwordx4 %0, %1, off" : "+v"(rb[slot][p][n]) : "v"(q + bf[n]));
  };
  auto issue_bp = [&](int slot, int st, int p) {
#pragma unroll
    for (int n = 0; n < TCF; ++n) issue_b1(slot, st, p, n);
  };
  auto issue_b = [&](int slot, int st) {
#pragma unroll
    for (int p = 0; p < NP; ++p) issue_bp(slot, st, p);
  };
  // fragment reads of step jj into fr (fp8: 8 bytes each, widened after the wait).  Each read lands in the very
  // registers the wait names ("=v" then "+v"): a copy out of an asm read's result before its wait would copy data
  // that has not arrived.
  using FragT = typename std::conditional<AT != 0, u32x2, u32x4>::type;
  // s_waitcnt vmcnt(C) naming B slot `slot`'s registers (so nothing reads them before the wait), and a no-op that
  // names a slot's registers (so the loads into them count as used)
#define SDC_TALL_WAIT_B(C, slot)                                                                                   \
  do {                                                                                                            \
    if constexpr (NP == 3 && TCF == 2)                                                                            \
      asm volatile("s_waitcnt vmcnt(%6)"                                                                          \
                   : "+v"(rb[slot][0][0]), "+v"(rb[slot][0][TCF - 1]), "+v"(rb[slot][1][0]),                      \
                     "+v"(rb[slot][1][TCF - 1]), "+v"(rb[slot][NP - 1][0]), "+v"(rb[slot][NP - 1][TCF - 1])       \
                   : "n"(C));                                                                                     \
    else if constexpr (TCF == 2)                                                                                  \
      asm volatile("s_waitcnt vmcnt(%4)"                                                                          \
                   : "+v"(rb[slot][0][0]), "+v"(rb[slot][0][TCF - 1]), "+v"(rb[slot][NP - 1][0]),                 \
                     "+v"(rb[slot][NP - 1][TCF - 1])                                                              \
                   : "n"(C));                                                                                     \
    else if constexpr (NP == 3)                                                                                   \
      asm volatile("s_waitcnt vmcnt(%3)"                                                                          \
                   : "+v"(rb[slot][0][0]), "+v"(rb[slot][1][0]), "+v"(rb[slot][NP - 1][0])                        \
                   : "n"(C));                                                                                     \
    else                                                                                                          \
      asm volatile("s_waitcnt vmcnt(%2)" : "+v"(rb[slot][0][0]), "+v"(rb[slot][NP - 1][0]) : "n"(C));             \
  } while (0)
#define SDC_TALL_NAME_B(slot)                                                                                      \
  do {                                                                                                            \
    if constexpr (NP == 3 && TCF == 2)                                                                            \
      asm volatile("" : "+v"(rb[slot][0][0]), "+v"(rb[slot][0][TCF - 1]), "+v"(rb[slot][1][0]),                   \
                   "+v"(rb[slot][1][TCF - 1]), "+v"(rb[slot][NP - 1][0]), "+v"(rb[slot][NP - 1][TCF - 1]));        \
    else if constexpr (TCF == 2)                                                                                  \
      asm volatile("" : "+v"(rb[slot][0][0]), "+v"(rb[slot][0][TCF - 1]), "+v"(rb[slot][NP - 1][0]),              \
                   "+v"(rb[slot][NP - 1][TCF - 1]));                                                              \
    else if constexpr (NP == 3)                                                                                   \
      asm volatile("" : "+v"(rb[slot][0][0]), "+v"(rb[slot][1][0]), "+v"(rb[slot][NP - 1][0]));                   \
    else                                                                                                          \
      asm volatile("" : "+v"(rb[slot][0][0]), "+v"(rb[slot][NP - 1][0]));                                         \
  } while (0)
  auto read_frag1 = [&](uint32_t L, int jj, FragT* fr, int i) {
    if constexpr (AT) asm volatile("ds_read_b64 %0, %1" : "=v"(fr[i]) : "v"(L + (uint32_t)ard[i][jj]));
    else asm volatile("ds_read_b128 %0, %1" : "=v"(fr[i]) : "v"(L + (uint32_t)ard[i][jj]));
  };
  auto read_frags = [&](uint32_t L, int jj, FragT* fr) {
#pragma unroll
    for (int i = 0; i < TRF; ++i) read_frag1(L, jj, fr, i);
  };
  const uint32_t lds0 = (uint32_t)(uintptr_t)abuf;
  f32x16 acc[NACC][TRF][TCF];                   // (int8: the int32 sums' bits)
#pragma unroll
  for (int pa = 0; pa < NACC; ++pa)
#pragma unroll
    for (int i = 0; i < TRF; ++i)
#pragma unroll
      for (int n = 0; n < TCF; ++n)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[pa][i][n][e] = 0.f;
  float xsq[TRF], xab[TRF];
#pragma unroll
  for (int i = 0; i < TRF; ++i) xsq[i] = xab[i] = 0.f;
#pragma unroll
  for (int q = 0; q < RB; ++q)
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int n = 0; n < TCF; ++n) rb[q][p][n] = BT{};
  if (per > 0) {
    // prologue: segment 0's A and B(0 .. 3) as the steps before the first would issue them (its A shares of those
    // steps; with 8 steps a segment, the shares of steps 0 .. 3 go out first)
#pragma unroll
    for (int q = 0; q < SPS - RB; ++q) issue_a4(0, APS * q);
#pragma unroll
    for (int q = 0; q < RB; ++q) {
      issue_a4(0, APS * (q + (SPS - RB)));
      issue_b(q, q);
    }
    // A step issues its MFMAs part by part, each part column by column, and after each MFMA at most one load, so
    // that the load's issue (which stalls the wave while the CU's memory pipeline is busy) overlaps the MFMA just
    // issued instead of leaving the matrix core idle: in part 0 the step's share of the next segment's A (a piece
    // after each of the first APS MFMAs), and in every part each column's B fragment for RB steps ahead, right
    // after the last MFMA that reads that column's registers (in part 0, after the A pieces).  So the loads still
    // go out in the order A, B part 0, 1, 2 that the wait counts assume.  The next step's A fragments are read from
    // LDS during part 1 (inside a segment; the first step of a segment reads its own after the wait).
    FragT fr[2][TRF];
    using AOpT = typename std::conditional<AT == 2, u32x2, u32x4>::type;
    for (int sg = 0; sg < per; ++sg) {
      const uint32_t L = lds0 + (uint32_t)((sg & 1) * RT_SEGB);
#pragma unroll
      for (int jj = 0; jj < SPS; ++jj) {
        static_assert(RB == 4, "the wait counts below assume B four steps ahead");
        const int st = SPS * sg + jj, cur = jj & 1, sl = jj & 3;
        if (jj == 0) {
          SDC_TALL_WAIT_B(NP * TCF, 0);
          read_frags(L, 0, fr[0]);
        } else {
          SDC_TALL_WAIT_B((RB - 1) * (APS + NP * TCF), sl);
        }
        if constexpr (TRF == 4)
          asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(fr[cur][0]), "+v"(fr[cur][1]), "+v"(fr[cur][2]), "+v"(fr[cur][3]));
        else
          asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(fr[cur][0]), "+v"(fr[cur][1]));
        AOpT a[TRF];
#pragma unroll
        for (int i = 0; i < TRF; ++i) {
          if constexpr (AT == 1) a[i] = fp8x8_to_bf16(fr[cur][i]);
          else a[i] = fr[cur][i];
        }
        auto mma = [&](int i, int n, int p) {
          if constexpr (AT == 2)
            acc[p][i][n] = __builtin_bit_cast(
                f32x16, __builtin_amdgcn_mfma_i32_32x32x16_i8(__builtin_bit_cast(long, a[i]),
                                                               __builtin_bit_cast(long, rb[sl][p][n]),
                                                               __builtin_bit_cast(i32x16, acc[p][i][n]), 0, 0, 0));
          else
            acc[0][i][n] = sdc_pipe::mfma32<MDT>(a[i], rb[sl][p][n], acc[0][i][n]);
        };
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
          for (int n = 0; n < TCF; ++n)
#pragma unroll
            for (int i = 0; i < TRF; ++i) {
              const int q = n * TRF + i;                          // the MFMA's place in its part
              mma(i, n, p);
              __builtin_amdgcn_sched_barrier(0);
              if (p == 0 && q < APS) issue_a1(sg + 1, APS * jj + q);
              if (p == 1 && n == 0 && jj < SPS - 1) read_frag1(L, jj + 1, fr[cur ^ 1], i);
#pragma unroll
              for (int c = 0; c < TCF; ++c) {                     // column c's B load: after its last reader (and
                const int qc = c * TRF + TRF - 1;                 // in part 0 after the A pieces, at the part's
                const int qs = p == 0 && qc < APS ? APS : qc;     // last MFMA at the latest)
                if (q == (qs < TRF * TCF ? qs : TRF * TCF - 1)) issue_b1(sl, st + RB, p, c);
              }
              __builtin_amdgcn_sched_barrier(0);
            }
        if constexpr (XNORM) {
          if (do_xn) {
          // the rows' norms over this step's 8 depths of each fragment (packed dot products)
          constexpr uint32_t ONES = MDT == SDC_BF16 ? 0x3F803F80u : 0x3C003C00u;
#pragma unroll
          for (int i = 0; i < TRF; ++i) {
            const uint32_t* ww = reinterpret_cast<const uint32_t*>(&a[i]);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              xsq[i] = pk_dot2<MDT>(ww[q], ww[q], xsq[i]);
              xab[i] = pk_dot2<MDT>(ww[q] & 0x7FFF7FFFu, ONES, xab[i]);
            }
          }
        }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    SDC_TALL_WAIT_B(0, 0);
#pragma unroll
    for (int q = 1; q < RB; ++q) SDC_TALL_NAME_B(q);
    __builtin_amdgcn_sched_barrier(0);
  }
  if constexpr (XNORM) {
    if (do_xn) {
      // the two depth halves of a row (lanes r, r + 32), then the four waves' depth quarters in LDS, in wave order
#pragma unroll
      for (int i = 0; i < TRF; ++i) {
        xsq[i] += __shfl_xor(xsq[i], 32, 64);
        xab[i] += __shfl_xor(xab[i], 32, 64);
        if (h == 0) {
          xred[w][32 * i + r][0] = xsq[i];
          xred[w][32 * i + r][1] = xab[i];
        }
      }
    }
  }
  __syncthreads();
  if constexpr (XNORM) {
    if (do_xn && t < TR) {
      float sq = xred[0][t][0], ab = xred[0][t][1];
#pragma unroll
      for (int q = 1; q < RS_WAVES; ++q) {
        sq += xred[q][t][0];
        ab += xred[q][t][1];
      }
      const int64_t row = r0 + t;
      if (row < rend) {
        g.XN[half * 2 * m + row] = sq;
        g.XN[half * 2 * m + m + row] = ab;
      }
    }
  }
  // The waves' accumulators meet in LDS column by column ([wave][column][row], rows padded to TR + 4 floats so a
  // wave's 16-byte writes spread over the banks) and are added in wave (depth) order; each store instruction then
  // writes two whole columns of the tile (2 x TR floats, contiguous in the transposed plane).
  constexpr int RP = TR + 4;
  float* red = reinterpret_cast<float*>(smem);                  // [RS_WAVES][TC][RP]
  static_assert(RS_WAVES * TC * RP * 4 <= (int)sizeof(smem), "the reduction fits the shared memory");
  const int64_t me = g.m;
  constexpr int LPC = TR / 4;                                   // lanes per column (4 rows each)
  constexpr int CPI = 64 / LPC;                                 // columns per store instruction
  const int lr = lane % LPC, lc = lane / LPC;
  // (int8: one round per digit, its plane after the other's; the wave partials are int32 and added as integers)
#pragma unroll
  for (int pa = 0; pa < NACC; ++pa) {
    if (pa > 0) __syncthreads();                                // (the previous round's reads are done)
#pragma unroll
    for (int i = 0; i < TRF; ++i)
#pragma unroll
      for (int n = 0; n < TCF; ++n)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4)
          *reinterpret_cast<f32x4*>(red + (w * TC + 32 * n + r) * RP + 32 * i + 8 * r4 + 4 * h) =
              f32x4{acc[pa][i][n][4 * r4], acc[pa][i][n][4 * r4 + 1], acc[pa][i][n][4 * r4 + 2],
                    acc[pa][i][n][4 * r4 + 3]};
    __syncthreads();
    float* const Eh = g.E + (half * NACC + pa) * N * me;
    if constexpr (TCF == 2) {                                   // (row-major planes: 64-column tiles only;
    if (!g.et) {                                                //  the launcher asks transposed ones otherwise)
      // a row-major plane ([m][N]): each store instruction writes 4 rows x 64 columns, lane l row 4 gq + l / 16
      // of the wave's quarter of the tile's rows, columns 4 (l % 16) .. + 3 (the four waves' partials added in
      // wave order, as below)
      const int c4 = 4 * (lane & 15);
#pragma unroll
      for (int gq = 0; gq < TR / 16; ++gq) {
        const int rl = w * (TR / 4) + 4 * gq + (lane >> 4);
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float x = red[(c4 + e) * RP + rl];
#pragma unroll
          for (int q = 1; q < RS_WAVES; ++q) {
            const float u = red[(q * TC + c4 + e) * RP + rl];
            if constexpr (AT == 2) x = __int_as_float(__float_as_int(x) + __float_as_int(u));
            else x += u;
          }
          v[e] = x;
        }
        const int64_t row = r0 + rl, col = c0 + c4;
        if (row < rend) {
          float* Er = Eh + row * N;
          if (col + 4 <= N && (N % 4) == 0) {
            *reinterpret_cast<f32x4*>(Er + col) = v;
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (col + e < N) Er[col + e] = v[e];
          }
        }
      }
      continue;
    }
    }
#pragma unroll
    for (int gq = 0; gq < TC / (RS_WAVES * CPI); ++gq) {
      const int cl = (w * (TC / (RS_WAVES * CPI)) + gq) * CPI + lc;   // the tile's column
      f32x4 v = *reinterpret_cast<const f32x4*>(red + cl * RP + 4 * lr);
#pragma unroll
      for (int q = 1; q < RS_WAVES; ++q) {
        const f32x4 u = *reinterpret_cast<const f32x4*>(red + (q * TC + cl) * RP + 4 * lr);
        if constexpr (AT == 2)
          v = __builtin_bit_cast(f32x4, __builtin_bit_cast(i32x4, v) + __builtin_bit_cast(i32x4, u));
        else
          v += u;
      }
      const int64_t row = r0 + 4 * lr;
      const int64_t col = c0 + cl;
      if (col < N) {
        float* Ec = Eh + col * me;
        if (row + 4 <= rend && (me % 4) == 0 && (row % 4) == 0) {
          *reinterpret_cast<f32x4*>(Ec + row) = v;
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (row + e < rend) Ec[row + e] = v[e];
        }
      }
    }
  }
}

#undef SDC_TALL_WAIT_B
#undef SDC_TALL_NAME_B

// Parts [3][N][kp] (k-contiguous per column, column stride spc) -> fragment order for rs_gemm_kernel: element e of
// lane l of fragment (step s, part p, column fragment f) is part p, column 32 f + l % 32 (zero past N), depth
// 64 (s / 4) + 32 (l / 32) + 8 (s % 4) + e.  One thread per 16-byte piece.
__global__ __launch_bounds__(256) void parts_frag_kernel(const uint16_t* parts, int64_t spc, int64_t N, int64_t k,
                                                         uint16_t* out, int64_t sgp) {
  const int64_t ncf = sdc_cdiv(N, 32), nst = k / 16;
  const int64_t total = nst * 3 * ncf * 64;
  parts += blockIdx.y * sgp;                      // group blockIdx.y: its parts, and its fragments after the last's
  out += blockIdx.y * total * 8;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int lane = (int)(i % 64);
    const int64_t fr = i / 64, f = fr % ncf, p = (fr / ncf) % 3, s = fr / (3 * ncf);
    const int64_t col = 32 * f + lane % 32;
    const int64_t kk = 64 * (s / 4) + 32 * (lane / 32) + 8 * (s % 4);
    u32x4 v = {0u, 0u, 0u, 0u};
    if (col < N) v = *reinterpret_cast<const u32x4*>(parts + (p * N + col) * spc + kk);
    *reinterpret_cast<u32x4*>(out + i * 8) = v;
  }
}

// int8 digits [2][N][spc] (bytes, k-contiguous per column) -> the tall GEMM's int8 fragment order: byte e of lane l
// of fragment (step s, digit p, column fragment f) is digit p, column 32 f + l % 32 (zero past N), depth
// 64 (s / 4) + 32 (l / 32) + 8 (s % 4) + e -- the depths the A fragment of that lane reads.  One thread per 8 bytes.
__global__ __launch_bounds__(256) void digit_frag_kernel(const uint8_t* parts, int64_t spc, int64_t N, int64_t k,
                                                         uint8_t* out) {
  const int64_t ncf = sdc_cdiv(N, 32), nst = k / 16;
  const int64_t total = nst * 2 * ncf * 64;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int lane = (int)(i % 64);
    const int64_t fr = i / 64, f = fr % ncf, p = (fr / ncf) % 2, s = fr / (2 * ncf);
    const int64_t col = 32 * f + lane % 32;
    const int64_t kk = 64 * (s / 4) + 32 * (lane / 32) + 8 * (s % 4);
    u32x2 v = {0u, 0u};
    if (col < N) v = *reinterpret_cast<const u32x2*>(parts + (p * N + col) * spc + kk);
    *reinterpret_cast<u32x2*>(out + i * 8) = v;
  }
}

}  // namespace

// The register-streamed GEMM applies to k-contiguous 16-bit A with depth a multiple of 256 and 16-byte rows, B in
// fragment order (sdc_parts_fragments): one plane of E (transposed), 64 x 64 tiles; role 0 / 1 (column / row
// check) only names the kernel.  Returns SDC_EUNSUPPORTED otherwise.
int sdc_rs_gemm_launch(int dtype, GemmArgs g, int role, hipStream_t stream) {
  if (dtype != SDC_BF16 && dtype != SDC_FP16) return SDC_EUNSUPPORTED;
  if (g.sak != 1 || g.k % RS_KMULT || g.k < RS_KMULT || g.sam % 8 || ((uintptr_t)g.A | (uintptr_t)g.B) % 16 ||
      !g.et || g.goffs)
    return SDC_EUNSUPPORTED;
  if (g.m < 1 || g.N < 1) return SDC_EINVAL;
  if (g.N > 0x7FFFFFFF) return SDC_EUNSUPPORTED;
  const int64_t tiles = sdc_cdiv(g.m, 64) * sdc_cdiv(g.N, 64);
  if (tiles > 0x7FFFFFFF) return SDC_EUNSUPPORTED;
  SdcProf prof(g.prof_name ? g.prof_name : "expected_gemm", stream);
  const dim3 grid((unsigned)tiles), block(64 * RS_WAVES);
  if (role == 1) {
    if (dtype == SDC_BF16) hipLaunchKernelGGL((rs_gemm_kernel<SDC_BF16, RS_RB, 1>), grid, block, 0, stream, g);
    else hipLaunchKernelGGL((rs_gemm_kernel<SDC_FP16, RS_RB, 1>), grid, block, 0, stream, g);
  } else {
    if (dtype == SDC_BF16) hipLaunchKernelGGL((rs_gemm_kernel<SDC_BF16, RS_RB, 0>), grid, block, 0, stream, g);
    else hipLaunchKernelGGL((rs_gemm_kernel<SDC_FP16, RS_RB, 0>), grid, block, 0, stream, g);
  }
  SDC_LAUNCH_CHECK();
  return SDC_OK;
}

// The tall-tile variant: 128 x 64 tiles (64 x 64 with g.short_rows, fp8 only) over g.splits (1 .. SDC_MAX_SPLITS)
// depth parts, one plane of E per part (the depth a multiple of 256 splits, of 512 splits for an fp8 A; A's rows
// 16-byte aligned); with g.XN set, also A's row norms, one plane per part.  dtype SDC_FP8: an fp8 e4m3 A widened to bf16 (B's parts bf16).  With g.goffs (16-bit A
// only): rows grouped by the groups' cumulative ends, group q's fragments at g.B + q g.sbb, row norms always.
// Returns SDC_EUNSUPPORTED where it does not apply.
int sdc_rs_gemm_tall_launch(int dtype, GemmArgs g, int role, hipStream_t stream) {
  if (dtype != SDC_BF16 && dtype != SDC_FP16 && dtype != SDC_FP8 && dtype != SDC_I8) return SDC_EUNSUPPORTED;
  const bool byte_a = dtype == SDC_FP8 || dtype == SDC_I8;
  const int64_t es = byte_a ? 1 : 2, kmul = (byte_a ? RS_WAVES * 128 : RS_KMULT) * g.splits;
  if (g.splits < 1 || g.splits > SDC_MAX_SPLITS || g.sak != 1 || g.k % kmul || (g.sam * es) % 16 ||
      ((uintptr_t)g.A | (uintptr_t)g.B) % 16 || (!g.et && (g.goffs || ((uintptr_t)g.E % 16))))
    return SDC_EUNSUPPORTED;
  if (g.goffs && (dtype == SDC_FP8 || g.ngroups < 1 || g.ngroups > GSCAN || g.sbb % 8)) return SDC_EUNSUPPORTED;
  if (g.m < 1 || g.N < 1) return SDC_EINVAL;
  if ((g.short_rows || dtype == SDC_I8) && (!byte_a || g.goffs || g.xf_blocks || (dtype == SDC_I8 && g.XN)))
    return SDC_EUNSUPPORTED;
  if (dtype == SDC_I8) g.short_rows = 1;                        // (int8: 64-row tiles only)
  const int64_t rtiles = sdc_cdiv(g.m, g.short_rows ? 64 : 32 * SDC_TALL_TRF) + (g.goffs ? g.ngroups : 0);
  if (g.xf_blocks < 0 || (g.xf_blocks && (g.goffs || dtype == SDC_FP8))) return SDC_EINVAL;
  // (grouped outputs of at most 32 columns: one-fragment tiles, whose grid counts 32-column tiles)
  const bool narrow = g.goffs && g.N <= 32;
  const int64_t blocks = g.splits * rtiles * sdc_cdiv(g.N, narrow ? 32 : 64) + g.xf_blocks;
  if (blocks > 0x7FFFFFFF) return SDC_EUNSUPPORTED;
  SdcProf prof(g.prof_name ? g.prof_name : "expected_gemm", stream);
  const dim3 grid((unsigned)blocks), block(64 * RS_WAVES);
  constexpr int T = SDC_TALL_TRF;
  if (g.goffs) {
    // (grouped: 16-bit A with its row norms)
    if (narrow && dtype == SDC_BF16)
      hipLaunchKernelGGL((rs_gemm_tall_kernel<SDC_BF16, 4, T, 0, true, true, 1>), grid, block, 0, stream, g);
    else if (narrow)
      hipLaunchKernelGGL((rs_gemm_tall_kernel<SDC_FP16, 4, T, 0, true, true, 1>), grid, block, 0, stream, g);
    else if (dtype == SDC_BF16)
      hipLaunchKernelGGL((rs_gemm_tall_kernel<SDC_BF16, 4, T, 0, true, true>), grid, block, 0, stream, g);
    else
      hipLaunchKernelGGL((rs_gemm_tall_kernel<SDC_FP16, 4, T, 0, true, true>), grid, block, 0, stream, g);
  } else if (dtype == SDC_I8) {
    hipLaunchKernelGGL((rs_gemm_tall_kernel<SDC_BF16, 5, 2, 2, false>), grid, block, 0, stream, g);
  } else if (dtype == SDC_FP8 && g.short_rows) {
    if (g.XN) hipLaunchKernelGGL((rs_gemm_tall_kernel<SDC_BF16, 3, 2, 1, true>), grid, block, 0, stream, g);
    else hipLaunchKernelGGL((rs_gemm_tall_kernel<SDC_BF16, 3, 2, 1, false>), grid, block, 0, stream, g);
  } else if (dtype == SDC_FP8) {
    if (g.XN) hipLaunchKernelGGL((rs_gemm_tall_kernel<SDC_BF16, 3, T, 1, true>), grid, block, 0, stream, g);
    else hipLaunchKernelGGL((rs_gemm_tall_kernel<SDC_BF16, 3, T, 1, false>), grid, block, 0, stream, g);
  } else if (role == 1) {
    if (dtype == SDC_BF16) hipLaunchKernelGGL((rs_gemm_tall_kernel<SDC_BF16, 1, T, 0, false>), grid, block, 0, stream, g);
    else hipLaunchKernelGGL((rs_gemm_tall_kernel<SDC_FP16, 1, T, 0, false>), grid, block, 0, stream, g);
  } else if (g.XN) {
    // (the serving check: its x row norms in the same pass)
    if (dtype == SDC_BF16) hipLaunchKernelGGL((rs_gemm_tall_kernel<SDC_BF16, 2, T, 0, true>), grid, block, 0, stream, g);
    else hipLaunchKernelGGL((rs_gemm_tall_kernel<SDC_FP16, 2, T, 0, true>), grid, block, 0, stream, g);
  } else {
    if (dtype == SDC_BF16) hipLaunchKernelGGL((rs_gemm_tall_kernel<SDC_BF16, 0, T, 0, false>), grid, block, 0, stream, g);
    else hipLaunchKernelGGL((rs_gemm_tall_kernel<SDC_FP16, 0, T, 0, false>), grid, block, 0, stream, g);
  }
  SDC_LAUNCH_CHECK();
  return SDC_OK;
}

// Bytes of the fragment-ordered copy of 3 x N 16-bit parts of depth k (k a multiple of 64).
extern "C" int64_t sdc_parts_fragments_bytes(int64_t N, int64_t k) {
  if (N < 1 || k < 64 || k % 64) return 0;
  return 3 * sdc_cdiv(N, 32) * 32 * k * 2;
}

// `groups` sets of 3 x N parts (set q at parts + q sgp elements, each [3][N][spc]: 16-bit, k-contiguous per column)
// -> fragment order for the register-streamed GEMM, set q's fragments at out + q sdc_parts_fragments_bytes(N, k).
int sdc_parts_fragments_sets(const void* parts, int64_t spc, int64_t sgp, int64_t groups, int64_t N, int64_t k,
                             void* out, hipStream_t stream) {
  if (!parts || !out || N < 1 || k < 64 || k % 64 || spc % 8 || spc < k || sgp % 8 || groups < 1 ||
      groups > 65535 || ((uintptr_t)parts | (uintptr_t)out) % 16)
    return SDC_EINVAL;
  const int64_t total = (k / 16) * 3 * sdc_cdiv(N, 32) * 64;
  const int64_t blocks = sdc_cdiv(total, 256) < 4096 ? sdc_cdiv(total, 256) : 4096;
  SdcProf prof("parts_frag", stream);
  hipLaunchKernelGGL(parts_frag_kernel, dim3((unsigned)blocks, (unsigned)groups), dim3(256), 0, stream,
                     (const uint16_t*)parts, spc, N, k, (uint16_t*)out, sgp);
  SDC_LAUNCH_CHECK();
  return SDC_OK;
}

// 3 x N parts [3][N][spc] (16-bit, k-contiguous per column) -> fragment order for the register-streamed GEMM.
extern "C" int sdc_parts_fragments(const void* parts, int64_t spc, int64_t N, int64_t k, void* out,
                                   hipStream_t stream) {
  SDC_CLEAR_ERRORS();
  return sdc_parts_fragments_sets(parts, spc, 0, 1, N, k, out, stream);
}

// Bytes of the int8 digits [2][N][k] in the tall GEMM's int8 fragment order (k a multiple of 64).
extern "C" int64_t sdc_digit_fragments_bytes(int64_t N, int64_t k) {
  if (N < 1 || k < 64 || k % 64) return 0;
  return 2 * sdc_cdiv(N, 32) * 32 * k;
}

// int8 digits [2][N][spc] (k-contiguous per column) -> the int8 fragment order of the tall GEMM.
extern "C" int sdc_digit_fragments(const void* parts, int64_t spc, int64_t N, int64_t k, void* out,
                                   hipStream_t stream) {
  SDC_CLEAR_ERRORS();
  if (!parts || !out || N < 1 || k < 64 || k % 64 || spc % 8 || spc < k || ((uintptr_t)parts | (uintptr_t)out) % 8)
    return SDC_EINVAL;
  const int64_t total = (k / 16) * 2 * sdc_cdiv(N, 32) * 64;
  const int64_t blocks = sdc_cdiv(total, 256) < 4096 ? sdc_cdiv(total, 256) : 4096;
  SdcProf prof("digit_frag", stream);
  hipLaunchKernelGGL(digit_frag_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, (const uint8_t*)parts, spc, N,
                     k, (uint8_t*)out);
  SDC_LAUNCH_CHECK();
  return SDC_OK;
}

// Split of the depth so that tiles x splits fill the GPU (one workgroup per CU), in multiples of the stage depth.
extern "C" int64_t sdc_expected_splits(int64_t m, int64_t k, int64_t ncols) {
  if (m <= 0 || k <= 0 || ncols <= 0) return 1;
  const int wgn = ncols > 64 ? 2 : 1;
  const int64_t tiles = sdc_cdiv(m, 64 * (8 / wgn)) * sdc_cdiv(ncols, 64 * wgn);
  int64_t s = sdc_cdiv(256, tiles);
  const int64_t smax = k / 256 > 1 ? k / 256 : 1;
  if (s > smax) s = smax;
  if (s > SDC_MAX_SPLITS) s = SDC_MAX_SPLITS;
  if (s < 1) s = 1;
  return s;
}

int sdc_gemm_launch(int dtype, GemmArgs g, int64_t batches, hipStream_t stream) {
  if (g.splits < 1 || g.splits > SDC_MAX_GEMM_SPLITS || batches < 1) return SDC_EINVAL;
  if (dtype < SDC_BF16 || dtype > SDC_I8) return SDC_EINVAL;
  g.kchunk = sdc_cdiv(sdc_cdiv(g.k, g.splits), KS) * KS;
  const int64_t ea = dtype == SDC_FP8 ? 1 : 2;                   // bytes per A element
  const bool vec = g.sak == 1 && (g.k % KS == 0) && ((g.sam * ea) % 16 == 0) && ((g.sab * ea) % 16 == 0) &&
                   ((uintptr_t)g.A % 16 == 0) && (g.sbc % 8 == 0) && (g.sbb % 8 == 0) && ((uintptr_t)g.B % 16 == 0);
  const int wgn = g.N > 64 ? 2 : 1;
  const int64_t rtiles = sdc_cdiv(g.m, 64 * (8 / wgn)) + (g.goffs ? g.ngroups : 0);
  if (g.goffs && batches != 1) return SDC_EINVAL;
  const int64_t blocks = rtiles * sdc_cdiv(g.N, 64 * wgn) * g.splits * batches;
  if (blocks > 0x7FFFFFFF) return SDC_EUNSUPPORTED;
  SdcProf prof(g.prof_name ? g.prof_name : "expected_gemm", stream);
  switch (dtype) {
    case SDC_BF16: return launch_mode<SDC_BF16>(g, vec, wgn, blocks, stream);
    case SDC_FP16: return launch_mode<SDC_FP16>(g, vec, wgn, blocks, stream);
    case SDC_FP8: return launch_mode<SDC_FP8>(g, vec, wgn, blocks, stream);
    default: return launch_mode<SDC_I8>(g, vec, wgn, blocks, stream);
  }
}

int sdc_split_launch(int dtype, const float* B2T, const float* scale, int64_t sscb, int64_t scale_stride,
                     int64_t ncols, int64_t k, int64_t kp, int64_t batches, uint16_t* parts, hipStream_t stream) {
  SplitArgs a{B2T, scale, sscb, scale_stride, ncols, k, kp, batches, parts};
  const int64_t total = batches * ncols * sdc_cdiv(kp, 8);
  const int64_t blocks = sdc_cdiv(total, 256) < 2048 ? sdc_cdiv(total, 256) : 2048;
  SdcProf prof("split", stream);
  if (dtype == SDC_BF16) hipLaunchKernelGGL(split_kernel<SDC_BF16>, dim3((unsigned)blocks), dim3(256), 0, stream, a);
  else hipLaunchKernelGGL(split_kernel<SDC_FP16>, dim3((unsigned)blocks), dim3(256), 0, stream, a);
  SDC_LAUNCH_CHECK();
  return SDC_OK;
}

// The serving check's call: one batch, precomputed parts (k-contiguous columns).
int sdc_expected_launch(int dtype, const void* x, int64_t sxm, int64_t sxk, const void* parts, int64_t spk,
                        int64_t spc, int nparts, int64_t m, int64_t k, int64_t ncols, int64_t splits, float* E,
                        float* XN, hipStream_t stream) {
  if (sxk != 1 || spk != 1) return SDC_EUNSUPPORTED;        // both operands must be k-contiguous
  if (nparts != 3) return SDC_EUNSUPPORTED;
  GemmArgs g{};
  g.A = (const uint16_t*)x; g.sab = 0; g.sam = sxm; g.sak = sxk;
  g.B = parts; g.sbb = 0; g.sbc = spc;
  g.m = m; g.k = k; g.N = ncols; g.splits = splits;
  g.E = E; g.XN = XN;
  return sdc_gemm_launch(dtype, g, 1, stream);
}

// Self-test of the MFMA operand layout this file assumes: C (32 x 32) = A (32 x 16) @ B (16 x 32), bf16 in,
// fp32 out, A given row-major (k contiguous) and B given column-major (k contiguous), one wave.
__global__ void mfma_layout_kernel(const uint16_t* A, const uint16_t* B, float* C) {
  const int lane = threadIdx.x;
  u32x4 a = *reinterpret_cast<const u32x4*>(A + (lane & 31) * 16 + (lane >> 5) * 8);
  u32x4 b = *reinterpret_cast<const u32x4*>(B + (lane & 31) * 16 + (lane >> 5) * 8);
  f32x16 c;
#pragma unroll
  for (int r = 0; r < 16; ++r) c[r] = 0.f;
  c = mfma32<SDC_BF16>(a, b, c);
#pragma unroll
  for (int r = 0; r < 16; ++r) C[(8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * 32 + (lane & 31)] = c[r];
}

extern "C" int sdc_mfma_layout_selftest(const void* A, const void* B, float* C, hipStream_t stream) {
  SDC_CLEAR_ERRORS();
  hipLaunchKernelGGL(mfma_layout_kernel, dim3(1), dim3(64), 0, stream, (const uint16_t*)A, (const uint16_t*)B, C);
  SDC_LAUNCH_CHECK();
  return SDC_OK;
}
