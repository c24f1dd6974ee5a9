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

}  // namespace

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
