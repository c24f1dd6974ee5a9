// Shared device helpers for the sdcguard HIP kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define SDC_WAVE 64
// most depth-split planes of the expected-side GEMM (its scorers add them with unrolled loads)
#define SDC_MAX_SPLITS 8
// depth splits the expected-side GEMM accepts (consumers that hold every split's value in registers take at most
// SDC_MAX_SPLITS; the quantized checks, whose GEMMs can be short in rows, loop over up to this many)
#define SDC_MAX_GEMM_SPLITS 32

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));

// Element kinds of the checked matmul's operands.  The expected-side GEMM also runs in two quantized modes:
// SDC_FP8 (A fp8 e4m3, converted exactly to bf16 on load; bf16 parts) and SDC_I8 (A int8; int8 parts).
enum SdcDtype { SDC_BF16 = 0, SDC_FP16 = 1, SDC_FP8 = 2, SDC_I8 = 3 };

// Status codes of the C ABI.
enum SdcStatus {
  SDC_OK = 0,
  SDC_EINVAL = -1,        // an argument is out of range (shape, stride, null pointer)
  SDC_EUNSUPPORTED = -2,  // a case this library does not implement (the caller must not pretend it ran)
  SDC_EWORKSPACE = -3,    // the workspace is smaller than the matching *_workspace() call asked for
  SDC_ELAUNCH = -4,       // a HIP launch error
};

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
__device__ __forceinline__ float f16_lo(uint32_t w) {
  _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)(w & 0xFFFFu));
  return (float)h;
}
__device__ __forceinline__ float f16_hi(uint32_t w) {
  _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
  return (float)h;
}

template <int DT>
__device__ __forceinline__ float lo_of(uint32_t w) { return DT == SDC_BF16 ? bf16_lo(w) : f16_lo(w); }
template <int DT>
__device__ __forceinline__ float hi_of(uint32_t w) { return DT == SDC_BF16 ? bf16_hi(w) : f16_hi(w); }
template <int DT>
__device__ __forceinline__ float half_to_f32(uint16_t h) {
  return DT == SDC_BF16 ? __uint_as_float((uint32_t)h << 16) : (float)__builtin_bit_cast(_Float16, h);
}

// DPP lane exchange inside a quad (xor 1 / xor 2): one VALU op each, no LDS traffic.
__device__ __forceinline__ float dpp_xor1(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
}
__device__ __forceinline__ float dpp_xor2(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
}
__device__ __forceinline__ float quad_sum(float v) {
  v += dpp_xor1(v);
  v += dpp_xor2(v);
  return v;
}

__device__ __forceinline__ int64_t shfl_xor_i64(int64_t v, int mask) {
  int lo = (int)(uint32_t)(uint64_t)v;
  int hi = (int)(uint32_t)((uint64_t)v >> 32);
  lo = __shfl_xor(lo, mask, SDC_WAVE);
  hi = __shfl_xor(hi, mask, SDC_WAVE);
  return (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}

__device__ __forceinline__ int64_t wave_max_i64(int64_t v) {
#pragma unroll
  for (int m = 1; m < SDC_WAVE; m <<= 1) {
    int64_t o = shfl_xor_i64(v, m);
    v = o > v ? o : v;
  }
  return v;
}

__device__ __forceinline__ int64_t wave_sum_i64(int64_t v) {
#pragma unroll
  for (int m = 1; m < SDC_WAVE; m <<= 1) v += shfl_xor_i64(v, m);
  return v;
}

__device__ __forceinline__ int wave_sum_i32(int v) {
#pragma unroll
  for (int m = 1; m < SDC_WAVE; m <<= 1) v += __shfl_xor(v, m, SDC_WAVE);
  return v;
}

__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
  for (int m = 1; m < SDC_WAVE; m <<= 1) v += __shfl_xor(v, m, SDC_WAVE);
  return v;
}

// Wave reductions on DPP lane moves: xor 1 and xor 2 (quad swaps), the half-row and row mirrors (every lane of a
// row of 16 then holds its row's result), then the four rows read through lanes 0, 16, 32 and 48.  No LDS round
// trips, unlike the shuffles above; every lane of the wave must be active.  (Integer maxima and sums: any order
// gives the same result.)
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ uint32_t wave_max_u32_dpp(uint32_t v) {
  v = max(v, dpp_u32<0xB1>(v));
  v = max(v, dpp_u32<0x4E>(v));
  v = max(v, dpp_u32<0x141>(v));
  v = max(v, dpp_u32<0x140>(v));
  const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)v, 0), b = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
  const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)v, 32), d = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
  return max(max(a, b), max(c, d));
}
__device__ __forceinline__ int wave_sum_i32_dpp(int v) {
  v += (int)dpp_u32<0xB1>((uint32_t)v);
  v += (int)dpp_u32<0x4E>((uint32_t)v);
  v += (int)dpp_u32<0x141>((uint32_t)v);
  v += (int)dpp_u32<0x140>((uint32_t)v);
  return (__builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16)) +
         (__builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48));
}
// (Float sums: the order is the lanes' pairs, then quads, eights and rows, then the rows in pairs.)
__device__ __forceinline__ float wave_sum_f32_dpp(float v) {
  v += __uint_as_float(dpp_u32<0xB1>(__float_as_uint(v)));
  v += __uint_as_float(dpp_u32<0x4E>(__float_as_uint(v)));
  v += __uint_as_float(dpp_u32<0x141>(__float_as_uint(v)));
  v += __uint_as_float(dpp_u32<0x140>(__float_as_uint(v)));
  const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (a + b) + (c + d);
}
__device__ __forceinline__ float wave_max_f32_dpp(float v) {
  v = fmaxf(v, __uint_as_float(dpp_u32<0xB1>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(dpp_u32<0x4E>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(dpp_u32<0x141>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(dpp_u32<0x140>(__float_as_uint(v))));
  const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return fmaxf(fmaxf(a, b), fmaxf(c, d));
}
template <int CTRL>
__device__ __forceinline__ int64_t dpp_i64(int64_t v) {
  const uint32_t lo = dpp_u32<CTRL>((uint32_t)(uint64_t)v), hi = dpp_u32<CTRL>((uint32_t)((uint64_t)v >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ int64_t readlane_i64(int64_t v, int l) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(uint64_t)v, l);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)v >> 32), l);
  return (int64_t)(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ int64_t wave_max_i64_dpp(int64_t v) {
  int64_t o = dpp_i64<0xB1>(v);
  v = o > v ? o : v;
  o = dpp_i64<0x4E>(v);
  v = o > v ? o : v;
  o = dpp_i64<0x141>(v);
  v = o > v ? o : v;
  o = dpp_i64<0x140>(v);
  v = o > v ? o : v;
  int64_t r = readlane_i64(v, 0);
#pragma unroll
  for (int l = 16; l < 64; l += 16) {
    const int64_t q = readlane_i64(v, l);
    r = q > r ? q : r;
  }
  return r;
}

// bits of a float as an int64 holding the unsigned 32-bit pattern
__device__ __forceinline__ int64_t fbits64(float f) { return (int64_t)(uint32_t)__float_as_uint(f); }

__host__ __device__ static inline int64_t sdc_cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// The HIP error behind the last SDC_ELAUNCH of this thread (sdc_last_error()).
void sdc_note_error(hipError_t e);

#define SDC_LAUNCH_CHECK()                                      \
  do {                                                          \
    hipError_t e_ = hipGetLastError();                          \
    if (e_ != hipSuccess) {                                     \
      sdc_note_error(e_);                                       \
      return SDC_ELAUNCH;                                       \
    }                                                           \
  } while (0)

// Entry points clear errors left by earlier HIP calls of the thread, so a launch check sees only its own.
#define SDC_CLEAR_ERRORS() (void)hipGetLastError()
