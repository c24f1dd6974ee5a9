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
