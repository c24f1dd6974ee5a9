// Building blocks of the MFMA GEMM pipelines (expected_gemm.hip, fused_check.hip): the bf16 / fp16 MFMA, the
// swizzled LDS tile layout, global-to-LDS loads and the wait-count immediates.
#pragma once
#include "common.h"

namespace sdc_pipe {

constexpr int KS = 32;                 // depth per pipeline stage (elements)

// C (32 x 32 fp32) += A (32 x 16) B (16 x 32): lane l holds A row l % 32 and B column l % 32, depths
// 8 (l / 32) .. 8 (l / 32) + 7; C[i][j] lands in lane j + 32 ((i / 4) % 2), register (i / 8) 4 + i % 4
template <int DT>
__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (DT == SDC_BF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                  0, 0, 0);
  }
}

// C (16 x 16 fp32) += A (16 x 32) B (32 x 16): lane l holds A row l % 16 and B column l % 16, depths
// 8 (l / 16) .. 8 (l / 16) + 7; C[i][j] lands in lane j + 16 (i / 4), register i % 4
template <int DT>
__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (DT == SDC_BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                  0, 0, 0);
  }
}

// LDS rows of KS 16-bit elements (64 bytes, four 16-byte chunks); chunk q of row r sits at position
// q ^ ((r / 2) % 4), so the eight lanes of each ds_read_b128 phase (eight consecutive rows, one chunk) and of each
// 16-byte write phase (two rows, four chunks each) hit 32 distinct banks
__device__ __forceinline__ int lds_at(int row, int chunk) { return row * KS + 8 * (chunk ^ ((row >> 1) & 3)); }

// s_waitcnt immediate that waits until at most n vector memory operations are outstanding (other counters free)
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
// ... until no LDS or scalar-memory operation is outstanding
constexpr int lgkmcnt0_imm() { return 15 | (3 << 14) | (7 << 4); }

// 16 bytes per lane from global memory straight into LDS: lane L's bytes land at lds + 16 L (lds wave-uniform)
__device__ __forceinline__ void lds_load16(const uint8_t* g, uint16_t* lds) {
  __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(g), lds, 16, 0, 0);
}

}  // namespace sdc_pipe
