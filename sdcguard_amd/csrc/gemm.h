// The expected-side GEMM shared by the checks (expected_gemm.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

struct GemmArgs {
  const uint16_t* A;            // bf16/fp16 rows; element (batch, row, kk) at A[batch * sab + row * sam + kk * sak]
  int64_t sab, sam, sak;
  const void* B;                // BSRC 0: parts (3 x N columns of the dtype), BSRC 1: fp32 B2^T (N columns)
  int64_t sbb, sbc;             // batch stride, column stride (columns are depth-contiguous)
  const float* scale;           // BSRC 1: per-column power of two to divide by before the split, at
  int64_t sscb;                 //   scale[batch * sscb + column * scale_stride]
  int64_t scale_stride;
  int64_t m, k, N, kchunk, splits;
  float* E;                     // [batch][split][m][N]
  float* XN;                    // [batch][split][2][m]: sum of squares and sum of |a| of each row's depth slice
};

// E and XN for `batches` batches (grid z = batches x splits); bsrc 0 or 1 as above.
int sdc_gemm_launch(int dtype, int bsrc, GemmArgs g, int64_t batches, hipStream_t stream);
