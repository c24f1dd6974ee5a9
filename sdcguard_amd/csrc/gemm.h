// The expected-side GEMM shared by the checks (expected_gemm.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "xfinish.h"

struct GemmArgs {
  const uint16_t* A;            // bf16/fp16 rows; element (batch, row, kk) at A[batch * sab + row * sam + kk * sak]
  int64_t sab, sam, sak;
  const void* B;                // parts: 3 x N depth-contiguous columns of the dtype, part p column c at
  int64_t sbb, sbc;             //   B[batch * sbb + (p * N + c) * sbc + kk]
  int64_t m, k, N, kchunk, splits;
  float* E;                     // [batch][split][m][N], or [batch][split][N][m] with et
  int et;                       // store E transposed (column-major per plane)
  const char* prof_name;        // name for per-kernel timing (null: "expected_gemm")
  // Grouped rows (a MoE grouped GEMM, tokens sorted by expert): when goffs is set, row r belongs to group g with
  // goffs[g-1] <= r < goffs[g] (cumulative ends, on the device) and is multiplied by group g's parts (batch
  // stride sbb); row tiles never cross a group, the grid covers cdiv(m, TM) + ngroups tiles and workgroups past the
  // last tile exit.  E and XN are indexed by the global row (batch 0).
  const int64_t* goffs;
  int64_t ngroups;
  float* XN;                    // [batch][split][2][m]: sum of squares and sum of |a| of each row's depth slice
  // 0: each XCD takes one depth slice of every row tile (its slice of the parts stays in its L2); 1: each XCD
  // takes every depth slice of some row tiles (its rows' 128-byte lines stay in its L2 between the two stages that
  // read their halves: for a tall A read once, whose parts fit one L2 whole)
  int rows_per_xcd;
  // (the tall-tile kernel) the grid's last xf_blocks workgroups run the x pass's finishing step for row blocks
  // 0 .. xf_blocks - 1 instead of tiles: sdc_linear_check's row GEMM leaves CUs idle, and xfinish has no other use
  // for them
  XStageArgs xf;
  int xf_blocks;
  // (the tall-tile kernel, an fp8 A) 64-row tiles instead of 128, for a short A whose 128-row tiles would leave
  // most CUs idle
  int short_rows;
};

// E and XN for `batches` batches.
int sdc_gemm_launch(int dtype, GemmArgs g, int64_t batches, hipStream_t stream);

// Register-streamed GEMMs over 16-bit parts in fragment order (E transposed): 64 x 64 tiles, one plane of E; and
// 128 x 64 tiles over g.splits depth parts (fp8 or 16-bit A, optional row norms, grouped rows).  Both return
// SDC_EUNSUPPORTED, launching nothing, where their shape or alignment rules do not hold.
int sdc_rs_gemm_launch(int dtype, GemmArgs g, int role, hipStream_t stream);
int sdc_rs_gemm_tall_launch(int dtype, GemmArgs g, int role, hipStream_t stream);
extern "C" int64_t sdc_expected_splits(int64_t m, int64_t k, int64_t ncols);
extern "C" int64_t sdc_parts_fragments_bytes(int64_t N, int64_t k);
extern "C" int sdc_parts_fragments(const void* parts, int64_t spc, int64_t N, int64_t k, void* out, hipStream_t stream);
int sdc_parts_fragments_sets(const void* parts, int64_t spc, int64_t sgp, int64_t groups, int64_t N, int64_t k,
                             void* out, hipStream_t stream);
extern "C" int64_t sdc_digit_fragments_bytes(int64_t N, int64_t k);
extern "C" int sdc_digit_fragments(const void* parts, int64_t spc, int64_t N, int64_t k, void* out, hipStream_t stream);

// parts[batch][3 * ncols][kp] from B2T[batch][ncols][k] (fp32), each column divided by
// scale[batch * sscb + col * scale_stride] first (null: 1); depth kp >= k padded with zeros.
int sdc_split_launch(int dtype, const float* B2T, const float* scale, int64_t sscb, int64_t scale_stride,
                     int64_t ncols, int64_t k, int64_t kp, int64_t batches, uint16_t* parts, hipStream_t stream);
