// Internal interface of the grouped MFMA GEMM, shared by the kernel
// families that call it (recurrent input projection, attention projections).
#pragma once

#include "wc_common.h"

namespace wc {

// C[i][m][o] = act( sum_k A[i][m][k] W[i][o][k] + bias[i][o] + R[i][m][o] ),
// rows m of A / C / R addressed as (m / rows_inner) * s_outer + (m % rows_inner) * s_inner.
struct GemmParams {
  int n, m, o, k;
  int act;
  int tiles_m, tiles_o;
  int remap;
  const void* a;
  int64_t a_sn, a_so, a_si;
  FastDiv a_ri;
  const void* w;
  int64_t w_sn;
  const void* bias;
  int64_t b_sn;
  const void* r;
  int64_t r_sn, r_so, r_si;
  void* c;
  int64_t c_sn, c_so, c_si;
  FastDiv c_ri;
  // persistent XL kernel only: dividers of the stage -> tile -> (model, column tile) map,
  // and the byte extents of one model's C and R regions (their buffer descriptors' range,
  // so a stray offset is dropped by the hardware instead of reaching other memory)
  FastDiv fd_ks, fd_tpm, fd_tm;
  int32_t c_bytes, r_bytes;
};

// dtype: A/W element type; out_dtype: WC_F32 or dtype; bias_dtype: WC_F32 or dtype.
int32_t grouped_gemm(const GemmParams& p, int32_t dtype, int32_t out_dtype, int32_t bias_dtype,
                     hipStream_t st);

}  // namespace wc
