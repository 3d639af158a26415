// Device helpers of the NVFP4 weight path shared by the GEMV and the prefill GEMM: exact dequantisation of a
// lane's codes to the f16 MFMA A operand.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "rowops.hpp"

namespace xtg::hip {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// 8 E2M1 codes (one 32-bit word, element 0 in the low nibble) times their group's E4M3 scale, as 8 f16: FP4 ->
// f16 pairs by v_cvt_scalef32_pk_f16_fp4 with a unit scale (the instruction's own scale uses only the exponent),
// then v_pk_mul_f16 by the scale, which f16 holds exactly; E2M1 x E4M3 products (at most 6 significant bits,
// 2^-10 .. 2688) are exact in f16.
__device__ inline f16x8 dequant8(uint32_t word, f16x2 s) {
  const f16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(word, 1.0f, 0) * s;
  const f16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(word, 1.0f, 1) * s;
  const f16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(word, 1.0f, 2) * s;
  const f16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(word, 1.0f, 3) * s;
  f16x8 a;
  a[0] = p0[0];
  a[1] = p0[1];
  a[2] = p1[0];
  a[3] = p1[1];
  a[4] = p2[0];
  a[5] = p2[1];
  a[6] = p3[0];
  a[7] = p3[1];
  return a;
}

// One of the two E4M3 scales of a lane's 16-bit scale word (which = 0: the low byte) as an f16 pair.
__device__ inline f16x2 scale_pair(uint32_t sbits, int which) {
  const _Float16 s = (_Float16)(which ? __builtin_amdgcn_cvt_f32_fp8(sbits, 1) : __builtin_amdgcn_cvt_f32_fp8(sbits, 0));
  f16x2 r;
  r[0] = s;
  r[1] = s;
  return r;
}

}  // namespace xtg::hip
