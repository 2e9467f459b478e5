// Per-lane RoPE and QK-norm arithmetic shared by the fused RoPE/append kernel
// and the fused decode-step kernel, so both produce the same bits.
//
//   rope.py:20-27   x.float() split into interleaved pairs (x[2j], x[2j+1]);
//                   out = (re*cos - im*sin, re*sin + im*cos) in fp32, then one
//                   rounding back to x's dtype (type_as).
//   rms_norm.py:7   F.rms_norm(x, (D,)) with eps=None: x * rsqrt(mean(x^2) + eps)
//                   in fp32 with eps = FLT_EPSILON, one rounding to x's dtype.
#pragma once

#include <float.h>

#include "dg_common.h"

namespace dg {

// RoPE on EPL consecutive elements (EPL/2 interleaved (re, im) pairs) with
// their interleaved (cos, sin) values: two separately rounded products and one
// rounded add/sub per output, never an FMA, then the rounding to T.
template <typename T, int EPL>
__device__ __forceinline__ void rope_rotate(float (&x)[EPL], const float (&cs)[EPL]) {
#pragma clang fp contract(off)
#pragma unroll
  for (int p = 0; p < EPL / 2; ++p) {
    const float re = x[2 * p], im = x[2 * p + 1];
    const float c = cs[2 * p], sn = cs[2 * p + 1];
    const float a0 = re * c, a1 = im * sn;
    const float b0 = re * sn, b1 = im * c;
    // rounding to the storage dtype happens here (type_as), before the norm
    if constexpr (__is_same(T, bf16_t)) {
      // both outputs rounded by one packed conversion, unpacked by shift and mask
      const uint32_t w = pack_pair<T>(a0 - a1, b0 + b1);
      x[2 * p] = __uint_as_float(w << 16);
      x[2 * p + 1] = __uint_as_float(w & 0xffff0000u);
    } else {
      x[2 * p] = to_f32(from_f32<T>(a0 - a1));
      x[2 * p + 1] = to_f32(from_f32<T>(b0 + b1));
    }
  }
}

// RMSNorm of a row of D elements held as EPL consecutive elements by each of
// LPK consecutive lanes (lanes past D hold zeros): squares rounded, summed by
// the pairwise tree over the row padded to a power of two (tree_sum inside the
// lane, then the xor-1, 2, ... butterfly across lanes), mean = sum / D,
// r = 1 / sqrt(mean + FLT_EPSILON) with correctly rounded sqrt and divide,
// y = x * r.  The caller rounds y to the storage dtype.  DPP selects the
// register-only butterfly (group_sum_dpp), which adds the same pairs in the
// same order: the same bits without LDS traffic.
template <int EPL, int LPK, bool DPP = false>
__device__ __forceinline__ void qk_rms_norm(float (&x)[EPL], int D) {
#pragma clang fp contract(off)
  float sq[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) sq[i] = x[i] * x[i];
  float ss = tree_sum<EPL>(sq);
  ss = DPP ? group_sum_dpp<LPK>(ss) : group_sum<LPK>(ss);
  const float mean = ss / (float)D;
  const float r = 1.0f / sqrtf(mean + FLT_EPSILON);
#pragma unroll
  for (int i = 0; i < EPL; ++i) x[i] = x[i] * r;
}

}  // namespace dg
