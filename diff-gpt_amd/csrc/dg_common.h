// Shared device helpers of libdgattn: element conversion, 64-lane butterfly
// reductions and the error slot used by every C entry point.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/dgattn.h"

namespace dg {

// ---------------------------------------------------------------------------
// Element types.  bf16 is held as its 16-bit pattern so loads/stores are plain
// integer moves; conversion to fp32 is exact (append 16 zero bits) and the
// conversion back rounds to nearest-even, matching torch's Tensor.to(bfloat16)
// and the single rounding of type_as() in rope.py:27.
// ---------------------------------------------------------------------------
struct bf16_t {
  uint16_t bits;
};
struct f16_t {
  uint16_t bits;
};

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16_t x) {
  return __uint_as_float(static_cast<uint32_t>(x.bits) << 16);
}
__device__ __forceinline__ float to_f32(f16_t x) {
  _Float16 h = __builtin_bit_cast(_Float16, x.bits);
  return static_cast<float>(h);
}

template <typename T>
__device__ __forceinline__ T from_f32(float x);

template <>
__device__ __forceinline__ float from_f32<float>(float x) {
  return x;
}
template <>
__device__ __forceinline__ bf16_t from_f32<bf16_t>(float x) {
  // v_cvt_pk_bf16_f32: round to nearest, ties to even (NaN stays a quiet
  // NaN), no data-dependent branch; x is materialised as an fp32 register
  // first so that no producer is folded into the conversion
  asm("" : "+v"(x));
  bf16_t r;
  r.bits = __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));
  return r;
}
template <>
__device__ __forceinline__ f16_t from_f32<f16_t>(float x) {
  // x is materialised as an fp32 register first: otherwise the backend may fold
  // the product that made x into the conversion (v_fma_mix*_f16), rounding
  // once where fp32 arithmetic followed by .to(float16) rounds twice
  asm("" : "+v"(x));
  _Float16 h = static_cast<_Float16>(x);  // v_cvt_f16_f32: round to nearest even
  f16_t r;
  r.bits = __builtin_bit_cast(uint16_t, h);
  return r;
}

// Two fp32 values rounded to T (nearest even) in one 32-bit word, a in the
// low half: bf16 pairs through one v_cvt_pk_bf16_f32, with the same guard
// as from_f32 against folding a producer into the conversion.
template <typename T>
__device__ __forceinline__ uint32_t pack_pair(float a, float b) {
  if constexpr (__is_same(T, bf16_t)) {
    asm("" : "+v"(a), "+v"(b));
    typedef float f2_t __attribute__((ext_vector_type(2)));
    typedef __bf16 b2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2_t{a, b}, b2_t));
  } else {
    return (uint32_t)from_f32<T>(a).bits | ((uint32_t)from_f32<T>(b).bits << 16);
  }
}

// ---------------------------------------------------------------------------
// Vector loads of EPL consecutive elements (EPL*sizeof(T) bytes, naturally
// aligned by the host-side checks) converted to fp32.
// ---------------------------------------------------------------------------
template <int BYTES>
struct raw_vec;
template <>
struct raw_vec<4> {
  using type = uint32_t;
};
template <>
struct raw_vec<8> {
  using type = uint2;
};
template <>
struct raw_vec<16> {
  using type = uint4;
};

template <typename T, int EPL>
__device__ __forceinline__ void load_vec(const T* __restrict__ p, float (&out)[EPL]) {
  constexpr int BYTES = EPL * (int)sizeof(T);
  T e[EPL];
  if constexpr (BYTES > 16) {
    static_assert(BYTES % 16 == 0, "vector width");
#pragma unroll
    for (int c = 0; c < BYTES / 16; ++c) {
      uint4 r = reinterpret_cast<const uint4*>(p)[c];
      __builtin_memcpy(reinterpret_cast<char*>(e) + 16 * c, &r, 16);
    }
  } else {
    static_assert(BYTES == 4 || BYTES == 8 || BYTES == 16, "vector width");
    using R = typename raw_vec<BYTES>::type;
    R r = *reinterpret_cast<const R*>(p);
    __builtin_memcpy(e, &r, BYTES);
  }
#pragma unroll
  for (int i = 0; i < EPL; ++i) out[i] = to_f32(e[i]);
}

template <typename T, int EPL>
__device__ __forceinline__ void store_vec(T* __restrict__ p, const float (&in)[EPL]) {
  constexpr int BYTES = EPL * (int)sizeof(T);
  T e[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) e[i] = from_f32<T>(in[i]);
  if constexpr (BYTES > 16) {
    static_assert(BYTES % 16 == 0, "vector width");
#pragma unroll
    for (int c = 0; c < BYTES / 16; ++c) {
      uint4 r;
      __builtin_memcpy(&r, reinterpret_cast<const char*>(e) + 16 * c, 16);
      reinterpret_cast<uint4*>(p)[c] = r;
    }
  } else {
    static_assert(BYTES == 4 || BYTES == 8 || BYTES == 16, "vector width");
    using R = typename raw_vec<BYTES>::type;
    R r;
    __builtin_memcpy(&r, e, BYTES);
    *reinterpret_cast<R*>(p) = r;
  }
}

// Pairwise-tree sum of N (power of two) values held by one lane: adjacent
// pairs first, then pairs of pairs.  Together with group_sum over the lanes
// of a row this is the canonical reduction order of the row norms.
template <int N>
__device__ __forceinline__ float tree_sum(float (&v)[N]) {
#pragma unroll
  for (int w = 1; w < N; w <<= 1) {
#pragma unroll
    for (int i = 0; i < N; i += 2 * w) v[i] = v[i] + v[i + w];
  }
  return v[0];
}

// ---------------------------------------------------------------------------
// Cross-lane exchange inside a 64-wide wavefront.  ds_swizzle / DPP are picked
// by the compiler for __shfl_xor with constant offsets.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float shfl_xor(float v, int off) { return __shfl_xor(v, off, 64); }

// Butterfly sum over groups of G consecutive lanes (G a power of two).  Every
// lane of a group ends with the same value: IEEE addition is commutative, so
// partners compute bit-identical sums.  The pairing order (xor 1, 2, 4, ...)
// is the tail of a pairwise tree over the lanes' partial sums.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int off = 1; off < G; off <<= 1) v = v + shfl_xor(v, off);
  return v;
}

constexpr float kNegInf = -__builtin_huge_valf();

// ---------------------------------------------------------------------------
// Register-only cross-lane sums (no LDS traffic): DPP quad permutes and row
// mirrors inside a 16-lane row, v_permlane16/32_swap across rows.  The
// pairings are those of group_sum (partner = lane ^ 1, ^ 2, then the other
// half of each 8-, 16-, 32- and 64-lane group), every pair adds the same two
// values in both lanes, so all G lanes of a group end with identical bits.
// ---------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
constexpr int kDppQuadXor1 = 0xB1;    // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;    // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7-i inside each 8
constexpr int kDppMirror = 0x140;     // lane i <-> 15-i inside each 16

// {own value, value of the partner row / half} in some order (which one comes
// first depends on the lane); combine them with a commutative operation.
__device__ __forceinline__ void pair16(float x, float& a, float& b) {
  const uint32_t u = __float_as_uint(x);
  auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}
__device__ __forceinline__ void pair32(float x, float& a, float& b) {
  const uint32_t u = __float_as_uint(x);
  auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}

constexpr int kDppRowRor4 = 0x124;    // rotate each 16-lane row by 4
constexpr int kDppRowRor8 = 0x128;    // rotate each 16-lane row by 8

// Maximum over the 64 lanes of the wave (identical in every lane).
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<kDppQuadXor1>(v));
  v = fmaxf(v, dpp<kDppQuadXor2>(v));
  v = fmaxf(v, dpp<kDppHalfMirror>(v));
  v = fmaxf(v, dpp<kDppMirror>(v));
  float a, b;
  pair16(v, a, b);
  v = fmaxf(a, b);
  pair32(v, a, b);
  return fmaxf(a, b);
}

// Sum over the 64/LPK groups of LPK consecutive lanes, element-wise for lanes
// of equal index inside their group (lane offsets that are multiples of
// LPK).  Every lane receives the full sum; the addition order may differ
// between lanes of one group, so only one group's result should be used.
template <int LPK>
__device__ __forceinline__ float sum_over_groups(float v) {
  static_assert(LPK >= 1 && LPK <= 64 && (LPK & (LPK - 1)) == 0, "group size");
  if constexpr (LPK <= 1) v = v + dpp<kDppQuadXor1>(v);
  if constexpr (LPK <= 2) v = v + dpp<kDppQuadXor2>(v);
  if constexpr (LPK <= 4) v = v + dpp<kDppRowRor4>(v);
  if constexpr (LPK <= 8) v = v + dpp<kDppRowRor8>(v);
  if constexpr (LPK <= 16) {
    float a, b;
    pair16(v, a, b);
    v = a + b;
  }
  if constexpr (LPK <= 32) {
    float a, b;
    pair32(v, a, b);
    v = a + b;
  }
  return v;
}

template <int G>
__device__ __forceinline__ float group_sum_dpp(float v) {
  static_assert(G >= 1 && G <= 64 && (G & (G - 1)) == 0, "group size");
  if constexpr (G >= 2) v = v + dpp<kDppQuadXor1>(v);
  if constexpr (G >= 4) v = v + dpp<kDppQuadXor2>(v);
  if constexpr (G >= 8) v = v + dpp<kDppHalfMirror>(v);
  if constexpr (G >= 16) v = v + dpp<kDppMirror>(v);
  if constexpr (G >= 32) {
    float a, b;
    pair16(v, a, b);
    v = a + b;
  }
  if constexpr (G >= 64) {
    float a, b;
    pair32(v, a, b);
    v = a + b;
  }
  return v;
}

// ---------------------------------------------------------------------------
// A lane's slice of one cache row: EPL consecutive elements held as raw
// 32-bit words, loaded with 16/8/4-byte vector loads, and the partial dot
// product of two such slices (fp32 FMAs, or v_dot2_f32_{bf16,f16} on the
// packed 16-bit data: products of two 16-bit floats are exact in fp32).
// ---------------------------------------------------------------------------
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2v_t;
typedef _Float16 __attribute__((ext_vector_type(2))) f16x2v_t;

// EPL elements of one row as raw 32-bit words (EPL*sizeof(T) bytes).
template <typename T, int EPL>
struct RowRegs {
  static constexpr int BYTES = EPL * (int)sizeof(T);
  static constexpr int WORDS = BYTES / 4;
  static_assert(BYTES % 4 == 0, "row slice must be whole 32-bit words");
  uint32_t w[WORDS];
};

template <typename T, int EPL>
__device__ __forceinline__ void load_row(RowRegs<T, EPL>& r, const T* p) {
  constexpr int W = RowRegs<T, EPL>::WORDS;
  if constexpr (W % 4 == 0) {
#pragma unroll
    for (int c = 0; c < W / 4; ++c) {
      const u32x4_t x = reinterpret_cast<const u32x4_t*>(p)[c];
      r.w[4 * c] = x[0];
      r.w[4 * c + 1] = x[1];
      r.w[4 * c + 2] = x[2];
      r.w[4 * c + 3] = x[3];
    }
  } else if constexpr (W == 2) {
    const u32x2_t x = *reinterpret_cast<const u32x2_t*>(p);
    r.w[0] = x[0];
    r.w[1] = x[1];
  } else {
    static_assert(W == 1, "row slice width");
    r.w[0] = *reinterpret_cast<const uint32_t*>(p);
  }
}

// EPL fp32 values rounded to T and packed as the raw words of a row slice.
template <typename T, int EPL>
__device__ __forceinline__ void pack_row(RowRegs<T, EPL>& r, const float (&x)[EPL]) {
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int e = 0; e < EPL; ++e) r.w[e] = __float_as_uint(x[e]);
  } else {
#pragma unroll
    for (int w = 0; w < EPL / 2; ++w) r.w[w] = pack_pair<T>(x[2 * w], x[2 * w + 1]);
  }
}

// The row slice's raw words to memory (naturally aligned by the host checks).
template <typename T, int EPL>
__device__ __forceinline__ void store_row(T* p, const RowRegs<T, EPL>& r) {
  constexpr int W = RowRegs<T, EPL>::WORDS;
  if constexpr (W % 4 == 0) {
#pragma unroll
    for (int c4 = 0; c4 < W / 4; ++c4)
      reinterpret_cast<u32x4_t*>(p)[c4] = u32x4_t{r.w[4 * c4], r.w[4 * c4 + 1], r.w[4 * c4 + 2], r.w[4 * c4 + 3]};
  } else if constexpr (W == 2) {
    *reinterpret_cast<u32x2_t*>(p) = u32x2_t{r.w[0], r.w[1]};
  } else {
    static_assert(W == 1, "row slice width");
    *reinterpret_cast<uint32_t*>(p) = r.w[0];
  }
}

// ---------------------------------------------------------------------------
// Slice access by (re, im) pairs, for head dims whose lane slices cannot all
// be whole vectors: the slice may run past the end of the row (D not a
// multiple of EPL) or its operands may be aligned to a pair only.  The first
// npairs pairs are read or written, one 4-byte (16-bit T) or 8-byte (fp32)
// access each; the rest of the slice reads as zeros and is not written.
// With PAIRS false the whole slice goes by vectors and npairs is unused.
// ---------------------------------------------------------------------------
template <typename T, int EPL, bool PAIRS>
__device__ __forceinline__ void load_slice(RowRegs<T, EPL>& r, const T* p, int npairs) {
  if constexpr (!PAIRS) {
    load_row<T, EPL>(r, p);
  } else {
#pragma unroll
    for (int j = 0; j < EPL / 2; ++j) {
      if constexpr (sizeof(T) == 4) {
        u32x2_t x = {0u, 0u};
        if (j < npairs) x = *reinterpret_cast<const u32x2_t*>(p + 2 * j);
        r.w[2 * j] = x[0];
        r.w[2 * j + 1] = x[1];
      } else {
        r.w[j] = j < npairs ? *reinterpret_cast<const uint32_t*>(p + 2 * j) : 0u;
      }
    }
  }
}

template <typename T, int EPL, bool PAIRS>
__device__ __forceinline__ void store_slice(T* p, const RowRegs<T, EPL>& r, int npairs) {
  if constexpr (!PAIRS) {
    store_row<T, EPL>(p, r);
  } else {
#pragma unroll
    for (int j = 0; j < EPL / 2; ++j) {
      if (j >= npairs) break;
      if constexpr (sizeof(T) == 4)
        *reinterpret_cast<u32x2_t*>(p + 2 * j) = u32x2_t{r.w[2 * j], r.w[2 * j + 1]};
      else
        *reinterpret_cast<uint32_t*>(p + 2 * j) = r.w[j];
    }
  }
}

template <typename T, int EPL, bool PAIRS>
__device__ __forceinline__ void load_vec_slice(const T* p, float (&out)[EPL], int npairs) {
  if constexpr (!PAIRS) {
    load_vec<T, EPL>(p, out);
  } else {
#pragma unroll
    for (int j = 0; j < EPL / 2; ++j) {
      float v[2] = {0.f, 0.f};
      if (j < npairs) load_vec<T, 2>(p + 2 * j, v);
      out[2 * j] = v[0];
      out[2 * j + 1] = v[1];
    }
  }
}

template <typename T, int EPL, bool PAIRS>
__device__ __forceinline__ void store_vec_slice(T* p, const float (&in)[EPL], int npairs) {
  if constexpr (!PAIRS) {
    store_vec<T, EPL>(p, in);
  } else {
#pragma unroll
    for (int j = 0; j < EPL / 2; ++j) {
      if (j >= npairs) break;
      const float v[2] = {in[2 * j], in[2 * j + 1]};
      store_vec<T, 2>(p + 2 * j, v);
    }
  }
}

// Pairs of the slice starting at element d0 that lie inside a row of D.
template <int EPL>
__device__ __forceinline__ int slice_pairs(int d0, int D) {
  const int n = (D - d0) >> 1;
  return n < 0 ? 0 : (n < EPL / 2 ? n : EPL / 2);
}

// Element e of the slice as fp32.
template <typename T, int EPL>
__device__ __forceinline__ float elem(const RowRegs<T, EPL>& r, int e) {
  if constexpr (sizeof(T) == 4) {
    return __uint_as_float(r.w[e]);
  } else if constexpr (__is_same(T, bf16_t)) {
    const uint32_t w = r.w[e >> 1];
    return __uint_as_float((e & 1) ? (w & 0xffff0000u) : (w << 16));
  } else {
    const uint32_t w = r.w[e >> 1];
    const uint16_t hbits = (e & 1) ? (uint16_t)(w >> 16) : (uint16_t)(w & 0xffffu);
    return (float)__builtin_bit_cast(_Float16, hbits);
  }
}

// Partial dot product of the lane's slices of q and k.
template <typename T, int EPL>
__device__ __forceinline__ float slice_dot(const RowRegs<T, EPL>& q, const RowRegs<T, EPL>& k) {
  float d = 0.f;
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int e = 0; e < EPL; ++e) d = __builtin_fmaf(__uint_as_float(q.w[e]), __uint_as_float(k.w[e]), d);
  } else if constexpr (__is_same(T, bf16_t)) {
#pragma unroll
    for (int w = 0; w < EPL / 2; ++w)
      d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v_t, q.w[w]),
                                          __builtin_bit_cast(bf16x2v_t, k.w[w]), d, false);
  } else {
#pragma unroll
    for (int w = 0; w < EPL / 2; ++w)
      d = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2v_t, q.w[w]),
                                 __builtin_bit_cast(f16x2v_t, k.w[w]), d, false);
  }
  return d;
}

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));

// 16 x 16 tile product D += A B^T over the lanes' slices, on the matrix
// cores: lane (c, g) = (l & 15, l >> 4) feeds row c of A and row c of B, each
// with its DQ contiguous elements of the contraction (the same permutation of
// the contraction index for both operands, so the dot products are
// unchanged), and gets back D[c][4g .. 4g+3] read as: row 4g + r of A against
// row c of B, i.e. D^T.  fp32 takes v_mfma_f32_16x16x4_f32 (fp32 products);
// bf16 / fp16 take v_mfma_f32_16x16x16_{bf16,f16} (exact products of two
// 16-bit floats, fp32 accumulation).
template <typename T, int DQ>
__device__ __forceinline__ f32x4_t qk_mfma(const RowRegs<T, DQ>& kop, const RowRegs<T, DQ>& qop, f32x4_t acc) {
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int s = 0; s < DQ; ++s)
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(kop.w[s]), __uint_as_float(qop.w[s]), acc,
                                                 0, 0, 0);
  } else {
    static_assert(DQ % 4 == 0, "16-bit operands come in runs of 4");
#pragma unroll
    for (int s = 0; s < DQ / 4; ++s) {
      const uint32_t ka[2] = {kop.w[2 * s], kop.w[2 * s + 1]};
      const uint32_t qa[2] = {qop.w[2 * s], qop.w[2 * s + 1]};
      if constexpr (__is_same(T, bf16_t))
        acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4_t, ka),
                                                        __builtin_bit_cast(i16x4_t, qa), acc, 0, 0, 0);
      else
        acc = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4_t, ka),
                                                    __builtin_bit_cast(f16x4_t, qa), acc, 0, 0, 0);
    }
  }
  return acc;
}

// Third dword of a raw buffer resource on gfx9-family chips (gfx950 included):
// 32-bit data format, no swizzle, no stride.
constexpr int kBufferWord3 = 0x00020000;

// Global -> LDS copy through a buffer resource: 16 bytes per lane from byte
// offset voff + soff of the resource (zeros past its range) into lds + 16*l
// (buffer_load_dwordx4 ... lds).  The address-space cast stays inside this
// device function.
__device__ __forceinline__ void lds_copy16_buf(__amdgpu_buffer_rsrc_t rs, int voff, int soff, void* lds) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 0);
}

// The 16 accumulators of a 32 x 32 MFMA block: lane l, register r holds row
// 8*(r/4) + 4*(l/32) + r%4 of column l%32.
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float floatx16_t;

// max / sum of x over lanes l and l^32.  v_permlane32_swap with the same
// value in both operands leaves every lane holding its own value in one
// result and lane l^32's in the other (which one depends on the half), so a
// commutative op over the pair gives both halves the same bits.
__device__ __forceinline__ float half_pair_max(float x) {
  const uint32_t u = __float_as_uint(x);
  auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float half_pair_sum(float x) {
  const uint32_t u = __float_as_uint(x);
  auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// ds_read_b64_tr_b16: within each 16 lanes, lane t receives element t & 3 of
// the 8-byte chunks addressed by lanes t/4, 4 + t/4, 8 + t/4, 12 + t/4
__device__ __forceinline__ uint2 lds_read_tr16(const void* lds) {
  const i16x4_t r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4_t*)lds);
  return __builtin_bit_cast(uint2, r);
}

}  // namespace dg

// ---------------------------------------------------------------------------
// Host side: thread-local error slot and launch checking.
// ---------------------------------------------------------------------------
namespace dg {
void set_error(const char* fmt, ...);
int check_launch(const char* what);

// Lane slices of a row of D elements of es bytes (the RoPE and vector
// attention kernels): the row padded to DPAD = the next power of two spreads
// over LPK = DPAD / EPL <= 64 lanes, EPL elements each.  Vector slices are
// max(16 bytes, DPAD / 64) elements read by 16-byte loads (4 or 8 bytes for
// rows that short); they need D to be a multiple of EPL and every operand
// aligned to a load.  Pair slices, max(2, DPAD / 64) elements, need only
// pair alignment: one pair per lane up to DPAD = 128, beyond that read pair
// by pair (load_slice with PAIRS).
constexpr int kMaxHeadDim = 1024;
// Bytes per element of a dg_dtype.
inline int64_t dtype_bytes(int dtype) { return dtype == DG_F64 ? 8 : dtype == DG_F32 ? 4 : 2; }
constexpr int vec_slice_epl(int dpad, int es) {
  const int e = 16 / es < dpad ? 16 / es : dpad;
  return dpad / 64 > e ? dpad / 64 : e;
}
constexpr int pair_slice_epl(int dpad) { return dpad / 64 > 2 ? dpad / 64 : 2; }
// Elements per load of a slice of epl elements: the operands' alignment unit.
constexpr int slice_load_elems(int epl, int es) { return epl * es > 16 ? 16 / es : epl; }

// A shared prefix (dg_prefix) as the kernels read it: keys t < len of row b
// at k + (b / group) * kb + t * (the cache's t stride) + h * kh (likewise v).
// The cache pointers the kernels receive are shifted so that position t >=
// own_start of row b is at cache + b*kb_cache + t*kt + h*kh_cache; they never
// read the cache below own_start, nor write it.  len = 0: no prefix.
struct PrefixRef {
  const void* k;
  const void* v;
  int64_t kb, kh, vb, vh;
  int len, group, own_start;
};
}  // namespace dg

#define DG_REQUIRE(cond, code, ...) \
  do {                              \
    if (!(cond)) {                  \
      ::dg::set_error(__VA_ARGS__); \
      return (code);                \
    }                               \
  } while (0)
