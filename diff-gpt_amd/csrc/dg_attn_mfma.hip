// bf16 / fp16 MFMA prefill attention for gfx950 (the causal / chunked
// branches of mha.py:61-81 when Tq is large and head_dim is 64 or 128).
//
// Workgroup = 4 wavefronts = 128 queries of one (b, h); each wavefront owns 32
// queries.  Keys stream through LDS in tiles of 64.  Both products are issued
// transposed so that a lane's statistics all belong to ONE query:
//
//   S^T (64 keys x 32 queries) = K (64 x D) . Q^T (D x 32)
//        A = K rows from LDS, B = Q^T held in registers for the whole loop
//   O^T (D x 32 queries)      = V^T (D x 64) . P^T (64 x 32)
//        A = V^T from the transposed LDS copy of V, B = P^T straight from
//        the S^T accumulators (converted to bf16, no lane exchange)
//
// with v_mfma_f32_32x32x16_{bf16,f16}.  Lane l (half hh = l/32) holds, in a
// 32x32 accumulator block, row 8*(r/4) + 4*hh + r%4 of column l%32 for
// register r; the column is the lane's query for both S^T and O^T, so the
// online-softmax max / sum / rescale of a query stay inside lanes l and l^32.
// The contraction order of P^T.V^T follows that register order (keys
// 16c + 4hh + {0..3} and 16c + 8 + 4hh + {0..3} for chunk c); V^T is read from
// LDS in exactly that permuted order, so P^T needs no shuffling.
//
// Causality: query i sees key j iff j <= i + (Tk - Tq).  Tiles entirely above
// a wavefront's diagonal are skipped by that wavefront; only tiles crossing
// it evaluate the mask.  Workgroups are mapped so that all query blocks of a
// (b, h) run on the same XCD (blockIdx round-robins over the 8 XCDs), keeping
// that head's K/V resident in one L2, and the longest (last) query blocks of a
// head start first.
#include "dg_common.h"

namespace dg {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float floatx16_t;

struct PrefillArgs {
  const void* q;
  const void* k;
  const void* v;
  void* y;
  int64_t qb, qt, qh;
  int64_t kb, kt, kh;
  int64_t vb, vt, vh;
  int64_t yb, yt, yh;
  int H, Tq, Tk, q_offset;
  int nqb;     // query blocks per (b, h)
  int nwg;     // total workgroups
  float scale_log2;
};

template <typename T>
struct MfmaOps;

template <>
struct MfmaOps<bf16_t> {
  using vec8 = bf16x8_t;
  __device__ static floatx16_t mma(vec8 a, vec8 b, floatx16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  // hardware round-to-nearest-even conversion (v_cvt_pk_bf16_f32)
  __device__ static vec8 pack(const float* x) {
    vec8 r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = (__bf16)x[i];
    return r;
  }
};
template <>
struct MfmaOps<f16_t> {
  using vec8 = f16x8_t;
  __device__ static floatx16_t mma(vec8 a, vec8 b, floatx16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  __device__ static vec8 pack(const float* x) {
    vec8 r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = (_Float16)x[i];
    return r;
  }
};

constexpr int kBM = 128;  // queries per workgroup
constexpr int kBN = 64;   // keys per tile

template <typename T, int D>
__global__ __launch_bounds__(256) void prefill_mfma_kernel(const PrefillArgs a) {
  using Ops = MfmaOps<T>;
  using vec8 = typename Ops::vec8;
  constexpr int KP = D + 8;    // padded K row (elements): 16-byte aligned, bank-shifted
  constexpr int VP = kBN + 8;  // padded V^T row
  constexpr int NC = D / 16;   // 16-wide contraction chunks of QK^T
  constexpr int NB = D / 32;   // 32-row blocks of O^T
  constexpr int CPR = D / 8;   // 16-byte chunks per K/V row
  constexpr int CPT = kBN * CPR / 256;  // chunks per thread per tile (K and V each)
  static_assert(CPT >= 1 && (kBN * CPR) % 256 == 0, "tile mapping");

  __shared__ __attribute__((aligned(16))) uint16_t Ks[kBN * KP];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[D * VP];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int hh = lane >> 5;
  const int r32 = lane & 31;

  // XCD-aware placement: consecutive logical blocks land on one XCD.
  int logical = blockIdx.x;
  if ((a.nwg & 7) == 0) logical = (blockIdx.x & 7) * (a.nwg >> 3) + (blockIdx.x >> 3);
  const int bh = logical / a.nqb;
  const int qblk = a.nqb - 1 - (logical % a.nqb);  // longest query blocks first
  const int head = bh % a.H;
  const int64_t b = bh / a.H;

  const int q0 = qblk * kBM;
  const int qw = q0 + 32 * wv;  // first query of this wavefront
  const int qi = qw + r32;      // this lane's query
  const int qoff = a.q_offset;

  const T* qp = static_cast<const T*>(a.q) + b * a.qb + (int64_t)head * a.qh;
  const T* kp = static_cast<const T*>(a.k) + b * a.kb + (int64_t)head * a.kh;
  const T* vp = static_cast<const T*>(a.v) + b * a.vb + (int64_t)head * a.vh;

  // Q^T fragments (B operand): lane holds Q[qi][16c + 8hh .. +8]
  vec8 qf[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    uint4 raw = make_uint4(0, 0, 0, 0);
    if (qi < a.Tq) raw = *reinterpret_cast<const uint4*>(qp + (int64_t)qi * a.qt + 16 * c + 8 * hh);
    qf[c] = __builtin_bit_cast(vec8, raw);
  }

  const int kv_end = min(a.Tk, q0 + kBM + qoff);
  const int ntiles = (kv_end + kBN - 1) / kBN;
  const bool wave_live = qw < a.Tq;
  const int wave_last_key = qw + 31 + qoff;  // largest key any query of this wave sees

  floatx16_t o[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[nb][r] = 0.f;
  float m = kNegInf, l = 0.f;

  uint4 kreg[CPT], vreg[CPT];
  auto gload = [&](int kt0) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int chunk = tid + 256 * i;
      const int key = chunk / CPR, dc = chunk % CPR;
      const int t = kt0 + key;
      if (t < a.Tk) {
        kreg[i] = *reinterpret_cast<const uint4*>(kp + (int64_t)t * a.kt + 8 * dc);
        vreg[i] = *reinterpret_cast<const uint4*>(vp + (int64_t)t * a.vt + 8 * dc);
      } else {
        kreg[i] = make_uint4(0, 0, 0, 0);
        vreg[i] = make_uint4(0, 0, 0, 0);
      }
    }
  };

  if (ntiles > 0) gload(0);
  for (int tile = 0; tile < ntiles; ++tile) {
    const int kt0 = tile * kBN;
    __syncthreads();  // previous tile's LDS reads are done
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int chunk = tid + 256 * i;
      const int key = chunk / CPR, dc = chunk % CPR;
      *reinterpret_cast<uint4*>(&Ks[key * KP + 8 * dc]) = kreg[i];
      uint16_t e[8];
      __builtin_memcpy(e, &vreg[i], 16);
#pragma unroll
      for (int j = 0; j < 8; ++j) Vt[(8 * dc + j) * VP + key] = e[j];
    }
    __syncthreads();
    if (tile + 1 < ntiles) gload(kt0 + kBN);  // in flight while this tile computes

    if (!wave_live || kt0 > wave_last_key) continue;  // tile entirely above this wave's diagonal

    // S^T = K . Q^T for the two 32-key halves of the tile
    floatx16_t s[2];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[mb][r] = 0.f;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const uint4 raw = *reinterpret_cast<const uint4*>(&Ks[(32 * mb + r32) * KP + 16 * c + 8 * hh]);
        s[mb] = Ops::mma(__builtin_bit_cast(vec8, raw), qf[c], s[mb]);
      }
    }

    // scale into log2 units, mask, tile max
    const bool needs_mask = (kt0 + kBN - 1 > qw + qoff) || (kt0 + kBN > a.Tk);
    float mt = kNegInf;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float x = s[mb][r] * a.scale_log2;
        if (needs_mask) {
          const int key = kt0 + 32 * mb + 8 * (r >> 2) + 4 * hh + (r & 3);
          if (key > qi + qoff || key >= a.Tk) x = kNegInf;
        }
        s[mb][r] = x;
        mt = fmaxf(mt, x);
      }
    }
    mt = fmaxf(mt, shfl_xor(mt, 32));
    const float m_new = fmaxf(m, mt);
    const float alpha = (m == kNegInf) ? 0.f : __builtin_amdgcn_exp2f(m - m_new);
    m = m_new;
    l *= alpha;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[nb][r] *= alpha;

    // P^T fragments: chunk c = 2*mb + r/8, item r%8
    vec8 pf[4];
    float ls = 0.f;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        // m is finite here (key 0 is visible to every query and tile 0 is
        // never skipped), so masked scores give exp2(-inf) = 0
        const float p = __builtin_amdgcn_exp2f(s[mb][r] - m);
        ls += p;
        s[mb][r] = p;
      }
#pragma unroll
      for (int c2 = 0; c2 < 2; ++c2) {
        float t8[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) t8[i] = s[mb][8 * c2 + i];
        pf[2 * mb + c2] = Ops::pack(t8);
      }
    }
    l += ls;

    // O^T += V^T . P^T
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const uint16_t* vrow = &Vt[(32 * nb + r32) * VP + 4 * hh];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint2 lo = *reinterpret_cast<const uint2*>(vrow + 16 * c);
        const uint2 hi = *reinterpret_cast<const uint2*>(vrow + 16 * c + 8);
        const uint4 raw = make_uint4(lo.x, lo.y, hi.x, hi.y);
        o[nb] = Ops::mma(__builtin_bit_cast(vec8, raw), pf[c], o[nb]);
      }
    }
  }

  if (!wave_live || qi >= a.Tq) return;
  const float lt = l + shfl_xor(l, 32);
  const float inv = 1.0f / lt;
  T* yp = static_cast<T*>(a.y) + b * a.yb + (int64_t)qi * a.yt + (int64_t)head * a.yh;
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      T e[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) e[i] = from_f32<T>(o[nb][4 * g + i] * inv);
      uint2 raw;
      __builtin_memcpy(&raw, e, 8);
      *reinterpret_cast<uint2*>(yp + 32 * nb + 8 * g + 4 * hh) = raw;
    }
  }
}

namespace {

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
bool strides8(const dg_stride3* s) { return s->b % 8 == 0 && s->t % 8 == 0 && s->h % 8 == 0; }

template <typename T, int D>
int launch_prefill(const PrefillArgs& a, hipStream_t s) {
  hipLaunchKernelGGL((prefill_mfma_kernel<T, D>), dim3((unsigned)a.nwg), dim3(256), 0, s, a);
  return check_launch("prefill_mfma_kernel");
}

}  // namespace

bool mfma_prefill_applicable(int B, int H, int Tq, int Tk, int D, int dtype, const void* q,
                             const dg_stride3* q_st, const void* k, const dg_stride3* k_st,
                             const void* v, const dg_stride3* v_st, const void* y,
                             const dg_stride3* y_st) {
  if (dtype != DG_BF16 && dtype != DG_F16) return false;
  if (D != 64 && D != 128) return false;
  if (Tq < 16) return false;  // decode and tiny chunks: vector kernel
  const int64_t nwg = (int64_t)B * H * ((Tq + kBM - 1) / kBM);
  if (nwg <= 0 || nwg > 0x7fffffffLL) return false;
  return aligned16(q) && aligned16(k) && aligned16(v) && aligned16(y) && strides8(q_st) &&
         strides8(k_st) && strides8(v_st) && strides8(y_st);
}

int mfma_prefill(int B, int H, int Tq, int Tk, int D, int dtype, const void* q,
                 const dg_stride3* q_st, const void* k, const dg_stride3* k_st, const void* v,
                 const dg_stride3* v_st, void* y, const dg_stride3* y_st, float scale,
                 hipStream_t s) {
  PrefillArgs a{};
  a.q = q; a.k = k; a.v = v; a.y = y;
  a.qb = q_st->b; a.qt = q_st->t; a.qh = q_st->h;
  a.kb = k_st->b; a.kt = k_st->t; a.kh = k_st->h;
  a.vb = v_st->b; a.vt = v_st->t; a.vh = v_st->h;
  a.yb = y_st->b; a.yt = y_st->t; a.yh = y_st->h;
  a.H = H; a.Tq = Tq; a.Tk = Tk;
  a.q_offset = Tk - Tq;
  a.nqb = (Tq + kBM - 1) / kBM;
  a.nwg = B * H * a.nqb;
  a.scale_log2 = scale * 1.44269504088896340736f;
  if (dtype == DG_BF16) return D == 64 ? launch_prefill<bf16_t, 64>(a, s) : launch_prefill<bf16_t, 128>(a, s);
  return D == 64 ? launch_prefill<f16_t, 64>(a, s) : launch_prefill<f16_t, 128>(a, s);
}

}  // namespace dg
