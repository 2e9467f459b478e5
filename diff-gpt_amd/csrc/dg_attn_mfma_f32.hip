// fp32 MFMA prefill attention for gfx950 (the causal / chunked branches of
// mha.py:61-81 for an fp32 model when Tq is large and head_dim is 64 or 128).
//
// Same schedule as the bf16 / fp16 kernel (dg_attn_mfma.hip): a workgroup is
// 4 wavefronts of 32 queries of one (b, h); keys stream through two LDS
// stages in tiles of 32, each wave copying its share of the next tile
// straight from global memory into LDS (buffer_load_dwordx4 ... lds) while
// the current tile is computed; one barrier per tile; the longest query
// blocks of a head start first and all blocks of a head share one XCD.
//
// The products run on v_mfma_f32_32x32x2_f32 (fp32 operands, fp32
// accumulation: 64 matrix cycles per 4096 FLOP, 157 TFLOP/s at the chip's
// 2.4 GHz), transposed so that a lane's softmax statistics all belong to one
// query, as in the bf16 kernel:
//
//   S^T (32 keys x 32 queries) = K (32 x D) . Q^T (D x 32)
//       contraction step c (two dims per step) takes dim (D/2)*hh + c in
//       lane half hh = l/32, so a lane's K operands are D/2 consecutive
//       floats of its key row (one ds_read_b128 per four steps) and its Q^T
//       operands D/2 consecutive floats of its query row, held in registers
//       for the whole loop
//   O^T (D x 32 queries) = V^T (D x 32 keys) . P^T (32 keys x 32 queries)
//       contraction step c takes key 8*(c/4) + 4*hh + c%4 in half hh: the key
//       accumulator register c of S^T holds, so P^T's operand is that register
//       itself (no lane exchange); row i of O^T block nb is dim NB*i + nb
//       (NB = D/32 blocks), so a lane's V operands for the NB blocks are NB
//       consecutive floats of one key row (one ds_read_b64 / b128 per step)
//
// Lane l, accumulator register r of a 32x32 block holds row
// 8*(r/4) + 4*(l/32) + r%4 of column l%32.  The softmax keeps a running
// maximum with the bf16 kernel's lazy rescale (the offset is raised only when
// a row's maximum outgrows it by more than kLazyLog2 in log2 units) and sums
// the fp32 probabilities that feed the PV products.  P stays fp32: no
// rounding beyond the fp32 arithmetic.
//
// LDS: K and V tiles row-major, the 16-byte pieces of row r at slot
// piece ^ (r & 15): the K operand reads (16 rows, one piece each, per 16
// lanes) and the V reads (one whole row per 32 lanes) are free of bank
// conflicts.
//
// ROPE instances (dg_prefill_rope) rotate and normalise each query row as it
// is loaded (mha.py:44-48) with rope_qknorm_kernel's arithmetic: a lane's
// half row rotates with its (cos, sin) pairs (rope_rotate), its squares sum
// by the pairwise tree (tree_sum) and meet the other half's in lane l^32 --
// the top level of the same tree over the row -- so the operand has the bits
// dg_rope_qknorm_append would store.
#include "dg_prefill.h"
#include "dg_rope_math.h"

namespace dg {

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4v_t __attribute__((ext_vector_type(4)));

template <int D>
struct PrefillF32Cfg {
  static constexpr int WAVES = 4;
  static constexpr int NT = 64 * WAVES;          // threads per workgroup
  static constexpr int BM = 32 * WAVES;          // queries per workgroup
  static constexpr int BN = 32;                  // keys per tile
  static constexpr int QC = D / 2;               // contraction steps of S^T (and q registers per lane)
  static constexpr int NB = D / 32;              // 32-row blocks of O^T
  static constexpr int PPR = D / 4;              // 16-byte pieces per row
  static constexpr int TILE = BN * D;            // floats of one K or V tile
  static constexpr int ROWS_PER_DMA = 64 / PPR;  // rows one wave-wide 1 KB copy covers
  static constexpr int DMA_PER_WAVE = BN / ROWS_PER_DMA / WAVES;
  static_assert(DMA_PER_WAVE >= 1 && BN % (ROWS_PER_DMA * WAVES) == 0, "tile copy split");
};

__device__ __forceinline__ int f32_slot(int piece, int row) { return piece ^ (row & 15); }

__device__ __forceinline__ floatx16_t mma_f32(float a, float b, floatx16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// Resident workgroups per CU: D = 64 fits 4 (32 KB of LDS, <= 128 VGPRs);
// D = 128 two (64 KB of LDS each).
template <int D>
constexpr int prefill_f32_wgs_per_cu() {
  return D == 64 ? 4 : 2;
}

template <int D, bool ROPE>
__global__ __launch_bounds__(256, (prefill_f32_wgs_per_cu<D>()))
void prefill_mfma_f32_kernel(const PrefillArgs a) {
  using C = PrefillF32Cfg<D>;
  constexpr int QC = C::QC, NB = C::NB, PPR = C::PPR, BN = C::BN;

  // two ring stages, each an array of its own (K tile, then V tile)
  __shared__ __attribute__((aligned(16))) float kv0[2 * C::TILE];
  __shared__ __attribute__((aligned(16))) float kv1[2 * C::TILE];
  float* const ks0 = kv0;
  float* const vs0 = kv0 + C::TILE;
  float* const ks1 = kv1;
  float* const vs1 = kv1 + C::TILE;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hh = lane >> 5;
  const int r32 = lane & 31;

  // grid (win, nqb, windows): block (x, y, z) takes pair z*win + x and query
  // block nqb - 1 - y (the bf16 kernel's schedule)
  const int bh = blockIdx.z * a.win + blockIdx.x;
  if (bh >= a.nbh) return;  // the last window's spare columns (whole workgroup, before any barrier)
  const int qblk = a.nqb - 1 - blockIdx.y;
  const int head = bh % a.H;
  const int64_t b = bh / a.H;
  const int q0 = qblk * C::BM;
  const int qw = q0 + 32 * wv;  // first query of this wavefront
  const int qoff = a.q_offset;

  const float* qp = static_cast<const float*>(a.q) + b * a.qb + (int64_t)head * a.qh;
  const float* kp = static_cast<const float*>(a.k) + b * a.kb + (int64_t)head * a.kh;
  const float* vp = static_cast<const float*>(a.v) + b * a.vb + (int64_t)head * a.vh;

  // ---- global -> LDS copy of one key tile ----------------------------------
  // Wave wv copies DMA_PER_WAVE blocks of 1 KB of K and of V; lane l of a
  // block fills slot l % PPR of row l / PPR with the piece the swizzle puts
  // there.  Rows past Tk lie beyond the buffer's range and read as zeros
  // (their keys are masked).
  const int dma_row = lane / PPR, dma_slot = lane % PPR;
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(kp), 0, (int)(((int64_t)(a.Tk - 1) * a.kt + D) * 4), kBufferWord3);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(vp), 0, (int)(((int64_t)(a.Tk - 1) * a.vt + D) * 4), kBufferWord3);
  int kvo[C::DMA_PER_WAVE], vvo[C::DMA_PER_WAVE];
#pragma unroll
  for (int i = 0; i < C::DMA_PER_WAVE; ++i) {
    const int row = (wv * C::DMA_PER_WAVE + i) * C::ROWS_PER_DMA + dma_row;
    const int piece = f32_slot(dma_slot, row);  // the swizzle is its own inverse
    kvo[i] = (row * (int)a.kt + 4 * piece) * 4;
    vvo[i] = (row * (int)a.vt + 4 * piece) * 4;
  }
  auto dma_tile = [&](float* ks, float* vs, int kt0) __attribute__((always_inline)) {
    const int ko = kt0 * (int)a.kt * 4, vo = kt0 * (int)a.vt * 4;
#pragma unroll
    for (int i = 0; i < C::DMA_PER_WAVE; ++i) {
      const int blk = wv * C::DMA_PER_WAVE + i;
      lds_copy16_buf(krs, kvo[i], ko, ks + blk * 256);
      lds_copy16_buf(vrs, vvo[i], vo, vs + blk * 256);
    }
  };
  auto stage_ready = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_s_barrier();
  };

  // Q^T operands: lane (r32, hh) holds Q[qw + r32][(D/2)*hh + c], c < D/2.
  // Rows past Tq hold row Tq - 1 (finite) and are never stored.
  float qf[QC];
  const int qi0 = min(qw + r32, a.Tq - 1);
  {
    const f32x4v_t* src = reinterpret_cast<const f32x4v_t*>(qp + (int64_t)qi0 * a.qt + QC * hh);
#pragma unroll
    for (int m = 0; m < QC / 4; ++m) {
      const f32x4v_t x = src[m];
      qf[4 * m] = x[0];
      qf[4 * m + 1] = x[1];
      qf[4 * m + 2] = x[2];
      qf[4 * m + 3] = x[3];
    }
  }
  float cs[ROPE ? QC : 1];
  if constexpr (ROPE)
    load_vec<float, QC>(static_cast<const float*>(a.freqs) + b * a.fb + (int64_t)qi0 * a.ft + (int64_t)head * a.fh +
                            QC * hh,
                        cs);
  dma_tile(ks0, vs0, 0);
  if constexpr (ROPE) {
#pragma clang fp contract(off)
    rope_rotate<float, QC>(qf, cs);
    if (a.qknorm) {
      // lanes l and l^32 hold the same row, so both take this branch
      float sq[QC];
#pragma unroll
      for (int c = 0; c < QC; ++c) sq[c] = qf[c] * qf[c];
      const float mean = half_pair_sum(tree_sum<QC>(sq)) / (float)D;
      const float r = 1.0f / sqrtf(mean + FLT_EPSILON);
#pragma unroll
      for (int c = 0; c < QC; ++c) qf[c] = qf[c] * r;
    }
  }

  const int kv_end = min(a.Tk, q0 + C::BM + qoff);
  const int ntiles = (kv_end + BN - 1) / BN;
  const bool wave_live = qw < a.Tq;
  const int wave_last_key = qw + 31 + qoff;  // largest key any query of this wave sees

  floatx16_t o[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[nb][r] = 0.f;
  float m = kNegInf, l = 0.f;

  // per-lane parts of the LDS operand addresses
  const int kslot0 = (PPR / 2) * hh;  // first piece of the lane's K dims
  auto compute_tile = [&](const float* Ks, const float* Vs, int kt0) __attribute__((always_inline)) {
    // S^T = K . Q^T
    floatx16_t s;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = 0.f;
    const float* krow = Ks + r32 * D;
#pragma unroll
    for (int p = 0; p < QC / 4; ++p) {
      const f32x4v_t kf = *reinterpret_cast<const f32x4v_t*>(krow + 4 * f32_slot(kslot0 + p, r32));
#pragma unroll
      for (int e = 0; e < 4; ++e) s = mma_f32(kf[e], qf[4 * p + e], s);
    }
    // mask (only on tiles that cross the diagonal or the end of the keys)
    if (kt0 + BN - 1 > qw + qoff || kt0 + BN > a.Tk) {
      const int lim = min(qw + r32 + qoff, a.Tk - 1) - kt0 - 4 * hh;
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (8 * (r >> 2) + (r & 3) > lim) s[r] = kNegInf;
    }
    // online softmax with the lazy rescale (scale > 0 commutes with the max)
    float mt = s[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mt = fmaxf(mt, s[r]);
    mt = half_pair_max(mt);
    const float mnew = fmaxf(m, mt);
    if (__builtin_amdgcn_ballot_w64(mnew > m + a.lazy_raw) != 0) {
      // m == -inf only before the first tile; key 0 is visible to every
      // query, so mnew is finite from then on
      const float alpha = (m == kNegInf) ? 0.f : __builtin_amdgcn_exp2f((m - mnew) * a.scale_log2);
      m = mnew;
      l *= alpha;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[nb][r] *= alpha;
    }
    const float moff = m * a.scale_log2;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[r], a.scale_log2, -moff));
      l += s[r];
    }
    // O^T += V^T . P^T: step c takes key 8*(c/4) + 4*hh + c%4, the key of
    // accumulator register c
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      const int key = 8 * (c >> 2) + 4 * hh + (c & 3);
      const float* vrow = Vs + key * D;
      if constexpr (NB == 2) {
        // dims 2*r32, 2*r32 + 1: half of piece r32/2
        const f32x2_t vf = *reinterpret_cast<const f32x2_t*>(vrow + 4 * f32_slot(r32 >> 1, key) + 2 * (r32 & 1));
        o[0] = mma_f32(vf[0], s[c], o[0]);
        o[1] = mma_f32(vf[1], s[c], o[1]);
      } else {
        // dims 4*r32 .. 4*r32 + 3: piece r32
        const f32x4v_t vf = *reinterpret_cast<const f32x4v_t*>(vrow + 4 * f32_slot(r32, key));
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) o[nb] = mma_f32(vf[nb], s[c], o[nb]);
      }
    }
  };

  stage_ready();  // the first tile (Tk >= Tq >= 1, so every workgroup has one)
  for (int tile = 0; tile < ntiles; tile += 2) {
    const int kt0 = tile * BN;
    if (tile + 1 < ntiles) dma_tile(ks1, vs1, kt0 + BN);
    if (wave_live && kt0 <= wave_last_key) compute_tile(ks0, vs0, kt0);
    stage_ready();  // stage 1 filled; every wave is done with stage 0
    if (tile + 1 >= ntiles) break;
    if (tile + 2 < ntiles) dma_tile(ks0, vs0, kt0 + 2 * BN);
    if (wave_live && kt0 + BN <= wave_last_key) compute_tile(ks1, vs1, kt0 + BN);
    stage_ready();
  }

  if (!wave_live) return;
  const int qi = qw + r32;
  if (qi >= a.Tq) return;
  // O^T block nb, register 4g + e of half hh: dim NB*(8g + 4hh + e) + nb of the
  // lane's query, so group g gives 4*NB consecutive dims
  const float inv = __builtin_amdgcn_rcpf(half_pair_sum(l));
  float* yrow = static_cast<float*>(a.y) + b * a.yb + (int64_t)qi * a.yt + (int64_t)head * a.yh;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    float* dst = yrow + NB * (8 * g + 4 * hh);
    if constexpr (NB == 2) {
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        f32x4v_t w;
        w[0] = o[0][4 * g + 2 * h2] * inv;
        w[1] = o[1][4 * g + 2 * h2] * inv;
        w[2] = o[0][4 * g + 2 * h2 + 1] * inv;
        w[3] = o[1][4 * g + 2 * h2 + 1] * inv;
        *reinterpret_cast<f32x4v_t*>(dst + 4 * h2) = w;
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        f32x4v_t w;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) w[nb] = o[nb][4 * g + e] * inv;
        *reinterpret_cast<f32x4v_t*>(dst + 4 * e) = w;
      }
    }
  }
}

int launch_prefill_f32(PrefillArgs a, int D, hipStream_t s) {
  constexpr int BM = 128;
  a.nqb = (a.Tq + BM - 1) / BM;
  const int nwin = (a.nbh + a.win - 1) / a.win;
  DG_REQUIRE(a.nqb <= 65535 && nwin <= 65535, DG_EINVAL, "prefill: %d query blocks, %d windows, at most 65535 each",
             a.nqb, nwin);
  const dim3 grid((unsigned)a.win, (unsigned)a.nqb, (unsigned)nwin);
  static_assert(PrefillF32Cfg<64>::BM == BM && PrefillF32Cfg<128>::BM == BM, "query block size");
  DG_REQUIRE(D == 64 || D == 128, DG_EINVAL, "prefill_f32: head_dim %d (64 or 128)", D);
  const dim3 block(PrefillF32Cfg<64>::NT);
  if (a.freqs != nullptr) {
    if (D == 64) hipLaunchKernelGGL((prefill_mfma_f32_kernel<64, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((prefill_mfma_f32_kernel<128, true>), grid, block, 0, s, a);
  } else {
    if (D == 64) hipLaunchKernelGGL((prefill_mfma_f32_kernel<64, false>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((prefill_mfma_f32_kernel<128, false>), grid, block, 0, s, a);
  }
  return check_launch("prefill_mfma_f32_kernel");
}

}  // namespace dg
