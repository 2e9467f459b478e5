// bf16 / fp16 MFMA prefill attention for gfx950 (the causal / chunked
// branches of mha.py:61-81 when Tq is large and head_dim is 64 or 128).
//
// Workgroup = 4 wavefronts; each wavefront owns QW blocks of 32 queries of one
// (b, h), so a workgroup covers BM = 128*QW queries.  Keys stream through two
// LDS stages in tiles of BN keys (64 at D = 64, 32 at D = 128; the text below
// writes BN = 64): every wave copies its share of the next tile
// straight from global memory into LDS (buffer_load_dwordx4 ... lds: no
// registers, no shuffles) while the current tile is computed, then waits for
// its own copies and meets the others at one barrier per tile.  K and V tiles
// are kept row-major with the 16-byte pieces of row r XOR-swizzled
// (piece_swz), which makes both operand reads below free of bank conflicts.  Both products are
// issued transposed so that a lane's statistics all belong to ONE query:
//
//   S^T (64 keys x 32 queries) = K (64 x D) . Q^T (D x 32)
//        A = K rows from LDS (ds_read_b128), B = Q^T held in registers for the
//        whole loop
//   O^T (D x 32 queries)      = V^T (D x 64) . P^T (64 x 32)
//        A = V^T read from the row-major V tile with ds_read_b64_tr_b16 (the
//        transposing LDS read: 4 keys x 16 dims per 16 lanes), B = P^T
//        straight from the S^T accumulators (packed to bf16/fp16, no lane
//        exchange)
//
// with v_mfma_f32_32x32x16_{bf16,f16}.  Lane l (half hh = l/32) holds, in a
// 32x32 accumulator block, row 8*(r/4) + 4*hh + r%4 of column l%32 for
// register r; the column is the lane's query for both S^T and O^T, so the
// online-softmax statistics of a query live in lanes l and l^32 and meet
// through one v_permlane32_swap.  The contraction order of P^T.V^T follows
// that register order (keys 16c + 4hh + {0..3} and 16c + 8 + 4hh + {0..3} for
// chunk c); the two transposing reads fetch V^T in exactly that order.
//
// Softmax arithmetic per score: one max (v_max3), one FMA (scale and max
// subtraction in log2 units), one exp2, half a bf16 pack and half a dot2 (the
// row sum adds the packed bf16/fp16 probabilities that also feed the MFMA, so
// numerator and denominator use the same rounded values; the bounded form
// below sums the fp32 probabilities instead).  The running max
// used as the exponent offset is raised only when a row's new maximum exceeds
// it by more than kLazyLog2 (log2 units); in between, probabilities up to
// 2^kLazyLog2 are accumulated exactly as the online softmax would after a
// rescale, so the result is the same function -- only the rescale of the
// accumulators is skipped.
//
// The output leaves through LDS (the stage arrays are free after the last
// tile), so that every store instruction writes whole 128/256-byte rows.
//
// Causality: query i sees key j iff j <= i + (Tk - Tq).  Tiles entirely above
// a wavefront's diagonal are skipped by that wavefront; only tiles crossing
// it evaluate the mask.  Workgroups are mapped so that all query blocks of a
// (b, h) run on the same XCD (blockIdx round-robins over the 8 XCDs), keeping
// that head's K/V resident in one L2, and the longest (last) query blocks of a
// head start first.
#include "dg_prefill.h"
#include "dg_rope_math.h"

namespace dg {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8_t;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;
typedef _Float16 __attribute__((ext_vector_type(2))) f16x2_t;
// plain clang vector (not HIP's uint4 wrapper class) so staging arrays stay in registers
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));


template <typename T>
struct MfmaOps;

template <>
struct MfmaOps<bf16_t> {
  using vec8 = bf16x8_t;
  __device__ static floatx16_t mma(vec8 a, vec8 b, floatx16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  // v_cvt_pk_bf16_f32: round to nearest even, two values per instruction
  __device__ static uint32_t pack2(float a, float b) {
    bf16x2_t r;
    r[0] = (__bf16)a;
    r[1] = (__bf16)b;
    return __builtin_bit_cast(uint32_t, r);
  }
  // acc + lo + hi of a packed pair (v_dot2c_f32_bf16 against (1, 1))
  __device__ static float add_pair(uint32_t p, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, p),
                                           __builtin_bit_cast(bf16x2_t, 0x3f803f80u), acc, false);
  }
};
template <>
struct MfmaOps<f16_t> {
  using vec8 = f16x8_t;
  __device__ static floatx16_t mma(vec8 a, vec8 b, floatx16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  __device__ static uint32_t pack2(float a, float b) {
    f16x2_t r;
    r[0] = (_Float16)a;
    r[1] = (_Float16)b;
    return __builtin_bit_cast(uint32_t, r);
  }
  __device__ static float add_pair(uint32_t p, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, p),
                                  __builtin_bit_cast(f16x2_t, 0x3c003c00u), acc, false);
  }
};

// Keys per tile: 64 at D = 64; 32 at D = 128, which halves the S and P
// registers (168 VGPRs) and the LDS stages (32 KB per workgroup), so three
// workgroups share a CU instead of two (+4 to +10 % at configs[4]'s shapes).
template <int D>
constexpr int prefill_bn() {
  return D == 64 ? 64 : 32;
}
// Schedule of the bounded form's 32-key blocks, per head_dim (measured at
// configs[2] / [4]: D = 64 gains 3-4 % from the prefetch, while the
// prefetched V^T fragments do not fit D = 128's register budget and halve
// its rate; the in-wave overlap is neutral at D = 64 and kept at D = 128):
//   pipe     -- the S products of block mb + 1 are issued before the softmax
//               of block mb (two S blocks live)
//   prefetch -- a block's K fragments are all read before its S products and
//               its V^T fragments before its softmax (one LDS wait each)
template <int D>
constexpr bool prefill_pipe() {
  return D != 64;
}
template <int D>
constexpr bool prefill_prefetch() {
  return D == 64;
}

template <typename T, int D, int QW>
struct PrefillCfg {
  static constexpr int WAVES = 4;                 // wavefronts per workgroup
  static constexpr int NT = 64 * WAVES;           // threads per workgroup
  static constexpr int BM = 32 * QW * WAVES;      // queries per workgroup
  static constexpr int NC = D / 16;               // 16-wide contraction chunks of QK^T
  static constexpr int NB = D / 32;               // 32-row blocks of O^T
  static constexpr int PPR = D / 8;               // 16-byte pieces per K/V row
  static constexpr int BN = prefill_bn<D>();       // keys per tile
  static constexpr int MB = BN / 32;              // 32-key blocks of S^T per tile
  static constexpr int PC = BN / 16;              // 16-key chunks of P^T per tile
  static constexpr int TILE = BN * D;             // elements of one K or V tile
  static constexpr int ROWS_PER_DMA = 64 / PPR;   // rows one wave-wide 1 KB copy covers
  static constexpr int DMA_PER_WAVE = BN / ROWS_PER_DMA / WAVES;
  static_assert(DMA_PER_WAVE >= 1 && BN % (ROWS_PER_DMA * WAVES) == 0, "tile copy split");
  static constexpr int LDS_BYTES = 4 * TILE * 2;  // K and V, two stages
};

// XOR swizzle of the 16-byte pieces of K/V row r in LDS (slot = piece ^ f(r)):
// conflict-free both for the K operand reads (16 consecutive rows, one piece
// each) and for the transposed V reads (4 consecutive rows, 4 adjacent pieces,
// per 16 lanes).
template <int D>
__device__ __forceinline__ int piece_swz(int r) {
  if constexpr (D == 64) return ((r & 2) << 1) | ((r >> 2) & 3);
  else return ((r & 3) << 2) | ((r >> 2) & 3);
}

// Resident workgroups per CU the register allocation must allow: D = 64 fits
// 4 (<= 128 VGPRs -> 4 waves per SIMD to overlap one wave's MFMAs with
// another's softmax); D = 128 with 32-key tiles 3 (<= 168 VGPRs).
template <int D, bool BND>
constexpr int prefill_wgs_per_cu() {
  return D == 64 ? 4 : 3;
}

template <typename T, int D, int QW, bool ROPE, typename FT, bool BND>
__global__ __launch_bounds__(256, (prefill_wgs_per_cu<D, BND>()))
void prefill_mfma_kernel(const PrefillArgs a) {
  using Ops = MfmaOps<T>;
  using vec8 = typename Ops::vec8;
  using C = PrefillCfg<T, D, QW>;
  constexpr int NC = C::NC, NB = C::NB, PPR = C::PPR, BN = C::BN, MB = C::MB, PC = C::PC;
  constexpr bool kPrefillPipe = prefill_pipe<D>();
  constexpr bool kPrefillPrefetch = prefill_prefetch<D>();

  // two ring stages, each an array of its own (K tile, then V tile): the
  // compiler can then tell the stage being copied into from the one being
  // read.  32 KB per workgroup at D = 64 lets four workgroups share a CU
  // (measured: with 40 KB at most three were ever resident)
  __shared__ __attribute__((aligned(16))) uint16_t kv0[2 * C::TILE];
  __shared__ __attribute__((aligned(16))) uint16_t kv1[2 * C::TILE];
  uint16_t* const ks0 = kv0;
  uint16_t* const vs0 = kv0 + C::TILE;
  uint16_t* const ks1 = kv1;
  uint16_t* const vs1 = kv1 + C::TILE;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hh = lane >> 5;
  const int r32 = lane & 31;

  // Schedule: the (b, h) pairs go in windows of a.win; the grid is
  // (win, nqb, windows) and block (x, y, z) takes pair z*win + x and query
  // block nqb - 1 - y.  Blocks are dispatched in linear order
  // x + win*(y + nqb*z), so inside a window the blocks run longest query
  // block first (long ones start early, short ones fill in at the end) and
  // the window's K/V stays cache-resident while its query blocks run.  Block
  // i runs on XCD i % 8: with a.win a multiple of 8 all query blocks of a
  // (b, h) share one XCD and its L2.  (No divisions: this grid replaces the
  // index arithmetic of a 1-D one.)
  const int bh = blockIdx.z * a.win + blockIdx.x;
  if (bh >= a.nbh) return;  // the last window's spare columns (whole workgroup, before any barrier)
  const int qblk = a.nqb - 1 - blockIdx.y;
  const int head = bh % a.H;
  const int64_t b = bh / a.H;

  const int q0 = qblk * C::BM;
  const int qw = q0 + 32 * QW * wv;  // first query of this wavefront
  const int qoff = a.q_offset;

  const T* qp = static_cast<const T*>(a.q) + b * a.qb + (int64_t)head * a.qh;
  const T* kp = static_cast<const T*>(a.k) + b * a.kb + (int64_t)head * a.kh;
  const T* vp = static_cast<const T*>(a.v) + b * a.vb + (int64_t)head * a.vh;

  // ---- global -> LDS copy of one key tile (no registers involved) -----------
  // Wave wv copies DMA_PER_WAVE blocks of 1 KB of K and of V; lane l of a block
  // fills slot l % PPR of row l / PPR with the piece that the swizzle puts
  // there.
  const int dma_row = lane / PPR, dma_slot = lane % PPR;
  // Buffer loads over this head's K and V rows: the per-lane byte offsets of
  // a tile's pieces are fixed, the tile's start goes into the scalar offset,
  // so a tile's copies cost no vector arithmetic.  Rows past Tk lie beyond
  // the resource's range and read as zeros (their keys are masked).
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<T*>(kp), 0, (int)(((int64_t)(a.Tk - 1) * a.kt + D) * 2), kBufferWord3);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<T*>(vp), 0, (int)(((int64_t)(a.Tk - 1) * a.vt + D) * 2), kBufferWord3);
  int kvo[C::DMA_PER_WAVE], vvo[C::DMA_PER_WAVE];
#pragma unroll
  for (int i = 0; i < C::DMA_PER_WAVE; ++i) {
    const int row = (wv * C::DMA_PER_WAVE + i) * C::ROWS_PER_DMA + dma_row;
    const int piece = dma_slot ^ piece_swz<D>(row);
    kvo[i] = (row * (int)a.kt + 8 * piece) * 2;
    vvo[i] = (row * (int)a.vt + 8 * piece) * 2;
  }
  auto dma_tile = [&](uint16_t* ks, uint16_t* vs, int kt0) __attribute__((always_inline)) {
    const int ks0 = kt0 * (int)a.kt * 2, vs0 = kt0 * (int)a.vt * 2;
#pragma unroll
    for (int i = 0; i < C::DMA_PER_WAVE; ++i) {
      const int blk = wv * C::DMA_PER_WAVE + i;
      lds_copy16_buf(krs, kvo[i], ks0, ks + blk * 512);
      lds_copy16_buf(vrs, vvo[i], vs0, vs + blk * 512);
    }
  };
  // this wave's copies are in LDS (each wave waits for its own before the
  // barrier that hands the stage to all waves)
  auto stage_ready = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_s_barrier();
  };

  // Q^T fragments (B operand): lane holds Q[qi][16c + 8hh .. +8].  The first
  // key tile's copies go out right behind the query loads.
  vec8 qf[QW][NC];
  if constexpr (ROPE && D == 64 && QW == 1) {
    // RoPE instances at D = 64: the query rows and their (cos, sin) rows are
    // loaded whole-line coalesced -- 8 lanes per 128-byte row, lane
    // (r, p) = (l / 8, l % 8) holding elements 8p .. 8p+7 of rows r, r + 8,
    // r + 16, r + 24 of the wave -- and rotated, normalised and packed in
    // that layout; one LDS round trip then hands each lane its operand
    // chunks.  (Loaded in the operand layout, every load instruction touches
    // 32 rows for 32 bytes each: measured 3-4x the cost per byte through the
    // vector memory path.)  The exact form's lanes and reduction tree are
    // those of rope_qknorm_kernel at D = 64 (8 elements per lane, 8 lanes per
    // row), so its bits are the same.  Each wave stages its 32 rows (4 KB,
    // 16-byte pieces XOR-swizzled by row) in the second stage, which nothing
    // else touches before the barrier that precedes the loop.  (For the
    // general kernel's plain q loads the round trip measured neutral.)
    const int prow = lane >> 3, ppc = lane & 7;
    auto qswz = [](int r) { return (r >> 1) & 7; };
    uint4 packed[4];
    {
#pragma clang fp contract(off)
      float x[4][8], cs[4][8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // rows past Tq hold row Tq - 1 (finite, normalised) and are never stored
        const int qi = min(qw + 8 * i + prow, a.Tq - 1);
        load_vec<T, 8>(qp + (int64_t)qi * a.qt + 8 * ppc, x[i]);
        load_vec<FT, 8>(static_cast<const FT*>(a.freqs) + b * a.fb + (int64_t)qi * a.ft + (int64_t)head * a.fh + 8 * ppc,
                        cs[i]);
      }
      dma_tile(ks0, vs0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t w[4];
        if constexpr (BND) {
          // Bounded form (launched with the norm): the operand only has to
          // carry q's direction to the bf16 bar, so the row is rotated in fp32
          // (FMAs), its sum of squares taken on the fp32 rotation, and the
          // rotation times rsqrt(mean + eps) * scale * log2(e) rounded once --
          // one rounding where the reference rounds the rotation and the
          // normalised row.
          float acc = 0.f;
#pragma unroll
          for (int p = 0; p < 4; ++p) {
            const float re = x[i][2 * p], im = x[i][2 * p + 1];
            const float co = cs[i][2 * p], sn = cs[i][2 * p + 1];
            x[i][2 * p] = __builtin_fmaf(re, co, -(im * sn));
            x[i][2 * p + 1] = __builtin_fmaf(re, sn, im * co);
            acc = __builtin_fmaf(x[i][2 * p + 1], x[i][2 * p + 1], __builtin_fmaf(x[i][2 * p], x[i][2 * p], acc));
          }
          const float ss = group_sum_dpp<8>(acc);
          const float r = __builtin_amdgcn_rsqf(__builtin_fmaf(ss, 1.0f / (float)D, FLT_EPSILON)) * a.scale_log2;
#pragma unroll
          for (int p = 0; p < 4; ++p) w[p] = pack_pair<T>(x[i][2 * p] * r, x[i][2 * p + 1] * r);
        } else {
          rope_rotate<T, 8>(x[i], cs[i]);
          if (a.qknorm) qk_rms_norm<8, 8, true>(x[i], D);
#pragma unroll
          for (int p = 0; p < 4; ++p) w[p] = pack_pair<T>(x[i][2 * p], x[i][2 * p + 1]);
        }
        packed[i] = make_uint4(w[0], w[1], w[2], w[3]);
      }
    }
    // all four waves stage in the one array kv1 (a pointer chosen between two
    // arrays would leave the compiler unable to tell these accesses from the
    // copies into the first stage, and it would make them wait for those)
    uint16_t* qst = kv1 + wv * 32 * D;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 8 * i + prow;
      *reinterpret_cast<uint4*>(qst + r * D + 8 * (ppc ^ qswz(r))) = packed[i];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int c = 0; c < NC; ++c)
      qf[0][c] = __builtin_bit_cast(vec8, *reinterpret_cast<const uint4*>(qst + r32 * D + 8 * ((2 * c + hh) ^ qswz(r32))));
  } else if constexpr (ROPE) {
    // RoPE + QK-norm of the query rows as they are loaded (mha.py:44-48), with
    // the arithmetic and roundings of dg_rope_qknorm_append, so the operand
    // has the bits that kernel would store: each 8-element chunk 16c + 8hh
    // rotates with its (cos, sin) pairs; the norm's sum of squares follows the
    // same pairwise tree over the row (chunk sums, the partner lane l^32 for
    // 16-element sums, then across chunks).  Rows past Tq load zeros.
#pragma clang fp contract(off)
    float x[QW][NC][8], cs[QW][NC][8];
#pragma unroll
    for (int qb = 0; qb < QW; ++qb) {
      const int qi = min(qw + 32 * qb + r32, a.Tq - 1);
      const T* qrow = qp + (int64_t)qi * a.qt;
      const FT* frow = static_cast<const FT*>(a.freqs) + b * a.fb + (int64_t)qi * a.ft + (int64_t)head * a.fh;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        load_vec<T, 8>(qrow + 16 * c + 8 * hh, x[qb][c]);
        load_vec<FT, 8>(frow + 16 * c + 8 * hh, cs[qb][c]);
      }
    }
    dma_tile(ks0, vs0, 0);
#pragma unroll
    for (int qb = 0; qb < QW; ++qb) {
      // rows past Tq hold row Tq - 1 (finite, normalised) and are never stored
#pragma unroll
      for (int c = 0; c < NC; ++c) rope_rotate<T, 8>(x[qb][c], cs[qb][c]);
      // the bounded form is launched with the norm; lanes l and l^32 hold the
      // same row, so both take this branch
      if (BND || a.qknorm) {
        float s16[NC];
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          float sq[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) sq[i] = x[qb][c][i] * x[qb][c][i];
          s16[c] = half_pair_sum(tree_sum<8>(sq));
        }
        const float mean = tree_sum<NC>(s16) / (float)D;
        float r = 1.0f / sqrtf(mean + FLT_EPSILON);
        // bounded form: the operand is the normalised row times scale*log2(e),
        // rounded once, so the scores come out of the MFMA in log2 units
        if constexpr (BND) r = r * a.scale_log2;
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
          for (int i = 0; i < 8; ++i) x[qb][c][i] = x[qb][c][i] * r;
      }
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = pack_pair<T>(x[qb][c][2 * i], x[qb][c][2 * i + 1]);
        qf[qb][c] = __builtin_bit_cast(vec8, make_uint4(w[0], w[1], w[2], w[3]));
      }
    }
  } else {
#pragma unroll
    for (int qb = 0; qb < QW; ++qb) {
      const int qi = qw + 32 * qb + r32;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        uint4 raw = make_uint4(0, 0, 0, 0);
        if (qi < a.Tq) raw = *reinterpret_cast<const uint4*>(qp + (int64_t)qi * a.qt + 16 * c + 8 * hh);
        qf[qb][c] = __builtin_bit_cast(vec8, raw);
      }
    }
    dma_tile(ks0, vs0, 0);
  }

  const int kv_end = min(a.Tk, q0 + C::BM + qoff);
  const int ntiles = (kv_end + BN - 1) / BN;
  const bool wave_live = qw < a.Tq;
  const int wave_last_key = qw + 32 * QW - 1 + qoff;  // largest key any query of this wave sees

  floatx16_t o[QW][NB];
#pragma unroll
  for (int qb = 0; qb < QW; ++qb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[qb][nb][r] = 0.f;
  float m[QW], l[QW];
#pragma unroll
  for (int qb = 0; qb < QW; ++qb) {
    m[qb] = kNegInf;
    l[qb] = 0.f;
  }

  // per-lane parts of the LDS operand addresses
  const int kswz = piece_swz<D>(r32);  // rows 32mb + r32 share it
  const int g16 = lane >> 4, t16 = lane & 15;
  const int vhh = g16 >> 1, vhalf = g16 & 1;
  int voff[2][NB];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int row = 8 * u + 4 * vhh + (t16 >> 2);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int col = 32 * nb + 16 * vhalf + 4 * (t16 & 3);
      voff[u][nb] = row * D + 8 * ((col >> 3) ^ piece_swz<D>(row)) + (col & 7);
    }
  }

  // Bounded form (BND): q and k rows are RMS-normalised and the scale is
  // folded into q, so every score s is a log2-unit logit with
  // |s| <= scale * log2(e) * D * (1 + 2^-7) (11.7 at D = 64, 16.5 at D = 128
  // with the SDPA scale; the host takes this form only while the bound is at
  // most 64) and p = exp2(s) can neither overflow nor underflow: no running maximum,
  // no rescale.  Without a tile-wide maximum each 32-key block goes from S to
  // P to the PV products on its own, and the S products of block mb + 1 are
  // issued before the exponentials of block mb, so one wave's MFMAs overlap
  // its own softmax.
  auto s_block = [&](const uint16_t* Ks, int mb, floatx16_t (&s)[QW]) __attribute__((always_inline)) {
#pragma unroll
    for (int qb = 0; qb < QW; ++qb)
#pragma unroll
      for (int r = 0; r < 16; ++r) s[qb][r] = 0.f;
    if constexpr (kPrefillPrefetch) {
      // all NC fragments of the block in flight before the first product
      vec8 kf[NC];
#pragma unroll
      for (int c = 0; c < NC; ++c)
        kf[c] = __builtin_bit_cast(vec8, *reinterpret_cast<const uint4*>(
                                             &Ks[(32 * mb + r32) * D + 8 * ((2 * c + hh) ^ kswz)]));
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int qb = 0; qb < QW; ++qb) s[qb] = Ops::mma(kf[c], qf[qb][c], s[qb]);
    } else {
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const uint4 raw = *reinterpret_cast<const uint4*>(&Ks[(32 * mb + r32) * D + 8 * ((2 * c + hh) ^ kswz)]);
        const vec8 kf = __builtin_bit_cast(vec8, raw);
#pragma unroll
        for (int qb = 0; qb < QW; ++qb) s[qb] = Ops::mma(kf, qf[qb][c], s[qb]);
      }
    }
  };
  auto compute_tile_bounded = [&](const uint16_t* Ks, const uint16_t* Vs, int kt0) __attribute__((always_inline)) {
    floatx16_t sbuf[2][QW];
    if constexpr (kPrefillPipe) s_block(Ks, 0, sbuf[0]);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      if constexpr (!kPrefillPipe) {
        if (kt0 + 32 * mb > wave_last_key) break;
        s_block(Ks, mb, sbuf[mb & 1]);
      }
      floatx16_t(&s)[QW] = sbuf[mb & 1];
      // the next block holds a key visible to some query of the wave
      const bool more = mb + 1 < MB && kt0 + 32 * (mb + 1) <= wave_last_key;
      if constexpr (kPrefillPipe) {
        if (more) s_block(Ks, mb + 1, sbuf[(mb + 1) & 1]);
      }
      // V^T fragments of the block's PV products, read before the softmax so
      // that their LDS latency passes under the exponentials
      vec8 vfr[kPrefillPrefetch ? NB : 1][2];
      if constexpr (kPrefillPrefetch) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int c2 = 0; c2 < 2; ++c2) {
            const int c = 2 * mb + c2;
            const uint2 lo = lds_read_tr16(Vs + 16 * c * D + voff[0][nb]);
            const uint2 hi = lds_read_tr16(Vs + 16 * c * D + voff[1][nb]);
            vfr[nb][c2] = __builtin_bit_cast(vec8, make_uint4(lo.x, lo.y, hi.x, hi.y));
          }
      }
      const int kb0 = kt0 + 32 * mb;
      if (kb0 + 31 > qw + qoff || kb0 + 32 > a.Tk) {
#pragma unroll
        for (int qb = 0; qb < QW; ++qb) {
          const int lim = min(qw + 32 * qb + r32 + qoff, a.Tk - 1) - kb0 - 4 * hh;
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (8 * (r >> 2) + (r & 3) > lim) s[qb][r] = kNegInf;
        }
      }
      // The row sum adds the fp32 probabilities with plain adds: measured on
      // this chip, a v_dot2_f32_bf16 takes ~38 cycles instead of ~6 while
      // another wave's MFMAs run on the same SIMD; a v_add_f32 loses ~1.
      vec8 pf[QW][2];
#pragma unroll
      for (int qb = 0; qb < QW; ++qb) {
        float ls = l[qb];
#pragma unroll
        for (int c2 = 0; c2 < 2; ++c2) {
          uint32_t w[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float p0 = __builtin_amdgcn_exp2f(s[qb][8 * c2 + 2 * i]);
            const float p1 = __builtin_amdgcn_exp2f(s[qb][8 * c2 + 2 * i + 1]);
            w[i] = Ops::pack2(p0, p1);
            ls += p0 + p1;
          }
          pf[qb][c2] = __builtin_bit_cast(vec8, make_uint4(w[0], w[1], w[2], w[3]));
        }
        l[qb] = ls;
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
        for (int c2 = 0; c2 < 2; ++c2) {
          vec8 vf;
          if constexpr (kPrefillPrefetch) {
            vf = vfr[nb][c2];
          } else {
            const int c = 2 * mb + c2;
            const uint2 lo = lds_read_tr16(Vs + 16 * c * D + voff[0][nb]);
            const uint2 hi = lds_read_tr16(Vs + 16 * c * D + voff[1][nb]);
            vf = __builtin_bit_cast(vec8, make_uint4(lo.x, lo.y, hi.x, hi.y));
          }
#pragma unroll
          for (int qb = 0; qb < QW; ++qb) o[qb][nb] = Ops::mma(vf, pf[qb][c2], o[qb][nb]);
        }
      }
      if constexpr (kPrefillPipe) {
        if (!more) break;
      }
    }
  };

  auto compute_tile = [&](const uint16_t* Ks, const uint16_t* Vs, int kt0) __attribute__((always_inline)) {
    if constexpr (BND) {
      compute_tile_bounded(Ks, Vs, kt0);
    } else {
      // S^T = K . Q^T for the two 32-key halves of the tile
      floatx16_t s[QW][MB];
#pragma unroll
      for (int qb = 0; qb < QW; ++qb)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int r = 0; r < 16; ++r) s[qb][mb][r] = 0.f;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const uint4 raw =
              *reinterpret_cast<const uint4*>(&Ks[(32 * mb + r32) * D + 8 * ((2 * c + hh) ^ kswz)]);
          const vec8 kf = __builtin_bit_cast(vec8, raw);
#pragma unroll
          for (int qb = 0; qb < QW; ++qb) s[qb][mb] = Ops::mma(kf, qf[qb][c], s[qb][mb]);
        }
      }

      // mask (only on tiles that cross the diagonal or the end of the keys)
      const bool needs_mask = (kt0 + BN - 1 > qw + qoff) || (kt0 + BN > a.Tk);
      if (needs_mask) {
#pragma unroll
        for (int qb = 0; qb < QW; ++qb) {
          const int lim = min(qw + 32 * qb + r32 + qoff, a.Tk - 1) - kt0 - 4 * hh;
#pragma unroll
          for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int rel = 32 * mb + 8 * (r >> 2) + (r & 3);  // key - kt0 - 4hh
              if (rel > lim) s[qb][mb][r] = kNegInf;
            }
        }
      }

      vec8 pf[QW][PC];
#pragma unroll
      for (int qb = 0; qb < QW; ++qb) {
        // tile max of the raw scores (scale > 0, so it commutes with the max)
        float mt = s[qb][0][0];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int r = (mb == 0 ? 1 : 0); r < 16; ++r) mt = fmaxf(mt, s[qb][mb][r]);
        mt = half_pair_max(mt);
        // raise the exponent offset only when some row of the wave would
        // otherwise produce probabilities above 2^kLazyLog2
        const float mnew = fmaxf(m[qb], mt);
        if (__builtin_amdgcn_ballot_w64(mnew > m[qb] + a.lazy_raw) != 0) {
          // m == -inf only before the first tile; key 0 is visible to every
          // query, so mnew is finite from then on
          const float alpha = (m[qb] == kNegInf) ? 0.f : __builtin_amdgcn_exp2f((m[qb] - mnew) * a.scale_log2);
          m[qb] = mnew;
          l[qb] *= alpha;
#pragma unroll
          for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[qb][nb][r] *= alpha;
        }
        const float moff = m[qb] * a.scale_log2;
        float ls = l[qb];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
          for (int c2 = 0; c2 < 2; ++c2) {
            uint32_t w[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[qb][mb][8 * c2 + 2 * i], a.scale_log2, -moff));
              const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[qb][mb][8 * c2 + 2 * i + 1], a.scale_log2, -moff));
              w[i] = Ops::pack2(p0, p1);
              ls = Ops::add_pair(w[i], ls);
            }
            pf[qb][2 * mb + c2] = __builtin_bit_cast(vec8, make_uint4(w[0], w[1], w[2], w[3]));
          }
        }
        l[qb] = ls;
      }

      // O^T += V^T . P^T; the V^T operand comes straight from the row-major V
      // tile through the transposing LDS read (4 keys x 16 dims per 16 lanes)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
        for (int c = 0; c < PC; ++c) {
          const uint2 lo = lds_read_tr16(Vs + 16 * c * D + voff[0][nb]);
          const uint2 hi = lds_read_tr16(Vs + 16 * c * D + voff[1][nb]);
          const vec8 vf = __builtin_bit_cast(vec8, make_uint4(lo.x, lo.y, hi.x, hi.y));
#pragma unroll
          for (int qb = 0; qb < QW; ++qb) o[qb][nb] = Ops::mma(vf, pf[qb][c], o[qb][nb]);
        }
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
  // The output goes out through LDS, row-major: a lane's accumulators hold 4
  // dims of its query per register group, so stored directly every store
  // instruction would write 16 bytes into each of 32 rows (8 partial-line
  // writes per row).  Each wave owns one of the four stage arrays (every wave
  // has passed the barrier after its last tile, so none is read any more; one
  // array holds 32 rows of D elements); the 16-byte pieces of row r sit at
  // slot piece ^ (r mod D/8), which spreads the 32 rows' writes of one piece
  // over the banks.  Read back, PPQ lanes cover one whole row, so a store
  // instruction writes RPS full rows.
  constexpr int PPQ = D / 8;     // 16-byte pieces per output row
  constexpr int RPS = 64 / PPQ;  // rows per wave-wide store
  static_assert(32 * D <= C::TILE, "a stage array holds one wave's output rows");
  uint16_t* stg = wv == 0 ? ks0 : wv == 1 ? vs0 : wv == 2 ? ks1 : vs1;
  T* yb0 = static_cast<T*>(a.y) + b * a.yb + (int64_t)head * a.yh;
#pragma unroll
  for (int qb = 0; qb < QW; ++qb) {
    // rows past Tq carry finite values and are not stored
    const float inv = __builtin_amdgcn_rcpf(half_pair_sum(l[qb]));
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const uint32_t w0 = pack_pair<T>(o[qb][nb][4 * g] * inv, o[qb][nb][4 * g + 1] * inv);
        const uint32_t w1 = pack_pair<T>(o[qb][nb][4 * g + 2] * inv, o[qb][nb][4 * g + 3] * inv);
        const int slot = (4 * nb + g) ^ (r32 & (PPQ - 1));
        *reinterpret_cast<uint2*>(stg + r32 * D + 8 * slot + 4 * hh) = make_uint2(w0, w1);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int piece = lane % PPQ;
#pragma unroll
    for (int p = 0; p < 32 / RPS; ++p) {
      const int row = p * RPS + lane / PPQ;
      const u32x4_t val = *reinterpret_cast<const u32x4_t*>(stg + row * D + 8 * (piece ^ (row & (PPQ - 1))));
      const int qi = qw + 32 * qb + row;
      if (qi < a.Tq) *reinterpret_cast<u32x4_t*>(yb0 + (int64_t)qi * a.yt + 8 * piece) = val;
    }
    if (qb + 1 < QW) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  }
}


namespace {

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
// every (b, t, h) row start 16-byte aligned
bool strides16b(const dg_stride3* s, int64_t es) {
  const int64_t n = 16 / es;
  return s->b % n == 0 && s->t % n == 0 && s->h % n == 0;
}

// query blocks of 32 per wave (64 per wave spills at D = 64, and halves the
// resident workgroups at D = 128)
template <int D>
constexpr int qw_for() {
  return 1;
}

template <typename T, int D, bool ROPE = false, typename FT = T, bool BND = false>
int launch_prefill(PrefillArgs a, hipStream_t s) {
  constexpr int QW = qw_for<D>();
  constexpr int BM = PrefillCfg<T, D, QW>::BM;
  a.nqb = (a.Tq + BM - 1) / BM;
  const int nwin = (a.nbh + a.win - 1) / a.win;
  DG_REQUIRE(a.nqb <= 65535 && nwin <= 65535, DG_EINVAL, "prefill: %d query blocks, %d windows, at most 65535 each",
             a.nqb, nwin);
  hipLaunchKernelGGL((prefill_mfma_kernel<T, D, QW, ROPE, FT, BND>), dim3((unsigned)a.win, (unsigned)a.nqb, (unsigned)nwin),
                     dim3(PrefillCfg<T, D, QW>::NT), 0, s, a);
  return check_launch("prefill_mfma_kernel");
}

}  // namespace

bool mfma_prefill_applicable(int B, int H, int Tq, int Tk, int D, int dtype, const void* q,
                             const dg_stride3* q_st, const void* k, const dg_stride3* k_st,
                             const void* v, const dg_stride3* v_st, const void* y,
                             const dg_stride3* y_st, float scale) {
  if (!(scale > 0.f)) return false;  // the tile max of raw scores needs a positive scale
  // bf16 / fp16 here, fp32 in dg_attn_mfma_f32.hip
  if (dtype != DG_BF16 && dtype != DG_F16 && dtype != DG_F32) return false;
  if (D != 64 && D != 128) return false;
  if (Tq < 16) return false;  // decode and tiny chunks: vector kernel
  // grid (window, query blocks, windows): at most 65535 query blocks of 128
  // and 65535 windows (of kPrefillWindowLong pairs at the least)
  const int64_t nbh = (int64_t)B * H;
  if (nbh <= 0 || (Tq + 127) / 128 > 65535 || (nbh + kPrefillWindowLong - 1) / kPrefillWindowLong > 65535)
    return false;
  // per-head byte offsets (buffer ranges) are 32-bit signed inside the kernels
  const int64_t es = dtype == DG_F32 ? 4 : 2;
  const int64_t span = (int64_t)Tk * (k_st->t > v_st->t ? k_st->t : v_st->t);
  if (span * es >= (int64_t)1 << 31 || k_st->t < 0 || v_st->t < 0) return false;
  return aligned16(q) && aligned16(k) && aligned16(v) && aligned16(y) && strides16b(q_st, es) &&
         strides16b(k_st, es) && strides16b(v_st, es) && strides16b(y_st, es);
}

namespace {
PrefillArgs prefill_args(int B, int H, int Tq, int Tk, int D, const void* q, const dg_stride3* q_st, const void* k,
                         const dg_stride3* k_st, const void* v, const dg_stride3* v_st, void* y,
                         const dg_stride3* y_st, float scale) {
  PrefillArgs a{};
  a.q = q; a.k = k; a.v = v; a.y = y;
  a.qb = q_st->b; a.qt = q_st->t; a.qh = q_st->h;
  a.kb = k_st->b; a.kt = k_st->t; a.kh = k_st->h;
  a.vb = v_st->b; a.vt = v_st->t; a.vh = v_st->h;
  a.yb = y_st->b; a.yt = y_st->t; a.yh = y_st->h;
  a.H = H; a.Tq = Tq; a.Tk = Tk;
  a.q_offset = Tk - Tq;
  a.nbh = B * H;
  // (b, h) pairs per scheduling window.  All query blocks of a pair share one
  // XCD, so a window keeps win/8 heads' K and V in each XCD's 4 MB L2.  32
  // for long rows (a head's K/V of 1 MB or more in bf16: at configs[4] the
  // FETCH_SIZE traffic drops from 4.35 to 2.68 GB per launch and the time by
  // 1 %) and for large batches (B*H >= 2048: +1 to +2 % at configs[2] /
  // configs[3]); 64 otherwise (B*H = 256 and D = 64 at T = 3584 measured 0.5
  // to 2.5 % slower with 32)
  const int win = (B * H >= 2048 || (int64_t)Tk * D >= 262144) ? kPrefillWindowLong : kPrefillWindow;
  a.win = B * H < win ? B * H : win;
  a.scale_log2 = scale * 1.44269504088896340736f;
  a.lazy_raw = kLazyLog2 / a.scale_log2;
  return a;
}
}  // namespace

int mfma_prefill(int B, int H, int Tq, int Tk, int D, int dtype, const void* q,
                 const dg_stride3* q_st, const void* k, const dg_stride3* k_st, const void* v,
                 const dg_stride3* v_st, void* y, const dg_stride3* y_st, float scale,
                 hipStream_t s) {
  const PrefillArgs a = prefill_args(B, H, Tq, Tk, D, q, q_st, k, k_st, v, v_st, y, y_st, scale);
  if (dtype == DG_F32) return launch_prefill_f32(a, D, s);
  if (dtype == DG_BF16) return D == 64 ? launch_prefill<bf16_t, 64>(a, s) : launch_prefill<bf16_t, 128>(a, s);
  return D == 64 ? launch_prefill<f16_t, 64>(a, s) : launch_prefill<f16_t, 128>(a, s);
}

// The fused form takes what the plain MFMA prefill takes, with (cos, sin) rows
// that are 16-byte aligned, in the data's dtype or fp32.
bool mfma_prefill_rope_applicable(int B, int H, int Tq, int Tk, int D, int dtype, const void* q,
                                  const dg_stride3* q_st, const void* freqs, const dg_stride3* f_st,
                                  int fdtype, const void* k, const dg_stride3* k_st, const void* v,
                                  const dg_stride3* v_st, const void* y, const dg_stride3* y_st,
                                  float scale) {
  if (!mfma_prefill_applicable(B, H, Tq, Tk, D, dtype, q, q_st, k, k_st, v, v_st, y, y_st, scale)) return false;
  if (fdtype != dtype && fdtype != DG_F32) return false;
  const int64_t fes = fdtype == DG_F32 ? 4 : 2;
  if (!freqs || !aligned16(freqs)) return false;
  for (int64_t st : {f_st->b, f_st->t, f_st->h})
    if (st < 0 || (st * fes) % 16 != 0) return false;
  return true;
}

namespace {
template <typename T, bool BND>
int launch_rope_prefill(int D, bool f32, const PrefillArgs& a, hipStream_t s) {
  if (D == 64) return f32 ? launch_prefill<T, 64, true, float, BND>(a, s) : launch_prefill<T, 64, true, T, BND>(a, s);
  return f32 ? launch_prefill<T, 128, true, float, BND>(a, s) : launch_prefill<T, 128, true, T, BND>(a, s);
}
}  // namespace

int mfma_prefill_rope(int B, int H, int Tq, int Tk, int D, int dtype, const void* q, const dg_stride3* q_st,
                      const void* freqs, const dg_stride3* f_st, int fdtype, int qknorm, int keys_normed,
                      const void* k, const dg_stride3* k_st, const void* v, const dg_stride3* v_st, void* y,
                      const dg_stride3* y_st, float scale, hipStream_t s) {
  PrefillArgs a = prefill_args(B, H, Tq, Tk, D, q, q_st, k, k_st, v, v_st, y, y_st, scale);
  a.freqs = freqs;
  a.fb = f_st->b; a.ft = f_st->t; a.fh = f_st->h;
  a.qknorm = qknorm;
  const bool f32 = fdtype == DG_F32;
  // normalised queries (here) and keys (the caller's guarantee): bounded
  // scores, |s| <= scale * log2(e) * D * (1 + 2^-7) in log2 units.  The form
  // without a running maximum is taken while that bound is at most 64, so
  // that exp2(s) of every score and the sum of up to 2^30 of them stay inside
  // fp32's normal range (the SDPA scale 1/sqrt(D) gives 11.7 at D = 64, 16.5
  // at D = 128; a scale above 0.68 / 0.34 there runs the running-maximum
  // form).  bf16 only: p reaches 2^16.5 at D = 128 with the SDPA scale, beyond
  // fp16's range, while bf16 has fp32's exponent range
  if (dtype == DG_F32) return launch_prefill_f32(a, D, s);  // running maximum; fp32 table
  const bool small_scores = (double)scale * 1.4426950408889634 * D * (1.0 + 1.0 / 128.0) <= 64.0;
  const bool bounded = qknorm && keys_normed && dtype == DG_BF16 && small_scores;
  if (dtype == DG_BF16)
    return bounded ? launch_rope_prefill<bf16_t, true>(D, f32, a, s) : launch_rope_prefill<bf16_t, false>(D, f32, a, s);
  return launch_rope_prefill<f16_t, false>(D, f32, a, s);
}

}  // namespace dg
