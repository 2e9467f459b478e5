// Decode attention (Tq = 1, mha.py:65-68) over a batch whose rows come in
// groups sharing a cache prefix, with the prefix on the matrix cores.
//
// After KVCache.prefill from a batch-1 cache (kv_cache.py:77-79) the `group`
// consecutive rows of each group share the keys and values at positions
// 0 .. len-1 (dg_prefix: stored once per group, or in each group's first row
// of a broadcast cache).  For one decode step the scores of a group's rows
// against that prefix form a real matrix product, S = Q_rows K_prefix^T, and
// so does P V_prefix: this kernel runs both on MFMA, reading the prefix
// (L2-resident, shared by the tiles of a group) once per 16-row tile.  The
// rows' own keys, positions len .. Tk-1, differ from row to row and go through
// the vector ALUs.  The two parts run at the same time on two wavefronts and
// merge at the end.
//
// Work unit = one block of two wavefronts = (group, tile of 16 rows of the
// group, head).  Wave 0 takes the prefix, wave 1 the own keys.
//
// Prefix (wave 0, MFMA: v_mfma_f32_16x16x4_f32 or
// v_mfma_f32_16x16x16_{bf16,f16}); lane l: c = l & 15 is the tile row,
// g = l >> 4 one of four lanes per row:
//   S^T (16 keys x 16 rows) = K_tile Q^T: lane (c, g) feeds key row c and
//   query row c of the tile, each with the D/4 contiguous elements
//   g*D/4 .. g*D/4 + D/4 - 1 (a fixed permutation of the contraction index,
//   the same for both operands, so the dot products are unchanged); it gets
//   back the scores of row c against keys 4g .. 4g+3 of the tile.  The
//   online softmax runs over chunks of 64 keys (max over the chunk, lazy
//   rescale as in the vector kernel), then
//   O^T (D x 16 rows) += V^T P^T: lane (c, g) feeds V[4g+s][16t+c] and its
//   own probability of key 4g+s, and holds O^T for row c, columns
//   16t + 4g .. 16t + 4g + 3.  Each 64-key chunk of V goes through LDS, one
//   row per lane with wide loads: fp32 writes it transposed (column-wise,
//   padded rows) and takes four 16x16x4 products per key tile from one
//   ds_read_b128; bf16 / fp16 write it row-major, read it back transposed
//   (ds_read_b64_tr_b16) and take two 16x16x16 products, P split as hi + lo
//   in T.
// Own keys (wave 1, VALU): a quad of lanes holds one tile row, 16 bytes of a
//   cache row per lane (OwnCfg), so every quad reads whole cache rows; the
//   lanes of a key row add their partial dot products with DPP, and each
//   lane accumulates p * v for its slice of the row.  The wave streams its
//   keys from the start of the launch, two register sets in flight, while
//   wave 0's prefix phase (a few dependent cache round trips) runs.  Keys
//   are loaded through buffer resources with one 32-bit offset for K and V;
//   a key past the last cached position reads zeros from past the range.
// Merge: wave 1 writes each row's softmax offset, sum and weighted values to
//   LDS; after one barrier wave 0 rescales both parts to the larger offset,
//   adds them and stores its O^T columns.
//
// Fused decode step (FUSED = true; mha.py:44-68 for one new token): the same
// kernel first applies RoPE and QK-norm to the step's q and k projections
// (the arithmetic of rope_qknorm_kernel, shared through dg_rope_math.h),
// appends k and v to the cache at position pos (kv_cache.py:108-109), and
// attends over positions 0 .. pos, taking the new key and value from
// registers: one launch per layer-step instead of two.
#include "dg_rope_math.h"

namespace dg {

#ifdef DG_TIMELINE
// Measurement build only (build.py --timeline, read by timeline.py): every
// wave of attn_shared_kernel stamps the shader clock at its phase boundaries
// and writes 8 values per (block, wave) to the buffer set by
// dg_timeline_set -- 6 stamps, the end, and the HW_ID register.
__device__ unsigned long long* g_timeline;
__device__ __forceinline__ unsigned long long stamp_now() {
  unsigned long long t;
  asm volatile("s_memtime %0\n s_waitcnt lgkmcnt(0)" : "=s"(t) :: "memory");
  return t;
}
#define DG_STAMP(i) (tl_[i] = stamp_now())
#define DG_TIMELINE_FLUSH()                                                                               \
  do {                                                                                                    \
    const unsigned long long te_ = stamp_now();                                                           \
    if (g_timeline && lane < 8) {                                                                         \
      const unsigned long long v_ = lane == 0 ? tl_[0] : lane == 1 ? tl_[1] : lane == 2 ? tl_[2]          \
                                  : lane == 3 ? tl_[3] : lane == 4 ? tl_[4] : lane == 5 ? tl_[5]          \
                                  : lane == 6 ? te_ : (unsigned long long)__builtin_amdgcn_s_getreg((31 << 11) | 4); \
      g_timeline[((size_t)blockIdx.x * 2 + role) * 8 + lane] = v_;                                        \
    }                                                                                                     \
  } while (0)
#else
#define DG_STAMP(i) ((void)0)
#define DG_TIMELINE_FLUSH() ((void)0)
#endif

struct SharedArgs {
  const void* q;  // attention q (unfused), or the step's q projection (fused)
  const void* k;  // cache pages (keys at position t: k + b*kb + t*kt + h*kh)
  const void* v;
  void* y;
  int64_t qb, qh;
  int64_t kb, kt, kh;
  int64_t vb, vt, vh;
  int64_t yb, yh;
  int64_t units;  // ceil(B / group) * tiles * H
  int B, H, D, Tk, tiles;
  PrefixRef pre;  // the groups' prefix pages (pre.group rows per group)
  float scale_log2;  // scale * log2(e)
  float lazy_raw;    // kSharedLazyLog2 / scale_log2
  // graph-replayable form: keys are positions 0 .. *pos_dev, at most Tk
  const int* pos_dev;
  // fused step: projections of the new token (B,1,H,D) and the RoPE table at
  // position 0 with fpos elements per position; the new token goes to
  // position pos (Tk = pos + 1), or *pos_dev when set; nothing is computed or
  // written when that position is outside [0, max_pos)
  const void* kp;
  const void* vp;
  int64_t kpb, kph, vpb, vph;
  const void* freqs;
  int64_t fpos;
  int pos, max_pos, qknorm;
};

constexpr float kSharedLazyLog2 = 8.0f;
constexpr int kSharedMinGroup = 16;

// Max / sum over the four lanes c, c+16, c+32, c+48 of a tile row (identical
// bits in all four).
__device__ __forceinline__ float row_max4(float x) {
  float a, b;
  pair16(x, a, b);
  x = fmaxf(a, b);
  pair32(x, a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float row_sum4(float x) {
  float a, b;
  pair16(x, a, b);
  x = a + b;
  pair32(x, a, b);
  return a + b;
}

// Own-key lane layout: a quad of lanes holds one tile row, LPK lanes per key
// row with EPL contiguous elements each (16 bytes, 32 for fp32 at D = 32), so
// every quad reads whole cache rows and one load instruction covers 16 rows x
// KPQ keys: few L1 accesses per byte, like the vector kernel's layout.
template <typename T, int D>
struct OwnCfg {
  static constexpr int ROWB = D * (int)sizeof(T);
  static constexpr int LPK = ROWB >= 64 ? 4 : 2;  // lanes per key row
  static constexpr int KPQ = 4 / LPK;             // keys per quad and instruction
  static constexpr int EPL = D / LPK;             // elements per lane
  static constexpr int WORDS = EPL * (int)sizeof(T) / 4;
  static constexpr int UO = 32 / WORDS;           // key instructions per register set (K+V: 64 VGPRs)
  static constexpr int STEP = UO * KPQ;           // keys per row and register set
};

template <int N>
struct IntConst {
  static constexpr int value = N;
};

// Lane `src` of the wave's value x (ds_bpermute: a gather over the wave).
__device__ __forceinline__ float lane_get(float x, int src) {
  return __int_as_float(__builtin_amdgcn_ds_bpermute(src << 2, __float_as_int(x)));
}
__device__ __forceinline__ uint32_t lane_get_u(uint32_t x, int src) {
  return (uint32_t)__builtin_amdgcn_ds_bpermute(src << 2, (int)x);
}


// O^T += V^T P^T over one 16-key tile on the 16-bit matrix cores
// (v_mfma_f32_16x16x16_{bf16,f16}): lane (c, g) feeds va[t] = V[4g + i][16t + c]
// and P[c][4g + i], i = 0..3 -- the four scores it holds after the S^T product.
// P is split as hi + lo, both rounded to T (lo = the rounding error of hi), so
// the two products carry about twice T's mantissa of each probability; the
// values are exact in T and every product is accumulated in fp32.
template <typename T, int DT>
__device__ __forceinline__ void pv_mfma16(const uint32_t (&va)[DT][2], const f32x4_t& p, f32x4_t (&oacc)[DT]) {
  uint32_t hi[2], lo[2];
#pragma unroll
  for (int w = 0; w < 2; ++w) {
    if constexpr (__is_same(T, bf16_t)) {
      // pairs through v_cvt_pk_bf16_f32 (round to nearest even); p - hi is
      // exact in fp32
      typedef float f2_t __attribute__((ext_vector_type(2)));
      typedef __bf16 b2_t __attribute__((ext_vector_type(2)));
      const uint32_t h = __builtin_bit_cast(uint32_t, __builtin_convertvector(f2_t{p[2 * w], p[2 * w + 1]}, b2_t));
      const f2_t r{p[2 * w] - __uint_as_float(h << 16), p[2 * w + 1] - __uint_as_float(h & 0xffff0000u)};
      hi[w] = h;
      lo[w] = __builtin_bit_cast(uint32_t, __builtin_convertvector(r, b2_t));
    } else {
      const T h0 = from_f32<T>(p[2 * w]), h1 = from_f32<T>(p[2 * w + 1]);
      const T l0 = from_f32<T>(p[2 * w] - to_f32(h0)), l1 = from_f32<T>(p[2 * w + 1] - to_f32(h1));
      hi[w] = (uint32_t)h0.bits | ((uint32_t)h1.bits << 16);
      lo[w] = (uint32_t)l0.bits | ((uint32_t)l1.bits << 16);
    }
  }
#pragma unroll
  for (int t = 0; t < DT; ++t) {
    if constexpr (__is_same(T, bf16_t)) {
      oacc[t] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4_t, va[t]),
                                                          __builtin_bit_cast(i16x4_t, hi), oacc[t], 0, 0, 0);
      oacc[t] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4_t, va[t]),
                                                          __builtin_bit_cast(i16x4_t, lo), oacc[t], 0, 0, 0);
    } else {
      oacc[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4_t, va[t]),
                                                      __builtin_bit_cast(f16x4_t, hi), oacc[t], 0, 0, 0);
      oacc[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4_t, va[t]),
                                                      __builtin_bit_cast(f16x4_t, lo), oacc[t], 0, 0, 0);
    }
  }
}

// Two wavefronts per work unit, running at the same time: wave 0 takes the
// prefix on the matrix cores, wave 1 streams the rows' own keys on the vector
// ALUs from the start of the launch, so the prefix phase (latency-bound: a few
// dependent cache round trips) overlaps the HBM-bound own-key stream instead of
// preceding it.  Wave 1 hands its partial (offset, sum and weighted values of
// each row) to wave 0 through LDS; wave 0 merges and stores.  At most 128
// VGPRs (four waves per SIMD), so that decode grids of a few thousand waves
// are resident at once.
template <typename T, int D, bool FUSED, typename FT>
__global__ __launch_bounds__(128, 4) void attn_shared_kernel(const SharedArgs a) {
  constexpr int DQ = D / 4;   // contraction elements per lane and key tile
  constexpr int DT = D / 16;  // 16-column tiles of the output
  constexpr int NT = 4;       // prefix key tiles (16 keys) per softmax chunk
  using O = OwnCfg<T, D>;
  constexpr int LPK = O::LPK, KPQ = O::KPQ, EPL = O::EPL;
  using Op = RowRegs<T, DQ>;
  using Slice = RowRegs<T, EPL>;
  constexpr int UO = 16 / Slice::WORDS;  // key slots per register set (K + V: 32 VGPRs)
  constexpr int STEP = UO * KPQ;         // keys per row and register set
  constexpr int NSW = 2;                 // register sets of own keys in flight (64 VGPRs)
  constexpr int RS = D + 4;              // floats per row of a hand-over buffer (16-byte rows)
  constexpr int NCB = D == 16 ? 2 : 1;   // prefix chunk buffers
  using VRow = RowRegs<T, D>;            // a whole value row
  // Prefix values go through LDS, 64 keys per buffer.  16-bit types: row-major
  // (64 rows of D), read transposed by ds_read_b64_tr_b16.  fp32: transposed
  // on the write, D rows of 64 keys padded to VT_STRIDE floats, so that one
  // ds_read_b128 gives a lane the 4 consecutive keys of one column that its
  // four 16x16x4 products take, with no bank conflicts (16 lanes of one read
  // sit 4 banks apart).
  constexpr int VT_STRIDE = 68;
  constexpr int VBUF_BYTES = sizeof(T) == 2 ? 64 * D * 2 : D * VT_STRIDE * 4;
  __shared__ __attribute__((aligned(16))) float part[16 * RS];  // wave 1's partial
  __shared__ __attribute__((aligned(16))) unsigned char vst[NCB * VBUF_BYTES];

  const int lane = threadIdx.x & 63;
  const int role = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // 0: prefix, 1: own keys
#ifdef DG_TIMELINE
  unsigned long long tl_[6] = {stamp_now(), 0, 0, 0, 0, 0};
#endif
  // the tiles and heads of one group run on one XCD, whose L2 keeps the prefix
  int unit = blockIdx.x;
  if ((gridDim.x & 7) == 0) unit = (blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3);
  if (unit >= a.units) return;  // both waves of the block; no barrier reached
  const int h = unit % a.H;
  const int rest = unit / a.H;
  const int tile = rest % a.tiles;
  const int grp = rest / a.tiles;

  const int64_t b0 = (int64_t)grp * a.pre.group;  // the group's first row
  // tile row r of the unit -> batch row (rows past the group compute on b0
  // and store nothing)
  auto row_of = [&](int r, bool& ok) __attribute__((always_inline)) {
    const int rin = tile * 16 + r;
    ok = rin < a.pre.group && b0 + rin < a.B;
    return ok ? b0 + rin : b0;
  };

  // keys 0 .. Tk-1; the fused step appends key Tk-1 = pos and takes it from
  // registers, so the cache is read for keys below Tc only
  int Tc;
  if constexpr (FUSED) {
    const int pos = a.pos_dev != nullptr ? *a.pos_dev : a.pos;
    // uniform over the grid; the append goes to the rows' own pages
    if (pos < a.pre.own_start || pos >= a.max_pos) return;
    Tc = pos;
  } else {
    int Tk = a.Tk;
    if (a.pos_dev != nullptr) Tk = min(*a.pos_dev + 1, a.Tk);
    Tc = Tk;
  }
  const int P = min(a.pre.len, Tc);
  const float cl = a.scale_log2;
  const int kt = (int)a.kt, vt = (int)a.vt;  // host: Tk * stride < 2^31
  const T* kbase = static_cast<const T*>(a.k) + (int64_t)h * a.kh;
  const T* vbase = static_cast<const T*>(a.v) + (int64_t)h * a.vh;
  const T* qbase = static_cast<const T*>(a.q) + (int64_t)h * a.qh;

  // --- quad layout (own keys): a quad of lanes holds one tile row ------------
  const int orow = lane >> 2, kk = (lane & 3) / LPK, piece = (lane & 3) % LPK;
  bool ovalid;
  const int64_t bo = row_of(orow, ovalid);
  // RoPE + QK-norm of the new token's q (mha.py:44-48), rounded to T as the
  // standalone kernel stores it; both waves compute it (same bits)
  auto rotate_q = [&](float (&xq)[EPL], const float (&cs)[EPL], Slice& qs) __attribute__((always_inline)) {
    rope_rotate<T, EPL>(xq, cs);
    if (a.qknorm) qk_rms_norm<EPL, LPK, true>(xq, D);
    pack_row<T, EPL>(qs, xq);
  };
  const FT* fbase = FUSED ? static_cast<const FT*>(a.freqs) + (int64_t)Tc * a.fpos + piece * EPL : nullptr;

  // --- own keys P .. Tc-1 (wave 1), in sets of STEP keys per row: set i
  // holds keys P + i*STEP ...  Loads go through buffer resources on the
  // head's K and V pages with one 32-bit byte offset for both (the host takes
  // this kernel only when the pages share their row and position strides and
  // every offset is below 2^31): key j of the lane's row at rowoff + j * ktb.
  // A key lane at or past Tc gets an offset past the resource's range, which
  // reads zeros without touching memory, so every set issues the same loads
  // on every path (the compiler's wait counts stay exact) and no masked key
  // reads uninitialised memory.
  constexpr uint32_t kOobOffset = 0x80000000u;  // past the 2^31 - 1 byte range, no wrap-around
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(kbase), (short)0, 0x7fffffff, kBufferWord3);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(vbase), (short)0, 0x7fffffff, kBufferWord3);
  const uint32_t ktb = (uint32_t)kt * (uint32_t)sizeof(T);
  // rows past the group start past the range too: their keys read zeros
  // without touching memory (rowoff + j * ktb stays in [2^31, 2^32))
  const uint32_t rowoff = ovalid ? (uint32_t)(bo * a.kb + piece * EPL) * (uint32_t)sizeof(T) : kOobOffset;
  auto load_kv = [&](Slice& kr, Slice& vr, int jb) __attribute__((always_inline)) {
    const int j = jb + kk;  // jb wave-uniform
    const uint32_t off = j < Tc ? rowoff + (uint32_t)j * ktb : kOobOffset;
    static_assert(Slice::WORDS % 4 == 0, "own-key slices are whole 16-byte pieces");
#pragma unroll
    for (int c4 = 0; c4 < Slice::WORDS / 4; ++c4) {
      const u32x4_t x = __builtin_amdgcn_raw_buffer_load_b128(krs, (int)(off + 16 * c4), 0, 0);
      const u32x4_t y = __builtin_amdgcn_raw_buffer_load_b128(vrs, (int)(off + 16 * c4), 0, 0);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        kr.w[4 * c4 + w] = x[w];
        vr.w[4 * c4 + w] = y[w];
      }
    }
  };
  Slice kr[NSW][UO], vr[NSW][UO];
  auto load_set = [&](int k, int i) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < UO; ++u) load_kv(kr[k][u], vr[k][u], P + i * STEP + KPQ * u);
  };

  float mo = kNegInf, lo = 0.f;
  float acc[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) acc[e] = 0.f;
  // raise the quad's offset to mt when a score exceeds it by more than the
  // lazy margin (one offset per quad row)
  auto raise_offset = [&](float mt) __attribute__((always_inline)) {
    if constexpr (KPQ == 2) mt = fmaxf(mt, dpp<kDppQuadXor2>(mt));
    if (mt > mo + a.lazy_raw) {
      const float alpha = (mo == kNegInf) ? 0.f : __builtin_amdgcn_exp2f((mo - mt) * cl);
      mo = mt;
      lo *= alpha;
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[e] *= alpha;
    }
  };
  auto add_key = [&](float score, const Slice& vs, float moff) __attribute__((always_inline)) {
    const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(score, cl, -moff));
    lo += p;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[e] = __builtin_fmaf(p, elem<T, EPL>(vs, e), acc[e]);
  };
  // one register set: a key lane at or past Tc (zeros in its registers)
  // scores -inf and adds p = 0; a set that starts at or past Tc is skipped
  auto process = [&](const Slice (&ks)[UO], const Slice (&vs)[UO], int j0, const Slice& qs)
                     __attribute__((always_inline)) {
    float sv[UO];
    float mt = kNegInf;
#pragma unroll
    for (int u = 0; u < UO; ++u) {
      const float dot = group_sum_dpp<LPK>(slice_dot<T, EPL>(qs, ks[u]));
      sv[u] = (j0 + KPQ * u + kk < Tc) ? dot : kNegInf;
      mt = fmaxf(mt, sv[u]);
    }
    raise_offset(mt);
    const float moff = mo * cl;
#pragma unroll
    for (int u = 0; u < UO; ++u) add_key(sv[u], vs[u], moff);
  };
  // Sets 0 and 1 are in flight on entry (nsets >= 2).  Rounds that refill
  // both sets run while sets i + 2 and i + 3 exist; the last two or three
  // sets are then consumed with at most one refill.  No load is issued for
  // a set past the last key: such loads touch no memory but still take the
  // CU's address-unit issue slots, which every wave of the CU shares.  Each
  // path issues a fixed number of loads, so the compiler's wait counts stay
  // exact (a data-dependent number would make it wait for every load).
  static_assert(NSW == 2, "the own-key stream is written for two register sets");
  auto own_stream = [&](const Slice& qs, int nsets) __attribute__((always_inline)) {
    int i = 0;
    for (; i + 2 * NSW <= nsets; i += NSW) {
      process(kr[0], vr[0], P + i * STEP, qs);
      load_set(0, i + 2);
      process(kr[1], vr[1], P + (i + 1) * STEP, qs);
      load_set(1, i + 3);
    }
    process(kr[0], vr[0], P + i * STEP, qs);
    if (nsets - i == 3) {
      load_set(0, i + 2);
      process(kr[1], vr[1], P + (i + 1) * STEP, qs);
      process(kr[0], vr[0], P + (i + 2) * STEP, qs);
    } else {
      process(kr[1], vr[1], P + (i + 1) * STEP, qs);
    }
  };
  // wave 1's partial to LDS: row orow's offset, sum and weighted values
  auto hand_over = [&]() __attribute__((always_inline)) {
    if constexpr (KPQ == 2) {  // the two keys of a quad: same offset, partials add
      lo += dpp<kDppQuadXor2>(lo);
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[e] += dpp<kDppQuadXor2>(acc[e]);
    }
    if (kk == 0) {
      float* pr = part + orow * RS;
#pragma unroll
      for (int e4 = 0; e4 < EPL / 4; ++e4)
        *reinterpret_cast<f32x4_t*>(pr + piece * EPL + 4 * e4) =
            f32x4_t{acc[4 * e4], acc[4 * e4 + 1], acc[4 * e4 + 2], acc[4 * e4 + 3]};
      if (piece == 0) {
        pr[D] = mo;
        pr[D + 1] = lo;
      }
    }
  };

  // wave 0's prefix state, merged after the hand-over
  const int c = lane & 15, g = lane >> 4;  // MFMA layout: tile row c, lane group g
  bool cvalid;
  const int64_t bc = row_of(c, cvalid);
  float m = kNegInf, lp = 0.f;
  f32x4_t oacc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) oacc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // Each wave issues its first cache loads right behind its query loads (wave
  // 1 with a scheduling barrier between them: waits count loads in the order
  // they were issued), so that waiting for the query does not wait for them.
  if (role == 0) {
    // --- prefix on MFMA: lane (c, g) -------------------------------------------
    const T* kpre = static_cast<const T*>(a.pre.k) + grp * a.pre.kb + (int64_t)h * a.pre.kh;
    const T* vpre = static_cast<const T*>(a.pre.v) + grp * a.pre.vb + (int64_t)h * a.pre.vh;
    Op kopA[NT], kopB[NT];  // B: the second chunk buffer (D = 16 only)
    VRow vrA, vrB;
    // Values of one 64-key chunk: lane l loads value row c0 + l (whole rows,
    // wide loads) and later writes it to an LDS buffer.  Rows past the prefix
    // re-read its last key (masked, probability 0).
    auto load_values = [&](int c0, int last, VRow& vrow) __attribute__((always_inline)) {
      load_row<T, D>(vrow, vpre + min(c0 + lane, last) * vt);
    };
    // the first 128 prefix keys (64 at D = 32)
    auto first_chunks = [&]() __attribute__((always_inline)) {
      const int last = max(P - 1, 0);
#pragma unroll
      for (int half = 0; half < NCB; ++half) {
#pragma unroll
        for (int j = 0; j < NT; ++j) {
          Op& kop = half ? kopB[j] : kopA[j];
          load_row<T, DQ>(kop, kpre + min(16 * NT * half + 16 * j + c, last) * kt + g * DQ);
        }
        load_values(16 * NT * half, last, half ? vrB : vrA);
      }
    };
    Op qop;  // q row c, elements g*DQ .. g*DQ + DQ - 1
    if constexpr (FUSED) {
      float xq[EPL], cs[EPL];
      load_vec<T, EPL>(qbase + bo * a.qb + piece * EPL, xq);
      load_vec<FT, EPL>(fbase, cs);
      first_chunks();
      DG_STAMP(1);  // wave 0: q and the first prefix chunks issued
      Slice qs;
      rotate_q(xq, cs, qs);
      // gathered from the quad layout: own lane 4c + (g*DQ)/EPL (key lane 0)
      // holds them at word (g*DQ % EPL) * sizeof(T) / 4 of its slice
      constexpr int OPW = Op::WORDS, SW = Slice::WORDS;
      const int src = 4 * c + (g * DQ) / EPL;
      const int wo = ((g * DQ) % EPL) * (int)sizeof(T) / 4;
#pragma unroll
      for (int w = 0; w < OPW; ++w) {
        uint32_t x = 0;
#pragma unroll
        for (int cand = 0; cand + OPW <= SW; cand += OPW) {
          const uint32_t y = lane_get_u(qs.w[cand + w], src);
          x = (wo == cand) ? y : x;
        }
        qop.w[w] = x;
      }
    } else {
      load_row<T, DQ>(qop, qbase + bc * a.qb + g * DQ);
      first_chunks();
    }
    auto load_chunk = [&](int c0, Op (&kop)[NT], VRow& vrow) __attribute__((always_inline)) {
#pragma unroll
      for (int j = 0; j < NT; ++j)
        load_row<T, DQ>(kop[j], kpre + min(c0 + 16 * j + c, P - 1) * kt + g * DQ);
      load_values(c0, P - 1, vrow);
    };
    // the chunk's value rows into LDS buffer buf: 16-bit types row l from
    // lane l; fp32 column d of key l at d * VT_STRIDE + l
    auto stage_values = [&](const VRow& vrow, int buf) __attribute__((always_inline)) {
      unsigned char* vb = vst + buf * VBUF_BYTES;
      if constexpr (sizeof(T) == 2) {
        u32x4_t* dst = reinterpret_cast<u32x4_t*>(vb) + lane * (D / 8);
#pragma unroll
        for (int c4 = 0; c4 < VRow::WORDS / 4; ++c4)
          dst[c4] = u32x4_t{vrow.w[4 * c4], vrow.w[4 * c4 + 1], vrow.w[4 * c4 + 2], vrow.w[4 * c4 + 3]};
      } else {
        float* dst = reinterpret_cast<float*>(vb) + lane;
#pragma unroll
        for (int d = 0; d < D; ++d) dst[d * VT_STRIDE] = __uint_as_float(vrow.w[d]);
      }
    };
    auto prefix_chunk = [&](int c0, const Op (&kop)[NT], int buf) __attribute__((always_inline)) {
      f32x4_t sc[NT];
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        sc[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        if (c0 + 16 * j >= P) continue;  // wave-uniform
        sc[j] = qk_mfma<T, DQ>(kop[j], qop, sc[j]);
      }
      // keys past the prefix: a tile wholly past it at once, element by
      // element only in the tile that holds key P - 1 (wave-uniform tests)
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const int k0 = c0 + 16 * j;
        if (k0 + 16 <= P) continue;
        if (k0 >= P) {
          sc[j] = f32x4_t{kNegInf, kNegInf, kNegInf, kNegInf};
          continue;
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) sc[j][r] = (k0 + 4 * g + r < P) ? sc[j][r] : kNegInf;
      }
      float mx = kNegInf;
#pragma unroll
      for (int j = 0; j < NT; ++j) {
#pragma unroll
        for (int r = 0; r < 4; ++r) mx = fmaxf(mx, sc[j][r]);
      }
      mx = row_max4(mx);  // every chunk holds a prefix key: finite
      if (mx > m + a.lazy_raw) {
        const float alpha = (m == kNegInf) ? 0.f : __builtin_amdgcn_exp2f((m - mx) * cl);
        m = mx;
        lp *= alpha;
#pragma unroll
        for (int t = 0; t < DT; ++t) oacc[t] *= alpha;
      }
      const float moff = m * cl;
#pragma unroll
      for (int j = 0; j < NT; ++j) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[j][r], cl, -moff));
          sc[j][r] = p;
          lp += p;
        }
      }
      const unsigned char* vb = vst + buf * VBUF_BYTES;
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        if (c0 + 16 * j >= P) continue;  // wave-uniform
        if constexpr (sizeof(T) == 2) {
          // V^T operand: lane l reads the 8 bytes at row 16j + l/4, columns
          // 16t + 4(l & 3) .. +3 of the buffer
          const uint16_t* vb16 = reinterpret_cast<const uint16_t*>(vb);
          uint32_t va[DT][2];
#pragma unroll
          for (int t = 0; t < DT; ++t) {
            const uint2 w = lds_read_tr16(vb16 + (16 * j + (lane >> 2)) * D + 16 * t + 4 * (lane & 3));
            va[t][0] = w.x;
            va[t][1] = w.y;
          }
          pv_mfma16<T, DT>(va, sc[j], oacc);
        } else {
          // lane (c, g): V[16j + 4g + s][16t + c], s = 0..3, in one read
          const float* vbf = reinterpret_cast<const float*>(vb);
#pragma unroll
          for (int t = 0; t < DT; ++t) {
            const f32x4_t w = *reinterpret_cast<const f32x4_t*>(vbf + (16 * t + c) * VT_STRIDE + 16 * j + 4 * g);
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4)
              oacc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(w[s4], sc[j][s4], oacc[t], 0, 0, 0);
          }
        }
      }
    };
    // the first chunks' values go to LDS as soon as they arrive (their
    // registers are then free while the own keys stream in); a later chunk's
    // right before its products, after the previous reads of its buffer fed
    // their products
    stage_values(vrA, 0);
    if constexpr (NCB == 2) stage_values(vrB, 1);
    if constexpr (D == 16) {  // two chunk buffers fit the register budget at D = 16
      for (int c0 = 0; c0 < P; c0 += 32 * NT) {
        if (c0 > 0 && c0 + 16 * NT < P) load_chunk(c0 + 16 * NT, kopB, vrB);
        if (c0 > 0) stage_values(vrA, 0);
        prefix_chunk(c0, kopA, 0);
        if (c0 + 16 * NT >= P) break;
        if (c0 + 32 * NT < P) load_chunk(c0 + 32 * NT, kopA, vrA);
        if (c0 > 0) stage_values(vrB, 1);
        prefix_chunk(c0 + 16 * NT, kopB, 1);
      }
    } else {
      for (int c0 = 0; c0 < P; c0 += 16 * NT) {
        if (c0 > 0) {
          load_chunk(c0, kopA, vrA);
          stage_values(vrA, 0);
        }
        prefix_chunk(c0, kopA, 0);
      }
    }
    DG_STAMP(2);  // wave 0: prefix done
  } else {
    // --- wave 1: own keys on the vector ALUs; fused: the new token -----------------
    // One path per number of register sets issued up front (wave-uniform):
    // the query, projection and table loads are issued before the sets, and
    // their waits count the sets issued after them.
    const int nsets = Tc > P ? (Tc - P + STEP - 1) / STEP : 0;
    auto own_wave = [&](auto ns) __attribute__((always_inline)) {
      constexpr int NS = decltype(ns)::value;
      Slice qs;
      Slice knew, vnew;  // fused: the appended key and value
      float xq[EPL], xk[EPL], cs[EPL];
      if constexpr (FUSED) {
        load_vec<T, EPL>(qbase + bo * a.qb + piece * EPL, xq);
        load_vec<T, EPL>(static_cast<const T*>(a.kp) + bo * a.kpb + (int64_t)h * a.kph + piece * EPL, xk);
        load_row<T, EPL>(vnew, static_cast<const T*>(a.vp) + bo * a.vpb + (int64_t)h * a.vph + piece * EPL);
        load_vec<FT, EPL>(fbase, cs);
      } else {
        load_row<T, EPL>(qs, qbase + bo * a.qb + piece * EPL);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int k = 0; k < NS; ++k) load_set(k, k);
      __builtin_amdgcn_sched_barrier(0);
      DG_STAMP(1);  // wave 1: q and the first register sets issued
      if constexpr (FUSED) {
        rotate_q(xq, cs, qs);
        rope_rotate<T, EPL>(xk, cs);
        if (a.qknorm) qk_rms_norm<EPL, LPK, true>(xk, D);
        pack_row<T, EPL>(knew, xk);
        // the append (kv_cache.py:108-109)
        if (ovalid && kk == 0) {
          store_row<T, EPL>(const_cast<T*>(kbase) + bo * a.kb + (int64_t)Tc * kt + piece * EPL, knew);
          store_row<T, EPL>(const_cast<T*>(vbase) + bo * a.vb + (int64_t)Tc * vt + piece * EPL, vnew);
        }
      }
      DG_STAMP(2);  // wave 1: RoPE, QK-norm and the append done
      if constexpr (NS == 2) own_stream(qs, nsets);
      if constexpr (NS == 1) process(kr[0], vr[0], P, qs);
      DG_STAMP(3);  // wave 1: own-key stream done
      if constexpr (FUSED) {  // the appended key, from registers (key lane 0 of each quad)
        const float dot = group_sum_dpp<LPK>(slice_dot<T, EPL>(qs, knew));
        const float sn = kk == 0 ? dot : kNegInf;
        raise_offset(sn);
        add_key(sn, vnew, mo * cl);
      }
      hand_over();
      DG_STAMP(4);  // wave 1: new key and hand-over done
    };
    if (nsets >= 2) own_wave(IntConst<2>{});
    else if (nsets == 1) own_wave(IntConst<1>{});
    else own_wave(IntConst<0>{});
  }
  __syncthreads();
  DG_STAMP(5);  // both: past the barrier
  if (role == 1) {
    DG_TIMELINE_FLUSH();
    return;
  }

  // --- merge (wave 0): lane (c, g) holds columns 16t + 4g + r of row c --------
  const float* pr = part + c * RS;
  const float m_own = pr[D], l_own = pr[D + 1];
  const float M = fmaxf(m, m_own);
  const float ao = (m_own == kNegInf) ? 0.f : __builtin_amdgcn_exp2f((m_own - M) * cl);
  const float ap = (m == kNegInf) ? 0.f : __builtin_amdgcn_exp2f((m - M) * cl);
  const float inv = 1.0f / (row_sum4(lp) * ap + l_own * ao);
#pragma unroll
  for (int t = 0; t < DT; ++t) {
    const f32x4_t own = *reinterpret_cast<const f32x4_t*>(pr + 16 * t + 4 * g);
    float out[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) out[r] = __builtin_fmaf(oacc[t][r], ap, own[r] * ao) * inv;
    if (cvalid)
      store_vec<T, 4>(static_cast<T*>(a.y) + bc * a.yb + (int64_t)h * a.yh + 16 * t + 4 * g, out);
  }
  DG_TIMELINE_FLUSH();
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
namespace {

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <typename T, int D, bool FUSED, typename FT>
int launch_shared(const SharedArgs& a, hipStream_t s) {
  hipLaunchKernelGGL((attn_shared_kernel<T, D, FUSED, FT>), dim3((unsigned)a.units), dim3(128), 0, s, a);
  return check_launch("attn_shared_kernel");
}

template <typename T, bool FUSED, typename FT>
int launch_shared_d(const SharedArgs& a, hipStream_t s) {
  return a.D == 16 ? launch_shared<T, 16, FUSED, FT>(a, s) : launch_shared<T, 32, FUSED, FT>(a, s);
}

void fill_common(SharedArgs& a, int B, int H, int D, int Tk, const void* q, const dg_stride3* q_st,
                 const void* k, const dg_stride3* k_st, const void* v, const dg_stride3* v_st, void* y,
                 const dg_stride3* y_st, float scale, const PrefixRef& pre, const int* pos_dev) {
  const int group = pre.group;
  a.q = q; a.k = k; a.v = v; a.y = y;
  a.qb = q_st->b; a.qh = q_st->h;
  a.kb = k_st->b; a.kt = k_st->t; a.kh = k_st->h;
  a.vb = v_st->b; a.vt = v_st->t; a.vh = v_st->h;
  a.yb = y_st->b; a.yh = y_st->h;
  a.B = B; a.H = H; a.D = D; a.Tk = Tk; a.pre = pre;
  a.tiles = (group + 15) / 16;
  a.units = (((int64_t)B + group - 1) / group) * a.tiles * H;
  a.scale_log2 = scale * 1.44269504088896340736f;
  a.lazy_raw = kSharedLazyLog2 / a.scale_log2;
  a.pos_dev = pos_dev;
}

}  // namespace

// The matrix-core path takes single-token decode over groups of at least 16
// rows, head_dim 16 or 32, 16-byte aligned rows; everything else stays on the
// vector kernel.
bool shared_attention_applicable(int B, int H, int Tq, int Tk, int D, int dtype, const PrefixRef& pre,
                                 const void* q, const dg_stride3* q_st, const void* k,
                                 const dg_stride3* k_st, const void* v, const dg_stride3* v_st,
                                 const void* y, const dg_stride3* y_st) {
  const int group = pre.group;
  if (Tq != 1 || group < kSharedMinGroup || pre.len < 1 || pre.len > Tk) return false;
  if (D != 16 && D != 32) return false;
  if (dtype != DG_F32 && dtype != DG_BF16 && dtype != DG_F16) return false;
  const int64_t es = dtype == DG_F32 ? 4 : 2;
  if (!al16(q) || !al16(k) || !al16(v) || !al16(y)) return false;
  auto st16 = [&](int64_t st) { return (st * es) % 16 == 0; };
  if (!st16(q_st->b) || !st16(q_st->h) || !st16(y_st->b) || !st16(y_st->h)) return false;
  if (!st16(k_st->b) || !st16(k_st->t) || !st16(k_st->h)) return false;
  if (!st16(v_st->b) || !st16(v_st->t) || !st16(v_st->h)) return false;
  if (!al16(pre.k) || !al16(pre.v) || !st16(pre.kb) || !st16(pre.kh) || !st16(pre.vb) || !st16(pre.vh))
    return false;
  if (k_st->t < 0 || v_st->t < 0 || k_st->b < 0) return false;
  if ((int64_t)Tk * k_st->t >= ((int64_t)1 << 31) || (int64_t)Tk * v_st->t >= ((int64_t)1 << 31)) return false;
  // the rows' own keys are addressed by one 32-bit byte offset for K and V
  if (k_st->b != v_st->b || k_st->t != v_st->t) return false;
  if (((int64_t)(B - 1) * k_st->b + (int64_t)(Tk - 1) * k_st->t + D) * es >= ((int64_t)1 << 31)) return false;
  const int64_t groups = ((int64_t)B + group - 1) / group;
  const int64_t tiles = (group + 15) / 16;
  const int64_t units = groups * tiles * H;
  return units < ((int64_t)1 << 31) - 4;
}

int shared_attention(int B, int H, int Tk, int D, int dtype, const void* q, const dg_stride3* q_st,
                     const void* k, const dg_stride3* k_st, const void* v, const dg_stride3* v_st,
                     void* y, const dg_stride3* y_st, float scale, const PrefixRef& pre,
                     const int* pos_dev, hipStream_t s) {
  DG_REQUIRE(scale > 0.f, DG_EINVAL, "attention: scale must be positive (got %g)", (double)scale);
  SharedArgs a{};
  fill_common(a, B, H, D, Tk, q, q_st, k, k_st, v, v_st, y, y_st, scale, pre, pos_dev);
  if (dtype == DG_F32) return launch_shared_d<float, false, float>(a, s);
  if (dtype == DG_BF16) return launch_shared_d<bf16_t, false, bf16_t>(a, s);
  return launch_shared_d<f16_t, false, f16_t>(a, s);
}

// The fused decode step takes what shared_attention takes, with the cache as
// (B, max_pos, H, D) pages, plus 16-byte aligned projection rows and RoPE
// table rows (table dtype: the data's or fp32).
bool shared_step_applicable(int B, int H, int D, int dtype, const PrefixRef& pre, int max_pos,
                            const void* q, const dg_stride3* q_st, const void* k, const dg_stride3* k_st,
                            const void* v, const dg_stride3* v_st, const void* kc, const dg_stride3* kc_st,
                            const void* vc, const dg_stride3* vc_st, const void* freqs, int64_t fpos,
                            int fdtype, const void* y, const dg_stride3* y_st) {
  if (!shared_attention_applicable(B, H, 1, max_pos, D, dtype, pre, q, q_st, kc, kc_st, vc,
                                   vc_st, y, y_st))
    return false;
  const int64_t es = dtype == DG_F32 ? 4 : 2;
  const int64_t fes = fdtype == DG_F32 ? 4 : 2;
  if (fdtype != dtype && fdtype != DG_F32) return false;
  auto st16 = [&](int64_t st, int64_t e) { return (st * e) % 16 == 0; };
  if (!al16(k) || !al16(v) || !al16(freqs)) return false;
  if (!st16(k_st->b, es) || !st16(k_st->h, es) || !st16(v_st->b, es) || !st16(v_st->h, es)) return false;
  return fpos >= 0 && st16(fpos, fes);
}

int shared_decode_step(int B, int H, int D, int dtype, const void* q, const dg_stride3* q_st, const void* k,
                       const dg_stride3* k_st, const void* v, const dg_stride3* v_st, void* kc,
                       const dg_stride3* kc_st, void* vc, const dg_stride3* vc_st, const void* freqs,
                       int64_t fpos, int fdtype, int pos, const int* pos_dev, int max_pos, void* y,
                       const dg_stride3* y_st, float scale, const PrefixRef& pre, int qknorm,
                       hipStream_t s) {
  DG_REQUIRE(scale > 0.f, DG_EINVAL, "decode_step: scale must be positive (got %g)", (double)scale);
  SharedArgs a{};
  fill_common(a, B, H, D, max_pos, q, q_st, kc, kc_st, vc, vc_st, y, y_st, scale, pre, pos_dev);
  a.kp = k; a.vp = v;
  a.kpb = k_st->b; a.kph = k_st->h; a.vpb = v_st->b; a.vph = v_st->h;
  a.freqs = freqs; a.fpos = fpos;
  a.pos = pos; a.max_pos = max_pos; a.qknorm = qknorm;
  if (dtype == DG_F32) return launch_shared_d<float, true, float>(a, s);
  if (dtype == DG_BF16)
    return fdtype == DG_F32 ? launch_shared_d<bf16_t, true, float>(a, s) : launch_shared_d<bf16_t, true, bf16_t>(a, s);
  return fdtype == DG_F32 ? launch_shared_d<f16_t, true, float>(a, s) : launch_shared_d<f16_t, true, f16_t>(a, s);
}

}  // namespace dg

#ifdef DG_TIMELINE
// Measurement build only: where the shared kernel's waves write their stamps
// (NULL: nowhere), and an empty kernel of a given grid for the launch floor.
namespace dg {
__global__ void timeline_empty_kernel() {}
}  // namespace dg
extern "C" __attribute__((visibility("default"))) int dg_timeline_set(void* buffer) {
  return (int)hipMemcpyToSymbol(HIP_SYMBOL(dg::g_timeline), &buffer, sizeof(buffer));
}
extern "C" __attribute__((visibility("default"))) int dg_timeline_empty(int blocks, int threads, void* stream) {
  hipLaunchKernelGGL(dg::timeline_empty_kernel, dim3(blocks), dim3(threads), 0, static_cast<hipStream_t>(stream));
  return (int)hipGetLastError();
}
#endif
