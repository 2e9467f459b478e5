// Fused RoPE + QK-norm + KV append, and the standalone row RMSNorm.
//
// Reference semantics (fxeqxmulfx/diff-gpt):
//   rope.py:20-27   x.float() split into interleaved pairs (x[2j], x[2j+1]);
//                   out = (re*cos - im*sin, re*sin + im*cos) in fp32, then one
//                   rounding back to x's dtype (type_as).
//   rms_norm.py:7   F.rms_norm(x, (D,)) with eps=None: x * rsqrt(mean(x^2) + eps)
//                   in fp32 with eps = FLT_EPSILON, one rounding to x's dtype.
//   mha.py:44-56    q,k -> rope -> QK-norm -> transpose -> KVCache.insert_kv.
//
// Arithmetic contract (what makes the cache contents reproducible bit for bit):
//   * RoPE: two separately rounded products and one rounded add/sub, never an
//     FMA (contraction is switched off below), cos/sin read from the caller's
//     table -- never recomputed on the device.
//   * Norm: squares rounded, summed by a pairwise tree over the row padded with
//     zeros to a power of two (adjacent pairs, then pairs of pairs ...),
//     mean = sum / D, r = 1 / sqrt(mean + FLT_EPSILON) with correctly rounded
//     sqrt and divide, y = x * r.
//   * The V half of the append is an exact copy.
#include "dg_rope_math.h"

namespace dg {

struct RopeArgs {
  const void* src[3];
  void* dst[3];
  int64_t sb[3], st[3], sh[3];  // source strides (b, t, h)
  int64_t db[3], dt[3], dh[3];  // destination strides (b, t, h)
  const void* freqs;
  int64_t fb, ft, fh;
  int64_t rows;  // B*T*H
  int T, H, D;
  int qknorm;
  // Decode-step form (graph-replayable): when pos_dev is set, the number of
  // positions already cached is read on the device; destinations advance by
  // pstep[w] and the table by fpos elements per position.  Positions outside
  // [min_pos, max_pos) write nothing.
  const int* pos_dev;
  int min_pos, max_pos;
  int64_t pstep[3];
  int64_t fpos;
};

// One row (b,t,h) of D elements is owned by LPK = DPAD/EPL consecutive lanes,
// each holding EPL consecutive elements (EPL even, so a (re, im) pair never
// straddles lanes).  Lanes whose slice starts at or beyond D (only when D is
// not a power of two) hold zeros and store nothing.  A lane group takes RPT
// rows, RPB apart (so that each wave instruction still covers consecutive
// rows), and issues every load of them before any arithmetic: RPT times the
// bytes in flight per wave, which a single row per lane leaves too few of to
// keep HBM busy.  Each row's arithmetic is the same whatever RPT is.
// PAIRS: slices read and written pair by pair, pairs past D skipped (head
// dims past 128 whose slices are not whole vectors).
template <typename T, typename FT, int DPAD, int EPL, int RPT, bool PAIRS>
__global__ __launch_bounds__(256) void rope_qknorm_kernel(const RopeArgs a) {
#pragma clang fp contract(off)
  constexpr int LPK = DPAD / EPL;
  static_assert(LPK >= 1 && LPK <= 64 && (EPL % 2) == 0, "row mapping");
  constexpr int RPB = 256 / LPK;  // rows of a block in one pass

  const int sub = threadIdx.x % LPK;
  const int64_t row0 = (int64_t)blockIdx.x * RPB * RPT + threadIdx.x / LPK;
  if (row0 >= a.rows) return;  // a whole lane group leaves together; no barriers follow
  int64_t pos = 0;
  if (a.pos_dev != nullptr) {  // uniform over the grid
    pos = *a.pos_dev;
    if (pos < a.min_pos || pos >= a.max_pos) return;
  }
  const int d0 = sub * EPL;
  const bool active = d0 < a.D;
  const int np = slice_pairs<EPL>(d0, a.D);  // PAIRS: pairs of the slice inside D

  // all sources of all RPT rows are read before anything is stored: the
  // destinations may alias them as far as the compiler knows, so this order
  // keeps every load in flight together
  RowRegs<FT, EPL> cr[RPT];      // (cos, sin) of the lane's EPL/2 pairs, interleaved
  RowRegs<T, EPL> xr[3][RPT];
  int64_t off_b[RPT];
  int off_t[RPT], off_h[RPT];
  bool live[RPT];
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    const int64_t row = row0 + (int64_t)j * RPB;
    live[j] = row < a.rows;  // uniform over the lane group
    // the host keeps B*T*H below 2^31: 32-bit division
    const uint32_t row32 = (uint32_t)(live[j] ? row : row0);
    off_h[j] = (int)(row32 % (uint32_t)a.H);
    const uint32_t bt = row32 / (uint32_t)a.H;
    off_t[j] = (int)(bt % (uint32_t)a.T);
    off_b[j] = (int64_t)(bt / (uint32_t)a.T);
#pragma unroll
    for (int w = 0; w < RowRegs<FT, EPL>::WORDS; ++w) cr[j].w[w] = 0u;
    if (active && live[j]) {
      const FT* f = static_cast<const FT*>(a.freqs) + pos * a.fpos + off_b[j] * a.fb + (int64_t)off_t[j] * a.ft +
                    (int64_t)off_h[j] * a.fh + d0;
      load_slice<FT, EPL, PAIRS>(cr[j], f, np);
    }
#pragma unroll
    for (int w = 0; w < 3; ++w) {
#pragma unroll
      for (int i = 0; i < RowRegs<T, EPL>::WORDS; ++i) xr[w][j].w[i] = 0u;
      if (a.src[w] == nullptr || !active || !live[j]) continue;  // src: uniform over the grid
      const T* sp = static_cast<const T*>(a.src[w]) + off_b[j] * a.sb[w] + (int64_t)off_t[j] * a.st[w] +
                    (int64_t)off_h[j] * a.sh[w] + d0;
      load_slice<T, EPL, PAIRS>(xr[w][j], sp, np);
    }
  }

#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    float cs[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) cs[e] = elem<FT, EPL>(cr[j], e);
#pragma unroll
    for (int w = 0; w < 3; ++w) {
      if (a.src[w] == nullptr) continue;  // uniform over the grid
      float x[EPL];
#pragma unroll
      for (int e = 0; e < EPL; ++e) x[e] = elem<T, EPL>(xr[w][j], e);
      if (w < 2) {
        rope_rotate<T, EPL>(x, cs);
        if (a.qknorm) qk_rms_norm<EPL, LPK, true>(x, a.D);
      }
      if (active && live[j]) {
        T* d = static_cast<T*>(a.dst[w]) + pos * a.pstep[w] + off_b[j] * a.db[w] + (int64_t)off_t[j] * a.dt[w] +
               (int64_t)off_h[j] * a.dh[w] + d0;
        store_vec_slice<T, EPL, PAIRS>(d, x, np);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Row RMSNorm over N elements (rms_norm.py:5-7).  G = NPAD/CH lanes per row,
// each lane owns CH consecutive elements; same canonical tree as above.
// ---------------------------------------------------------------------------
struct RowNormArgs {
  const void* x;
  void* out;
  int64_t x_ld, out_ld, M;
  int N;
  int vec;  // 1 when every lane slice is aligned for CH-element vector access
  // dg_embed_norm: row r of x is row ids[r] of the table (ids outside
  // [0, V) give NaN rows), and out2, when set, receives the norm of the
  // stored (rounded) out row
  const int64_t* ids;
  int64_t V;
  void* out2;
  int64_t out2_ld;
};

template <typename T, int NPAD, int CH>
__global__ __launch_bounds__(256) void rms_norm_kernel(const RowNormArgs a) {
#pragma clang fp contract(off)
  constexpr int G = NPAD / CH;
  static_assert(G >= 1 && G <= 64, "row mapping");
  constexpr int ROWS_PER_BLOCK = 256 / G;
  const int sub = threadIdx.x % G;
  const int64_t row = (int64_t)blockIdx.x * ROWS_PER_BLOCK + threadIdx.x / G;
  if (row >= a.M) return;
  const int c0 = sub * CH;
  int64_t src = row;
  bool bad = false;
  if (a.ids != nullptr) {  // uniform over the grid
    const int64_t id = a.ids[row];
    bad = id < 0 || id >= a.V;
    src = bad ? 0 : id;
  }
  const T* xs = static_cast<const T*>(a.x) + src * a.x_ld + c0;
  float x[CH];
  if (a.vec && c0 + CH <= a.N) {
    load_vec<T, CH>(xs, x);
  } else {
#pragma unroll
    for (int i = 0; i < CH; ++i) x[i] = (c0 + i < a.N) ? to_f32(xs[i]) : 0.f;
  }
  if (bad) {
#pragma unroll
    for (int i = 0; i < CH; ++i) x[i] = __builtin_nanf("");
  }
  auto norm = [&](float (&v)[CH]) __attribute__((always_inline)) {
    float sq[CH];
#pragma unroll
    for (int i = 0; i < CH; ++i) sq[i] = v[i] * v[i];
    float ss = tree_sum<CH>(sq);
    ss = group_sum<G>(ss);
    const float mean = ss / (float)a.N;
    const float r = 1.0f / sqrtf(mean + FLT_EPSILON);
#pragma unroll
    for (int i = 0; i < CH; ++i) v[i] = v[i] * r;
  };
  norm(x);
  if (a.out2 != nullptr) {  // uniform over the grid
    // the second norm reads the first one's stored values
    float y[CH];
#pragma unroll
    for (int i = 0; i < CH; ++i) y[i] = (c0 + i < a.N) ? to_f32(from_f32<T>(x[i])) : 0.f;
    norm(y);
    T* o2 = static_cast<T*>(a.out2) + row * a.out2_ld + c0;
    if (a.vec && c0 + CH <= a.N) {
      store_vec<T, CH>(o2, y);
    } else {
#pragma unroll
      for (int i = 0; i < CH; ++i)
        if (c0 + i < a.N) o2[i] = from_f32<T>(y[i]);
    }
  }
  T* os = static_cast<T*>(a.out) + row * a.out_ld + c0;
  if (a.vec && c0 + CH <= a.N) {
    store_vec<T, CH>(os, x);
  } else {
#pragma unroll
    for (int i = 0; i < CH; ++i)
      if (c0 + i < a.N) os[i] = from_f32<T>(x[i]);
  }
}

// ---------------------------------------------------------------------------
// float64 rows (a GPT.double() model).  rope.py:20-27 rounds x to fp32
// (x.float()) and multiplies by the table in the promoted dtype of the two:
// with a float64 table (GPT.double() converts the buffer) two rounded
// products and a rounded sum or difference in float64; with an fp32 table the
// same in fp32, converted exactly to float64 (type_as).  The QK-norm is
// F.rms_norm on float64 rows: x / sqrt(mean(x^2) + DBL_EPSILON) in float64.
// One wave per row; lane l holds pairs l, l + 64, ... (D <= 1024: at most 8),
// so every load and store of a wave covers consecutive pairs.
// ---------------------------------------------------------------------------
constexpr int kF64RopePairs = 8;  // 1024 / 2 / 64

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <typename FT>
__global__ __launch_bounds__(256) void rope_qknorm_f64_kernel(const RopeArgs a) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;  // whole waves leave; no barriers follow
  int64_t pos = 0;
  if (a.pos_dev != nullptr) {  // uniform over the grid
    pos = *a.pos_dev;
    if (pos < a.min_pos || pos >= a.max_pos) return;
  }
  const uint32_t r32 = (uint32_t)row;  // the host keeps B*T*H below 2^31
  const int h = (int)(r32 % (uint32_t)a.H);
  const uint32_t bt = r32 / (uint32_t)a.H;
  const int t = (int)(bt % (uint32_t)a.T);
  const int64_t b = (int64_t)(bt / (uint32_t)a.T);
  const int npairs = a.D / 2;
  const FT* f = static_cast<const FT*>(a.freqs) + pos * a.fpos + b * a.fb + (int64_t)t * a.ft + (int64_t)h * a.fh;
  for (int w = 0; w < 3; ++w) {
    if (a.src[w] == nullptr) continue;  // uniform over the grid
    const double* sp = static_cast<const double*>(a.src[w]) + b * a.sb[w] + (int64_t)t * a.st[w] + (int64_t)h * a.sh[w];
    double* dp = static_cast<double*>(a.dst[w]) + pos * a.pstep[w] + b * a.db[w] + (int64_t)t * a.dt[w] +
                 (int64_t)h * a.dh[w];
    double re[kF64RopePairs], im[kF64RopePairs];
#pragma unroll
    for (int j = 0; j < kF64RopePairs; ++j) {
      const int p = lane + 64 * j;
      re[j] = p < npairs ? sp[2 * p] : 0.0;
      im[j] = p < npairs ? sp[2 * p + 1] : 0.0;
    }
    if (w < 2) {
      double ss = 0.0;
#pragma unroll
      for (int j = 0; j < kF64RopePairs; ++j) {
        const int p = lane + 64 * j;
        // FT is the arithmetic type: float * float stays fp32, float * double
        // promotes to float64
        const FT c = p < npairs ? f[2 * p] : FT(0);
        const FT sn = p < npairs ? f[2 * p + 1] : FT(0);
        const FT xr = (FT)(float)re[j], xi = (FT)(float)im[j];
        const FT a0 = xr * c, a1 = xi * sn, b0 = xr * sn, b1 = xi * c;
        re[j] = (double)(a0 - a1);
        im[j] = (double)(b0 + b1);
        ss += re[j] * re[j] + im[j] * im[j];
      }
      if (a.qknorm) {
        const double r = 1.0 / sqrt(wave_sum_f64(ss) / (double)a.D + DBL_EPSILON);
#pragma unroll
        for (int j = 0; j < kF64RopePairs; ++j) {
          re[j] *= r;
          im[j] *= r;
        }
      }
    }
#pragma unroll
    for (int j = 0; j < kF64RopePairs; ++j) {
      const int p = lane + 64 * j;
      if (p < npairs) {
        dp[2 * p] = re[j];
        dp[2 * p + 1] = im[j];
      }
    }
  }
}

// Row RMSNorm in float64 (rms_norm.py:5-7 on float64 rows): one wave per row,
// two passes over the row (N <= 8192).
__global__ __launch_bounds__(256) void rms_norm_f64_kernel(const RowNormArgs a) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.M) return;
  const double* x = static_cast<const double*>(a.x) + row * a.x_ld;
  double* o = static_cast<double*>(a.out) + row * a.out_ld;
  double ss = 0.0;
  for (int c = lane; c < a.N; c += 64) ss += x[c] * x[c];
  const double r = 1.0 / sqrt(wave_sum_f64(ss) / (double)a.N + DBL_EPSILON);
  for (int c = lane; c < a.N; c += 64) o[c] = x[c] * r;
}

// ---------------------------------------------------------------------------
// Host dispatch
// ---------------------------------------------------------------------------
namespace {

int elem_size(int dtype) { return (int)dtype_bytes(dtype); }

bool aligned(const void* p, int64_t bytes) {
  return p == nullptr || (reinterpret_cast<uintptr_t>(p) % (uintptr_t)bytes) == 0;
}
bool strides_multiple(const dg_stride3* s, int64_t m) {
  return s == nullptr || (s->b % m == 0 && s->t % m == 0 && s->h % m == 0);
}

int next_pow2(int x) {
  int p = 1;
  while (p < x) p <<= 1;
  return p;
}

// Rows per lane group: 4 once the launch still has >= 2048 workgroups with
// them (a prefill's many rows), else 1 (a decode step's few rows would leave
// CUs idle).
constexpr int kRopeRowsPerGroup = 4;
constexpr int64_t kRopeMinBlocks = 2048;

template <typename T, typename FT, int DPAD, int EPL, bool PAIRS>
int launch_rope(const RopeArgs& a, hipStream_t s) {
  constexpr int LPK = DPAD / EPL;
  constexpr int RPB = 256 / LPK;
  DG_REQUIRE(a.rows < 0x7fffffffLL, DG_EINVAL, "rope: B*T*H = %lld rows, at most 2^31 - 1", (long long)a.rows);
  // slices past 16 bytes hold enough bytes in flight with one row per group
  constexpr int R = EPL * (int)sizeof(T) > 16 ? 1 : kRopeRowsPerGroup;
  if (R > 1 && a.rows >= kRopeMinBlocks * RPB * R) {
    const int64_t blocks = (a.rows + RPB * R - 1) / (RPB * R);
    hipLaunchKernelGGL((rope_qknorm_kernel<T, FT, DPAD, EPL, R, PAIRS>), dim3((unsigned)blocks), dim3(256), 0, s,
                       a);
  } else {
    const int64_t blocks = (a.rows + RPB - 1) / RPB;
    hipLaunchKernelGGL((rope_qknorm_kernel<T, FT, DPAD, EPL, 1, PAIRS>), dim3((unsigned)blocks), dim3(256), 0, s,
                       a);
  }
  return check_launch("rope_qknorm_kernel");
}

// The kernel for a slice choice: vector slices (vec_slice_epl) or pair
// slices (pair_slice_epl; read pair by pair past one pair per lane).
template <typename T, typename FT, int DPAD>
int rope_pick_epl(int epl, bool pairs, const RopeArgs& a, hipStream_t s) {
  constexpr int VEC = vec_slice_epl(DPAD, (int)sizeof(T));
  constexpr int PAIR = pair_slice_epl(DPAD);
  if (!pairs && epl == VEC) return launch_rope<T, FT, DPAD, VEC, false>(a, s);
  if (pairs && epl == PAIR) return launch_rope<T, FT, DPAD, PAIR, (PAIR > 2)>(a, s);
  set_error("rope: no kernel for D pad %d with %d elements per lane", DPAD, epl);
  return DG_EUNSUPPORTED;
}

template <typename T, typename FT>
int rope_pick_d(int dpad, int epl, bool pairs, const RopeArgs& a, hipStream_t s) {
  switch (dpad) {
    case 2: return rope_pick_epl<T, FT, 2>(epl, pairs, a, s);
    case 4: return rope_pick_epl<T, FT, 4>(epl, pairs, a, s);
    case 8: return rope_pick_epl<T, FT, 8>(epl, pairs, a, s);
    case 16: return rope_pick_epl<T, FT, 16>(epl, pairs, a, s);
    case 32: return rope_pick_epl<T, FT, 32>(epl, pairs, a, s);
    case 64: return rope_pick_epl<T, FT, 64>(epl, pairs, a, s);
    case 128: return rope_pick_epl<T, FT, 128>(epl, pairs, a, s);
    case 256: return rope_pick_epl<T, FT, 256>(epl, pairs, a, s);
    case 512: return rope_pick_epl<T, FT, 512>(epl, pairs, a, s);
    case 1024: return rope_pick_epl<T, FT, 1024>(epl, pairs, a, s);
  }
  set_error("rope: head_dim %d unsupported", a.D);
  return DG_EUNSUPPORTED;
}

template <typename T, int NPAD>
int launch_rms(const RowNormArgs& a, hipStream_t s) {
  constexpr int PREF = 16 / (int)sizeof(T);
  constexpr int CH0 = NPAD / 64 > PREF ? NPAD / 64 : PREF;
  constexpr int CH = CH0 < NPAD ? CH0 : NPAD;
  constexpr int G = NPAD / CH;
  constexpr int RPB = 256 / G;
  const int64_t blocks = (a.M + RPB - 1) / RPB;
  DG_REQUIRE(blocks <= 0x7fffffffLL, DG_EINVAL, "rms_norm: too many rows (%lld)", (long long)a.M);
  RowNormArgs b = a;
  const int64_t vb = (int64_t)CH * (int64_t)sizeof(T);
  const bool pow2_vec = (vb == 4 || vb == 8 || vb % 16 == 0);
  b.vec = pow2_vec && aligned(a.x, vb) && aligned(a.out, vb) &&
          (a.x_ld * (int64_t)sizeof(T)) % vb == 0 && (a.out_ld * (int64_t)sizeof(T)) % vb == 0 &&
          (CH * (int)sizeof(T)) >= 4 &&
          (a.out2 == nullptr || (aligned(a.out2, vb) && (a.out2_ld * (int64_t)sizeof(T)) % vb == 0));
  hipLaunchKernelGGL((rms_norm_kernel<T, NPAD, CH>), dim3((unsigned)blocks), dim3(256), 0, s, b);
  return check_launch("rms_norm_kernel");
}

template <typename T>
int rms_pick(int npad, const RowNormArgs& a, hipStream_t s) {
  switch (npad) {
    case 1: return launch_rms<T, 2>(a, s);
    case 2: return launch_rms<T, 2>(a, s);
    case 4: return launch_rms<T, 4>(a, s);
    case 8: return launch_rms<T, 8>(a, s);
    case 16: return launch_rms<T, 16>(a, s);
    case 32: return launch_rms<T, 32>(a, s);
    case 64: return launch_rms<T, 64>(a, s);
    case 128: return launch_rms<T, 128>(a, s);
    case 256: return launch_rms<T, 256>(a, s);
    case 512: return launch_rms<T, 512>(a, s);
    case 1024: return launch_rms<T, 1024>(a, s);
    case 2048: return launch_rms<T, 2048>(a, s);
    case 4096: return launch_rms<T, 4096>(a, s);
    case 8192: return launch_rms<T, 8192>(a, s);
  }
  set_error("rms_norm: N=%d unsupported (max 8192)", a.N);
  return DG_EUNSUPPORTED;
}

}  // namespace
}  // namespace dg

using namespace dg;

namespace dg {
namespace {

// Shared body of the two RoPE entry points; pos_dev == nullptr is the plain form.
int rope_entry(int B, int T, int H, int D, int dtype, const void* q, const dg_stride3* q_st,
               void* q_out, const dg_stride3* qo_st, const void* k, const dg_stride3* k_st,
               void* k_out, const dg_stride3* ko_st, const void* v, const dg_stride3* v_st,
               void* v_out, const dg_stride3* vo_st, const void* freqs, const dg_stride3* f_st,
               int freqs_dtype, int flags, const int32_t* pos_dev, int min_pos, int max_pos,
               const int64_t (&pstep)[3], int64_t fpos, void* stream) {
  DG_REQUIRE(B >= 0 && T >= 0 && H >= 0, DG_EINVAL, "rope: negative size");
  DG_REQUIRE(D >= 2 && D % 2 == 0, DG_EINVAL, "rope: head_dim must be even and >= 2 (got %d)", D);
  DG_REQUIRE(dtype == DG_F32 || dtype == DG_BF16 || dtype == DG_F16 || dtype == DG_F64, DG_EUNSUPPORTED,
             "rope: dtype %d unsupported", dtype);
  DG_REQUIRE(freqs_dtype == DG_F32 || freqs_dtype == dtype, DG_EUNSUPPORTED,
             "rope: freqs dtype must be fp32 or equal to the data dtype");
  if ((int64_t)B * T * H == 0) return DG_OK;
  const void* src[3] = {q, k, v};
  void* dst[3] = {q_out, k_out, v_out};
  const dg_stride3* sst[3] = {q_st, k_st, v_st};
  const dg_stride3* dst_st[3] = {qo_st, ko_st, vo_st};
  bool any = false;
  for (int w = 0; w < 3; ++w) {
    DG_REQUIRE((src[w] == nullptr) == (dst[w] == nullptr), DG_EINVAL,
               "rope: input %d and its output must both be given or both be NULL", w);
    if (src[w]) {
      DG_REQUIRE(sst[w] && dst_st[w], DG_EINVAL, "rope: missing strides for tensor %d", w);
      any = true;
    }
  }
  if (!any) return DG_OK;
  const bool need_freqs = (q != nullptr) || (k != nullptr);
  DG_REQUIRE(!need_freqs || (freqs != nullptr && f_st != nullptr), DG_EINVAL,
             "rope: freqs table required");

  const int es = elem_size(dtype);
  const int fes = elem_size(freqs_dtype);
  const int dpad = next_pow2(D);
  DG_REQUIRE(D <= kMaxHeadDim, DG_EUNSUPPORTED, "rope: head_dim %d > %d", D, kMaxHeadDim);
  if (dtype == DG_F64) {
    // element-aligned float64 rows, one wave per row (rope_qknorm_f64_kernel)
    for (int w = 0; w < 3; ++w)
      DG_REQUIRE(aligned(src[w], 8) && aligned(dst[w], 8), DG_EINVAL, "rope: float64 rows must be 8-byte aligned");
    DG_REQUIRE(!need_freqs || aligned(freqs, fes), DG_EINVAL, "rope: freqs not aligned to its element size");
    const int64_t rows = (int64_t)B * T * H;
    DG_REQUIRE(rows < 0x7fffffffLL, DG_EINVAL, "rope: B*T*H = %lld rows, at most 2^31 - 1", (long long)rows);
    RopeArgs a{};
    for (int w = 0; w < 3; ++w) {
      a.src[w] = src[w];
      a.dst[w] = dst[w];
      if (src[w]) {
        a.sb[w] = sst[w]->b;  a.st[w] = sst[w]->t;  a.sh[w] = sst[w]->h;
        a.db[w] = dst_st[w]->b; a.dt[w] = dst_st[w]->t; a.dh[w] = dst_st[w]->h;
      }
      a.pstep[w] = pstep[w];
    }
    a.freqs = freqs;
    if (f_st) { a.fb = f_st->b; a.ft = f_st->t; a.fh = f_st->h; }
    a.rows = rows;
    a.T = T; a.H = H; a.D = D;
    a.qknorm = (flags & DG_QKNORM) ? 1 : 0;
    a.pos_dev = pos_dev; a.min_pos = min_pos; a.max_pos = max_pos;
    a.fpos = fpos;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 grid((unsigned)((rows + 3) / 4));
    if (freqs_dtype == DG_F32) hipLaunchKernelGGL(rope_qknorm_f64_kernel<float>, grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL(rope_qknorm_f64_kernel<double>, grid, dim3(256), 0, s, a);
    return check_launch("rope_qknorm_f64_kernel");
  }

  // Vector slices (16 bytes of data per lane, or the whole row when it is
  // shorter) where D is a multiple of them and every pointer / stride
  // allows it; otherwise pair slices.
  auto fits = [&](int epl, bool pairs) {
    if (!pairs && D % epl != 0) return false;
    const int w = pairs ? 2 : slice_load_elems(epl, es);        // data elements per access
    const int wf = pairs ? 2 : slice_load_elems(epl, fes);      // table elements per access
    for (int i = 0; i < 3; ++i) {
      if (!src[i]) continue;
      if (!aligned(src[i], (int64_t)w * es) || !aligned(dst[i], (int64_t)w * es)) return false;
      if (!strides_multiple(sst[i], w) || !strides_multiple(dst_st[i], w)) return false;
      if (pstep[i] % w != 0) return false;
    }
    if (need_freqs) {
      if (!aligned(freqs, (int64_t)wf * fes) || !strides_multiple(f_st, wf)) return false;
      if (fpos % wf != 0) return false;
    }
    return true;
  };
  int epl = 0;
  bool pairs = false;
  if (fits(vec_slice_epl(dpad, es), false)) {
    epl = vec_slice_epl(dpad, es);
  } else if (fits(pair_slice_epl(dpad), true)) {
    epl = pair_slice_epl(dpad);
    pairs = true;
  }
  DG_REQUIRE(epl != 0, DG_EINVAL,
             "rope: pointers/strides not aligned to an element pair (D=%d); pass contiguous rows", D);

  RopeArgs a{};
  for (int w = 0; w < 3; ++w) {
    a.src[w] = src[w];
    a.dst[w] = dst[w];
    if (src[w]) {
      a.sb[w] = sst[w]->b;  a.st[w] = sst[w]->t;  a.sh[w] = sst[w]->h;
      a.db[w] = dst_st[w]->b; a.dt[w] = dst_st[w]->t; a.dh[w] = dst_st[w]->h;
    }
  }
  a.freqs = freqs;
  if (f_st) { a.fb = f_st->b; a.ft = f_st->t; a.fh = f_st->h; }
  a.rows = (int64_t)B * T * H;
  a.T = T;
  a.H = H;
  a.D = D;
  a.qknorm = (flags & DG_QKNORM) ? 1 : 0;
  a.pos_dev = pos_dev;
  a.min_pos = min_pos;
  a.max_pos = max_pos;
  for (int w = 0; w < 3; ++w) a.pstep[w] = pstep[w];
  a.fpos = fpos;
  hipStream_t s = static_cast<hipStream_t>(stream);

  if (dtype == DG_F32) return rope_pick_d<float, float>(dpad, epl, pairs, a, s);
  if (dtype == DG_BF16) {
    if (freqs_dtype == DG_F32) return rope_pick_d<bf16_t, float>(dpad, epl, pairs, a, s);
    return rope_pick_d<bf16_t, bf16_t>(dpad, epl, pairs, a, s);
  }
  if (freqs_dtype == DG_F32) return rope_pick_d<f16_t, float>(dpad, epl, pairs, a, s);
  return rope_pick_d<f16_t, f16_t>(dpad, epl, pairs, a, s);
}

}  // namespace
}  // namespace dg

extern "C" int dg_rope_qknorm_append(int B, int T, int H, int D, int dtype, const void* q,
                                     const dg_stride3* q_st, void* q_out, const dg_stride3* qo_st,
                                     const void* k, const dg_stride3* k_st, void* k_out,
                                     const dg_stride3* ko_st, const void* v,
                                     const dg_stride3* v_st, void* v_out,
                                     const dg_stride3* vo_st, const void* freqs,
                                     const dg_stride3* f_st, int freqs_dtype, int flags,
                                     void* stream) {
  const int64_t none[3] = {0, 0, 0};
  return rope_entry(B, T, H, D, dtype, q, q_st, q_out, qo_st, k, k_st, k_out, ko_st, v, v_st, v_out,
                    vo_st, freqs, f_st, freqs_dtype, flags, nullptr, 0, 0, none, 0, stream);
}

namespace dg {
// dg_rope_qknorm_append_at with a lower bound on the position: nothing is
// written when *pos is outside [min_pos, max_pos) (the decode step's cache
// pages may start at a shared prefix's end).
int rope_append_at(int B, int H, int D, int dtype, const void* q, const dg_stride3* q_st, void* q_out,
                   const dg_stride3* qo_st, const void* k, const dg_stride3* k_st, void* k_cache,
                   const dg_stride3* kc_st, const void* v, const dg_stride3* v_st, void* v_cache,
                   const dg_stride3* vc_st, const void* freqs, int64_t freqs_pos_stride, int freqs_dtype,
                   const int32_t* pos, int min_pos, int max_pos, int flags, void* stream) {
  DG_REQUIRE(pos != nullptr, DG_EINVAL, "rope_at: NULL position pointer");
  DG_REQUIRE(max_pos >= 1 && min_pos >= 0, DG_EINVAL, "rope_at: bad position range [%d, %d)", min_pos, max_pos);
  DG_REQUIRE((k == nullptr || kc_st != nullptr) && (v == nullptr || vc_st != nullptr), DG_EINVAL,
             "rope_at: missing cache strides");
  const int64_t pstep[3] = {0, k ? kc_st->t : 0, v ? vc_st->t : 0};
  const dg_stride3 fst = {0, 0, 0};  // one position per call, broadcast over rows and heads
  return rope_entry(B, 1, H, D, dtype, q, q_st, q_out, qo_st, k, k_st, k_cache, kc_st, v, v_st,
                    v_cache, vc_st, freqs, &fst, freqs_dtype, flags, pos, min_pos, max_pos, pstep,
                    freqs_pos_stride, stream);
}
}  // namespace dg

extern "C" int dg_rope_qknorm_append_at(int B, int H, int D, int dtype, const void* q,
                                        const dg_stride3* q_st, void* q_out,
                                        const dg_stride3* qo_st, const void* k,
                                        const dg_stride3* k_st, void* k_cache,
                                        const dg_stride3* kc_st, const void* v,
                                        const dg_stride3* v_st, void* v_cache,
                                        const dg_stride3* vc_st, const void* freqs,
                                        int64_t freqs_pos_stride, int freqs_dtype,
                                        const int32_t* pos, int max_pos, int flags, void* stream) {
  return rope_append_at(B, H, D, dtype, q, q_st, q_out, qo_st, k, k_st, k_cache, kc_st, v, v_st, v_cache, vc_st,
                        freqs, freqs_pos_stride, freqs_dtype, pos, 0, max_pos, flags, stream);
}

extern "C" int dg_rms_norm(int64_t M, int N, int dtype, const void* x, int64_t x_ld, void* out,
                           int64_t out_ld, void* stream) {
  DG_REQUIRE(M >= 0 && N >= 1, DG_EINVAL, "rms_norm: bad sizes M=%lld N=%d", (long long)M, N);
  DG_REQUIRE(N <= 8192, DG_EUNSUPPORTED, "rms_norm: N=%d > 8192", N);
  DG_REQUIRE(dtype == DG_F32 || dtype == DG_BF16 || dtype == DG_F16 || dtype == DG_F64, DG_EUNSUPPORTED,
             "rms_norm: dtype %d unsupported", dtype);
  if (M == 0) return DG_OK;
  DG_REQUIRE(x != nullptr && out != nullptr, DG_EINVAL, "rms_norm: NULL pointer");
  DG_REQUIRE(x_ld >= N && out_ld >= N, DG_EINVAL, "rms_norm: row stride smaller than N");
  RowNormArgs a{};
  a.x = x;
  a.out = out;
  a.x_ld = x_ld;
  a.out_ld = out_ld;
  a.M = M;
  a.N = N;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == DG_F64) {
    DG_REQUIRE((M + 3) / 4 <= 0x7fffffffLL, DG_EINVAL, "rms_norm: too many rows (%lld)", (long long)M);
    hipLaunchKernelGGL(rms_norm_f64_kernel, dim3((unsigned)((M + 3) / 4)), dim3(256), 0, s, a);
    return check_launch("rms_norm_f64_kernel");
  }
  const int npad = next_pow2(N);
  if (dtype == DG_F32) return rms_pick<float>(npad, a, s);
  if (dtype == DG_BF16) return rms_pick<bf16_t>(npad, a, s);
  return rms_pick<f16_t>(npad, a, s);
}

extern "C" int dg_embed_norm(int64_t M, int C, int dtype, const int64_t* ids, int64_t V, const void* table,
                             int64_t table_ld, void* x_out, int64_t x_ld, void* xn_out, int64_t xn_ld,
                             void* stream) {
  DG_REQUIRE(M >= 0 && C >= 1 && V >= 1, DG_EINVAL, "embed_norm: bad sizes M=%lld C=%d V=%lld", (long long)M, C,
             (long long)V);
  DG_REQUIRE(C <= 8192, DG_EUNSUPPORTED, "embed_norm: C=%d > 8192", C);
  DG_REQUIRE(dtype == DG_F32 || dtype == DG_BF16 || dtype == DG_F16, DG_EUNSUPPORTED,
             "embed_norm: dtype %d unsupported", dtype);
  if (M == 0) return DG_OK;
  DG_REQUIRE(ids && table && x_out, DG_EINVAL, "embed_norm: NULL pointer");
  DG_REQUIRE(table_ld >= C && x_ld >= C && (xn_out == nullptr || xn_ld >= C), DG_EINVAL,
             "embed_norm: row stride smaller than C");
  RowNormArgs a{};
  a.x = table;
  a.out = x_out;
  a.x_ld = table_ld;
  a.out_ld = x_ld;
  a.M = M;
  a.N = C;
  a.ids = ids;
  a.V = V;
  a.out2 = xn_out;
  a.out2_ld = xn_ld;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int npad = next_pow2(C);
  if (dtype == DG_F32) return rms_pick<float>(npad, a, s);
  if (dtype == DG_BF16) return rms_pick<bf16_t>(npad, a, s);
  return rms_pick<f16_t>(npad, a, s);
}
