// Row kernels for the layers around attention in a decode step (the
// "neighbours" of the hot path), one launch each where torch issues several:
//
//   attn_res_norm_kernel  rms_norm(block_attn_res(V, w)) (block.py:10-44 then
//                         rms_norm.py:5-7): per row, the scores
//                         rms_norm(V_n) . w over the sources V_0 .. V_N, their
//                         softmax over n, the weighted sum h = sum_n p_n V_n,
//                         and the RMSNorm of h.  Torch runs stack, rms_norm,
//                         matmul, softmax, mul and sum, then rms_norm.
//   gate_kernel           y * sigmoid(g) (mha.py:84)
//   swiglu_kernel         clamped SwiGLU on interleaved (gate, linear) pairs
//                         (swi_glu.py:11-19)
//   softcap_kernel        cap * tanh(x / cap) (gpt.py:182-186)
//   lm_head_kernel        the tied lm_head GEMM, the softcap and, for greedy
//                         sampling, the argmax of each row (gpt.py:181-186,
//                         temperature.py:22-23) in one pass: the logits are
//                         written once and not read back
//
// Every intermediate is rounded to the storage dtype where the torch op
// sequence rounds it (each op returns a tensor of the input dtype; fp32
// arithmetic inside, as ATen's opmath does), so bf16 results follow the same
// rounding steps.  The RMSNorms use the lane mapping and reduction tree of
// rms_norm_kernel, so they produce its bits for the same row.
#include <float.h>

#include <type_traits>

#include "dg_common.h"

namespace dg {

constexpr int kMaxResSources = 32;

struct AttnResArgs {
  const void* src[kMaxResSources];
  int64_t ld[kMaxResSources];  // row strides (elements)
  const void* w;               // (C,) pseudo-query
  void* out;
  int64_t out_ld, M;
  int nsrc, N;
};

// round-trip through the storage dtype
template <typename T>
__device__ __forceinline__ float rt(float x) {
  return to_f32(from_f32<T>(x));
}

// RMSNorm of one row slice with rms_norm_kernel's arithmetic (squares summed
// by tree_sum inside the lane, then the butterfly over the G lanes of the row,
// here in registers: group_sum_dpp pairs the lanes as group_sum does, so the
// bits are the same)
template <int CH, int G>
__device__ __forceinline__ void row_rms(float (&x)[CH], int N) {
#pragma clang fp contract(off)
  float sq[CH];
#pragma unroll
  for (int i = 0; i < CH; ++i) sq[i] = x[i] * x[i];
  float ss = tree_sum<CH>(sq);
  ss = group_sum_dpp<G>(ss);
  const float mean = ss / (float)N;
  const float r = 1.0f / sqrtf(mean + FLT_EPSILON);
#pragma unroll
  for (int i = 0; i < CH; ++i) x[i] = x[i] * r;
}

template <typename T, int CH>
__device__ __forceinline__ void load_slice(const T* p, int c0, int N, bool vec, float (&x)[CH]) {
  if (vec && c0 + CH <= N) {
    load_vec<T, CH>(p, x);
  } else {
#pragma unroll
    for (int i = 0; i < CH; ++i) x[i] = (c0 + i < N) ? to_f32(p[i]) : 0.f;
  }
}

// Sources a lane loads into registers together, up front, to serve both
// passes of the mixture (one round trip to memory for them, instead of one
// per source and pass): about 32 registers of slices inside dg_block_out,
// whose GEMM stages need the rest, and about 64 in attn_res_norm_kernel (at
// n_embd 512, bf16, 10 sources took 21 us with 4 held).
template <int CH>
constexpr int res_held() {
  return CH <= 4 ? 8 : CH <= 8 ? 4 : CH <= 16 ? 2 : 1;
}
template <int CH>
constexpr int res_held_norm() {
  return CH <= 4 ? 16 : CH <= 8 ? 8 : CH <= 16 ? 4 : CH <= 32 ? 2 : 1;
}

template <typename T, int NPAD, int CH>
__global__ __launch_bounds__(256) void attn_res_norm_kernel(const AttnResArgs a, const int vec) {
#pragma clang fp contract(off)
  constexpr int G = NPAD / CH;
  constexpr int HELD = res_held_norm<CH>();
  static_assert(G >= 1 && G <= 64, "row mapping");
  constexpr int ROWS_PER_BLOCK = 256 / G;
  const int sub = threadIdx.x % G;
  const int64_t row = (int64_t)blockIdx.x * ROWS_PER_BLOCK + threadIdx.x / G;
  if (row >= a.M) return;  // whole lane groups leave together; no barriers
  const int c0 = sub * CH;
  auto load = [&](int n, float (&x)[CH]) __attribute__((always_inline)) {
    load_slice<T, CH>(static_cast<const T*>(a.src[n]) + row * a.ld[n] + c0, c0, a.N, vec, x);
  };
  float held[HELD][CH];
#pragma unroll
  for (int n = 0; n < HELD; ++n)
    if (n < a.nsrc) load(n, held[n]);  // uniform; no use before all are issued
  auto get = [&](int n, float (&x)[CH]) __attribute__((always_inline)) {
    if (n < HELD) {
#pragma unroll
      for (int i = 0; i < CH; ++i) x[i] = held[n][i];
    } else {
      load(n, x);
    }
  };
  float w[CH];
  load_slice<T, CH>(static_cast<const T*>(a.w) + c0, c0, a.N, vec, w);

  // pass 1: score_n = rms_norm(V_n) . w, each rounded as its tensor is
  float score[kMaxResSources];
  float mx = -INFINITY;
#pragma unroll
  for (int n = 0; n < kMaxResSources; ++n) {
    score[n] = -INFINITY;
    if (n >= a.nsrc) continue;  // uniform
    float x[CH];
    get(n, x);
    row_rms<CH, G>(x, a.N);
    float prod[CH];
#pragma unroll
    for (int i = 0; i < CH; ++i) prod[i] = rt<T>(x[i]) * w[i];
    float dot = tree_sum<CH>(prod);
    dot = group_sum_dpp<G>(dot);
    score[n] = rt<T>(dot);
    mx = fmaxf(mx, score[n]);
  }
  // softmax over the sources (fp32 inside, rounded output)
  float e[kMaxResSources];
  float sum = 0.f;
#pragma unroll
  for (int n = 0; n < kMaxResSources; ++n) {
    e[n] = 0.f;
    if (n >= a.nsrc) continue;
    e[n] = expf(score[n] - mx);
    sum += e[n];
  }
  // pass 2: h = sum_n rt(p_n * V_n), fp32 sum in source order, rounded
  float h[CH];
#pragma unroll
  for (int i = 0; i < CH; ++i) h[i] = 0.f;
#pragma unroll
  for (int n = 0; n < kMaxResSources; ++n) {
    if (n >= a.nsrc) continue;
    const float p = rt<T>(e[n] / sum);
    float x[CH];
    get(n, x);
#pragma unroll
    for (int i = 0; i < CH; ++i) h[i] = h[i] + rt<T>(p * x[i]);
  }
#pragma unroll
  for (int i = 0; i < CH; ++i) h[i] = (c0 + i < a.N) ? rt<T>(h[i]) : 0.f;
  row_rms<CH, G>(h, a.N);
  T* os = static_cast<T*>(a.out) + row * a.out_ld + c0;
  if (vec && c0 + CH <= a.N) {
    store_vec<T, CH>(os, h);
  } else {
#pragma unroll
    for (int i = 0; i < CH; ++i)
      if (c0 + i < a.N) os[i] = from_f32<T>(h[i]);
  }
}

// attn_res_norm_kernel for few wide rows (one row per wave there, G = 64):
// a workgroup of 4 waves takes one row, so a decode step's few hundred rows
// keep four times the waves in flight and each wave's dependent chain of
// per-source reductions is a quarter as long.  Wave w scores sources w,
// w + 4, ... (each in the lane mapping, arithmetic and reduction tree of
// attn_res_norm_kernel, so each score has its bits); the scores meet in LDS;
// every wave takes the softmax over them in source order; wave w forms the
// weighted sum for a quarter of the columns (each column summed over the
// sources in source order, as before) into LDS; wave 0 normalises the row in
// attn_res_norm_kernel's lane mapping and stores it.  Same bits throughout.
template <int CH>
constexpr int res_held_split() {
  return CH <= 8 ? 8 : 64 / CH;
}

template <typename T, int NPAD, int CH>
__global__ __launch_bounds__(256) void attn_res_norm_split_kernel(const AttnResArgs a, const int vec) {
#pragma clang fp contract(off)
  constexpr int G = NPAD / CH;
  static_assert(G == 64, "one row per wave in attn_res_norm_kernel's mapping");
  constexpr int HELD = res_held_split<CH>();  // sources a wave holds in registers
  constexpr int CQ = CH / 4;                  // columns per lane in the weighted sum
  static_assert(CQ >= 1 && CQ * 4 == CH, "column split");
  __shared__ float sc[kMaxResSources];
  __shared__ __attribute__((aligned(16))) float hrow[NPAD];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int64_t row = blockIdx.x;  // the host launches one workgroup per row
  const int c0 = lane * CH;
  float w[CH];
  load_slice<T, CH>(static_cast<const T*>(a.w) + c0, c0, a.N, vec, w);
  auto load = [&](int n, float (&x)[CH]) __attribute__((always_inline)) {
    load_slice<T, CH>(static_cast<const T*>(a.src[n]) + row * a.ld[n] + c0, c0, a.N, vec, x);
  };
  float held[HELD][CH];
#pragma unroll
  for (int j = 0; j < HELD; ++j)
    if (wv + 4 * j < a.nsrc) load(wv + 4 * j, held[j]);  // wave-uniform; no use before all are issued
  // pass 1: this wave's scores
#pragma unroll
  for (int j = 0; j < kMaxResSources / 4; ++j) {
    const int n = wv + 4 * j;
    if (n >= a.nsrc) break;  // wave-uniform
    float x[CH];
    if (j < HELD) {
#pragma unroll
      for (int i = 0; i < CH; ++i) x[i] = held[j][i];
    } else {
      load(n, x);
    }
    row_rms<CH, G>(x, a.N);
    float prod[CH];
#pragma unroll
    for (int i = 0; i < CH; ++i) prod[i] = rt<T>(x[i]) * w[i];
    float dot = tree_sum<CH>(prod);
    dot = group_sum_dpp<G>(dot);
    if (lane == 0) sc[n] = rt<T>(dot);
  }
  __syncthreads();
  // softmax over the sources (fp32 inside, rounded output), in source order
  float mx = -INFINITY;
#pragma unroll
  for (int n = 0; n < kMaxResSources; ++n)
    if (n < a.nsrc) mx = fmaxf(mx, sc[n]);
  float e[kMaxResSources];
  float sum = 0.f;
#pragma unroll
  for (int n = 0; n < kMaxResSources; ++n) {
    e[n] = 0.f;
    if (n >= a.nsrc) continue;
    e[n] = expf(sc[n] - mx);
    sum += e[n];
  }
  // pass 2: columns [16 CH wv, 16 CH (wv + 1)) of the weighted sum, CQ per lane
  const int cq = 16 * CH * wv + lane * CQ;
  float h[CQ];
#pragma unroll
  for (int i = 0; i < CQ; ++i) h[i] = 0.f;
#pragma unroll
  for (int n = 0; n < kMaxResSources; ++n) {
    if (n >= a.nsrc) continue;
    const float p = rt<T>(e[n] / sum);
    float x[CQ];
    load_slice<T, CQ>(static_cast<const T*>(a.src[n]) + row * a.ld[n] + cq, cq, a.N, vec, x);
#pragma unroll
    for (int i = 0; i < CQ; ++i) h[i] = h[i] + rt<T>(p * x[i]);
  }
#pragma unroll
  for (int i = 0; i < CQ; ++i) hrow[cq + i] = (cq + i < a.N) ? rt<T>(h[i]) : 0.f;
  __syncthreads();
  if (wv != 0) return;  // no barrier follows
  float hn[CH];
#pragma unroll
  for (int i = 0; i < CH; ++i) hn[i] = hrow[c0 + i];
  row_rms<CH, G>(hn, a.N);
  T* os = static_cast<T*>(a.out) + row * a.out_ld + c0;
  if (vec && c0 + CH <= a.N) {
    store_vec<T, CH>(os, hn);
  } else {
#pragma unroll
    for (int i = 0; i < CH; ++i)
      if (c0 + i < a.N) os[i] = from_f32<T>(hn[i]);
  }
}

// sigmoid as ATen evaluates it: 1 / (1 + exp(-x)) in fp32
__device__ __forceinline__ float sigmoid_f32(float x) {
#pragma clang fp contract(off)
  return 1.0f / (1.0f + expf(-x));
}

struct RowsArgs {
  const void* x;  // gate: y;  swiglu: interleaved input;  softcap: logits
  const void* g;  // gate: g
  void* out;
  int64_t x_ld, g_ld, out_ld, M;
  int N;          // output columns
  float p0, p1;   // swiglu: alpha, limit;  softcap: cap
  double d0, d1;  // the same in float64 (the float64 kernels)
};

template <typename T>
__global__ __launch_bounds__(256) void gate_kernel(const RowsArgs a) {
#pragma clang fp contract(off)
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= a.M * a.N) return;
  const int64_t r = idx / a.N;
  const int c = (int)(idx - r * a.N);
  const float y = to_f32(static_cast<const T*>(a.x)[r * a.x_ld + c]);
  const float s = rt<T>(sigmoid_f32(to_f32(static_cast<const T*>(a.g)[r * a.g_ld + c])));
  static_cast<T*>(a.out)[r * a.out_ld + c] = from_f32<T>(y * s);
}

template <typename T>
__global__ __launch_bounds__(256) void swiglu_kernel(const RowsArgs a) {
#pragma clang fp contract(off)
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= a.M * a.N) return;
  const int64_t r = idx / a.N;
  const int j = (int)(idx - r * a.N);
  const T* xr = static_cast<const T*>(a.x) + r * a.x_ld;
  const float alpha = a.p0, limit = a.p1;
  // clamp(max=limit) / clamp(-limit, limit) select existing values: exact
  const float gate = fminf(to_f32(xr[2 * j]), limit);
  const float lin = fminf(fmaxf(to_f32(xr[2 * j + 1]), -limit), limit);
  const float s = rt<T>(sigmoid_f32(rt<T>(alpha * gate)));
  const float gs = rt<T>(gate * s);
  const float l1 = rt<T>(lin + 1.0f);
  static_cast<T*>(a.out)[r * a.out_ld + j] = from_f32<T>(gs * l1);
}

template <typename T>
__global__ __launch_bounds__(256) void softcap_kernel(const RowsArgs a) {
#pragma clang fp contract(off)
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= a.M * a.N) return;
  const int64_t r = idx / a.N;
  const int c = (int)(idx - r * a.N);
  const float cap = a.p0;
  const float x = to_f32(static_cast<const T*>(a.x)[r * a.x_ld + c]);
  const float t = rt<T>(tanhf(rt<T>(x / cap)));
  static_cast<T*>(a.out)[r * a.out_ld + c] = from_f32<T>(cap * t);
}

// ---------------------------------------------------------------------------
// float64 rows (a GPT.double() model): the same ops in float64 arithmetic, as
// torch's float64 kernels evaluate them -- sigmoid 1 / (1 + exp(-x)), tanh,
// the RMSNorms with DBL_EPSILON, the source softmax with its maximum
// subtracted.  alpha, limit and cap are the ABI's float64 values.
// ---------------------------------------------------------------------------
__device__ __forceinline__ double sigmoid_f64(double x) { return 1.0 / (1.0 + exp(-x)); }

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// rms_norm(block_attn_res(V, w)) for one row per wave, two passes over the
// sources (C <= 2048, lane l holding columns l, l + 64, ...): the scores
// rms_norm(V_n) . w, their softmax over n, h = sum_n p_n V_n written out, then
// h's RMSNorm in place (each lane rescales the columns it wrote).
__global__ __launch_bounds__(256) void attn_res_norm_f64_kernel(const AttnResArgs a) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.M) return;  // whole waves leave; no barriers follow
  const double* w = static_cast<const double*>(a.w);
  double score[kMaxResSources];
  double mx = -__builtin_huge_val();
  for (int n = 0; n < a.nsrc; ++n) {
    const double* x = static_cast<const double*>(a.src[n]) + row * a.ld[n];
    double ss = 0.0;
    for (int c = lane; c < a.N; c += 64) ss += x[c] * x[c];
    const double r = 1.0 / sqrt(wave_sum_f64(ss) / (double)a.N + DBL_EPSILON);
    double dot = 0.0;
    for (int c = lane; c < a.N; c += 64) dot += (x[c] * r) * w[c];
    score[n] = wave_sum_f64(dot);
    mx = fmax(mx, score[n]);
  }
  double sum = 0.0;
  for (int n = 0; n < a.nsrc; ++n) {
    score[n] = exp(score[n] - mx);
    sum += score[n];
  }
  double* o = static_cast<double*>(a.out) + row * a.out_ld;
  double ss = 0.0;
  for (int c = lane; c < a.N; c += 64) {
    double h = 0.0;
    for (int n = 0; n < a.nsrc; ++n) h += (score[n] / sum) * static_cast<const double*>(a.src[n])[row * a.ld[n] + c];
    o[c] = h;
    ss += h * h;
  }
  const double r = 1.0 / sqrt(wave_sum_f64(ss) / (double)a.N + DBL_EPSILON);
  for (int c = lane; c < a.N; c += 64) o[c] = o[c] * r;
}

__global__ __launch_bounds__(256) void gate_kernel_f64(const RowsArgs a) {
#pragma clang fp contract(off)
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= a.M * a.N) return;
  const int64_t r = idx / a.N;
  const int c = (int)(idx - r * a.N);
  const double y = static_cast<const double*>(a.x)[r * a.x_ld + c];
  const double s = sigmoid_f64(static_cast<const double*>(a.g)[r * a.g_ld + c]);
  static_cast<double*>(a.out)[r * a.out_ld + c] = y * s;
}

__global__ __launch_bounds__(256) void swiglu_kernel_f64(const RowsArgs a) {
#pragma clang fp contract(off)
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= a.M * a.N) return;
  const int64_t r = idx / a.N;
  const int j = (int)(idx - r * a.N);
  const double* xr = static_cast<const double*>(a.x) + r * a.x_ld;
  const double alpha = a.d0, limit = a.d1;
  const double gate = fmin(xr[2 * j], limit);
  const double lin = fmin(fmax(xr[2 * j + 1], -limit), limit);
  const double s = sigmoid_f64(alpha * gate);
  static_cast<double*>(a.out)[r * a.out_ld + j] = (gate * s) * (lin + 1.0);
}

__global__ __launch_bounds__(256) void softcap_kernel_f64(const RowsArgs a) {
#pragma clang fp contract(off)
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= a.M * a.N) return;
  const int64_t r = idx / a.N;
  const int c = (int)(idx - r * a.N);
  const double cap = a.d0;
  const double x = static_cast<const double*>(a.x)[r * a.x_ld + c];
  static_cast<double*>(a.out)[r * a.out_ld + c] = cap * tanh(x / cap);
}

namespace {

bool al(const void* p, int64_t bytes) { return (reinterpret_cast<uintptr_t>(p) % (uintptr_t)bytes) == 0; }

int pow2_at_least(int x) {
  int p = 1;
  while (p < x) p <<= 1;
  return p;
}

// rows up to which wide rows (G = 64) take attn_res_norm_split_kernel
constexpr int64_t kResSplitRows = 4096;

template <typename T, int NPAD>
int launch_res(const AttnResArgs& a, hipStream_t s) {
  // the lane mapping of rms_norm_kernel for the same row length
  constexpr int PREF = 16 / (int)sizeof(T);
  constexpr int CH0 = NPAD / 64 > PREF ? NPAD / 64 : PREF;
  constexpr int CH = CH0 < NPAD ? CH0 : NPAD;
  constexpr int G = NPAD / CH;
  constexpr int RPB = 256 / G;
  const int64_t blocks = (a.M + RPB - 1) / RPB;
  DG_REQUIRE(blocks <= 0x7fffffffLL, DG_EINVAL, "attn_res_norm: too many rows (%lld)", (long long)a.M);
  const int64_t vb = (int64_t)CH * (int64_t)sizeof(T);
  bool vec = (vb == 4 || vb == 8 || vb % 16 == 0) && (CH * (int)sizeof(T)) >= 4 && al(a.w, vb) &&
             al(a.out, vb) && (a.out_ld * (int64_t)sizeof(T)) % vb == 0;
  for (int n = 0; n < a.nsrc; ++n) vec = vec && al(a.src[n], vb) && (a.ld[n] * (int64_t)sizeof(T)) % vb == 0;
  if constexpr (G == 64 && CH % 4 == 0) {
    // few wide rows (a decode step's): one row per workgroup of four waves
    if (a.M <= kResSplitRows) {
      hipLaunchKernelGGL((attn_res_norm_split_kernel<T, NPAD, CH>), dim3((unsigned)a.M), dim3(256), 0, s, a,
                         vec ? 1 : 0);
      return check_launch("attn_res_norm_split_kernel");
    }
  }
  hipLaunchKernelGGL((attn_res_norm_kernel<T, NPAD, CH>), dim3((unsigned)blocks), dim3(256), 0, s, a,
                     vec ? 1 : 0);
  return check_launch("attn_res_norm_kernel");
}

template <typename T>
int res_pick(int npad, const AttnResArgs& a, hipStream_t s) {
  switch (npad) {
    case 1:
    case 2: return launch_res<T, 2>(a, s);
    case 4: return launch_res<T, 4>(a, s);
    case 8: return launch_res<T, 8>(a, s);
    case 16: return launch_res<T, 16>(a, s);
    case 32: return launch_res<T, 32>(a, s);
    case 64: return launch_res<T, 64>(a, s);
    case 128: return launch_res<T, 128>(a, s);
    case 256: return launch_res<T, 256>(a, s);
    case 512: return launch_res<T, 512>(a, s);
    case 1024: return launch_res<T, 1024>(a, s);
    case 2048: return launch_res<T, 2048>(a, s);
  }
  set_error("attn_res_norm: C=%d unsupported (max 2048)", a.N);
  return DG_EUNSUPPORTED;
}

}  // namespace

// ---------------------------------------------------------------------------
// A layer's work after its attention, in one launch (mha.py:84-85,
// block.py:98-106, feed_forward.py:10-14):
//
//   block_out_kernel  a = y * sigmoid(g); attn_out = a @ W_proj^T; the
//                     partial sum (attn_out, or partial_in + attn_out inside
//                     a block); the MLP's mixture over the committed blocks
//                     and that partial, its norm; the FFN (C -> 4C, clamped
//                     SwiGLU, 2C -> C); and the residual
//
// A workgroup of 4 waves takes 16 token rows.  The stages meet in LDS (rows
// padded by 16 bytes, so the 16 rows of a matrix-core operand read fall on
// different banks); every GEMM is a sequence of 16 x 16 output tiles on the
// matrix cores (qk_mfma's lane mapping: lane (c, g) feeds weight row
// 16t + c and token row c with the contiguous quarter g of the contraction,
// and gets back token row c's outputs 16t + 4g .. 16t + 4g + 3), the tiles of a
// stage dealt round-robin to the 4 waves, each wave's weight fragments
// fetched a stage or a tile ahead.  Every intermediate is rounded to T where
// the torch sequence rounds it -- the gate as gate_kernel, each GEMM's fp32
// sum once, the mixture as attn_res_norm_kernel, the SwiGLU as swiglu_kernel,
// the residual adds -- so bf16 follows the same rounding steps; only the
// GEMMs' summation order differs from hipBLASLt's.  C is 64 or 128.
// (The same fusion before the attention -- the mixture, its norm and the
// q/k/v/g projection in one launch -- measured no faster than the two
// launches at 6400 rows and slower beyond: the mixture's dependent chain at
// the occupancy its registers allow costs what the saved launch gains.)
// ---------------------------------------------------------------------------
constexpr int kLayerRows = 16;

struct BlockOutArgs {
  const void* y;        // (M, C) attention output (before the gate)
  const void* g;        // (M, C) gate logits
  const void* w_proj;   // (C, C)
  const void* pin;      // (M, C) partial sum entering the layer; null when the layer commits it
  const void* blk[kMaxResSources];  // committed blocks (the MLP mixture's first sources)
  int64_t blk_ld[kMaxResSources];
  const void* w_mix;    // (C,)
  const void* w_up;     // (4C, C)
  const void* w_down;   // (C, 2C)
  void* out;            // (M, C) partial sum leaving the layer
  void* xn;             // (M, C) rms_norm(out) as stored, or null
  int64_t y_ld, g_ld, wp_ld, pin_ld, wu_ld, wd_ld, out_ld, xn_ld, M;
  int nblk;
  float alpha, limit;
};

// LDS row stride (elements) of a K-wide operand matrix: 16 bytes of padding
template <typename T, int K>
constexpr int lds_ld() {
  return K + 16 / (int)sizeof(T);
}

// A lane's weight fragment of one 16 x 16 output tile over a K-long
// contraction: weight row 16t + c (c = lane & 15), the contiguous quarter
// g = lane >> 4 of the contraction, in chunks of 16 elements.  Loaded apart
// from the product so that a wave can fetch it before the stage that
// produces the tile's other operand, or one tile ahead.
template <typename T, int K>
struct TileW {
  static constexpr int CQ = K / 4;  // contraction elements of a lane's quarter
  static constexpr int KCH = 16;
  static_assert(CQ % KCH == 0, "contraction chunking");
  RowRegs<T, KCH> r[CQ / KCH];
};

template <typename T, int K>
__device__ __forceinline__ void load_tile_w(TileW<T, K>& f, const T* __restrict__ w, int64_t w_ld, int t, int lane) {
  const int c = lane & 15, g = lane >> 4;
  const T* wr = w + (int64_t)(16 * t + c) * w_ld + g * TileW<T, K>::CQ;
#pragma unroll
  for (int i = 0; i < TileW<T, K>::CQ / 16; ++i) load_row<T, 16>(f.r[i], wr + 16 * i);
}

// The tile's product against the token rows of the LDS matrix x.
template <typename T, int K>
__device__ __forceinline__ f32x4_t layer_tile(const TileW<T, K>& f, const T* x, int lane) {
  constexpr int CQ = TileW<T, K>::CQ;
  const int c = lane & 15, g = lane >> 4;
  const T* xr = x + c * lds_ld<T, K>() + g * CQ;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < CQ / 16; ++i) {
    RowRegs<T, 16> xo;
    load_row<T, 16>(xo, xr + 16 * i);
    acc = qk_mfma<T, 16>(f.r[i], xo, acc);
  }
  return acc;
}

// rms_norm(block_attn_res(V, w)) of the 16 rows into LDS xn, with
// attn_res_norm_kernel's arithmetic; 16 lanes per row (CH = C / 16 elements
// each).  Sources 0 .. nmem-1 are rows of global tensors; with last != null
// the last source is that LDS matrix.  The caller has loaded the first
// res_held<CH>() global sources (held) and the lane's slice of the
// pseudo-query (w) into registers at the start of the kernel; they serve both
// passes, further global sources and the LDS one are read where used.
template <typename T, int C>
__device__ __forceinline__ void layer_mixture(const void* const* src, const int64_t* ld, int nmem, const T* last,
                                              const float (&held)[res_held<C / 16>()][C / 16],
                                              const float (&w)[C / 16], int64_t row0, int64_t M, T* xn) {
#pragma clang fp contract(off)
  constexpr int CH = C / 16;
  constexpr int G = 16;
  constexpr int HELD = res_held<CH>();
  const int r = threadIdx.x / G, sub = threadIdx.x % G, c0 = sub * CH;
  const int64_t row = min(row0 + r, M - 1);  // rows past M: a finite copy, never stored
  const int nsrc = nmem + (last != nullptr ? 1 : 0);
  auto get = [&](int n, float (&x)[CH]) __attribute__((always_inline)) {
    if (n < HELD && n < nmem) {
#pragma unroll
      for (int i = 0; i < CH; ++i) x[i] = held[n][i];
    } else if (n < nmem) {
      load_vec<T, CH>(static_cast<const T*>(src[n]) + row * ld[n] + c0, x);
    } else {
      load_vec<T, CH>(last + r * lds_ld<T, C>() + c0, x);
    }
  };
  float score[kMaxResSources];
  float mx = -INFINITY;
#pragma unroll
  for (int n = 0; n < kMaxResSources; ++n) {
    score[n] = -INFINITY;
    if (n >= nsrc) continue;  // uniform
    float x[CH];
    get(n, x);
    row_rms<CH, G>(x, C);
    float prod[CH];
#pragma unroll
    for (int i = 0; i < CH; ++i) prod[i] = rt<T>(x[i]) * w[i];
    float dot = tree_sum<CH>(prod);
    dot = group_sum_dpp<G>(dot);
    score[n] = rt<T>(dot);
    mx = fmaxf(mx, score[n]);
  }
  float e[kMaxResSources];
  float sum = 0.f;
#pragma unroll
  for (int n = 0; n < kMaxResSources; ++n) {
    e[n] = 0.f;
    if (n >= nsrc) continue;
    e[n] = expf(score[n] - mx);
    sum += e[n];
  }
  float h[CH];
#pragma unroll
  for (int i = 0; i < CH; ++i) h[i] = 0.f;
#pragma unroll
  for (int n = 0; n < kMaxResSources; ++n) {
    if (n >= nsrc) continue;
    const float p = rt<T>(e[n] / sum);
    float x[CH];
    get(n, x);
#pragma unroll
    for (int i = 0; i < CH; ++i) h[i] = h[i] + rt<T>(p * x[i]);
  }
#pragma unroll
  for (int i = 0; i < CH; ++i) h[i] = rt<T>(h[i]);
  row_rms<CH, G>(h, C);
  store_vec<T, CH>(xn + r * lds_ld<T, C>() + c0, h);
}

// FFN weight fragments loaded at the start of block_out_kernel: at C = 64 in
// 16-bit types all of a wave's up and down tiles (72 registers); otherwise
// the first up tile, each later one fetched while the one before runs, and
// the down tiles behind the last up tile (fp32 fragments are twice the
// registers, and loading all of them up front measured slower).
template <typename T, int C>
constexpr int block_up_depth() {
  return (C == 64 && sizeof(T) == 2) ? C / 16 : 1;
}

template <typename T, int C>
__global__ __launch_bounds__(256) void block_out_kernel(const BlockOutArgs a) {
#pragma clang fp contract(off)
  constexpr int LDC = lds_ld<T, C>(), LDH = lds_ld<T, 2 * C>();
  constexpr int CH = C / 16;
  constexpr int NPJ = C / 64;  // c_proj tiles per wave (C / 16 tiles over 4 waves)
  constexpr int NUP = C / 16;  // FFN-up tiles per wave (4C / 16 over 4 waves)
  constexpr int NDN = C / 64;  // FFN-down tiles per wave
  constexpr int UPD = block_up_depth<T, C>();
  constexpr bool kDownAtStart = UPD == NUP;  // else the down fragments follow the up tiles
  constexpr int NDP = kDownAtStart ? NDN : 1;
  constexpr int HELD = res_held<CH>();
  __shared__ __attribute__((aligned(16))) T ga[kLayerRows * LDC];  // gated attention output, then xn
  __shared__ __attribute__((aligned(16))) T pm[kLayerRows * LDC];  // the partial sum after the attention
  __shared__ __attribute__((aligned(16))) T hh[kLayerRows * LDH];  // SwiGLU output
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 15, g = lane >> 4;
  const int64_t row0 = (int64_t)blockIdx.x * kLayerRows;
  const T* w_proj = static_cast<const T*>(a.w_proj);
  const T* w_up = static_cast<const T*>(a.w_up);
  const T* w_down = static_cast<const T*>(a.w_down);

  // Every global operand of the wave goes out here, in the order the stages
  // use them, so that the stages wait on LDS and the matrix cores instead of
  // one memory round trip each: the gate's rows (16 lanes per row), the
  // c_proj fragments and the partial sum entering the layer (matrix-core
  // lane mapping), the mixture's committed blocks and pseudo-query (16 lanes
  // per row), the FFN fragments.
  const int gr = threadIdx.x / 16, gc0 = (threadIdx.x % 16) * CH;
  const int64_t grow = min(row0 + gr, a.M - 1);  // rows past M: a finite copy, never stored
  const int64_t crow = min(row0 + c, a.M - 1);
  float y[CH], gl[CH];
  load_vec<T, CH>(static_cast<const T*>(a.y) + grow * a.y_ld + gc0, y);
  load_vec<T, CH>(static_cast<const T*>(a.g) + grow * a.g_ld + gc0, gl);
  TileW<T, C> wp[NPJ];
#pragma unroll
  for (int j = 0; j < NPJ; ++j) load_tile_w<T, C>(wp[j], w_proj, a.wp_ld, wv + 4 * j, lane);
  float pin[NPJ][4];
  if (a.pin != nullptr) {  // uniform
#pragma unroll
    for (int j = 0; j < NPJ; ++j)
      load_vec<T, 4>(static_cast<const T*>(a.pin) + crow * a.pin_ld + 16 * (wv + 4 * j) + 4 * g, pin[j]);
  }
  float held[HELD][CH];
#pragma unroll
  for (int n = 0; n < HELD; ++n)
    if (n < a.nblk) load_vec<T, CH>(static_cast<const T*>(a.blk[n]) + grow * a.blk_ld[n] + gc0, held[n]);  // uniform
  float wmix[CH];
  load_vec<T, CH>(static_cast<const T*>(a.w_mix) + gc0, wmix);
  TileW<T, C> wu[UPD];
#pragma unroll
  for (int j = 0; j < UPD; ++j) load_tile_w<T, C>(wu[j], w_up, a.wu_ld, wv + 4 * j, lane);
  TileW<T, 2 * C> wd[NDP];
  if constexpr (kDownAtStart) {
#pragma unroll
    for (int j = 0; j < NDN; ++j) load_tile_w<T, 2 * C>(wd[j], w_down, a.wd_ld, wv + 4 * j, lane);
  }
  // keep the scheduler from sinking the loads toward their uses
  __builtin_amdgcn_sched_barrier(0);

  // 1) gate (gate_kernel's arithmetic)
#pragma unroll
  for (int i = 0; i < CH; ++i) y[i] = y[i] * rt<T>(sigmoid_f32(gl[i]));
  store_vec<T, CH>(ga + gr * LDC + gc0, y);
  __syncthreads();
  // 2) c_proj, then the partial sum
#pragma unroll
  for (int j = 0; j < NPJ; ++j) {
    const f32x4_t acc = layer_tile<T, C>(wp[j], ga, lane);
    const int f = 16 * (wv + 4 * j) + 4 * g;
    float p[4];
    if (a.pin != nullptr) {
#pragma unroll
      for (int i = 0; i < 4; ++i) p[i] = pin[j][i] + rt<T>(acc[i]);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) p[i] = acc[i];
    }
    store_vec<T, 4>(pm + c * LDC + f, p);
  }
  __syncthreads();
  // 3) the MLP's mixture over the committed blocks and the new partial; its
  //    norm overwrites the gated rows (no longer read)
  layer_mixture<T, C>(a.blk, a.blk_ld, a.nblk, pm, held, wmix, row0, a.M, ga);
  __syncthreads();
  // 4) FFN up + SwiGLU (swiglu_kernel's arithmetic on the interleaved
  //    (gate, linear) pairs: features 2j, 2j + 1 -> hidden j)
#pragma unroll
  for (int i = 0; i < NUP; ++i) {
    const int t = wv + 4 * i;
    TileW<T, C> next;
    if (i + UPD < NUP) load_tile_w<T, C>(next, w_up, a.wu_ld, t + 4 * UPD, lane);
    if constexpr (!kDownAtStart) {
      if (i + 1 == NUP) load_tile_w<T, 2 * C>(wd[0], w_down, a.wd_ld, wv, lane);
    }
    const f32x4_t acc = layer_tile<T, C>(wu[i % UPD], ga, lane);
    if (i + UPD < NUP) wu[i % UPD] = next;
    float hv[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const float gate = fminf(rt<T>(acc[2 * q]), a.limit);
      const float lin = fminf(fmaxf(rt<T>(acc[2 * q + 1]), -a.limit), a.limit);
      const float s = rt<T>(sigmoid_f32(rt<T>(a.alpha * gate)));
      hv[q] = rt<T>(gate * s) * rt<T>(lin + 1.0f);
    }
    store_vec<T, 2>(hh + c * LDH + 8 * t + 2 * g, hv);
  }
  __syncthreads();
  // 5) FFN down + residual
  const bool store = row0 + c < a.M;
  T* orow = static_cast<T*>(a.out) + (row0 + c) * a.out_ld;
#pragma unroll
  for (int j = 0; j < NDN; ++j) {
    const int t = wv + 4 * j;
    TileW<T, 2 * C> next;
    if constexpr (!kDownAtStart) {
      if (j + 1 < NDN) load_tile_w<T, 2 * C>(next, w_down, a.wd_ld, t + 4, lane);
    }
    const f32x4_t acc = layer_tile<T, 2 * C>(wd[kDownAtStart ? j : 0], hh, lane);
    if constexpr (!kDownAtStart) {
      if (j + 1 < NDN) wd[0] = next;
    }
    const int f = 16 * t + 4 * g;
    float pmv[4], o[4];
    load_vec<T, 4>(pm + c * LDC + f, pmv);
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = pmv[i] + rt<T>(acc[i]);
    if (store) store_vec<T, 4>(orow + f, o);
    // the same lane alone reads and writes this slice of pm
    if (a.xn != nullptr) store_vec<T, 4>(pm + c * LDC + f, o);  // uniform
  }
  // 6) dg_block_out_norm: the RMSNorm of the stored output rows (the head's
  //    input after the last layer), 16 lanes per row
  if (a.xn != nullptr) {  // uniform
    __syncthreads();
    float x[CH];
    load_vec<T, CH>(pm + gr * LDC + gc0, x);
    row_rms<CH, 16>(x, C);
    if (row0 + gr < a.M) store_vec<T, CH>(static_cast<T*>(a.xn) + (row0 + gr) * a.xn_ld + gc0, x);
  }
}

// ---------------------------------------------------------------------------
// lm_head + softcap + greedy argmax.  Block = 4 waves = 16 rows of x; wave w
// takes the vocabulary entries [w V/4, (w+1) V/4) in NTW tiles of 16.  Per
// tile, logits^T (16 entries x 16 rows) = W_tile x^T on the matrix cores with
// qk_mfma's lane mapping: lane (c, g) feeds embedding row 16t + c and x row c,
// each with the contiguous quarter g of the contraction (chunks of 16
// elements), and gets back row c's logits for entries 16t + 4g .. 16t + 4g + 3.
// The logit is rounded to T (F.linear's output), then capped with
// softcap_kernel's arithmetic and rounding, stored, and compared: the first
// maximum wins (torch.argmax), across the lane's values in entry order, the
// four lanes of a row, then the four waves through LDS.
// ---------------------------------------------------------------------------
struct LmHeadArgs {
  const void* x;  // (M, C) rows, already normalised (gpt.py:181 rms_norm)
  const void* w;  // (V, C) tied embedding table
  void* logits;   // (M, V)
  int64_t* ids;   // (M,) or null
  int64_t x_ld, w_ld, l_ld, M;
  int C, V;
  float cap;  // 0: no softcap
};

template <typename T, int NTW>
__global__ __launch_bounds__(256) void lm_head_kernel(const LmHeadArgs a) {
#pragma clang fp contract(off)
  constexpr int KCH = 16;  // contraction elements per lane and chunk
  __shared__ float red_v[4][16];
  __shared__ int red_i[4][16];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 15, g = lane >> 4;
  const int64_t row0 = (int64_t)blockIdx.x * 16;
  const bool row_ok = row0 + c < a.M;
  const int64_t row = row_ok ? row0 + c : a.M - 1;
  const int cq = a.C / 4;  // this lane's quarter of the contraction
  const int vbase = w * (a.V / 4);
  const T* xr = static_cast<const T*>(a.x) + row * a.x_ld + g * cq;
  const T* wr = static_cast<const T*>(a.w) + (int64_t)(vbase + c) * a.w_ld + g * cq;

  f32x4_t acc[NTW];
#pragma unroll
  for (int t = 0; t < NTW; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < cq; k0 += KCH) {
    RowRegs<T, KCH> xo;
    load_row<T, KCH>(xo, xr + k0);
#pragma unroll
    for (int t = 0; t < NTW; ++t) {
      RowRegs<T, KCH> wo;
      load_row<T, KCH>(wo, wr + (int64_t)16 * t * a.w_ld + k0);
      acc[t] = qk_mfma<T, KCH>(wo, xo, acc[t]);
    }
  }

  float best = kNegInf;
  int bidx = 0x7fffffff;
  T* lrow = static_cast<T*>(a.logits) + row * a.l_ld + vbase + 4 * g;
#pragma unroll
  for (int t = 0; t < NTW; ++t) {
    float out[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v = rt<T>(acc[t][r]);
      if (a.cap > 0.f) v = rt<T>(a.cap * rt<T>(tanhf(rt<T>(v / a.cap))));
      out[r] = v;
      const int e = vbase + 16 * t + 4 * g + r;  // increasing within the lane
      if (v > best) {
        best = v;
        bidx = e;
      }
    }
    if (row_ok) store_vec<T, 4>(lrow + 16 * t, out);
  }
  if (a.ids == nullptr) return;  // uniform over the grid
  // the row's four lanes: larger value, or equal value and smaller entry
#pragma unroll
  for (int off = 16; off <= 32; off <<= 1) {
    const float ov = __shfl_xor(best, off, 64);
    const int oi = __shfl_xor(bidx, off, 64);
    if (ov > best || (ov == best && oi < bidx)) {
      best = ov;
      bidx = oi;
    }
  }
  if (g == 0) {
    red_v[w][c] = best;
    red_i[w][c] = bidx;
  }
  __syncthreads();
  if (w != 0 || g != 0 || !row_ok) return;
  // waves in entry order: a strictly larger value replaces the earlier one
  float bv = red_v[0][c];
  int bi = red_i[0][c];
#pragma unroll
  for (int q = 1; q < 4; ++q) {
    if (red_v[q][c] > bv) {
      bv = red_v[q][c];
      bi = red_i[q][c];
    }
  }
  a.ids[row0 + c] = (int64_t)(bi == 0x7fffffff ? 0 : bi);
}

namespace {

template <typename T>
int launch_lm_head(const LmHeadArgs& a, hipStream_t s) {
  const int ntw = a.V / 64;
  const unsigned blocks = (unsigned)((a.M + 15) / 16);
  switch (ntw) {
    case 1: hipLaunchKernelGGL((lm_head_kernel<T, 1>), dim3(blocks), dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL((lm_head_kernel<T, 2>), dim3(blocks), dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL((lm_head_kernel<T, 4>), dim3(blocks), dim3(256), 0, s, a); break;
    case 8: hipLaunchKernelGGL((lm_head_kernel<T, 8>), dim3(blocks), dim3(256), 0, s, a); break;
    case 16: hipLaunchKernelGGL((lm_head_kernel<T, 16>), dim3(blocks), dim3(256), 0, s, a); break;
    default:
      set_error("lm_head: vocabulary %d unsupported (64, 128, 256, 512 or 1024)", a.V);
      return DG_EUNSUPPORTED;
  }
  return check_launch("lm_head_kernel");
}

// one thread per output element; K<T> for the dtype
#define DG_LAUNCH_ROWS(K, dtype, a, s)                                                        \
  do {                                                                                        \
    const int64_t n_ = (a).M * (int64_t)(a).N;                                                \
    if (n_ == 0) return DG_OK;                                                                \
    const int64_t blocks_ = (n_ + 255) / 256;                                                 \
    DG_REQUIRE(blocks_ <= 0x7fffffffLL, DG_EINVAL, #K ": too many elements (%lld)", (long long)n_); \
    if ((dtype) == DG_F64)                                                                    \
      hipLaunchKernelGGL(K##_f64, dim3((unsigned)blocks_), dim3(256), 0, (s), (a));           \
    else if ((dtype) == DG_F32)                                                               \
      hipLaunchKernelGGL(K<float>, dim3((unsigned)blocks_), dim3(256), 0, (s), (a));          \
    else if ((dtype) == DG_BF16)                                                              \
      hipLaunchKernelGGL(K<bf16_t>, dim3((unsigned)blocks_), dim3(256), 0, (s), (a));         \
    else                                                                                      \
      hipLaunchKernelGGL(K<f16_t>, dim3((unsigned)blocks_), dim3(256), 0, (s), (a));          \
    return check_launch(#K);                                                                  \
  } while (0)

bool dtype_ok(int dtype) { return dtype == DG_F32 || dtype == DG_BF16 || dtype == DG_F16; }
// the row kernels with float64 forms (dg_attn_res_norm, dg_gate, dg_swiglu, dg_softcap)
bool dtype_ok_f64(int dtype) { return dtype_ok(dtype) || dtype == DG_F64; }

}  // namespace
}  // namespace dg

using namespace dg;

extern "C" int dg_attn_res_norm(int64_t M, int C, int dtype, int nsrc, const void* const* src,
                                const int64_t* src_ld, const void* w, void* out, int64_t out_ld,
                                void* stream) {
  DG_REQUIRE(M >= 0 && C >= 1, DG_EINVAL, "attn_res_norm: bad sizes M=%lld C=%d", (long long)M, C);
  DG_REQUIRE(C <= 2048, DG_EUNSUPPORTED, "attn_res_norm: C=%d > 2048", C);
  DG_REQUIRE(dtype_ok_f64(dtype), DG_EUNSUPPORTED, "attn_res_norm: dtype %d unsupported", dtype);
  DG_REQUIRE(nsrc >= 1 && nsrc <= kMaxResSources, DG_EINVAL, "attn_res_norm: %d sources (1..%d)", nsrc,
             kMaxResSources);
  if (M == 0) return DG_OK;
  DG_REQUIRE(src != nullptr && src_ld != nullptr && w != nullptr && out != nullptr, DG_EINVAL,
             "attn_res_norm: NULL pointer");
  DG_REQUIRE(out_ld >= C, DG_EINVAL, "attn_res_norm: output row stride smaller than C");
  AttnResArgs a{};
  for (int n = 0; n < nsrc; ++n) {
    DG_REQUIRE(src[n] != nullptr && src_ld[n] >= C, DG_EINVAL,
               "attn_res_norm: source %d is NULL or its row stride is smaller than C", n);
    a.src[n] = src[n];
    a.ld[n] = src_ld[n];
  }
  a.w = w;
  a.out = out;
  a.out_ld = out_ld;
  a.M = M;
  a.nsrc = nsrc;
  a.N = C;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == DG_F64) {
    DG_REQUIRE((M + 3) / 4 <= 0x7fffffffLL, DG_EINVAL, "attn_res_norm: too many rows (%lld)", (long long)M);
    hipLaunchKernelGGL(attn_res_norm_f64_kernel, dim3((unsigned)((M + 3) / 4)), dim3(256), 0, s, a);
    return check_launch("attn_res_norm_f64_kernel");
  }
  const int npad = pow2_at_least(C);
  if (dtype == DG_F32) return res_pick<float>(npad, a, s);
  if (dtype == DG_BF16) return res_pick<bf16_t>(npad, a, s);
  return res_pick<f16_t>(npad, a, s);
}

extern "C" int dg_gate(int64_t M, int C, int dtype, const void* y, int64_t y_ld, const void* g,
                       int64_t g_ld, void* out, int64_t out_ld, void* stream) {
  DG_REQUIRE(M >= 0 && C >= 1, DG_EINVAL, "gate: bad sizes M=%lld C=%d", (long long)M, C);
  DG_REQUIRE(dtype_ok_f64(dtype), DG_EUNSUPPORTED, "gate: dtype %d unsupported", dtype);
  if (M == 0) return DG_OK;
  DG_REQUIRE(y != nullptr && g != nullptr && out != nullptr, DG_EINVAL, "gate: NULL pointer");
  DG_REQUIRE(y_ld >= C && g_ld >= C && out_ld >= C, DG_EINVAL, "gate: row stride smaller than C");
  RowsArgs a{};
  a.x = y; a.g = g; a.out = out;
  a.x_ld = y_ld; a.g_ld = g_ld; a.out_ld = out_ld; a.M = M; a.N = C;
  DG_LAUNCH_ROWS(gate_kernel, dtype, a, static_cast<hipStream_t>(stream));
}

extern "C" int dg_swiglu(int64_t M, int N, int dtype, const void* x, int64_t x_ld, void* out,
                         int64_t out_ld, double alpha, double limit, void* stream) {
  DG_REQUIRE(M >= 0 && N >= 1, DG_EINVAL, "swiglu: bad sizes M=%lld N=%d", (long long)M, N);
  DG_REQUIRE(dtype_ok_f64(dtype), DG_EUNSUPPORTED, "swiglu: dtype %d unsupported", dtype);
  if (M == 0) return DG_OK;
  DG_REQUIRE(x != nullptr && out != nullptr, DG_EINVAL, "swiglu: NULL pointer");
  DG_REQUIRE(x_ld >= 2 * (int64_t)N && out_ld >= N, DG_EINVAL, "swiglu: row stride too small");
  RowsArgs a{};
  a.x = x; a.out = out;
  a.x_ld = x_ld; a.out_ld = out_ld; a.M = M; a.N = N;
  a.p0 = (float)alpha; a.p1 = (float)limit;
  a.d0 = alpha; a.d1 = limit;
  DG_LAUNCH_ROWS(swiglu_kernel, dtype, a, static_cast<hipStream_t>(stream));
}

extern "C" int dg_softcap(int64_t M, int N, int dtype, const void* x, int64_t x_ld, void* out,
                          int64_t out_ld, double cap, void* stream) {
  DG_REQUIRE(M >= 0 && N >= 1, DG_EINVAL, "softcap: bad sizes M=%lld N=%d", (long long)M, N);
  DG_REQUIRE(dtype_ok_f64(dtype), DG_EUNSUPPORTED, "softcap: dtype %d unsupported", dtype);
  DG_REQUIRE(cap > 0.0, DG_EINVAL, "softcap: cap must be positive (got %g)", cap);
  if (M == 0) return DG_OK;
  DG_REQUIRE(x != nullptr && out != nullptr, DG_EINVAL, "softcap: NULL pointer");
  DG_REQUIRE(x_ld >= N && out_ld >= N, DG_EINVAL, "softcap: row stride smaller than N");
  RowsArgs a{};
  a.x = x; a.out = out;
  a.x_ld = x_ld; a.out_ld = out_ld; a.M = M; a.N = N;
  a.p0 = (float)cap;
  a.d0 = cap;
  DG_LAUNCH_ROWS(softcap_kernel, dtype, a, static_cast<hipStream_t>(stream));
}

extern "C" int dg_lm_head(int64_t M, int C, int V, int dtype, const void* x, int64_t x_ld, const void* w,
                          int64_t w_ld, float cap, void* logits, int64_t logits_ld, int64_t* ids, void* stream) {
  DG_REQUIRE(M >= 0 && C >= 1 && V >= 1, DG_EINVAL, "lm_head: bad sizes M=%lld C=%d V=%d", (long long)M, C, V);
  DG_REQUIRE(dtype_ok(dtype), DG_EUNSUPPORTED, "lm_head: dtype %d unsupported", dtype);
  DG_REQUIRE(cap >= 0.f, DG_EINVAL, "lm_head: cap must be >= 0 (got %g)", (double)cap);
  DG_REQUIRE(C % 64 == 0 && C <= 8192, DG_EUNSUPPORTED, "lm_head: n_embd %d unsupported (a multiple of 64)", C);
  DG_REQUIRE(V == 64 || V == 128 || V == 256 || V == 512 || V == 1024, DG_EUNSUPPORTED,
             "lm_head: vocabulary %d unsupported (64, 128, 256, 512 or 1024)", V);
  if (M == 0) return DG_OK;
  DG_REQUIRE(M <= (int64_t)16 * 0x7fffffffLL, DG_EINVAL, "lm_head: too many rows (%lld)", (long long)M);
  DG_REQUIRE(x != nullptr && w != nullptr && logits != nullptr, DG_EINVAL, "lm_head: NULL pointer");
  DG_REQUIRE(x_ld >= C && w_ld >= C && logits_ld >= V, DG_EINVAL, "lm_head: row stride smaller than the row");
  const int64_t es = dtype == DG_F32 ? 4 : 2;
  auto al = [](const void* p, int64_t n) { return (reinterpret_cast<uintptr_t>(p) % (uintptr_t)n) == 0; };
  DG_REQUIRE(al(x, 16) && al(w, 16) && al(logits, 4 * es) && (x_ld * es) % 16 == 0 && (w_ld * es) % 16 == 0 &&
                 (logits_ld * es) % (4 * es) == 0,
             DG_EUNSUPPORTED, "lm_head: rows must be 16-byte aligned");
  LmHeadArgs a{};
  a.x = x; a.w = w; a.logits = logits; a.ids = ids;
  a.x_ld = x_ld; a.w_ld = w_ld; a.l_ld = logits_ld; a.M = M;
  a.C = C; a.V = V; a.cap = cap;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == DG_F32) return launch_lm_head<float>(a, s);
  if (dtype == DG_BF16) return launch_lm_head<bf16_t>(a, s);
  return launch_lm_head<f16_t>(a, s);
}

namespace {
bool rows16(const void* p, int64_t ld, int64_t es) {
  return (reinterpret_cast<uintptr_t>(p) & 15) == 0 && (ld * es) % 16 == 0;
}
}  // namespace

static int block_out_impl(int64_t M, int C, int dtype, const void* y, int64_t y_ld, const void* g, int64_t g_ld,
                          const void* w_proj, int64_t wp_ld, const void* partial_in, int64_t pin_ld, int nblk,
                          const void* const* blocks, const int64_t* blocks_ld, const void* w_mix, const void* w_up,
                          int64_t wu_ld, const void* w_down, int64_t wd_ld, float alpha, float limit, void* out,
                          int64_t out_ld, void* xn, int64_t xn_ld, void* stream) {
  DG_REQUIRE(M >= 0 && C >= 1, DG_EINVAL, "block_out: bad sizes M=%lld C=%d", (long long)M, C);
  DG_REQUIRE(dtype_ok(dtype), DG_EUNSUPPORTED, "block_out: dtype %d unsupported", dtype);
  DG_REQUIRE(C == 64 || C == 128, DG_EUNSUPPORTED, "block_out: n_embd %d unsupported (64 or 128)", C);
  DG_REQUIRE(nblk >= 0 && nblk + 1 <= kMaxResSources, DG_EINVAL, "block_out: %d blocks (0..%d)", nblk,
             kMaxResSources - 1);
  if (M == 0) return DG_OK;
  DG_REQUIRE(y && g && w_proj && w_mix && w_up && w_down && out && (nblk == 0 || (blocks && blocks_ld)), DG_EINVAL,
             "block_out: NULL pointer");
  DG_REQUIRE(M <= (int64_t)kLayerRows * 0x7fffffffLL, DG_EINVAL, "block_out: too many rows (%lld)", (long long)M);
  const int64_t es = dtype == DG_F32 ? 4 : 2;
  BlockOutArgs a{};
  bool ok = rows16(y, y_ld, es) && rows16(g, g_ld, es) && rows16(w_proj, wp_ld, es) && rows16(w_mix, 0, es) &&
            rows16(w_up, wu_ld, es) && rows16(w_down, wd_ld, es) && rows16(out, out_ld, es) &&
            (partial_in == nullptr || rows16(partial_in, pin_ld, es)) && (xn == nullptr || rows16(xn, xn_ld, es));
  DG_REQUIRE(y_ld >= C && g_ld >= C && wp_ld >= C && wu_ld >= C && wd_ld >= 2 * C && out_ld >= C &&
                 (partial_in == nullptr || pin_ld >= C) && (xn == nullptr || xn_ld >= C),
             DG_EINVAL, "block_out: a row stride is narrower than its row");
  for (int n = 0; n < nblk; ++n) {
    DG_REQUIRE(blocks[n] != nullptr && blocks_ld[n] >= C, DG_EINVAL, "block_out: block %d is NULL or narrower than C",
               n);
    ok = ok && rows16(blocks[n], blocks_ld[n], es);
    a.blk[n] = blocks[n];
    a.blk_ld[n] = blocks_ld[n];
  }
  DG_REQUIRE(ok, DG_EUNSUPPORTED, "block_out: rows must be 16-byte aligned");
  a.y = y; a.g = g; a.w_proj = w_proj; a.pin = partial_in; a.w_mix = w_mix; a.w_up = w_up; a.w_down = w_down;
  a.out = out; a.xn = xn;
  a.y_ld = y_ld; a.g_ld = g_ld; a.wp_ld = wp_ld; a.pin_ld = pin_ld; a.wu_ld = wu_ld; a.wd_ld = wd_ld;
  a.out_ld = out_ld; a.xn_ld = xn_ld; a.M = M; a.nblk = nblk; a.alpha = alpha; a.limit = limit;
  const dim3 grid((unsigned)((M + kLayerRows - 1) / kLayerRows));
  hipStream_t s = static_cast<hipStream_t>(stream);
#define DG_BLOCK_OUT(T)                                                                             \
  do {                                                                                            \
    if (C == 64) hipLaunchKernelGGL((block_out_kernel<T, 64>), grid, dim3(256), 0, s, a);         \
    else hipLaunchKernelGGL((block_out_kernel<T, 128>), grid, dim3(256), 0, s, a);                \
  } while (0)
  if (dtype == DG_F32) DG_BLOCK_OUT(float);
  else if (dtype == DG_BF16) DG_BLOCK_OUT(bf16_t);
  else DG_BLOCK_OUT(f16_t);
#undef DG_BLOCK_OUT
  return check_launch("block_out_kernel");
}

extern "C" int dg_block_out(int64_t M, int C, int dtype, const void* y, int64_t y_ld, const void* g, int64_t g_ld,
                            const void* w_proj, int64_t wp_ld, const void* partial_in, int64_t pin_ld, int nblk,
                            const void* const* blocks, const int64_t* blocks_ld, const void* w_mix,
                            const void* w_up, int64_t wu_ld, const void* w_down, int64_t wd_ld, float alpha,
                            float limit, void* out, int64_t out_ld, void* stream) {
  return block_out_impl(M, C, dtype, y, y_ld, g, g_ld, w_proj, wp_ld, partial_in, pin_ld, nblk, blocks, blocks_ld,
                        w_mix, w_up, wu_ld, w_down, wd_ld, alpha, limit, out, out_ld, nullptr, 0, stream);
}

extern "C" int dg_block_out_norm(int64_t M, int C, int dtype, const void* y, int64_t y_ld, const void* g,
                                 int64_t g_ld, const void* w_proj, int64_t wp_ld, const void* partial_in,
                                 int64_t pin_ld, int nblk, const void* const* blocks, const int64_t* blocks_ld,
                                 const void* w_mix, const void* w_up, int64_t wu_ld, const void* w_down,
                                 int64_t wd_ld, float alpha, float limit, void* out, int64_t out_ld, void* xn,
                                 int64_t xn_ld, void* stream) {
  DG_REQUIRE(M == 0 || xn != nullptr, DG_EINVAL, "block_out_norm: NULL pointer");
  return block_out_impl(M, C, dtype, y, y_ld, g, g_ld, w_proj, wp_ld, partial_in, pin_ld, nblk, blocks, blocks_ld,
                        w_mix, w_up, wu_ld, w_down, wd_ld, alpha, limit, out, out_ld, xn, xn_ld, stream);
}

// ---------------------------------------------------------------------------
// The sampler's draw (torch.multinomial's one-sample method, temperature.py:
// 24-25 after the softmax): ids[r] = the first maximum over j of
// probs[r, j] / q[r, j], with q the caller's Exp(1) variates.  The quotient
// is rounded to the storage dtype as torch's division returns it (fp32
// arithmetic, correctly rounded; fp64 for fp64 data), and compared as
// torch.argmax compares: a NaN is above every number, the first of equal
// values (or of NaNs) wins.  One wave per row; lane l takes entries l,
// l + 64, ... so each lane meets its entries in increasing order.
// ---------------------------------------------------------------------------
namespace dg {

template <typename C>
__device__ __forceinline__ bool draw_better(C v, int i, C bv, int bi) {
  const bool vn = v != v, bn = bv != bv;
  if (vn || bn) return vn && (!bn || i < bi);
  return v > bv || (v == bv && i < bi);
}

template <typename T>
__global__ __launch_bounds__(256) void draw_argmax_kernel(const T* probs, int64_t p_ld, const T* q, int64_t q_ld,
                                                          int64_t* ids, int64_t M, int V) {
  using C = typename std::conditional<sizeof(T) == 8, double, float>::type;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;  // whole waves
  const T* pr = probs + row * p_ld;
  const T* qr = q + row * q_ld;
  C best = (C)0;
  int bi = 0x7fffffff;
  for (int j = lane; j < V; j += 64) {
    C v;
    if constexpr (sizeof(T) == 8) {
      v = (C)pr[j] / (C)qr[j];
    } else {
      v = (C)to_f32(from_f32<T>(to_f32(pr[j]) / to_f32(qr[j])));
    }
    if (bi == 0x7fffffff || draw_better<C>(v, j, best, bi)) {
      best = v;
      bi = j;
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const C ov = __shfl_xor(best, off, 64);
    const int oi = __shfl_xor(bi, off, 64);
    if (oi != 0x7fffffff && (bi == 0x7fffffff || draw_better<C>(ov, oi, best, bi))) {
      best = ov;
      bi = oi;
    }
  }
  if (lane == 0) ids[row] = bi;
}

}  // namespace dg

extern "C" int dg_draw_argmax(int64_t M, int V, int dtype, const void* probs, int64_t p_ld, const void* q,
                              int64_t q_ld, int64_t* ids, void* stream) {
  using namespace dg;
  DG_REQUIRE(M >= 0 && V >= 1, DG_EINVAL, "draw_argmax: bad sizes M=%lld V=%d", (long long)M, V);
  DG_REQUIRE(dtype_ok_f64(dtype), DG_EUNSUPPORTED, "draw_argmax: dtype %d unsupported", dtype);
  if (M == 0) return DG_OK;
  DG_REQUIRE(probs && q && ids, DG_EINVAL, "draw_argmax: NULL pointer");
  DG_REQUIRE(p_ld >= V && q_ld >= V, DG_EINVAL, "draw_argmax: a row stride is narrower than its row");
  DG_REQUIRE(M <= 4 * 0x7fffffffLL, DG_EINVAL, "draw_argmax: too many rows (%lld)", (long long)M);
  const dim3 grid((unsigned)((M + 3) / 4));
  hipStream_t s = static_cast<hipStream_t>(stream);
#define DG_DRAW(T)                                                                                 \
  hipLaunchKernelGGL((draw_argmax_kernel<T>), grid, dim3(256), 0, s, static_cast<const T*>(probs), p_ld, \
                     static_cast<const T*>(q), q_ld, ids, M, V)
  if (dtype == DG_F32) DG_DRAW(float);
  else if (dtype == DG_BF16) DG_DRAW(bf16_t);
  else if (dtype == DG_F16) DG_DRAW(f16_t);
  else DG_DRAW(double);
#undef DG_DRAW
  return check_launch("draw_argmax_kernel");
}
