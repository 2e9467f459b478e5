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
//
// Every intermediate is rounded to the storage dtype where the torch op
// sequence rounds it (each op returns a tensor of the input dtype; fp32
// arithmetic inside, as ATen's opmath does), so bf16 results follow the same
// rounding steps.  The RMSNorms use the lane mapping and reduction tree of
// rms_norm_kernel, so they produce its bits for the same row.
#include <float.h>

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
// by tree_sum inside the lane, then the butterfly over the G lanes of the row)
template <int CH, int G>
__device__ __forceinline__ void row_rms(float (&x)[CH], int N) {
#pragma clang fp contract(off)
  float sq[CH];
#pragma unroll
  for (int i = 0; i < CH; ++i) sq[i] = x[i] * x[i];
  float ss = tree_sum<CH>(sq);
  ss = group_sum<G>(ss);
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

template <typename T, int NPAD, int CH>
__global__ __launch_bounds__(256) void attn_res_norm_kernel(const AttnResArgs a, const int vec) {
#pragma clang fp contract(off)
  constexpr int G = NPAD / CH;
  static_assert(G >= 1 && G <= 64, "row mapping");
  constexpr int ROWS_PER_BLOCK = 256 / G;
  const int sub = threadIdx.x % G;
  const int64_t row = (int64_t)blockIdx.x * ROWS_PER_BLOCK + threadIdx.x / G;
  if (row >= a.M) return;  // whole lane groups leave together; no barriers
  const int c0 = sub * CH;
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
    load_slice<T, CH>(static_cast<const T*>(a.src[n]) + row * a.ld[n] + c0, c0, a.N, vec, x);
    row_rms<CH, G>(x, a.N);
    float prod[CH];
#pragma unroll
    for (int i = 0; i < CH; ++i) prod[i] = rt<T>(x[i]) * w[i];
    float dot = tree_sum<CH>(prod);
    dot = group_sum<G>(dot);
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
    load_slice<T, CH>(static_cast<const T*>(a.src[n]) + row * a.ld[n] + c0, c0, a.N, vec, x);
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

namespace {

bool al(const void* p, int64_t bytes) { return (reinterpret_cast<uintptr_t>(p) % (uintptr_t)bytes) == 0; }

int pow2_at_least(int x) {
  int p = 1;
  while (p < x) p <<= 1;
  return p;
}

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

// one thread per output element; K<T> for the dtype
#define DG_LAUNCH_ROWS(K, dtype, a, s)                                                        \
  do {                                                                                        \
    const int64_t n_ = (a).M * (int64_t)(a).N;                                                \
    if (n_ == 0) return DG_OK;                                                                \
    const int64_t blocks_ = (n_ + 255) / 256;                                                 \
    DG_REQUIRE(blocks_ <= 0x7fffffffLL, DG_EINVAL, #K ": too many elements (%lld)", (long long)n_); \
    if ((dtype) == DG_F32)                                                                    \
      hipLaunchKernelGGL(K<float>, dim3((unsigned)blocks_), dim3(256), 0, (s), (a));          \
    else if ((dtype) == DG_BF16)                                                              \
      hipLaunchKernelGGL(K<bf16_t>, dim3((unsigned)blocks_), dim3(256), 0, (s), (a));         \
    else                                                                                      \
      hipLaunchKernelGGL(K<f16_t>, dim3((unsigned)blocks_), dim3(256), 0, (s), (a));          \
    return check_launch(#K);                                                                  \
  } while (0)

bool dtype_ok(int dtype) { return dtype == DG_F32 || dtype == DG_BF16 || dtype == DG_F16; }

}  // namespace
}  // namespace dg

using namespace dg;

extern "C" int dg_attn_res_norm(int64_t M, int C, int dtype, int nsrc, const void* const* src,
                                const int64_t* src_ld, const void* w, void* out, int64_t out_ld,
                                void* stream) {
  DG_REQUIRE(M >= 0 && C >= 1, DG_EINVAL, "attn_res_norm: bad sizes M=%lld C=%d", (long long)M, C);
  DG_REQUIRE(C <= 2048, DG_EUNSUPPORTED, "attn_res_norm: C=%d > 2048", C);
  DG_REQUIRE(dtype_ok(dtype), DG_EUNSUPPORTED, "attn_res_norm: dtype %d unsupported", dtype);
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
  const int npad = pow2_at_least(C);
  if (dtype == DG_F32) return res_pick<float>(npad, a, s);
  if (dtype == DG_BF16) return res_pick<bf16_t>(npad, a, s);
  return res_pick<f16_t>(npad, a, s);
}

extern "C" int dg_gate(int64_t M, int C, int dtype, const void* y, int64_t y_ld, const void* g,
                       int64_t g_ld, void* out, int64_t out_ld, void* stream) {
  DG_REQUIRE(M >= 0 && C >= 1, DG_EINVAL, "gate: bad sizes M=%lld C=%d", (long long)M, C);
  DG_REQUIRE(dtype_ok(dtype), DG_EUNSUPPORTED, "gate: dtype %d unsupported", dtype);
  if (M == 0) return DG_OK;
  DG_REQUIRE(y != nullptr && g != nullptr && out != nullptr, DG_EINVAL, "gate: NULL pointer");
  DG_REQUIRE(y_ld >= C && g_ld >= C && out_ld >= C, DG_EINVAL, "gate: row stride smaller than C");
  RowsArgs a{};
  a.x = y; a.g = g; a.out = out;
  a.x_ld = y_ld; a.g_ld = g_ld; a.out_ld = out_ld; a.M = M; a.N = C;
  DG_LAUNCH_ROWS(gate_kernel, dtype, a, static_cast<hipStream_t>(stream));
}

extern "C" int dg_swiglu(int64_t M, int N, int dtype, const void* x, int64_t x_ld, void* out,
                         int64_t out_ld, float alpha, float limit, void* stream) {
  DG_REQUIRE(M >= 0 && N >= 1, DG_EINVAL, "swiglu: bad sizes M=%lld N=%d", (long long)M, N);
  DG_REQUIRE(dtype_ok(dtype), DG_EUNSUPPORTED, "swiglu: dtype %d unsupported", dtype);
  if (M == 0) return DG_OK;
  DG_REQUIRE(x != nullptr && out != nullptr, DG_EINVAL, "swiglu: NULL pointer");
  DG_REQUIRE(x_ld >= 2 * (int64_t)N && out_ld >= N, DG_EINVAL, "swiglu: row stride too small");
  RowsArgs a{};
  a.x = x; a.out = out;
  a.x_ld = x_ld; a.out_ld = out_ld; a.M = M; a.N = N;
  a.p0 = alpha; a.p1 = limit;
  DG_LAUNCH_ROWS(swiglu_kernel, dtype, a, static_cast<hipStream_t>(stream));
}

extern "C" int dg_softcap(int64_t M, int N, int dtype, const void* x, int64_t x_ld, void* out,
                          int64_t out_ld, float cap, void* stream) {
  DG_REQUIRE(M >= 0 && N >= 1, DG_EINVAL, "softcap: bad sizes M=%lld N=%d", (long long)M, N);
  DG_REQUIRE(dtype_ok(dtype), DG_EUNSUPPORTED, "softcap: dtype %d unsupported", dtype);
  DG_REQUIRE(cap > 0.f, DG_EINVAL, "softcap: cap must be positive (got %g)", (double)cap);
  if (M == 0) return DG_OK;
  DG_REQUIRE(x != nullptr && out != nullptr, DG_EINVAL, "softcap: NULL pointer");
  DG_REQUIRE(x_ld >= N && out_ld >= N, DG_EINVAL, "softcap: row stride smaller than N");
  RowsArgs a{};
  a.x = x; a.out = out;
  a.x_ld = x_ld; a.out_ld = out_ld; a.M = M; a.N = N;
  a.p0 = cap;
  DG_LAUNCH_ROWS(softcap_kernel, dtype, a, static_cast<hipStream_t>(stream));
}
