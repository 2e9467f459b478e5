// Vector-ALU attention: single-token decode over the KV cache (mha.py:68) and
// the general masked case (mha.py:61-81) for every dtype / head_dim the MFMA
// prefill kernel does not take.
//
// Work unit = one wavefront = one (row b, head h, query i, key split).  Inside
// the wave, LPK = DPAD/EPL lanes hold one key row (EPL consecutive elements
// each, 16 bytes when the layout allows), so one wave instruction touches
// KPI = 64/LPK consecutive cache rows: a contiguous, fully coalesced stretch of
// the (b,h) page.  Each lane group keeps its own online-softmax state (running
// max m, running sum l, the group's EPL-slice of sum p*v); the KPI groups are
// merged with xor-butterflies at the end.  Scores use exp2 with log2(e) folded
// into the scale.  With several key splits, unnormalised partials (acc, m, l)
// go to the caller's workspace and attn_combine_kernel merges them.
#include "dg_common.h"

namespace dg {

struct AttnArgs {
  const void* q;
  const void* k;
  const void* v;
  void* y;
  float* part;
  int64_t qb, qt, qh;
  int64_t kb, kt, kh;
  int64_t vb, vt, vh;
  int64_t yb, yt, yh;
  int64_t units;  // B*H*Tq*nsplit
  int H, Tq, Tk, D;
  int q_offset;  // Tk - Tq: query i sees keys j <= i + q_offset
  int nsplit, split_len;
  float scale_log2;  // scale * log2(e)
};

template <typename T, int DPAD, int EPL, int U>
__global__ __launch_bounds__(256) void attn_vec_kernel(const AttnArgs a) {
  constexpr int LPK = DPAD / EPL;
  constexpr int KPI = 64 / LPK;
  static_assert(LPK >= 1 && LPK <= 64, "lane mapping");

  const int lane = threadIdx.x & 63;
  const int64_t unit = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (unit >= a.units) return;  // whole wave exits; kernel has no barriers

  const int sub = lane % LPK;
  const int grp = lane / LPK;
  int64_t r = unit;
  const int split = (int)(r % a.nsplit);
  r /= a.nsplit;
  const int i = (int)(r % a.Tq);
  r /= a.Tq;
  const int h = (int)(r % a.H);
  const int64_t b = r / a.H;

  const int d0 = sub * EPL;
  const bool active = d0 < a.D;
  const int kvis = min(a.Tk, i + a.q_offset + 1);
  const int kbeg = split * a.split_len;
  const int kend = min(kvis, kbeg + a.split_len);

  float qf[EPL];
  if (active) {
    load_vec<T, EPL>(static_cast<const T*>(a.q) + b * a.qb + (int64_t)i * a.qt + (int64_t)h * a.qh + d0,
                     qf);
  } else {
#pragma unroll
    for (int e = 0; e < EPL; ++e) qf[e] = 0.f;
  }
#pragma unroll
  for (int e = 0; e < EPL; ++e) qf[e] *= a.scale_log2;

  const T* kp = static_cast<const T*>(a.k) + b * a.kb + (int64_t)h * a.kh + d0;
  const T* vp = static_cast<const T*>(a.v) + b * a.vb + (int64_t)h * a.vh + d0;

  float m = kNegInf, l = 0.f;
  float acc[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) acc[e] = 0.f;

  for (int t0 = kbeg; t0 < kend; t0 += KPI * U) {
    float s[U];
    float vv[U][EPL];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = t0 + u * KPI + grp;
      const bool valid = t < kend;
      float kk[EPL];
      if (valid && active) {
        load_vec<T, EPL>(kp + (int64_t)t * a.kt, kk);
        load_vec<T, EPL>(vp + (int64_t)t * a.vt, vv[u]);
      } else {
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
          kk[e] = 0.f;
          vv[u][e] = 0.f;
        }
      }
      float dot = 0.f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) dot += qf[e] * kk[e];
      dot = group_sum<LPK>(dot);
      s[u] = valid ? dot : kNegInf;
    }
    float mloc = s[0];
#pragma unroll
    for (int u = 1; u < U; ++u) mloc = fmaxf(mloc, s[u]);
    const float mnew = fmaxf(m, mloc);
    if (mnew != kNegInf) {
      const float alpha = exp2f(m - mnew);
      l *= alpha;
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[e] *= alpha;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float p = exp2f(s[u] - mnew);
        l += p;
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[e] += p * vv[u][e];
      }
      m = mnew;
    }
  }

  // merge the KPI lane groups (xor over the group index keeps the d-slice)
#pragma unroll
  for (int off = LPK; off < 64; off <<= 1) {
    const float mo = shfl_xor(m, off);
    const float lo = shfl_xor(l, off);
    float ao[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) ao[e] = shfl_xor(acc[e], off);
    const float mn = fmaxf(m, mo);
    if (mn != kNegInf) {
      const float c1 = exp2f(m - mn), c2 = exp2f(mo - mn);
      l = l * c1 + lo * c2;
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[e] = acc[e] * c1 + ao[e] * c2;
      m = mn;
    }
  }

  if (grp != 0 || !active) return;
  if (a.nsplit == 1) {
    const float inv = 1.0f / l;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[e] *= inv;
    store_vec<T, EPL>(static_cast<T*>(a.y) + b * a.yb + (int64_t)i * a.yt + (int64_t)h * a.yh + d0,
                      acc);
  } else {
    float* pp = a.part + unit * (int64_t)(DPAD + 2);
#pragma unroll
    for (int e = 0; e < EPL; ++e) pp[d0 + e] = acc[e];
    if (sub == 0) {
      pp[DPAD] = m;
      pp[DPAD + 1] = l;
    }
  }
}

// Merge the nsplit partials of each (b, h, i): one lane group per query row.
template <typename T, int DPAD, int EPL>
__global__ __launch_bounds__(256) void attn_combine_kernel(const AttnArgs a) {
  constexpr int LPK = DPAD / EPL;
  constexpr int RPB = 256 / LPK;
  const int64_t rows = a.units / a.nsplit;
  const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / LPK;
  if (row >= rows) return;
  const int sub = threadIdx.x % LPK;
  const int d0 = sub * EPL;
  if (d0 >= a.D) return;
  int64_t r = row;
  const int i = (int)(r % a.Tq);
  r /= a.Tq;
  const int h = (int)(r % a.H);
  const int64_t b = r / a.H;

  const float* base = a.part + row * a.nsplit * (int64_t)(DPAD + 2);
  float M = kNegInf;
  for (int s = 0; s < a.nsplit; ++s) M = fmaxf(M, base[s * (DPAD + 2) + DPAD]);
  float L = 0.f;
  float acc[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) acc[e] = 0.f;
  for (int s = 0; s < a.nsplit; ++s) {
    const float* pp = base + s * (DPAD + 2);
    const float ms = pp[DPAD];
    if (ms == kNegInf) continue;
    const float c = exp2f(ms - M);
    L += c * pp[DPAD + 1];
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[e] += c * pp[d0 + e];
  }
  const float inv = 1.0f / L;
#pragma unroll
  for (int e = 0; e < EPL; ++e) acc[e] *= inv;
  store_vec<T, EPL>(static_cast<T*>(a.y) + b * a.yb + (int64_t)i * a.yt + (int64_t)h * a.yh + d0, acc);
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
namespace {

constexpr int kUnroll = 4;        // key slots per lane group per loop trip
constexpr int64_t kTargetWaves = 8192;  // 256 CUs x 32 resident waves
constexpr int kMinSplitKeys = 128;
constexpr int kMaxSplits = 64;

int next_pow2(int x) {
  int p = 1;
  while (p < x) p <<= 1;
  return p;
}
bool aligned(const void* p, int64_t bytes) {
  return (reinterpret_cast<uintptr_t>(p) % (uintptr_t)bytes) == 0;
}
bool strides_multiple(const dg_stride3* s, int64_t m) {
  return s->b % m == 0 && s->t % m == 0 && s->h % m == 0;
}

// Number of key splits for a launch; 1 unless the (b, h, i) units alone cannot
// fill the chip and the rows are long.
int pick_splits(int64_t base_units, int Tk) {
  if (base_units <= 0) return 1;
  int64_t want = (kTargetWaves + base_units - 1) / base_units;
  int64_t by_len = Tk / kMinSplitKeys;
  int64_t n = want < by_len ? want : by_len;
  if (n > kMaxSplits) n = kMaxSplits;
  if (n < 1) n = 1;
  return (int)n;
}

template <typename T, int DPAD, int EPL>
int launch_attn(AttnArgs a, hipStream_t s) {
  const int64_t blocks = (a.units + 3) / 4;
  DG_REQUIRE(blocks <= 0x7fffffffLL, DG_EINVAL, "attention: too many units");
  hipLaunchKernelGGL((attn_vec_kernel<T, DPAD, EPL, kUnroll>), dim3((unsigned)blocks), dim3(256), 0,
                     s, a);
  int rc = check_launch("attn_vec_kernel");
  if (rc != DG_OK || a.nsplit == 1) return rc;
  constexpr int LPK = DPAD / EPL;
  constexpr int RPB = 256 / LPK;
  const int64_t rows = a.units / a.nsplit;
  hipLaunchKernelGGL((attn_combine_kernel<T, DPAD, EPL>), dim3((unsigned)((rows + RPB - 1) / RPB)),
                     dim3(256), 0, s, a);
  return check_launch("attn_combine_kernel");
}

template <typename T, int DPAD>
int attn_pick_epl(int epl, const AttnArgs& a, hipStream_t s) {
  constexpr int PREF = (16 / (int)sizeof(T)) < DPAD ? (16 / (int)sizeof(T)) : DPAD;
  if constexpr (PREF != 2) {
    if (epl == PREF) return launch_attn<T, DPAD, PREF>(a, s);
  }
  if constexpr (DPAD / 2 <= 64) {
    if (epl == 2) return launch_attn<T, DPAD, 2>(a, s);
  }
  set_error("attention: no kernel for D pad %d with %d elements per lane", DPAD, epl);
  return DG_EUNSUPPORTED;
}

template <typename T>
int attn_pick_d(int dpad, int epl, const AttnArgs& a, hipStream_t s) {
  switch (dpad) {
    case 2: return attn_pick_epl<T, 2>(epl, a, s);
    case 4: return attn_pick_epl<T, 4>(epl, a, s);
    case 8: return attn_pick_epl<T, 8>(epl, a, s);
    case 16: return attn_pick_epl<T, 16>(epl, a, s);
    case 32: return attn_pick_epl<T, 32>(epl, a, s);
    case 64: return attn_pick_epl<T, 64>(epl, a, s);
    case 128: return attn_pick_epl<T, 128>(epl, a, s);
    case 256: return attn_pick_epl<T, 256>(epl, a, s);
  }
  set_error("attention: head_dim %d unsupported", a.D);
  return DG_EUNSUPPORTED;
}

}  // namespace

// Used by the C entry points in dg_abi.hip.
int vec_attention_splits(int B, int H, int Tq, int Tk, int D) {
  (void)D;
  if (Tq != 1) return 1;  // prefill rows are plentiful; split only decode
  return pick_splits((int64_t)B * H * Tq, Tk);
}

size_t vec_attention_workspace(int B, int H, int Tq, int Tk, int D) {
  const int ns = vec_attention_splits(B, H, Tq, Tk, D);
  if (ns <= 1) return 0;
  return (size_t)B * H * Tq * ns * (size_t)(next_pow2(D) + 2) * sizeof(float);
}

int vec_attention(int B, int H, int Tq, int Tk, int D, int dtype, const void* q,
                  const dg_stride3* q_st, const void* k, const dg_stride3* k_st, const void* v,
                  const dg_stride3* v_st, void* y, const dg_stride3* y_st, float scale,
                  void* workspace, size_t workspace_bytes, hipStream_t s) {
  const int es = dtype == DG_F32 ? 4 : 2;
  const int dpad = next_pow2(D);
  DG_REQUIRE(dpad <= 256, DG_EUNSUPPORTED, "attention: head_dim %d > 256", D);
  int pref = 16 / es;
  if (pref > dpad) pref = dpad;
  auto fits = [&](int epl) {
    if (epl != 2 && dpad != D) return false;
    if (dpad / epl > 64) return false;
    const int64_t bytes = (int64_t)epl * es;
    return aligned(q, bytes) && aligned(k, bytes) && aligned(v, bytes) && aligned(y, bytes) &&
           strides_multiple(q_st, epl) && strides_multiple(k_st, epl) &&
           strides_multiple(v_st, epl) && strides_multiple(y_st, epl);
  };
  int epl = 0;
  if (fits(pref)) epl = pref;
  else if (fits(2)) epl = 2;
  DG_REQUIRE(epl != 0, DG_EINVAL,
             "attention: pointers/strides not aligned to an element pair (D=%d); pass contiguous rows", D);

  AttnArgs a{};
  a.q = q; a.k = k; a.v = v; a.y = y;
  a.qb = q_st->b; a.qt = q_st->t; a.qh = q_st->h;
  a.kb = k_st->b; a.kt = k_st->t; a.kh = k_st->h;
  a.vb = v_st->b; a.vt = v_st->t; a.vh = v_st->h;
  a.yb = y_st->b; a.yt = y_st->t; a.yh = y_st->h;
  a.H = H; a.Tq = Tq; a.Tk = Tk; a.D = D;
  a.q_offset = Tk - Tq;
  a.scale_log2 = scale * 1.44269504088896340736f;

  int ns = vec_attention_splits(B, H, Tq, Tk, D);
  const size_t need = vec_attention_workspace(B, H, Tq, Tk, D);
  if (ns > 1 && (workspace == nullptr || workspace_bytes < need)) {
    DG_REQUIRE(workspace == nullptr, DG_EWORKSPACE,
               "attention: workspace of %zu bytes given, %zu needed", workspace_bytes, need);
    ns = 1;  // no workspace: single pass over all keys
  }
  a.nsplit = ns;
  a.split_len = ns == 1 ? Tk : (((Tk + ns - 1) / ns + 15) / 16) * 16;
  a.part = ns == 1 ? nullptr : static_cast<float*>(workspace);
  DG_REQUIRE(ns == 1 || aligned(workspace, 16), DG_EINVAL, "attention: workspace must be 16-byte aligned");
  a.units = (int64_t)B * H * Tq * ns;

  if (dtype == DG_F32) return attn_pick_d<float>(dpad, epl, a, s);
  if (dtype == DG_BF16) return attn_pick_d<bf16_t>(dpad, epl, a, s);
  return attn_pick_d<f16_t>(dpad, epl, a, s);
}

}  // namespace dg
