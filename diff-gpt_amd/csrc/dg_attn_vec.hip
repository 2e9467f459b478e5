// Vector-ALU attention: single-token decode over the KV cache (mha.py:68) and
// the general masked case (mha.py:61-81) for every dtype / head_dim the MFMA
// prefill kernel does not take.
//
// Work unit = one wavefront = one (row b, head h, query i, key split).  Inside
// the wave, LPK = DPAD/EPL lanes hold one key row (EPL consecutive elements
// each, 16 bytes when the layout allows), so one wave instruction touches
// KPI = 64/LPK consecutive cache rows: a contiguous, fully coalesced stretch of
// the (b,h) page.  Keys are processed in trips of U slots (U*KPI keys); the
// K/V registers of the next trip are loaded while the current trip computes
// (two register sets, loop unrolled by two), so every wave keeps 2*U*2
// sixteen-byte loads per lane in flight.
//
// Arithmetic per key slot and lane: the partial q.k over the lane's EPL
// elements (fp32 FMAs, or v_dot2_f32_{bf16,f16} straight on the packed
// 16-bit data -- products of two 16-bit floats are exact in fp32), a
// register-only sum over the LPK lanes of the key (DPP / permlane, no LDS),
// then the online softmax in log2 units with the SDPA scale folded into one
// FMA: p = exp2(s*c - m*c), c = scale*log2(e), on raw scores s.  The offset m
// is shared by the whole wave (a DPP max over the trip's scores): it is raised
// only when a score exceeds it by more than kLazyLog2/c, so probabilities stay
// <= 2^kLazyLog2 and the rescale of (l, acc) is skipped on most trips; the
// result is the same function.  Because m is common to all KPI lane groups,
// they merge at the end by plain register sums of l and acc.  With key
// splits, up to 16 splits of one (b, h, i) are the waves of one workgroup
// and merge their unnormalised partials (acc, m, l) in LDS; more go to the
// caller's workspace and attn_combine_kernel merges them.
//
// FUSED instances are the whole decode step of one new token (dg_decode_step,
// mha.py:44-68): every wave rotates and normalises its q and the new k from
// the projections, the wave whose split holds the position appends k and v
// to the cache, and the new key enters the softmax from registers in the
// trip slot where the two-launch form reads it back, so y has that form's
// bits.
#include "dg_rope_math.h"

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
  PrefixRef pre;     // keys j < pre.len of row b come from its group's prefix pages
  float scale_log2;  // scale * log2(e)
  float lazy_raw;    // kLazyLog2 / scale_log2
  // Decode-step form (graph-replayable, Tq == 1): when pos_dev is set, the
  // keys are positions 0 .. *pos_dev (the token of this step was appended at
  // *pos_dev), at most Tk of them; split_len follows from that count.
  const int* pos_dev;
  // Fused decode step (FUSED instances, Tq == 1, mha.py:44-68 for one new
  // token): q is the new token's query projection, kn / vn its key and value
  // projections ((b, h) strides); the (cos, sin) row of position p is at
  // freqs + p * fpos (fp32 when f32freqs, else T).  The position is pos_dev's
  // value when set, else pos.  k and v (the cache pages) are written at it.
  const void* kn;
  const void* vn;
  int64_t knb, knh, vnb, vnh;
  const void* freqs;
  int64_t fpos;
  int f32freqs, qknorm, pos;
};

constexpr float kVecLazyLog2 = 8.0f;
// Key splits of one (b, h, i) run as the waves of one workgroup and merge in
// LDS when there are at most this many (16, or 8 for rows padded to 1024,
// whose (acc, m, l) partials would not fit 32 KB of LDS); more go through
// the workspace and attn_combine_kernel.
constexpr int kMaxBlockSplits = 16;
constexpr int block_splits(int dpad) { return dpad * kMaxBlockSplits * 4 <= 32768 ? kMaxBlockSplits : 32768 / (dpad * 4); }

// MERGE: the workgroup's nsplit waves are the key splits of one (b, h, i)
// (blockDim = 64 * nsplit); otherwise a workgroup holds 4 independent units.
// FUSED: the decode step of one new token in the same launch -- q and the new
// key rotated (and normalised) with rope_qknorm_kernel's arithmetic, the key
// and value appended by the wave whose split holds the position, and the new
// key taken from registers in the trip slot where the two-call form reads it
// back from the cache, so y has the two calls' bits.
// PAIRS: the lanes' slices are read and written pair by pair (load_slice),
// pairs past D skipped.
template <typename T, int DPAD, int EPL, int U, bool MERGE, bool FUSED, bool PAIRS>
__global__ __launch_bounds__(MERGE ? 64 * block_splits(DPAD) : 256) void attn_vec_kernel(const AttnArgs a) {
  constexpr int LPK = DPAD / EPL;
  constexpr int KPI = 64 / LPK;
  constexpr int STEP = KPI * U;  // keys per trip
  static_assert(LPK >= 1 && LPK <= 64, "lane mapping");
  using Row = RowRegs<T, EPL>;

  const int lane = threadIdx.x & 63;
  // Consecutive blocks (rows of one group, heads of one row) go to one XCD:
  // workgroups are dealt round-robin over the 8 XCDs, each with its own L2.
  int blk = blockIdx.x;
  if ((gridDim.x & 7) == 0) blk = (blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3);
  // wave-uniform unit index (the host keeps units below 2^31)
  const int unit = blk * (int)(blockDim.x >> 6) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if constexpr (!MERGE) {
    if (unit >= a.units) return;  // whole wave exits; no barrier follows
  }

  const int sub = lane % LPK;
  const int grp = lane / LPK;
  int r = unit;
  const int split = r % a.nsplit;
  r /= a.nsplit;
  const int i = r % a.Tq;
  r /= a.Tq;
  const int h = r % a.H;
  const int64_t b = r / a.H;

  const int d0 = sub * EPL;
  const bool active = d0 < a.D;
  const int dl = active ? d0 : 0;  // inactive lanes (D not a power of two) read a valid slice
  const int np = slice_pairs<EPL>(d0, a.D);  // PAIRS: pairs of the slice inside D
  int Tk = a.Tk, q_offset = a.q_offset, split_len = a.split_len;
  int pos = -1;         // fused: the new token's position
  bool pos_ok = false;  // fused: the position lies in the rows' own pages (a.Tk = max_pos)
  if (FUSED || a.pos_dev != nullptr) {  // uniform over the grid
    if constexpr (FUSED) {
      pos = a.pos_dev != nullptr ? *a.pos_dev : a.pos;
      pos_ok = pos >= a.pre.own_start && pos < a.Tk;
      Tk = min(pos + 1, a.Tk);
    } else {
      Tk = min(*a.pos_dev + 1, a.Tk);
    }
    q_offset = Tk - 1;
    split_len = a.nsplit == 1 ? Tk : (((Tk + a.nsplit - 1) / a.nsplit + 15) / 16) * 16;
  }
  const int kvis = min(Tk, i + q_offset + 1);
  const int kbeg = split * split_len;
  const int kend = min(kvis, kbeg + split_len);
  const float c = a.scale_log2;

  Row qr;
  Row knew, vnew;              // fused: the appended key and value
  float xq[EPL], xk[EPL], cs[EPL];  // fused: q and k before RoPE, the (cos, sin) pairs
  if constexpr (FUSED) {
    load_vec_slice<T, EPL, PAIRS>(static_cast<const T*>(a.q) + b * a.qb + (int64_t)h * a.qh + dl, xq, np);
    load_vec_slice<T, EPL, PAIRS>(static_cast<const T*>(a.kn) + b * a.knb + (int64_t)h * a.knh + dl, xk, np);
    load_slice<T, EPL, PAIRS>(vnew, static_cast<const T*>(a.vn) + b * a.vnb + (int64_t)h * a.vnh + dl, np);
    // a position outside the pages writes nothing and reads table row 0
    // (its y is undefined, as in the two-launch form)
    const int64_t frow = pos_ok ? pos : 0;
    if (a.f32freqs)
      load_vec_slice<float, EPL, PAIRS>(static_cast<const float*>(a.freqs) + frow * a.fpos + dl, cs, np);
    else
      load_vec_slice<T, EPL, PAIRS>(static_cast<const T*>(a.freqs) + frow * a.fpos + dl, cs, np);
  } else {
    load_slice<T, EPL, PAIRS>(qr, static_cast<const T*>(a.q) + b * a.qb + (int64_t)i * a.qt + (int64_t)h * a.qh + dl,
                              np);
    if (!active) {
#pragma unroll
      for (int w = 0; w < Row::WORDS; ++w) qr.w[w] = 0u;  // contributes 0 to every dot
    }
  }

  // wave-uniform page bases; per-lane offsets of slot u inside a trip
  const T* kbase = static_cast<const T*>(a.k) + b * a.kb + (int64_t)h * a.kh;
  const T* vbase = static_cast<const T*>(a.v) + b * a.vb + (int64_t)h * a.vh;
  // shared prefix: keys below pre.len come from the group's prefix pages
  // (same t stride as the cache); own keys are at or past it
  const int64_t grp_of = b / a.pre.group;
  const T* kpre = static_cast<const T*>(a.pre.k) + grp_of * a.pre.kb + (int64_t)h * a.pre.kh;
  const T* vpre = static_cast<const T*>(a.pre.v) + grp_of * a.pre.vb + (int64_t)h * a.pre.vh;
  const int P = a.pre.len;
  const int kt = (int)a.kt, vt = (int)a.vt;  // host: Tk * stride < 2^31
  int koff[U], voff[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    koff[u] = (u * KPI + grp) * kt + dl;
    voff[u] = (u * KPI + grp) * vt + dl;
  }

  float m = kNegInf, l = 0.f;
  float acc[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) acc[e] = 0.f;

  Row kA[U], vA[U], kB[U], vB[U];
  auto load_trip = [&](Row (&kr)[U], Row (&vr)[U], int t0) __attribute__((always_inline)) {
    if (t0 + STEP <= kend && (t0 >= P || t0 + STEP <= P)) {
      // full trip inside one source page (own rows, or the shared prefix)
      const bool pre = t0 < P;
      const T* kb = (pre ? kpre : kbase) + (int64_t)t0 * kt;
      const T* vb = (pre ? vpre : vbase) + (int64_t)t0 * vt;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        load_slice<T, EPL, PAIRS>(kr[u], kb + koff[u], np);
        load_slice<T, EPL, PAIRS>(vr[u], vb + voff[u], np);
      }
    } else {
      // trip straddling the end of the prefix or the end of the keys: slots
      // wholly past kend are skipped (wave-uniform); inside the last slot,
      // rows past kend re-read row kend-1 (always valid) and their scores
      // are masked
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (t0 + u * KPI >= kend) break;
        const int t = min(t0 + u * KPI + grp, kend - 1);
        const bool pre = t < P;
        load_slice<T, EPL, PAIRS>(kr[u], (pre ? kpre : kbase) + t * kt + dl, np);
        load_slice<T, EPL, PAIRS>(vr[u], (pre ? vpre : vbase) + t * vt + dl, np);
      }
    }
  };
  auto process = [&](Row (&kr)[U], Row (&vr)[U], int t0) __attribute__((always_inline)) {
    if constexpr (FUSED) {
      // the trip holding the new position takes its key and value from
      // registers in every lane the cache read would fill from that row: the
      // position's own slot and the slots past the last key, which re-read
      // the last row (kend - 1 = pos) and are masked -- the row's old
      // contents, read before the append, could be any bits
      if (pos_ok && pos >= t0 && pos < t0 + STEP) {  // wave-uniform
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const bool mine = t0 + u * KPI + grp >= pos;
#pragma unroll
          for (int w = 0; w < Row::WORDS; ++w) {
            kr[u].w[w] = mine ? knew.w[w] : kr[u].w[w];
            vr[u].w[w] = mine ? vnew.w[w] : vr[u].w[w];
          }
        }
      }
    }
    float s[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      s[u] = kNegInf;
      if (t0 + u * KPI >= kend) continue;  // slot not loaded (wave-uniform)
      const float dot = group_sum_dpp<LPK>(slice_dot<T, EPL>(qr, kr[u]));
      s[u] = (t0 + u * KPI + grp < kend) ? dot : kNegInf;
    }
    float mt = s[0];
#pragma unroll
    for (int u = 1; u < U; ++u) mt = fmaxf(mt, s[u]);
    // every trip holds at least one visible key, so mt is finite
    mt = wave_max(mt);
    if (mt > m + a.lazy_raw) {  // wave-uniform
      const float alpha = (m == kNegInf) ? 0.f : __builtin_amdgcn_exp2f((m - mt) * c);
      m = mt;
      l *= alpha;
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[e] *= alpha;
    }
    const float moff = m * c;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (t0 + u * KPI >= kend) continue;
      const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[u], c, -moff));
      l += p;
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[e] = __builtin_fmaf(p, elem<T, EPL>(vr[u], e), acc[e]);
    }
  };

  int t0 = kbeg;
  if (t0 < kend) load_trip(kA, vA, t0);
  if constexpr (FUSED) {
    // rope_qknorm_kernel's arithmetic on the lane's EPL elements (lanes past
    // D hold zeros, which leave the row norm unchanged), while the first
    // trip's keys are in flight; then the append (kv_cache.py:108-109) by the
    // split that holds the position, after those loads in program order (the
    // slot they read at the position is replaced from registers anyway)
    if (!active) {
#pragma unroll
      for (int e = 0; e < EPL; ++e) xq[e] = xk[e] = 0.f;
    }
    rope_rotate<T, EPL>(xq, cs);
    rope_rotate<T, EPL>(xk, cs);
    if (a.qknorm) {
      qk_rms_norm<EPL, LPK, true>(xq, a.D);
      qk_rms_norm<EPL, LPK, true>(xk, a.D);
    }
    pack_row<T, EPL>(qr, xq);
    pack_row<T, EPL>(knew, xk);
    if (pos_ok && pos >= kbeg && pos < kend && grp == 0 && active) {
      store_slice<T, EPL, PAIRS>(const_cast<T*>(kbase) + (int64_t)pos * kt + d0, knew, np);
      store_slice<T, EPL, PAIRS>(const_cast<T*>(vbase) + (int64_t)pos * vt + d0, vnew, np);
    }
  }
  if (t0 < kend) {
    while (true) {
      if (t0 + STEP < kend) load_trip(kB, vB, t0 + STEP);
      process(kA, vA, t0);
      t0 += STEP;
      if (t0 >= kend) break;
      if (t0 + STEP < kend) load_trip(kA, vA, t0 + STEP);
      process(kB, vB, t0);
      t0 += STEP;
      if (t0 >= kend) break;
    }
  }

  // the KPI lane groups share m: their partials add up
  l = sum_over_groups<LPK>(l);
#pragma unroll
  for (int e = 0; e < EPL; ++e) acc[e] = sum_over_groups<LPK>(acc[e]);

  if constexpr (MERGE) {
    // each wave (split) leaves its partial in LDS; after the barrier the
    // workgroup's threads take the output dims in pairs and merge the splits:
    // weights exp2((m_j - M) c) against the largest offset M, as the combine
    // kernel does.  Every wave reaches the barrier (no early exit above).
    __shared__ float lds_acc[block_splits(DPAD)][DPAD];
    __shared__ float lds_ml[block_splits(DPAD)][2];
    if (grp == 0 && active) {
#pragma unroll
      for (int e = 0; e < EPL; ++e) lds_acc[split][d0 + e] = acc[e];
    }
    if (lane == 0) {
      lds_ml[split][0] = m;
      lds_ml[split][1] = l;
    }
    __syncthreads();
    const int ns = a.nsplit;
    float M = kNegInf;
    for (int j = 0; j < ns; ++j) M = fmaxf(M, lds_ml[j][0]);  // split 0 holds key 0: M is finite
    T* yp = static_cast<T*>(a.y) + b * a.yb + (int64_t)i * a.yt + (int64_t)h * a.yh;
    for (int d = 2 * (int)threadIdx.x; d < a.D; d += 2 * (int)blockDim.x) {
      float L = 0.f, o[2] = {0.f, 0.f};
      for (int j = 0; j < ns; ++j) {
        const float mj = lds_ml[j][0];
        const float w = mj == kNegInf ? 0.f : __builtin_amdgcn_exp2f((mj - M) * c);
        L += w * lds_ml[j][1];
        o[0] += w * lds_acc[j][d];
        o[1] += w * lds_acc[j][d + 1];
      }
      const float inv = 1.0f / L;
      o[0] *= inv;
      o[1] *= inv;
      store_vec<T, 2>(yp + d, o);  // D is even; y is aligned to a pair (host check)
    }
    return;
  }
  if (grp != 0 || !active) return;
  if (a.nsplit == 1) {
    const float inv = 1.0f / l;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[e] *= inv;
    store_vec_slice<T, EPL, PAIRS>(static_cast<T*>(a.y) + b * a.yb + (int64_t)i * a.yt + (int64_t)h * a.yh + d0,
                                   acc, np);
  } else {
    // workspace: acc of every unit ([units][DPAD] fp32), then its (m, l)
    store_vec<float, EPL>(a.part + (int64_t)unit * DPAD + d0, acc);
    if (sub == 0) {
      float* ml = a.part + a.units * DPAD + 2 * (int64_t)unit;
      ml[0] = m;
      ml[1] = l;
    }
  }
}

// Merge the nsplit partials of each (b, h, i).  A row's threads are C chunks
// of CW floats times SP split slots (SP a power of two, C * SP <= 256): slot j
// folds splits j, j + SP, ... into a running (m, l, acc) -- all its loads are
// independent of one another, so a row's partials arrive in about one memory
// latency -- and the SP slot states meet in LDS, where slot 0 merges them.
// PAIRS (y aligned to a pair only, D any even size): stored pair by pair.
template <typename T, int DPAD, int EPL, bool PAIRS>
__global__ __launch_bounds__(256) void attn_combine_kernel(const AttnArgs a, const int sp_shift) {
  constexpr int CW = DPAD < 4 ? DPAD : 4;
  constexpr int C = DPAD / CW;
  constexpr int LOG2C = __builtin_ctz(C);
  __shared__ float red_acc[256 * CW];
  __shared__ float red_m[256], red_l[256];

  const int t = threadIdx.x;
  const int tpr_shift = sp_shift + LOG2C;  // threads per row = 2^tpr_shift <= 256
  const int SP = 1 << sp_shift;
  const int j = (t >> LOG2C) & (SP - 1);
  const int cidx = t & (C - 1);
  const int64_t rows = a.units / a.nsplit;
  const int64_t row = ((int64_t)blockIdx.x << (8 - tpr_shift)) + (t >> tpr_shift);
  const bool live = row < rows;
  const int64_t r0 = live ? row : 0;  // threads past the last row read row 0 and store nothing
  const int ns = a.nsplit;
  const float* ml = a.part + a.units * DPAD + r0 * ns * 2;
  const float* pacc = a.part + r0 * ns * (int64_t)DPAD + cidx * CW;
  const float c = a.scale_log2;

  float m = kNegInf, l = 0.f;
  float acc[CW];
#pragma unroll
  for (int e = 0; e < CW; ++e) acc[e] = 0.f;
  for (int s = j; s < ns; s += SP) {
    const float2 mls = *reinterpret_cast<const float2*>(ml + 2 * s);
    float v[CW];
    load_vec<float, CW>(pacc + (int64_t)s * DPAD, v);
    if (mls.x == kNegInf) continue;  // a split with no visible key
    const float mn = fmaxf(m, mls.x);
    const float w_old = m == kNegInf ? 0.f : __builtin_amdgcn_exp2f((m - mn) * c);
    const float w_new = __builtin_amdgcn_exp2f((mls.x - mn) * c);
    l = w_old * l + w_new * mls.y;
#pragma unroll
    for (int e = 0; e < CW; ++e) acc[e] = w_old * acc[e] + w_new * v[e];
    m = mn;
  }
#pragma unroll
  for (int e = 0; e < CW; ++e) red_acc[t * CW + e] = acc[e];
  red_m[t] = m;
  red_l[t] = l;
  __syncthreads();
  if (!live || j != 0) return;

  float M = m;
  for (int jj = 1; jj < SP; ++jj) M = fmaxf(M, red_m[t + (jj << LOG2C)]);
  const float w0 = m == kNegInf ? 0.f : __builtin_amdgcn_exp2f((m - M) * c);
  float L = w0 * l;
#pragma unroll
  for (int e = 0; e < CW; ++e) acc[e] *= w0;
  for (int jj = 1; jj < SP; ++jj) {
    const int o = t + (jj << LOG2C);
    const float mj = red_m[o];
    const float w = mj == kNegInf ? 0.f : __builtin_amdgcn_exp2f((mj - M) * c);
    L += w * red_l[o];
#pragma unroll
    for (int e = 0; e < CW; ++e) acc[e] += w * red_acc[o * CW + e];
  }
  const float inv = 1.0f / L;
#pragma unroll
  for (int e = 0; e < CW; ++e) acc[e] *= inv;

  int64_t r = row;
  const int i = (int)(r % a.Tq);
  r /= a.Tq;
  const int h = (int)(r % a.H);
  const int64_t b = r / a.H;
  T* yp = static_cast<T*>(a.y) + b * a.yb + (int64_t)i * a.yt + (int64_t)h * a.yh;
  const int d0 = cidx * CW;
  if constexpr (EPL >= CW && !PAIRS) {
    // EPL-element alignment of y (host check) covers a CW-element store
    if (d0 < a.D) store_vec<T, CW>(yp + d0, acc);
  } else {
    static_assert(CW == 4, "combine store width");
    // D is even here (2-element alignment); store the pairs inside D
    const float lo[2] = {acc[0], acc[1]}, hi[2] = {acc[2], acc[3]};
    if (d0 < a.D) store_vec<T, 2>(yp + d0, lo);
    if (d0 + 2 < a.D) store_vec<T, 2>(yp + d0 + 2, hi);
  }
}

// ---------------------------------------------------------------------------
// float64 attention (a GPT.double() model; SDPA in float64, mha.py:61-81):
// one wave per (b, h, i), every key in turn, lane l holding elements
// l, l + 64, ... of the rows (D <= 1024: at most 16); the scores, the online
// softmax (exact running maximum) and the output in float64.  Same masks,
// shared prefix and device position as attn_vec_kernel; no key splits.
// ---------------------------------------------------------------------------
constexpr int kF64Elems = 16;  // 1024 / 64

__global__ __launch_bounds__(256) void attn_f64_kernel(const AttnArgs a, const double scale) {
  const int lane = threadIdx.x & 63;
  const int64_t unit = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (unit >= a.units) return;  // whole waves leave; no barriers follow
  int64_t r = unit;
  const int i = (int)(r % a.Tq);
  r /= a.Tq;
  const int h = (int)(r % a.H);
  const int64_t b = r / a.H;
  int Tk = a.Tk, q_offset = a.q_offset;
  if (a.pos_dev != nullptr) {  // uniform over the grid
    Tk = min(*a.pos_dev + 1, a.Tk);
    q_offset = Tk - 1;
  }
  const int kvis = min(Tk, i + q_offset + 1);
  const double* qp = static_cast<const double*>(a.q) + b * a.qb + (int64_t)i * a.qt + (int64_t)h * a.qh;
  double q[kF64Elems], acc[kF64Elems];
#pragma unroll
  for (int e = 0; e < kF64Elems; ++e) {
    const int d = lane + 64 * e;
    q[e] = d < a.D ? qp[d] : 0.0;
    acc[e] = 0.0;
  }
  const double* kbase = static_cast<const double*>(a.k) + b * a.kb + (int64_t)h * a.kh;
  const double* vbase = static_cast<const double*>(a.v) + b * a.vb + (int64_t)h * a.vh;
  const int64_t grp = b / a.pre.group;
  const double* kpre = static_cast<const double*>(a.pre.k) + grp * a.pre.kb + (int64_t)h * a.pre.kh;
  const double* vpre = static_cast<const double*>(a.pre.v) + grp * a.pre.vb + (int64_t)h * a.pre.vh;
  double m = -__builtin_huge_val(), l = 0.0;
  for (int j = 0; j < kvis; ++j) {
    const bool pre = j < a.pre.len;
    const double* kr = (pre ? kpre : kbase) + (int64_t)j * a.kt;
    const double* vr = (pre ? vpre : vbase) + (int64_t)j * a.vt;
    double dot = 0.0;
#pragma unroll
    for (int e = 0; e < kF64Elems; ++e) {
      const int d = lane + 64 * e;
      if (d < a.D) dot += q[e] * kr[d];
    }
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) dot += __shfl_xor(dot, off, 64);
    const double s = dot * scale;
    if (s > m) {  // wave-uniform: every lane holds the same sum
      const double alpha = exp(m - s);  // 0 for the first key
      l *= alpha;
#pragma unroll
      for (int e = 0; e < kF64Elems; ++e) acc[e] *= alpha;
      m = s;
    }
    const double p = exp(s - m);
    l += p;
#pragma unroll
    for (int e = 0; e < kF64Elems; ++e) {
      const int d = lane + 64 * e;
      if (d < a.D) acc[e] += p * vr[d];
    }
  }
  double* yp = static_cast<double*>(a.y) + b * a.yb + (int64_t)i * a.yt + (int64_t)h * a.yh;
#pragma unroll
  for (int e = 0; e < kF64Elems; ++e) {
    const int d = lane + 64 * e;
    if (d < a.D) yp[d] = acc[e] / l;
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
namespace {

// Key splits aim at 4096 waves: 16 per CU, all resident from the start (the
// kernel takes 72 VGPRs, room for 7 waves per SIMD).  Measured at the
// configs[3] and configs[4] decode shapes: 1.3-2.5 % faster than 8192 waves
// of 4-slot trips (144 VGPRs, 3 waves per SIMD, the grid in 2.7 rounds), and
// within 1-3 % of a bare kernel streaming the same pages.
constexpr int64_t kTargetWaves = 4096;
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

// Key slots per trip: 2 with 16-byte lane slices, 4 with narrower ones (the
// same bytes in flight per wave).  Two register sets of two slots keep the
// kernel at 72 VGPRs.
// Slices of 32 bytes or more (head dims past 256) take one slot per trip.
template <typename T, int EPL>
constexpr int slots_for() {
  return EPL * (int)sizeof(T) >= 32 ? 1 : EPL * (int)sizeof(T) >= 16 ? 2 : 4;
}

template <typename T, int DPAD, int EPL, bool FUSED, bool PAIRS>
int launch_attn(AttnArgs a, hipStream_t s) {
  constexpr int U = slots_for<T, EPL>();
  if (a.nsplit > 1 && a.nsplit <= block_splits(DPAD)) {
    // one workgroup per (b, h, i), one wave per key split, merged in LDS
    const int64_t blocks = a.units / a.nsplit;
    DG_REQUIRE(blocks <= 0x7fffffffLL, DG_EINVAL, "attention: too many units");
    hipLaunchKernelGGL((attn_vec_kernel<T, DPAD, EPL, U, true, FUSED, PAIRS>), dim3((unsigned)blocks),
                       dim3(64 * a.nsplit), 0, s, a);
    return check_launch("attn_vec_kernel");
  }
  const int64_t blocks = (a.units + 3) / 4;
  DG_REQUIRE(blocks <= 0x7fffffffLL, DG_EINVAL, "attention: too many units");
  hipLaunchKernelGGL((attn_vec_kernel<T, DPAD, EPL, U, false, FUSED, PAIRS>), dim3((unsigned)blocks),
                     dim3(256), 0, s, a);
  int rc = check_launch("attn_vec_kernel");
  if (rc != DG_OK || a.nsplit == 1) return rc;
  // combine: C chunks of 4 floats per row times SP split slots, SP <= nsplit
  constexpr int C = DPAD < 4 ? 1 : DPAD / 4;
  int sp_shift = 0;
  while ((1 << sp_shift) < a.nsplit && (C << (sp_shift + 1)) <= 256) ++sp_shift;
  const int64_t rows = a.units / a.nsplit;
  const int64_t rpb = 256 / (C << sp_shift);
  hipLaunchKernelGGL((attn_combine_kernel<T, DPAD, EPL, PAIRS>), dim3((unsigned)((rows + rpb - 1) / rpb)),
                     dim3(256), 0, s, a, sp_shift);
  return check_launch("attn_combine_kernel");
}

// The kernel for a slice choice: vector slices (vec_slice_epl) or pair
// slices (pair_slice_epl; read pair by pair past one pair per lane).
template <typename T, int DPAD, bool FUSED>
int attn_pick_epl(int epl, bool pairs, const AttnArgs& a, hipStream_t s) {
  constexpr int VEC = vec_slice_epl(DPAD, (int)sizeof(T));
  constexpr int PAIR = pair_slice_epl(DPAD);
  if (!pairs && epl == VEC) return launch_attn<T, DPAD, VEC, FUSED, false>(a, s);
  if (pairs && epl == PAIR) return launch_attn<T, DPAD, PAIR, FUSED, (PAIR > 2)>(a, s);
  set_error("attention: no kernel for D pad %d with %d elements per lane", DPAD, epl);
  return DG_EUNSUPPORTED;
}

template <typename T, bool FUSED = false>
int attn_pick_d(int dpad, int epl, bool pairs, const AttnArgs& a, hipStream_t s) {
  switch (dpad) {
    case 2: return attn_pick_epl<T, 2, FUSED>(epl, pairs, a, s);
    case 4: return attn_pick_epl<T, 4, FUSED>(epl, pairs, a, s);
    case 8: return attn_pick_epl<T, 8, FUSED>(epl, pairs, a, s);
    case 16: return attn_pick_epl<T, 16, FUSED>(epl, pairs, a, s);
    case 32: return attn_pick_epl<T, 32, FUSED>(epl, pairs, a, s);
    case 64: return attn_pick_epl<T, 64, FUSED>(epl, pairs, a, s);
    case 128: return attn_pick_epl<T, 128, FUSED>(epl, pairs, a, s);
    case 256: return attn_pick_epl<T, 256, FUSED>(epl, pairs, a, s);
    case 512: return attn_pick_epl<T, 512, FUSED>(epl, pairs, a, s);
    case 1024: return attn_pick_epl<T, 1024, FUSED>(epl, pairs, a, s);
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
  if (ns <= block_splits(next_pow2(D))) return 0;  // merged inside the workgroup
  return (size_t)B * H * Tq * ns * (size_t)(next_pow2(D) + 2) * sizeof(float);
}

// The fused decode step's extra inputs (dg_decode_step): the new token's key
// and value projections and the (cos, sin) table.
struct VecStep {
  const void* kn;
  const dg_stride3* kn_st;
  const void* vn;
  const dg_stride3* vn_st;
  const void* freqs;
  int64_t fpos;
  int fdtype, qknorm, pos;
};

namespace {

// The vector kernel's launch.  With step != nullptr (Tq == 1, Tk = max_pos)
// it is the fused decode step; when the projections or the table are not
// aligned to the kernel's lane slices it launches nothing and sets *declined.
int vec_launch(int B, int H, int Tq, int Tk, int D, int dtype, const void* q, const dg_stride3* q_st,
               const void* k, const dg_stride3* k_st, const void* v, const dg_stride3* v_st, void* y,
               const dg_stride3* y_st, float scale, const PrefixRef& pre, const int* pos_dev, void* workspace,
               size_t workspace_bytes, int size_keys, const VecStep* step, bool* declined, hipStream_t s) {
  // size_keys (>= Tk) sizes the key splits and the workspace: a decode step
  // passes its max_pos, so that the host- and device-position forms split
  // the same way and give the same bits
  const int es = (int)dtype_bytes(dtype);
  const int dpad = next_pow2(D);
  DG_REQUIRE(D <= kMaxHeadDim, DG_EUNSUPPORTED, "attention: head_dim %d > %d", D, kMaxHeadDim);
  DG_REQUIRE(scale > 0.f, DG_EINVAL, "attention: scale must be positive (got %g)", (double)scale);
  if (dtype == DG_F64) {
    if (step != nullptr) {  // the decode step of a float64 model runs as two launches
      *declined = true;
      return DG_OK;
    }
    DG_REQUIRE(aligned(q, 8) && aligned(k, 8) && aligned(v, 8) && aligned(y, 8) && (pre.len == 0 ||
               (aligned(pre.k, 8) && aligned(pre.v, 8))), DG_EINVAL, "attention: float64 rows must be 8-byte aligned");
    DG_REQUIRE(k_st->t >= 0 && v_st->t >= 0, DG_EINVAL, "attention: negative key/value row stride");
    AttnArgs a{};
    a.q = q; a.k = k; a.v = v; a.y = y;
    a.qb = q_st->b; a.qt = q_st->t; a.qh = q_st->h;
    a.kb = k_st->b; a.kt = k_st->t; a.kh = k_st->h;
    a.vb = v_st->b; a.vt = v_st->t; a.vh = v_st->h;
    a.yb = y_st->b; a.yt = y_st->t; a.yh = y_st->h;
    a.H = H; a.Tq = Tq; a.Tk = Tk; a.D = D;
    a.q_offset = Tk - Tq;
    a.pre = pre;
    a.pos_dev = pos_dev;
    a.nsplit = 1;
    a.units = (int64_t)B * H * Tq;
    DG_REQUIRE((a.units + 3) / 4 <= 0x7fffffffLL, DG_EINVAL, "attention: too many units");
    // the ABI's scale is fp32; its rounding of SDPA's default 1/sqrt(D) stands
    // for 1/sqrt(D) in float64, as a float64 model's SDPA applies it
    const double d_inv = 1.0 / sqrt((double)D);
    const double dscale = scale == (float)d_inv ? d_inv : (double)scale;
    hipLaunchKernelGGL(attn_f64_kernel, dim3((unsigned)((a.units + 3) / 4)), dim3(256), 0, s, a, dscale);
    return check_launch("attn_f64_kernel");
  }
  // row offsets inside one (b, h) page are 32-bit in the kernel
  const int64_t span_k = (int64_t)Tk * (k_st->t < 0 ? -k_st->t : k_st->t);
  const int64_t span_v = (int64_t)Tk * (v_st->t < 0 ? -v_st->t : v_st->t);
  DG_REQUIRE(span_k < ((int64_t)1 << 31) && span_v < ((int64_t)1 << 31) && k_st->t >= 0 && v_st->t >= 0,
             DG_EINVAL, "attention: Tk * key/value row stride must be below 2^31 elements");
  // vector slices where D is a multiple of them and every operand is aligned
  // to a load; else pair slices (each operand aligned to a pair)
  auto fits = [&](int epl, bool pairs) {
    if (!pairs && D % epl != 0) return false;
    const int w = pairs ? 2 : slice_load_elems(epl, es);  // elements per access
    const int64_t bytes = (int64_t)w * es;
    const bool pre_ok = pre.len == 0 || (aligned(pre.k, bytes) && aligned(pre.v, bytes) && pre.kb % w == 0 &&
                                         pre.kh % w == 0 && pre.vb % w == 0 && pre.vh % w == 0);
    bool step_ok = true;
    if (step != nullptr) {
      // the table row's slice of a lane: epl elements of the table's dtype
      const int64_t fes = step->fdtype == DG_F32 ? 4 : 2;
      const int64_t fbytes = pairs ? 2 * fes : (epl * fes < 16 ? epl * fes : 16);
      step_ok = aligned(step->kn, bytes) && aligned(step->vn, bytes) && step->kn_st->b % w == 0 &&
                step->kn_st->h % w == 0 && step->vn_st->b % w == 0 && step->vn_st->h % w == 0 &&
                aligned(step->freqs, fbytes) && (step->fpos * fes) % fbytes == 0;
    }
    return aligned(q, bytes) && aligned(k, bytes) && aligned(v, bytes) && aligned(y, bytes) &&
           strides_multiple(q_st, w) && strides_multiple(k_st, w) &&
           strides_multiple(v_st, w) && strides_multiple(y_st, w) && pre_ok && step_ok;
  };
  int epl = 0;
  bool pairs = false;
  if (fits(vec_slice_epl(dpad, es), false)) {
    epl = vec_slice_epl(dpad, es);
  } else if (fits(pair_slice_epl(dpad), true)) {
    epl = pair_slice_epl(dpad);
    pairs = true;
  }
  if (epl == 0 && step != nullptr) {
    *declined = true;
    return DG_OK;
  }
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
  a.lazy_raw = kVecLazyLog2 / a.scale_log2;
  a.pre = pre;
  a.pos_dev = pos_dev;
  if (step != nullptr) {
    a.kn = step->kn; a.vn = step->vn;
    a.knb = step->kn_st->b; a.knh = step->kn_st->h; a.vnb = step->vn_st->b; a.vnh = step->vn_st->h;
    a.freqs = step->freqs; a.fpos = step->fpos;
    a.f32freqs = step->fdtype == DG_F32 ? 1 : 0;
    a.qknorm = step->qknorm;
    a.pos = step->pos;
  }

  DG_REQUIRE(size_keys >= Tk, DG_EINVAL, "attention: split sizing for %d keys below Tk = %d", size_keys, Tk);
  int ns = vec_attention_splits(B, H, Tq, size_keys, D);
  const size_t need = vec_attention_workspace(B, H, Tq, size_keys, D);
  const int in_block = block_splits(dpad);
  if (ns > in_block && (workspace == nullptr || workspace_bytes < need)) {
    DG_REQUIRE(workspace == nullptr, DG_EWORKSPACE,
               "attention: workspace of %zu bytes given, %zu needed", workspace_bytes, need);
    ns = in_block;  // no workspace: as many splits as one workgroup merges
  }
  a.nsplit = ns;
  a.split_len = ns == 1 ? Tk : (((Tk + ns - 1) / ns + 15) / 16) * 16;
  const bool global_splits = ns > in_block;
  a.part = global_splits ? static_cast<float*>(workspace) : nullptr;
  DG_REQUIRE(!global_splits || aligned(workspace, 16), DG_EINVAL, "attention: workspace must be 16-byte aligned");
  a.units = (int64_t)B * H * Tq * ns;
  DG_REQUIRE(a.units < ((int64_t)1 << 31), DG_EINVAL, "attention: B*H*Tq*splits must be below 2^31");

  if (step != nullptr) {
    if (dtype == DG_F32) return attn_pick_d<float, true>(dpad, epl, pairs, a, s);
    if (dtype == DG_BF16) return attn_pick_d<bf16_t, true>(dpad, epl, pairs, a, s);
    return attn_pick_d<f16_t, true>(dpad, epl, pairs, a, s);
  }
  if (dtype == DG_F32) return attn_pick_d<float>(dpad, epl, pairs, a, s);
  if (dtype == DG_BF16) return attn_pick_d<bf16_t>(dpad, epl, pairs, a, s);
  return attn_pick_d<f16_t>(dpad, epl, pairs, a, s);
}

}  // namespace

int vec_attention(int B, int H, int Tq, int Tk, int D, int dtype, const void* q,
                  const dg_stride3* q_st, const void* k, const dg_stride3* k_st, const void* v,
                  const dg_stride3* v_st, void* y, const dg_stride3* y_st, float scale,
                  const PrefixRef& pre, const int* pos_dev, void* workspace,
                  size_t workspace_bytes, int size_keys, hipStream_t s) {
  return vec_launch(B, H, Tq, Tk, D, dtype, q, q_st, k, k_st, v, v_st, y, y_st, scale, pre, pos_dev, workspace,
                    workspace_bytes, size_keys, nullptr, nullptr, s);
}

// The decode step of one new token in one launch of the vector kernel
// (dg_decode_step where the attention runs on it): q, k, v are the token's
// projections, kc / vc the cache pages (written at the position: pos_dev's
// value when set, else pos), keys 0 .. position attended.  The kernel, its
// key splits and the workspace follow max_pos, as in the two-launch form,
// whose y it reproduces bit for bit.  *declined: the projections or the
// table are not aligned to the kernel's lane slices; nothing was launched.
int vec_decode_step(int B, int H, int D, int dtype, const void* q, const dg_stride3* q_st, const void* k,
                    const dg_stride3* k_st, const void* v, const dg_stride3* v_st, void* kc,
                    const dg_stride3* kc_st, void* vc, const dg_stride3* vc_st, const void* freqs, int64_t fpos,
                    int fdtype, int pos, const int* pos_dev, int max_pos, void* y, const dg_stride3* y_st,
                    float scale, const PrefixRef& pre, int qknorm, void* workspace, size_t workspace_bytes,
                    bool* declined, hipStream_t s) {
  *declined = false;
  const VecStep step{k, k_st, v, v_st, freqs, fpos, fdtype, qknorm, pos};
  return vec_launch(B, H, 1, max_pos, D, dtype, q, q_st, kc, kc_st, vc, vc_st, y, y_st, scale, pre, pos_dev,
                    workspace, workspace_bytes, max_pos, &step, declined, s);
}

}  // namespace dg
