// C entry points that are not a single kernel family: version, error slot,
// attention dispatch (MFMA prefill vs. vector kernel) and the strided copy.
#include "dg_common.h"

#include <stdarg.h>
#include <stdio.h>

namespace dg {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return DG_ELAUNCH;
  }
  return DG_OK;
}

// dg_attn_vec.hip
int vec_attention_splits(int B, int H, int Tq, int Tk, int D);
size_t vec_attention_workspace(int B, int H, int Tq, int Tk, int D);
int vec_attention(int B, int H, int Tq, int Tk, int D, int dtype, const void* q,
                  const dg_stride3* q_st, const void* k, const dg_stride3* k_st, const void* v,
                  const dg_stride3* v_st, void* y, const dg_stride3* y_st, float scale,
                  const PrefixRef& pre, const int* pos_dev, void* workspace,
                  size_t workspace_bytes, int size_keys, hipStream_t s);
int vec_decode_step(int B, int H, int D, int dtype, const void* q, const dg_stride3* q_st, const void* k,
                    const dg_stride3* k_st, const void* v, const dg_stride3* v_st, void* kc,
                    const dg_stride3* kc_st, void* vc, const dg_stride3* vc_st, const void* freqs, int64_t fpos,
                    int fdtype, int pos, const int* pos_dev, int max_pos, void* y, const dg_stride3* y_st,
                    float scale, const PrefixRef& pre, int qknorm, void* workspace, size_t workspace_bytes,
                    bool* declined, hipStream_t s);
// dg_attn_shared.hip
bool shared_attention_applicable(int B, int H, int Tq, int Tk, int D, int dtype, const PrefixRef& pre,
                                 const void* q, const dg_stride3* q_st, const void* k,
                                 const dg_stride3* k_st, const void* v, const dg_stride3* v_st,
                                 const void* y, const dg_stride3* y_st);
int shared_attention(int B, int H, int Tk, int D, int dtype, const void* q, const dg_stride3* q_st,
                     const void* k, const dg_stride3* k_st, const void* v, const dg_stride3* v_st,
                     void* y, const dg_stride3* y_st, float scale, const PrefixRef& pre,
                     const int* pos_dev, hipStream_t s);
bool shared_step_applicable(int B, int H, int D, int dtype, const PrefixRef& pre, int max_pos,
                            const void* q, const dg_stride3* q_st, const void* k, const dg_stride3* k_st,
                            const void* v, const dg_stride3* v_st, const void* kc, const dg_stride3* kc_st,
                            const void* vc, const dg_stride3* vc_st, const void* freqs, int64_t fpos,
                            int fdtype, const void* y, const dg_stride3* y_st);
int shared_decode_step(int B, int H, int D, int dtype, const void* q, const dg_stride3* q_st, const void* k,
                       const dg_stride3* k_st, const void* v, const dg_stride3* v_st, void* kc,
                       const dg_stride3* kc_st, void* vc, const dg_stride3* vc_st, const void* freqs,
                       int64_t fpos, int fdtype, int pos, const int* pos_dev, int max_pos, void* y,
                       const dg_stride3* y_st, float scale, const PrefixRef& pre, int qknorm,
                       hipStream_t s);
// dg_rope.hip
int rope_append_at(int B, int H, int D, int dtype, const void* q, const dg_stride3* q_st, void* q_out,
                   const dg_stride3* qo_st, const void* k, const dg_stride3* k_st, void* k_cache,
                   const dg_stride3* kc_st, const void* v, const dg_stride3* v_st, void* v_cache,
                   const dg_stride3* vc_st, const void* freqs, int64_t freqs_pos_stride, int freqs_dtype,
                   const int32_t* pos, int min_pos, int max_pos, int flags, void* stream);
// dg_attn_mfma.hip
bool mfma_prefill_applicable(int B, int H, int Tq, int Tk, int D, int dtype, const void* q,
                             const dg_stride3* q_st, const void* k, const dg_stride3* k_st,
                             const void* v, const dg_stride3* v_st, const void* y,
                             const dg_stride3* y_st, float scale);
int mfma_prefill(int B, int H, int Tq, int Tk, int D, int dtype, const void* q,
                 const dg_stride3* q_st, const void* k, const dg_stride3* k_st, const void* v,
                 const dg_stride3* v_st, void* y, const dg_stride3* y_st, float scale,
                 hipStream_t s);
bool mfma_prefill_rope_applicable(int B, int H, int Tq, int Tk, int D, int dtype, const void* q,
                                  const dg_stride3* q_st, const void* freqs, const dg_stride3* f_st,
                                  int fdtype, const void* k, const dg_stride3* k_st, const void* v,
                                  const dg_stride3* v_st, const void* y, const dg_stride3* y_st,
                                  float scale);
int mfma_prefill_rope(int B, int H, int Tq, int Tk, int D, int dtype, const void* q, const dg_stride3* q_st,
                      const void* freqs, const dg_stride3* f_st, int fdtype, int qknorm, int keys_normed,
                      const void* k, const dg_stride3* k_st, const void* v, const dg_stride3* v_st, void* y,
                      const dg_stride3* y_st, float scale, hipStream_t s);

// ---------------------------------------------------------------------------
// Strided 4-D copy (exact), element size 2, 4 or 8 bytes.
// ---------------------------------------------------------------------------
struct CopyArgs {
  const void* src;
  void* dst;
  int64_t n0, n1, n2, n3;
  int64_t s0, s1, s2, s3;
  int64_t d0, d1, d2, d3;
  int64_t total;
};

template <typename E>
__global__ __launch_bounds__(256) void copy4d_kernel(const CopyArgs a) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < a.total; idx += stride) {
    int64_t r = idx;
    const int64_t i3 = r % a.n3;
    r /= a.n3;
    const int64_t i2 = r % a.n2;
    r /= a.n2;
    const int64_t i1 = r % a.n1;
    const int64_t i0 = r / a.n1;
    const E* s = static_cast<const E*>(a.src) + i0 * a.s0 + i1 * a.s1 + i2 * a.s2 + i3 * a.s3;
    E* d = static_cast<E*>(a.dst) + i0 * a.d0 + i1 * a.d1 + i2 * a.d2 + i3 * a.d3;
    *d = *s;
  }
}

// Rows whose last dimension is contiguous on both sides and a whole number of
// 16-byte chunks: one workgroup per (i0, i1, i2) row, 16-byte loads and
// stores, the row index decomposed once per row.  Strides here are in bytes.
__global__ __launch_bounds__(256) void copy4d_rows_kernel(const CopyArgs a) {
  const int chunks = (int)a.n3;
  for (int64_t row = blockIdx.x; row < a.total; row += gridDim.x) {
    int64_t r = row;
    const int64_t i2 = r % a.n2;
    r /= a.n2;
    const int64_t i1 = r % a.n1;
    const int64_t i0 = r / a.n1;
    const uint4* src = reinterpret_cast<const uint4*>(static_cast<const char*>(a.src) + i0 * a.s0 +
                                                      i1 * a.s1 + i2 * a.s2);
    uint4* dst = reinterpret_cast<uint4*>(static_cast<char*>(a.dst) + i0 * a.d0 + i1 * a.d1 + i2 * a.d2);
    for (int c = threadIdx.x; c < chunks; c += blockDim.x) dst[c] = src[c];
  }
}

// The dg_prefix of a call as the kernels read it (PrefixRef), after checking
// it against the cache views: positions t < len of row b come from the
// group's prefix pages (the group's first row of the cache when prefix->k is
// NULL); the cache views, which start at position own_start, are shifted so
// that the kernels index every cache position absolutely.  limit is the
// number of positions the call covers (Tk, or max_pos).
int resolve_prefix(const dg_prefix* p, int limit, int dtype, const char* what, const void*& k,
                   const dg_stride3* k_st, const void*& v, const dg_stride3* v_st, PrefixRef& out) {
  out = PrefixRef{k, v, 0, 0, 0, 0, 0, 1, 0};
  if (p == nullptr) return DG_OK;
  DG_REQUIRE(p->group >= 1, DG_EINVAL, "%s: prefix group must be >= 1 (got %d)", what, p->group);
  DG_REQUIRE(p->len >= 0 && p->len <= limit, DG_EINVAL, "%s: prefix len %d outside [0, %d]", what, p->len,
             limit);
  DG_REQUIRE((p->k == nullptr) == (p->v == nullptr), DG_EINVAL, "%s: prefix k and v must both be given or NULL",
             what);
  DG_REQUIRE(p->own_start >= 0 && p->own_start <= p->len, DG_EINVAL,
             "%s: prefix own_start %d outside [0, len=%d]", what, p->own_start, p->len);
  DG_REQUIRE(p->k != nullptr || p->own_start == 0, DG_EINVAL,
             "%s: own_start > 0 needs prefix pages of their own (k, v)", what);
  if (p->k == nullptr && (p->group == 1 || p->len == 0)) return DG_OK;  // no sharing
  if (p->k != nullptr) {
    DG_REQUIRE(p->k_st.t == k_st->t && p->v_st.t == v_st->t, DG_EINVAL,
               "%s: prefix pages must have the cache's position stride", what);
    const int64_t es = dtype_bytes(dtype);
    k = static_cast<const char*>(k) - (int64_t)p->own_start * k_st->t * es;
    v = static_cast<const char*>(v) - (int64_t)p->own_start * v_st->t * es;
    out = PrefixRef{p->k, p->v, p->k_st.b, p->k_st.h, p->v_st.b, p->v_st.h, p->len, p->group, p->own_start};
  } else {
    out = PrefixRef{k, v, (int64_t)p->group * k_st->b, k_st->h, (int64_t)p->group * v_st->b, v_st->h,
                    p->len, p->group, 0};
  }
  if (p->len == 0) out.len = 0;
  return DG_OK;
}

}  // namespace dg

using namespace dg;

extern "C" int dg_abi_version(void) { return DG_ABI_VERSION; }

extern "C" const char* dg_last_error(void) { return g_err; }

extern "C" size_t dg_attention_workspace_size(int B, int H, int Tq, int Tk, int D, int dtype) {
  // float64 runs on a kernel without key splits
  if (B <= 0 || H <= 0 || Tq <= 0 || Tk <= 0 || D <= 0 || dtype == DG_F64) return 0;
  return vec_attention_workspace(B, H, Tq, Tk, D);
}

extern "C" int dg_attention_grouped(int B, int H, int Tq, int Tk, int D, int dtype, const void* q,
                                    const dg_stride3* q_st, const void* k, const dg_stride3* k_st,
                                    const void* v, const dg_stride3* v_st, void* y,
                                    const dg_stride3* y_st, float scale, const dg_prefix* prefix,
                                    void* workspace, size_t workspace_bytes, void* stream) {
  DG_REQUIRE(B >= 0 && H >= 0 && Tq >= 0 && Tk >= 0, DG_EINVAL, "attention: negative size");
  DG_REQUIRE(dtype == DG_F32 || dtype == DG_BF16 || dtype == DG_F16 || dtype == DG_F64, DG_EUNSUPPORTED,
             "attention: dtype %d unsupported", dtype);
  DG_REQUIRE(D >= 2 && D % 2 == 0, DG_EINVAL, "attention: head_dim must be even (got %d)", D);
  if ((int64_t)B * H * Tq == 0) return DG_OK;
  DG_REQUIRE(Tk >= Tq, DG_EINVAL, "attention: Tk (%d) < Tq (%d)", Tk, Tq);
  DG_REQUIRE(q && k && v && y && q_st && k_st && v_st && y_st, DG_EINVAL, "attention: NULL argument");
  const void* kk = k;
  const void* vv = v;
  PrefixRef pre;
  const int rc = resolve_prefix(prefix, Tk, dtype, "attention", kk, k_st, vv, v_st, pre);
  if (rc != DG_OK) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // The MFMA prefill kernel reads every row's own keys: equal results when
  // the rows hold the prefix themselves (identical within a group).
  const bool rows_hold_all = prefix == nullptr || prefix->k == nullptr;
  if (rows_hold_all &&
      mfma_prefill_applicable(B, H, Tq, Tk, D, dtype, q, q_st, k, k_st, v, v_st, y, y_st, scale))
    return mfma_prefill(B, H, Tq, Tk, D, dtype, q, q_st, k, k_st, v, v_st, y, y_st, scale, s);
  // Groups of at least 16 rows: the shared prefix as a matrix product (when the
  // vector kernel would not split the keys, so no workspace is involved).
  if (vec_attention_splits(B, H, Tq, Tk, D) == 1 &&
      shared_attention_applicable(B, H, Tq, Tk, D, dtype, pre, q, q_st, kk, k_st, vv, v_st, y, y_st))
    return shared_attention(B, H, Tk, D, dtype, q, q_st, kk, k_st, vv, v_st, y, y_st, scale, pre, nullptr, s);
  return vec_attention(B, H, Tq, Tk, D, dtype, q, q_st, kk, k_st, vv, v_st, y, y_st, scale, pre, nullptr,
                       workspace, workspace_bytes, Tk, s);
}

extern "C" int dg_prefill_rope(int B, int H, int Tq, int Tk, int D, int dtype, const void* q,
                               const dg_stride3* q_st, const void* freqs, const dg_stride3* f_st,
                               int freqs_dtype, int flags, const void* k, const dg_stride3* k_st,
                               const void* v, const dg_stride3* v_st, void* y, const dg_stride3* y_st,
                               float scale, void* stream) {
  DG_REQUIRE(B >= 0 && H >= 0 && Tq >= 0 && Tk >= 0, DG_EINVAL, "prefill_rope: negative size");
  DG_REQUIRE(dtype == DG_F32 || dtype == DG_BF16 || dtype == DG_F16, DG_EUNSUPPORTED,
             "prefill_rope: dtype %d unsupported", dtype);
  DG_REQUIRE(freqs_dtype == DG_F32 || freqs_dtype == DG_BF16 || freqs_dtype == DG_F16, DG_EUNSUPPORTED,
             "prefill_rope: freqs dtype %d unsupported", freqs_dtype);
  DG_REQUIRE(D >= 2 && D % 2 == 0, DG_EINVAL, "prefill_rope: head_dim must be even (got %d)", D);
  DG_REQUIRE((flags & ~(DG_QKNORM | DG_KEYS_NORMED)) == 0, DG_EINVAL, "prefill_rope: unknown flags 0x%x", flags);
  DG_REQUIRE(!(flags & DG_KEYS_NORMED) || (flags & DG_QKNORM), DG_EINVAL,
             "prefill_rope: DG_KEYS_NORMED needs DG_QKNORM (bounded scores need both rows normalised)");
  if ((int64_t)B * H * Tq == 0) return DG_OK;
  DG_REQUIRE(Tk >= Tq, DG_EINVAL, "prefill_rope: Tk (%d) < Tq (%d)", Tk, Tq);
  DG_REQUIRE(q && freqs && k && v && y && q_st && f_st && k_st && v_st && y_st, DG_EINVAL,
             "prefill_rope: NULL argument");
  DG_REQUIRE(mfma_prefill_rope_applicable(B, H, Tq, Tk, D, dtype, q, q_st, freqs, f_st, freqs_dtype, k, k_st, v,
                                          v_st, y, y_st, scale),
             DG_EUNSUPPORTED,
             "prefill_rope: not taken by the fused kernels (bf16/fp16/fp32, head_dim 64 or 128, Tq >= 16, "
             "16-byte aligned rows); use dg_rope_qknorm_append + dg_attention");
  return mfma_prefill_rope(B, H, Tq, Tk, D, dtype, q, q_st, freqs, f_st, freqs_dtype, (flags & DG_QKNORM) != 0,
                           (flags & DG_KEYS_NORMED) != 0, k, k_st, v, v_st, y, y_st, scale,
                           static_cast<hipStream_t>(stream));
}

extern "C" size_t dg_decode_attention_at_workspace_size(int B, int H, int max_keys, int D, int dtype) {
  return dg_attention_workspace_size(B, H, 1, max_keys, D, dtype);
}

extern "C" int dg_decode_attention_at(int B, int H, int D, int dtype, const void* q,
                                      const dg_stride3* q_st, const void* k_cache,
                                      const dg_stride3* kc_st, const void* v_cache,
                                      const dg_stride3* vc_st, void* y, const dg_stride3* y_st,
                                      float scale, const dg_prefix* prefix, const int32_t* pos,
                                      int max_keys, void* workspace, size_t workspace_bytes,
                                      void* stream) {
  DG_REQUIRE(B >= 0 && H >= 0, DG_EINVAL, "attention_at: negative size");
  DG_REQUIRE(dtype == DG_F32 || dtype == DG_BF16 || dtype == DG_F16 || dtype == DG_F64, DG_EUNSUPPORTED,
             "attention_at: dtype %d unsupported", dtype);
  DG_REQUIRE(D >= 2 && D % 2 == 0, DG_EINVAL, "attention_at: head_dim must be even (got %d)", D);
  DG_REQUIRE(max_keys >= 1, DG_EINVAL, "attention_at: max_keys must be >= 1 (got %d)", max_keys);
  if ((int64_t)B * H == 0) return DG_OK;
  DG_REQUIRE(pos && q && k_cache && v_cache && y && q_st && kc_st && vc_st && y_st, DG_EINVAL,
             "attention_at: NULL argument");
  const void* kk = k_cache;
  const void* vv = v_cache;
  PrefixRef pre;
  const int rc = resolve_prefix(prefix, max_keys, dtype, "attention_at", kk, kc_st, vv, vc_st, pre);
  if (rc != DG_OK) return rc;
  // The kernels read at most max_keys keys (Tk = min(*pos + 1, max_keys)); key
  // splits and the workspace are sized for max_keys.
  if (vec_attention_splits(B, H, 1, max_keys, D) == 1 &&
      shared_attention_applicable(B, H, 1, max_keys, D, dtype, pre, q, q_st, kk, kc_st, vv, vc_st, y, y_st))
    return shared_attention(B, H, max_keys, D, dtype, q, q_st, kk, kc_st, vv, vc_st, y, y_st, scale, pre, pos,
                            static_cast<hipStream_t>(stream));
  return vec_attention(B, H, 1, max_keys, D, dtype, q, q_st, kk, kc_st, vv, vc_st, y, y_st, scale, pre, pos,
                       workspace, workspace_bytes, max_keys, static_cast<hipStream_t>(stream));
}

extern "C" size_t dg_decode_step_workspace_size(int B, int H, int max_pos, int D, int dtype) {
  return dg_attention_workspace_size(B, H, 1, max_pos, D, dtype);
}

extern "C" int dg_decode_step(int B, int H, int D, int dtype, const void* q, const dg_stride3* q_st,
                              const void* k, const dg_stride3* k_st, const void* v, const dg_stride3* v_st,
                              void* k_cache, const dg_stride3* kc_st, void* v_cache, const dg_stride3* vc_st,
                              const void* freqs, int64_t freqs_pos_stride, int freqs_dtype, int pos,
                              const int32_t* pos_dev, int max_pos, void* y, const dg_stride3* y_st,
                              float scale, const dg_prefix* prefix, int flags, void* workspace,
                              size_t workspace_bytes, void* stream) {
  DG_REQUIRE(B >= 0 && H >= 0, DG_EINVAL, "decode_step: negative size");
  DG_REQUIRE(dtype == DG_F32 || dtype == DG_BF16 || dtype == DG_F16 || dtype == DG_F64, DG_EUNSUPPORTED,
             "decode_step: dtype %d unsupported", dtype);
  DG_REQUIRE(freqs_dtype == DG_F32 || freqs_dtype == dtype, DG_EUNSUPPORTED,
             "decode_step: freqs dtype %d unsupported (fp32 or the data's dtype)", freqs_dtype);
  DG_REQUIRE(D >= 2 && D % 2 == 0, DG_EINVAL, "decode_step: head_dim must be even (got %d)", D);
  DG_REQUIRE(max_pos >= 1, DG_EINVAL, "decode_step: max_pos must be >= 1 (got %d)", max_pos);
  DG_REQUIRE(freqs_pos_stride >= 0, DG_EINVAL, "decode_step: negative freqs_pos_stride");
  DG_REQUIRE(kc_st && vc_st, DG_EINVAL, "decode_step: NULL cache strides");
  const void* kk = k_cache;
  const void* vv = v_cache;
  PrefixRef pre;
  int rc = resolve_prefix(prefix, max_pos, dtype, "decode_step", kk, kc_st, vv, vc_st, pre);
  if (rc != DG_OK) return rc;
  DG_REQUIRE(pre.own_start < max_pos, DG_EINVAL, "decode_step: the cache pages hold no position (own_start %d, "
             "max_pos %d)", pre.own_start, max_pos);
  if (pos_dev == nullptr) {
    DG_REQUIRE(pos >= 0 && pos < max_pos, DG_EINVAL, "decode_step: position %d outside [0, max_pos=%d)", pos,
               max_pos);
    DG_REQUIRE(pos >= pre.len, DG_EINVAL, "decode_step: position %d inside the shared prefix (len %d)", pos,
               pre.len);
  }
  if ((int64_t)B * H == 0) return DG_OK;
  DG_REQUIRE(q && k && v && k_cache && v_cache && freqs && y && q_st && k_st && v_st && y_st, DG_EINVAL,
             "decode_step: NULL argument");
  void* kw = const_cast<void*>(kk);
  void* vw = const_cast<void*>(vv);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int qknorm = (flags & DG_QKNORM) ? 1 : 0;
  if (vec_attention_splits(B, H, 1, max_pos, D) == 1 &&
      shared_step_applicable(B, H, D, dtype, pre, max_pos, q, q_st, k, k_st, v, v_st, kw, kc_st, vw, vc_st,
                             freqs, freqs_pos_stride, freqs_dtype, y, y_st))
    return shared_decode_step(B, H, D, dtype, q, q_st, k, k_st, v, v_st, kw, kc_st, vw, vc_st, freqs,
                              freqs_pos_stride, freqs_dtype, pos, pos_dev, max_pos, y, y_st, scale, pre, qknorm,
                              s);
  // Where the attention runs on the vector kernel: one launch of its fused
  // form, with the two launches' bits (below), unless the projections or the
  // table are not aligned to its lane slices.
  const bool vector_attention =
      !(vec_attention_splits(B, H, 1, max_pos, D) == 1 &&
        shared_attention_applicable(B, H, 1, max_pos, D, dtype, pre, y, y_st, kw, kc_st, vw, vc_st, y, y_st));
  if (vector_attention && (freqs_dtype == DG_F32 || freqs_dtype == dtype)) {
    bool declined = false;
    rc = vec_decode_step(B, H, D, dtype, q, q_st, k, k_st, v, v_st, kw, kc_st, vw, vc_st, freqs, freqs_pos_stride,
                         freqs_dtype, pos, pos_dev, max_pos, y, y_st, scale, pre, qknorm, workspace,
                         workspace_bytes, &declined, s);
    if (!declined) return rc;
  }
  // Two launches: RoPE/QK-norm/append with the rotated q staged in y, then the
  // attention reading q from y (every attention kernel reads a query row
  // before it writes the output row at the same place).  Both index the
  // shifted cache pointers absolutely.
  if (pos_dev != nullptr) {
    rc = rope_append_at(B, H, D, dtype, q, q_st, y, y_st, k, k_st, kw, kc_st, v, v_st, vw, vc_st, freqs,
                        freqs_pos_stride, freqs_dtype, pos_dev, pre.own_start, max_pos, flags, stream);
    if (rc != DG_OK) return rc;
    return vec_attention_splits(B, H, 1, max_pos, D) == 1 &&
                   shared_attention_applicable(B, H, 1, max_pos, D, dtype, pre, y, y_st, kw, kc_st, vw, vc_st, y,
                                               y_st)
               ? shared_attention(B, H, max_pos, D, dtype, y, y_st, kw, kc_st, vw, vc_st, y, y_st, scale, pre,
                                  pos_dev, s)
               : vec_attention(B, H, 1, max_pos, D, dtype, y, y_st, kw, kc_st, vw, vc_st, y, y_st, scale, pre,
                               pos_dev, workspace, workspace_bytes, max_pos, s);
  }
  const int64_t es = dtype_bytes(dtype), fes = dtype_bytes(freqs_dtype);
  const dg_stride3 f_st = {0, 0, 0};
  rc = dg_rope_qknorm_append(B, 1, H, D, dtype, q, q_st, y, y_st, k, k_st,
                             static_cast<char*>(kw) + (int64_t)pos * kc_st->t * es, kc_st, v, v_st,
                             static_cast<char*>(vw) + (int64_t)pos * vc_st->t * es, vc_st,
                             static_cast<const char*>(freqs) + (int64_t)pos * freqs_pos_stride * fes, &f_st,
                             freqs_dtype, flags, stream);
  if (rc != DG_OK) return rc;
  // the kernel, its key splits and the workspace are chosen for max_pos, as
  // the device-position form must: both forms give the same bits
  return vec_attention_splits(B, H, 1, max_pos, D) == 1 &&
                 shared_attention_applicable(B, H, 1, max_pos, D, dtype, pre, y, y_st, kw, kc_st, vw, vc_st, y,
                                             y_st)
             ? shared_attention(B, H, pos + 1, D, dtype, y, y_st, kw, kc_st, vw, vc_st, y, y_st, scale, pre,
                                nullptr, s)
             : vec_attention(B, H, 1, pos + 1, D, dtype, y, y_st, kw, kc_st, vw, vc_st, y, y_st, scale, pre,
                             nullptr, workspace, workspace_bytes, max_pos, s);
}

extern "C" int dg_attention(int B, int H, int Tq, int Tk, int D, int dtype, const void* q,
                            const dg_stride3* q_st, const void* k, const dg_stride3* k_st,
                            const void* v, const dg_stride3* v_st, void* y,
                            const dg_stride3* y_st, float scale, void* workspace,
                            size_t workspace_bytes, void* stream) {
  return dg_attention_grouped(B, H, Tq, Tk, D, dtype, q, q_st, k, k_st, v, v_st, y, y_st, scale, nullptr,
                              workspace, workspace_bytes, stream);
}

extern "C" int dg_copy4d(int dtype, const int64_t* shape, const void* src, const int64_t* src_st,
                         void* dst, const int64_t* dst_st, void* stream) {
  DG_REQUIRE(dtype == DG_F32 || dtype == DG_BF16 || dtype == DG_F16 || dtype == DG_F64, DG_EUNSUPPORTED,
             "copy4d: dtype %d unsupported", dtype);
  DG_REQUIRE(shape && src_st && dst_st, DG_EINVAL, "copy4d: NULL shape/strides");
  for (int i = 0; i < 4; ++i) DG_REQUIRE(shape[i] >= 0, DG_EINVAL, "copy4d: negative extent");
  CopyArgs a{};
  a.total = shape[0] * shape[1] * shape[2] * shape[3];
  if (a.total == 0) return DG_OK;
  DG_REQUIRE(src && dst, DG_EINVAL, "copy4d: NULL pointer");
  a.src = src;
  a.dst = dst;
  a.n0 = shape[0]; a.n1 = shape[1]; a.n2 = shape[2]; a.n3 = shape[3];
  a.s0 = src_st[0]; a.s1 = src_st[1]; a.s2 = src_st[2]; a.s3 = src_st[3];
  a.d0 = dst_st[0]; a.d1 = dst_st[1]; a.d2 = dst_st[2]; a.d3 = dst_st[3];
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t es = dtype_bytes(dtype);
  const int64_t row_bytes = shape[3] * es;
  auto bytes16 = [&](int64_t stride) { return (stride * es) % 16 == 0; };
  if (src_st[3] == 1 && dst_st[3] == 1 && row_bytes % 16 == 0 &&
      (reinterpret_cast<uintptr_t>(src) & 15) == 0 && (reinterpret_cast<uintptr_t>(dst) & 15) == 0 &&
      bytes16(src_st[0]) && bytes16(src_st[1]) && bytes16(src_st[2]) && bytes16(dst_st[0]) &&
      bytes16(dst_st[1]) && bytes16(dst_st[2]) && row_bytes / 16 <= 0x7fffffffLL) {
    CopyArgs r = a;
    r.total = shape[0] * shape[1] * shape[2];  // rows
    r.n3 = row_bytes / 16;                     // 16-byte chunks per row
    r.s0 = src_st[0] * es; r.s1 = src_st[1] * es; r.s2 = src_st[2] * es;
    r.d0 = dst_st[0] * es; r.d1 = dst_st[1] * es; r.d2 = dst_st[2] * es;
    const int64_t grid = r.total < 262144 ? r.total : 262144;
    hipLaunchKernelGGL(copy4d_rows_kernel, dim3((unsigned)grid), dim3(256), 0, s, r);
    return check_launch("copy4d_rows_kernel");
  }
  int64_t blocks = (a.total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (dtype == DG_F64)
    hipLaunchKernelGGL(copy4d_kernel<uint64_t>, dim3((unsigned)blocks), dim3(256), 0, s, a);
  else if (dtype == DG_F32)
    hipLaunchKernelGGL(copy4d_kernel<uint32_t>, dim3((unsigned)blocks), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(copy4d_kernel<uint16_t>, dim3((unsigned)blocks), dim3(256), 0, s, a);
  return check_launch("copy4d_kernel");
}
