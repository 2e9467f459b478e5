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
                  int prefix_len, int group, const int* pos_dev, void* workspace,
                  size_t workspace_bytes, hipStream_t s);
// dg_attn_shared.hip
bool shared_attention_applicable(int B, int H, int Tq, int Tk, int D, int dtype, int prefix_len,
                                 int group, const void* q, const dg_stride3* q_st, const void* k,
                                 const dg_stride3* k_st, const void* v, const dg_stride3* v_st,
                                 const void* y, const dg_stride3* y_st);
int shared_attention(int B, int H, int Tk, int D, int dtype, const void* q, const dg_stride3* q_st,
                     const void* k, const dg_stride3* k_st, const void* v, const dg_stride3* v_st,
                     void* y, const dg_stride3* y_st, float scale, int prefix_len, int group,
                     const int* pos_dev, hipStream_t s);
bool shared_step_applicable(int B, int H, int D, int dtype, int prefix_len, int group, int max_pos,
                            const void* q, const dg_stride3* q_st, const void* k, const dg_stride3* k_st,
                            const void* v, const dg_stride3* v_st, const void* kc, const dg_stride3* kc_st,
                            const void* vc, const dg_stride3* vc_st, const void* freqs, int64_t fpos,
                            int fdtype, const void* y, const dg_stride3* y_st);
int shared_decode_step(int B, int H, int D, int dtype, const void* q, const dg_stride3* q_st, const void* k,
                       const dg_stride3* k_st, const void* v, const dg_stride3* v_st, void* kc,
                       const dg_stride3* kc_st, void* vc, const dg_stride3* vc_st, const void* freqs,
                       int64_t fpos, int fdtype, int pos, const int* pos_dev, int max_pos, void* y,
                       const dg_stride3* y_st, float scale, int prefix_len, int group, int qknorm,
                       hipStream_t s);
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
// Strided 4-D copy (exact), element size 2 or 4 bytes.
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

}  // namespace dg

using namespace dg;

extern "C" int dg_abi_version(void) { return DG_ABI_VERSION; }

extern "C" const char* dg_last_error(void) { return g_err; }

extern "C" size_t dg_attention_workspace_size(int B, int H, int Tq, int Tk, int D, int dtype) {
  (void)dtype;
  if (B <= 0 || H <= 0 || Tq <= 0 || Tk <= 0 || D <= 0) return 0;
  return vec_attention_workspace(B, H, Tq, Tk, D);
}

extern "C" int dg_attention_grouped(int B, int H, int Tq, int Tk, int D, int dtype, const void* q,
                                    const dg_stride3* q_st, const void* k, const dg_stride3* k_st,
                                    const void* v, const dg_stride3* v_st, void* y,
                                    const dg_stride3* y_st, float scale, int prefix_len, int group,
                                    void* workspace, size_t workspace_bytes, void* stream) {
  DG_REQUIRE(B >= 0 && H >= 0 && Tq >= 0 && Tk >= 0, DG_EINVAL, "attention: negative size");
  DG_REQUIRE(dtype == DG_F32 || dtype == DG_BF16 || dtype == DG_F16, DG_EUNSUPPORTED,
             "attention: dtype %d unsupported", dtype);
  DG_REQUIRE(D >= 2 && D % 2 == 0, DG_EINVAL, "attention: head_dim must be even (got %d)", D);
  DG_REQUIRE(group >= 1, DG_EINVAL, "attention: group must be >= 1 (got %d)", group);
  DG_REQUIRE(prefix_len >= 0 && prefix_len <= Tk, DG_EINVAL,
             "attention: prefix_len %d outside [0, Tk=%d]", prefix_len, Tk);
  if ((int64_t)B * H * Tq == 0) return DG_OK;
  DG_REQUIRE(Tk >= Tq, DG_EINVAL, "attention: Tk (%d) < Tq (%d)", Tk, Tq);
  DG_REQUIRE(q && k && v && y && q_st && k_st && v_st && y_st, DG_EINVAL, "attention: NULL argument");
  hipStream_t s = static_cast<hipStream_t>(stream);
  // The MFMA prefill kernel reads every row's own keys: equal results, since
  // the rows of a group hold identical prefixes.
  if (mfma_prefill_applicable(B, H, Tq, Tk, D, dtype, q, q_st, k, k_st, v, v_st, y, y_st, scale))
    return mfma_prefill(B, H, Tq, Tk, D, dtype, q, q_st, k, k_st, v, v_st, y, y_st, scale, s);
  if (group == 1) prefix_len = 0;
  // Groups of at least 16 rows: the shared prefix as a matrix product (when the
  // vector kernel would not split the keys, so no workspace is involved).
  if (vec_attention_splits(B, H, Tq, Tk, D) == 1 &&
      shared_attention_applicable(B, H, Tq, Tk, D, dtype, prefix_len, group, q, q_st, k, k_st, v, v_st,
                                  y, y_st))
    return shared_attention(B, H, Tk, D, dtype, q, q_st, k, k_st, v, v_st, y, y_st, scale, prefix_len,
                            group, nullptr, s);
  return vec_attention(B, H, Tq, Tk, D, dtype, q, q_st, k, k_st, v, v_st, y, y_st, scale, prefix_len,
                       group, nullptr, workspace, workspace_bytes, s);
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
             "prefill_rope: not taken by the fused kernel (bf16/fp16, head_dim 64 or 128, Tq >= 16, "
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
                                      float scale, int prefix_len, int group, const int32_t* pos,
                                      int max_keys, void* workspace, size_t workspace_bytes,
                                      void* stream) {
  DG_REQUIRE(B >= 0 && H >= 0, DG_EINVAL, "attention_at: negative size");
  DG_REQUIRE(dtype == DG_F32 || dtype == DG_BF16 || dtype == DG_F16, DG_EUNSUPPORTED,
             "attention_at: dtype %d unsupported", dtype);
  DG_REQUIRE(D >= 2 && D % 2 == 0, DG_EINVAL, "attention_at: head_dim must be even (got %d)", D);
  DG_REQUIRE(max_keys >= 1, DG_EINVAL, "attention_at: max_keys must be >= 1 (got %d)", max_keys);
  DG_REQUIRE(group >= 1, DG_EINVAL, "attention_at: group must be >= 1 (got %d)", group);
  DG_REQUIRE(prefix_len >= 0 && prefix_len <= max_keys, DG_EINVAL,
             "attention_at: prefix_len %d outside [0, max_keys=%d]", prefix_len, max_keys);
  if ((int64_t)B * H == 0) return DG_OK;
  DG_REQUIRE(pos && q && k_cache && v_cache && y && q_st && kc_st && vc_st && y_st, DG_EINVAL,
             "attention_at: NULL argument");
  if (group == 1) prefix_len = 0;
  // The kernels read at most max_keys keys (Tk = min(*pos + 1, max_keys)); key
  // splits and the workspace are sized for max_keys.
  if (vec_attention_splits(B, H, 1, max_keys, D) == 1 &&
      shared_attention_applicable(B, H, 1, max_keys, D, dtype, prefix_len, group, q, q_st, k_cache, kc_st,
                                  v_cache, vc_st, y, y_st))
    return shared_attention(B, H, max_keys, D, dtype, q, q_st, k_cache, kc_st, v_cache, vc_st, y, y_st,
                            scale, prefix_len, group, pos, static_cast<hipStream_t>(stream));
  return vec_attention(B, H, 1, max_keys, D, dtype, q, q_st, k_cache, kc_st, v_cache, vc_st, y, y_st,
                       scale, prefix_len, group, pos, workspace, workspace_bytes,
                       static_cast<hipStream_t>(stream));
}

extern "C" size_t dg_decode_step_workspace_size(int B, int H, int max_pos, int D, int dtype) {
  return dg_attention_workspace_size(B, H, 1, max_pos, D, dtype);
}

extern "C" int dg_decode_step(int B, int H, int D, int dtype, const void* q, const dg_stride3* q_st,
                              const void* k, const dg_stride3* k_st, const void* v, const dg_stride3* v_st,
                              void* k_cache, const dg_stride3* kc_st, void* v_cache, const dg_stride3* vc_st,
                              const void* freqs, int64_t freqs_pos_stride, int freqs_dtype, int pos,
                              const int32_t* pos_dev, int max_pos, void* y, const dg_stride3* y_st,
                              float scale, int prefix_len, int group, int flags, void* workspace,
                              size_t workspace_bytes, void* stream) {
  DG_REQUIRE(B >= 0 && H >= 0, DG_EINVAL, "decode_step: negative size");
  DG_REQUIRE(dtype == DG_F32 || dtype == DG_BF16 || dtype == DG_F16, DG_EUNSUPPORTED,
             "decode_step: dtype %d unsupported", dtype);
  DG_REQUIRE(freqs_dtype == DG_F32 || freqs_dtype == DG_BF16 || freqs_dtype == DG_F16, DG_EUNSUPPORTED,
             "decode_step: freqs dtype %d unsupported", freqs_dtype);
  DG_REQUIRE(D >= 2 && D % 2 == 0, DG_EINVAL, "decode_step: head_dim must be even (got %d)", D);
  DG_REQUIRE(max_pos >= 1, DG_EINVAL, "decode_step: max_pos must be >= 1 (got %d)", max_pos);
  DG_REQUIRE(group >= 1, DG_EINVAL, "decode_step: group must be >= 1 (got %d)", group);
  DG_REQUIRE(prefix_len >= 0 && prefix_len <= max_pos, DG_EINVAL,
             "decode_step: prefix_len %d outside [0, max_pos=%d]", prefix_len, max_pos);
  DG_REQUIRE(freqs_pos_stride >= 0, DG_EINVAL, "decode_step: negative freqs_pos_stride");
  if (pos_dev == nullptr) {
    DG_REQUIRE(pos >= 0 && pos < max_pos, DG_EINVAL, "decode_step: position %d outside [0, max_pos=%d)", pos,
               max_pos);
    DG_REQUIRE(group == 1 || prefix_len <= pos, DG_EINVAL,
               "decode_step: position %d inside the shared prefix (prefix_len %d)", pos, prefix_len);
  }
  if ((int64_t)B * H == 0) return DG_OK;
  DG_REQUIRE(q && k && v && k_cache && v_cache && freqs && y && q_st && k_st && v_st && kc_st && vc_st && y_st,
             DG_EINVAL, "decode_step: NULL argument");
  if (group == 1) prefix_len = 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int qknorm = (flags & DG_QKNORM) ? 1 : 0;
  if (vec_attention_splits(B, H, 1, max_pos, D) == 1 &&
      shared_step_applicable(B, H, D, dtype, prefix_len, group, max_pos, q, q_st, k, k_st, v, v_st, k_cache,
                             kc_st, v_cache, vc_st, freqs, freqs_pos_stride, freqs_dtype, y, y_st))
    return shared_decode_step(B, H, D, dtype, q, q_st, k, k_st, v, v_st, k_cache, kc_st, v_cache, vc_st, freqs,
                              freqs_pos_stride, freqs_dtype, pos, pos_dev, max_pos, y, y_st, scale, prefix_len,
                              group, qknorm, s);
  // Two launches: RoPE/QK-norm/append with the rotated q staged in y, then the
  // attention reading q from y (every attention kernel reads a query row
  // before it writes the output row at the same place).
  int rc;
  if (pos_dev != nullptr) {
    rc = dg_rope_qknorm_append_at(B, H, D, dtype, q, q_st, y, y_st, k, k_st, k_cache, kc_st, v, v_st, v_cache,
                                  vc_st, freqs, freqs_pos_stride, freqs_dtype, pos_dev, max_pos, flags, stream);
    if (rc != DG_OK) return rc;
    return dg_decode_attention_at(B, H, D, dtype, y, y_st, k_cache, kc_st, v_cache, vc_st, y, y_st, scale,
                                  prefix_len, group, pos_dev, max_pos, workspace, workspace_bytes, stream);
  }
  const int64_t es = dtype == DG_F32 ? 4 : 2, fes = freqs_dtype == DG_F32 ? 4 : 2;
  const dg_stride3 f_st = {0, 0, 0};
  rc = dg_rope_qknorm_append(B, 1, H, D, dtype, q, q_st, y, y_st, k, k_st,
                             static_cast<char*>(k_cache) + (int64_t)pos * kc_st->t * es, kc_st, v, v_st,
                             static_cast<char*>(v_cache) + (int64_t)pos * vc_st->t * es, vc_st,
                             static_cast<const char*>(freqs) + (int64_t)pos * freqs_pos_stride * fes, &f_st,
                             freqs_dtype, flags, stream);
  if (rc != DG_OK) return rc;
  return dg_attention_grouped(B, H, 1, pos + 1, D, dtype, y, y_st, k_cache, kc_st, v_cache, vc_st, y, y_st, scale,
                              prefix_len, group, workspace, workspace_bytes, stream);
}

extern "C" int dg_attention(int B, int H, int Tq, int Tk, int D, int dtype, const void* q,
                            const dg_stride3* q_st, const void* k, const dg_stride3* k_st,
                            const void* v, const dg_stride3* v_st, void* y,
                            const dg_stride3* y_st, float scale, void* workspace,
                            size_t workspace_bytes, void* stream) {
  return dg_attention_grouped(B, H, Tq, Tk, D, dtype, q, q_st, k, k_st, v, v_st, y, y_st, scale, 0, 1,
                              workspace, workspace_bytes, stream);
}

extern "C" int dg_copy4d(int dtype, const int64_t* shape, const void* src, const int64_t* src_st,
                         void* dst, const int64_t* dst_st, void* stream) {
  DG_REQUIRE(dtype == DG_F32 || dtype == DG_BF16 || dtype == DG_F16, DG_EUNSUPPORTED,
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
  const int64_t es = dtype == DG_F32 ? 4 : 2;
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
  if (dtype == DG_F32)
    hipLaunchKernelGGL(copy4d_kernel<uint32_t>, dim3((unsigned)blocks), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(copy4d_kernel<uint16_t>, dim3((unsigned)blocks), dim3(256), 0, s, a);
  return check_launch("copy4d_kernel");
}
