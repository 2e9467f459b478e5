/*
 * dgattn.h -- C-ABI of the MI355X (gfx950) attention hot path of diff-gpt.
 *
 * The library (libdgattn.so) exports plain C entry points over raw device
 * pointers, element strides and sizes.  No torch or HIP types appear in the
 * signatures: a stream is passed as `void*` (a hipStream_t; NULL = the null
 * stream).  Every entry point only enqueues work on that stream; none
 * synchronises the host, none allocates device memory.  Buffers are owned by
 * the caller.  Entry points return DG_OK (0) or a negative dg_status; the
 * calling thread's last error message is available from dg_last_error().
 *
 * Layout vocabulary: a "(B,T,H,D) view" is addressed as
 *     base + b*st.b + t*st.t + h*st.h + d          (element strides, d stride 1)
 * The KV cache of the reference (kv_cache.py:25) is (L, 2, B, H, Tcap, D),
 * i.e. for one layer and one of K/V the strides are b = H*Tcap*D, h = Tcap*D,
 * t = D: one contiguous page of Tcap*D elements per (layer, K|V, row, head).
 *
 * Reference interfaces replaced (paths relative to fxeqxmulfx/diff-gpt):
 *   src/diff_gpt/model/rope.py:4-27       apply_rotary_emb
 *   src/diff_gpt/model/rms_norm.py:5-7    rms_norm (QK-norm at mha.py:48 and the
 *                                         residual-stream norms of gpt.py/block.py)
 *   src/diff_gpt/model/kv_cache.py:77-79  KVCache.prefill broadcast copy
 *   src/diff_gpt/model/kv_cache.py:100-109 KVCache.insert_kv growth copy + append
 *   src/diff_gpt/model/mha.py:44-56       RoPE x2, QK-norm x2, transpose, insert_kv
 *   src/diff_gpt/model/mha.py:61-83       the three scaled_dot_product_attention
 *                                         branches and the head re-assembly
 */
#ifndef DGATTN_H
#define DGATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DG_ABI_VERSION 3

#if defined(__GNUC__)
#define DG_API __attribute__((visibility("default")))
#else
#define DG_API
#endif

/* Element types.  The reference computes in the model's dtype (fp32, or bf16
 * after GPT.to(torch.bfloat16)); fp16 and fp64 (a GPT.double() model) are
 * accepted as well.  fp64 runs on plain vector-ALU kernels in fp64 arithmetic
 * (the RoPE rotation of fp32-rounded inputs, as rope.py:20 does), taken by
 * dg_rope_qknorm_append(_at), dg_attention(_grouped), dg_decode_attention_at,
 * dg_decode_step (two launches), dg_rms_norm, dg_attn_res_norm, dg_gate,
 * dg_swiglu, dg_softcap and dg_copy4d; the other entry points return
 * DG_EUNSUPPORTED for it.  The attention scale is an fp32 argument: with
 * fp64 data its rounding of 1/sqrt(D) (SDPA's default) stands for 1/sqrt(D)
 * in fp64, any other scale acts as its fp32 value.  ABI version 3 added
 * DG_F64 and made dg_swiglu's alpha / limit and dg_softcap's cap double. */
enum dg_dtype { DG_F32 = 0, DG_BF16 = 1, DG_F16 = 2, DG_F64 = 3 };

enum dg_status {
  DG_OK = 0,
  DG_EINVAL = -1,       /* bad size, stride, alignment or pointer            */
  DG_EUNSUPPORTED = -2, /* dtype / head_dim combination not built            */
  DG_ELAUNCH = -3,      /* hipLaunchKernel / hipGetLastError reported failure */
  DG_EWORKSPACE = -4    /* workspace missing or smaller than required        */
};

/* Flags of dg_rope_qknorm_append and dg_prefill_rope. */
#define DG_QKNORM 1 /* apply the parameter-free RMSNorm after RoPE (mha.py:48) */
/* dg_prefill_rope only, with DG_QKNORM: every key row of k is RMS-normalised
 * (as dg_rope_qknorm_append with DG_QKNORM writes it, mha.py:48).  With both
 * rows normalised every scaled score lies within scale*log2(e)*D*(1+2^-7) in
 * log2 units (log2(e)*sqrt(D)*(1+2^-7) at the SDPA scale 1/sqrt(D)), and for
 * bf16 data, while that bound is at most 64, the kernel drops the running
 * maximum of the softmax (fp16 data keeps it: exp2 of the bound can exceed
 * fp16's range; so does a larger scale). */
#define DG_KEYS_NORMED 2

/* Element strides of a (B,T,H,D) view; the D stride is always 1. */
typedef struct dg_stride3 {
  int64_t b, t, h;
} dg_stride3;

/* Returns DG_ABI_VERSION of the built library. */
DG_API int dg_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
DG_API const char* dg_last_error(void);

/*
 * Fused RoPE + QK-norm + KV append.  Replaces mha.py:44-56: apply_rotary_emb on
 * q and k (rope.py:4-27), rms_norm on both (rms_norm.py:5-7, eps = FLT_EPSILON,
 * fp32 arithmetic), the (B,T,H,D)->(B,H,T,D) transposes and the two cache
 * copies of KVCache.insert_kv (kv_cache.py:108-109).
 *
 * For every (b,t,h) row:
 *   q_out[b,t,h,:] = norm(rope(q[b,t,h,:], freqs[b,t,h]))     if q != NULL
 *   k_out[b,t,h,:] = norm(rope(k[b,t,h,:], freqs[b,t,h]))     if k != NULL
 *   v_out[b,t,h,:] = v[b,t,h,:]                                if v != NULL
 * norm() is applied only with DG_QKNORM.  freqs points at the (cos, sin) pairs
 * of the row (the reference's (T, D/2, 2) table, kv_cache-position slice,
 * gpt.py:150-153); f_st gives its element strides over (b,t,h) -- 0 for the
 * broadcast dims -- and the D/2 pairs of a row are contiguous.  Pass k_out /
 * v_out as the cache page at position `pos` (e.g. &cache[l,0,0,0,pos,0] with
 * cache strides) to append.  Output dtype = input dtype (rope.py:27 type_as).
 * Supported: every even D up to 1024.  Rows aligned to 16 bytes (and D a
 * multiple of max(16 bytes, D's next power of two / 64) elements) go by
 * 16-byte accesses; other rows need alignment to an element pair.
 */
DG_API int dg_rope_qknorm_append(int B, int T, int H, int D, int dtype,
                          const void* q, const dg_stride3* q_st,
                          void* q_out, const dg_stride3* qo_st,
                          const void* k, const dg_stride3* k_st,
                          void* k_out, const dg_stride3* ko_st,
                          const void* v, const dg_stride3* v_st,
                          void* v_out, const dg_stride3* vo_st,
                          const void* freqs, const dg_stride3* f_st,
                          int freqs_dtype, int flags, void* stream);

/*
 * Scaled dot-product attention of mha.py:61-81 with the head re-assembly of
 * mha.py:83.  q is a (B,Tq,H,D) view, k and v are (B,Tk,H,D) views (for the
 * KV cache: strides b=H*Tcap*D, t=D, h=Tcap*D), y a (B,Tq,H,D) view.  Query i
 * sees key j iff j <= i + (Tk - Tq): this is is_causal=True when Tq == Tk
 * (mha.py:64), the unmasked single-query decode when Tq == 1 (mha.py:68) and
 * the bottom-right chunk mask otherwise (mha.py:69-81).  Softmax in fp32
 * (in fp64 for fp64 data).
 * scale is the SDPA scale (the reference uses the default 1/sqrt(D); see
 * dg_dtype for its meaning with fp64 data).
 * Prefills (Tq >= 16) at D = 64 or 128 with 16-byte aligned rows run on the
 * matrix cores: bf16 / fp16 products with fp32 accumulation, fp32 inputs on
 * fp32 products and accumulation; other shapes on the vector kernel, which
 * takes every even D up to 1024 (alignment as for dg_rope_qknorm_append).
 *
 * workspace: split-KV partials; dg_attention_workspace_size() gives the bytes
 * needed for these sizes: 0 unless a single-token decode splits the keys of
 * a (b, h) over more than 16 waves of one workgroup (8 for D > 512; B*H <
 * 256 with long rows; those merge inside the workgroup and need none).  With
 * workspace == NULL such a launch uses as many splits as one workgroup
 * merges (always correct, slower for very few long rows).
 */
DG_API size_t dg_attention_workspace_size(int B, int H, int Tq, int Tk, int D, int dtype);

DG_API int dg_attention(int B, int H, int Tq, int Tk, int D, int dtype,
                 const void* q, const dg_stride3* q_st,
                 const void* k, const dg_stride3* k_st,
                 const void* v, const dg_stride3* v_st,
                 void* y, const dg_stride3* y_st, float scale,
                 void* workspace, size_t workspace_bytes, void* stream);

/*
 * Prefill attention with RoPE and QK-norm of the queries fused in: "Prefill
 * fuses RoPE" of mha.py:44-48 + 61-81.  y = dg_attention(norm(rope(q)), k, v)
 * where norm(rope(q)) is what dg_rope_qknorm_append would store for q (the
 * same roundings and reduction order, so y is dg_attention's on that q bit
 * for bit) and k, v are the cache views (keys already rotated, e.g. by
 * dg_rope_qknorm_append with q = NULL appending them).  freqs / f_st /
 * freqs_dtype as in dg_rope_qknorm_append, for the Tq query rows; flags:
 * DG_QKNORM or 0, optionally with DG_KEYS_NORMED (DG_QKNORM | DG_KEYS_NORMED:
 * the keys are normalised too; for bf16 data the softmax then runs without a
 * running maximum, with the scale folded into the rounded query operand, so y
 * agrees with dg_attention's within the bf16 bar rather than bit for bit.
 * That form is taken only while scale * log2(e) * D * (1 + 2^-7) <= 64, the
 * bound on a score in log2 units that keeps exp2 of every score inside
 * fp32's normal range: scale up to about 0.68 at head_dim 64 and 0.34 at 128,
 * the SDPA scale 1/sqrt(D) well inside.  A larger scale, and fp16 data,
 * ignore the flag and give dg_attention's y bit for bit, as fp32 data always
 * does).  Only the MFMA prefill kernels' shapes are taken (bf16, fp16 or
 * fp32, head_dim 64 or 128, Tq >= 16, scale > 0, 16-byte aligned rows,
 * freqs in the data's dtype or fp32, Tq <= 65535 * 128 and B*H <= 65535 * 64,
 * one head's K and V rows within 2^31 bytes): anything else returns
 * DG_EUNSUPPORTED and does nothing, and the caller makes the two calls.
 */
DG_API int dg_prefill_rope(int B, int H, int Tq, int Tk, int D, int dtype,
                           const void* q, const dg_stride3* q_st,
                           const void* freqs, const dg_stride3* f_st, int freqs_dtype, int flags,
                           const void* k, const dg_stride3* k_st,
                           const void* v, const dg_stride3* v_st,
                           void* y, const dg_stride3* y_st, float scale, void* stream);

/*
 * A prefix shared by groups of rows: KVCache.prefill's batch broadcast
 * (kv_cache.py:77-79) gives the `group` consecutive rows of each group the
 * same positions 0 .. len-1.  Row b belongs to group b / group.
 *   k, v      -- the prefix's keys and values, one page set per group:
 *                position t, head h of group g at k + g*k_st.b + t*k_st.t
 *                + h*k_st.h (likewise v).  Their t strides must equal the
 *                cache view's.  NULL (both): each group's first row of the
 *                cache view holds the prefix (the broadcast cache itself).
 *   own_start -- the first position the per-row cache view holds: with
 *                own_start = s, position t >= s of row b is at
 *                cache + b*st.b + (t - s)*st.t + h*st.h.  0 for a cache that
 *                holds every position; len when the prefix is stored only in
 *                k / v and the rows' pages start after it.  Must be 0 with
 *                k = NULL, and at most len.
 * A NULL dg_prefix*, len = 0, or group = 1 with k = NULL means no shared
 * prefix.
 */
typedef struct dg_prefix {
  int len;
  int group;
  const void* k;
  const void* v;
  dg_stride3 k_st;
  dg_stride3 v_st;
  int own_start;
} dg_prefix;

/*
 * dg_attention over a batch whose rows come in groups sharing a prefix
 * (dg_prefix): for row b, keys j < prefix->len come from its group's prefix
 * pages, keys j >= len from row b's own cache pages.  This is the decode
 * attention of mha.py:65-68 over the cache that KVCache.prefill's batch
 * broadcast (kv_cache.py:77-79) leaves behind, with the prefix fetched from
 * HBM about once per group (rows of one group run on one XCD and hit its L2)
 * and, with separate prefix pages, stored once per group.  The caller
 * guarantees that the prefix pages hold what every row of the group would.
 * Single-token decode with group >= 16, head_dim 16 or 32 and no key splits
 * runs the prefix part as a matrix product on MFMA (fp32 products for fp32
 * inputs): equal to dg_attention within the fp32 rounding of a different
 * summation order.  Other shapes give dg_attention's bits exactly.  Prefill
 * launches the MFMA kernel takes (prefix in the cache rows themselves) read
 * every row's own keys.
 */
DG_API int dg_attention_grouped(int B, int H, int Tq, int Tk, int D, int dtype,
                                const void* q, const dg_stride3* q_st,
                                const void* k, const dg_stride3* k_st,
                                const void* v, const dg_stride3* v_st,
                                void* y, const dg_stride3* y_st, float scale,
                                const dg_prefix* prefix,
                                void* workspace, size_t workspace_bytes, void* stream);

/*
 * Decode-step forms for HIP graph capture.  The number of positions already in
 * the cache is read on the device from *pos (int32), so a captured decode step
 * (GPT.forward over one new token per row, gpt.py:140-200) replays unchanged
 * at every position; the caller advances *pos after the step.
 *
 * dg_rope_qknorm_append_at: dg_rope_qknorm_append with T = 1 at position *pos
 * (mha.py:44-56 with kv_cache.py:108-109): k_cache / v_cache are the cache
 * pages at position 0 viewed as (B,Tcap,H,D) (strides b, t = D, h), the new
 * key / value go to t = *pos; freqs is the (cos, sin) table at position 0
 * with freqs_pos_stride elements per position (gpt.py:150-153 slicing done on
 * the device).  Nothing is written when *pos is outside [0, max_pos).
 *
 * dg_decode_attention_at: dg_attention_grouped with Tq = 1 over the keys
 * 0 .. *pos of the cache pages (mha.py:65-68), at most max_keys of them (an
 * absolute position bound; with prefix->own_start = s the cache views hold
 * positions s .. max_keys-1).  Key splits and the workspace
 * (dg_decode_attention_at_workspace_size) are sized for max_keys.
 */
DG_API int dg_rope_qknorm_append_at(int B, int H, int D, int dtype,
                                    const void* q, const dg_stride3* q_st,
                                    void* q_out, const dg_stride3* qo_st,
                                    const void* k, const dg_stride3* k_st,
                                    void* k_cache, const dg_stride3* kc_st,
                                    const void* v, const dg_stride3* v_st,
                                    void* v_cache, const dg_stride3* vc_st,
                                    const void* freqs, int64_t freqs_pos_stride, int freqs_dtype,
                                    const int32_t* pos, int max_pos, int flags, void* stream);

DG_API size_t dg_decode_attention_at_workspace_size(int B, int H, int max_keys, int D, int dtype);

DG_API int dg_decode_attention_at(int B, int H, int D, int dtype,
                                  const void* q, const dg_stride3* q_st,
                                  const void* k_cache, const dg_stride3* kc_st,
                                  const void* v_cache, const dg_stride3* vc_st,
                                  void* y, const dg_stride3* y_st, float scale,
                                  const dg_prefix* prefix, const int32_t* pos, int max_keys,
                                  void* workspace, size_t workspace_bytes, void* stream);

/*
 * One decode step of a layer, fused: dg_rope_qknorm_append with T = 1 at
 * position p (mha.py:44-56, kv_cache.py:108-109) followed by
 * dg_attention_grouped with Tq = 1 over positions 0 .. p (mha.py:65-68).
 * q, k, v are the step's projections (B,1,H,D); k_cache / v_cache the cache
 * pages viewed as (B,positions,H,D) from position prefix->own_start (0
 * without a prefix) up to max_pos (absolute); freqs the (cos, sin) row of
 * position 0 with freqs_pos_stride elements per position (0: freqs already
 * points at position p's row); y (B,1,H,D) receives the attention output.
 * p = *pos_dev when pos_dev != NULL (graph-replayable: nothing is written when
 * *pos_dev is outside [own_start, max_pos)), else p = pos, which must lie in
 * [own_start, max_pos) and at or past the prefix's length.
 *
 * With a shared prefix (group >= 16, D 16 or 32) this is one launch: the new
 * key and value are appended and also used from registers.  The cache
 * contents are those of dg_rope_qknorm_append bit for bit; y equals the
 * two-call result within fp32 rounding (the new key is accumulated last).
 * Where the attention runs on the vector kernel (every other shape whose
 * rows, projections and table are aligned to its lane slices) it is one
 * launch too: each (row, head) wave rotates q and k itself, the wave whose
 * key split holds p appends them, and the new key enters the softmax from
 * registers in the slot where the two-launch form reads it back, so y has
 * the two-launch form's bits.  Any other shape runs those two launches, with
 * the rotated q staged in y: dg_rope_qknorm_append at p, then the decode
 * attention over 0 .. p.  Both choose the kernel and key splits for max_pos
 * -- in both position forms, since the device form must fix them for every
 * p a captured graph replays.  So y
 * equals dg_decode_attention_at's (max_keys = max_pos) bit for bit, host and
 * device position alike; it equals the two calls dg_rope_qknorm_append +
 * dg_attention_grouped over p + 1 keys bit for bit when both choose the same
 * number of key splits, and otherwise differs from them only in the order
 * of the fp32 accumulation (with B*H below 4096, p + 1 and max_pos can lie
 * on different sides of a multiple of 128 keys).  The workspace (dg_decode_step_workspace_size)
 * serves key splits beyond 16 per (b, h); NULL caps them at 16.
 */
DG_API size_t dg_decode_step_workspace_size(int B, int H, int max_pos, int D, int dtype);

DG_API int dg_decode_step(int B, int H, int D, int dtype,
                          const void* q, const dg_stride3* q_st,
                          const void* k, const dg_stride3* k_st,
                          const void* v, const dg_stride3* v_st,
                          void* k_cache, const dg_stride3* kc_st,
                          void* v_cache, const dg_stride3* vc_st,
                          const void* freqs, int64_t freqs_pos_stride, int freqs_dtype,
                          int pos, const int32_t* pos_dev, int max_pos,
                          void* y, const dg_stride3* y_st, float scale,
                          const dg_prefix* prefix, int flags,
                          void* workspace, size_t workspace_bytes, void* stream);

/*
 * dg_decode_step without a workspace argument: no counterpart in the
 * reference.  It is for callers that cannot allocate device memory (code
 * under HIP graph capture that must not allocate, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments, kernels and results as
 * dg_decode_step; the key-split partials live in a static device array of
 * dg_decode_step_noalloc_scratch_bytes() bytes (20 MiB) that the library
 * holds on every GPU it runs on until the process ends.  Every size fits:
 * the split workspace (dg_decode_step_workspace_size) is at most 19 MB; a
 * size beyond the array would return DG_EWORKSPACE before any GPU work.
 * It allocates nothing and frees nothing.  All calls on one GPU share that array: calls that
 * overlap on one GPU (other streams, other host threads) race and must be
 * serialised by the caller.  The stream must belong to the current device.
 */
DG_API size_t dg_decode_step_noalloc_scratch_bytes(void);

DG_API int dg_decode_step_noalloc(int B, int H, int D, int dtype,
                                  const void* q, const dg_stride3* q_st,
                                  const void* k, const dg_stride3* k_st,
                                  const void* v, const dg_stride3* v_st,
                                  void* k_cache, const dg_stride3* kc_st,
                                  void* v_cache, const dg_stride3* vc_st,
                                  const void* freqs, int64_t freqs_pos_stride, int freqs_dtype,
                                  int pos, const int32_t* pos_dev, int max_pos,
                                  void* y, const dg_stride3* y_st, float scale,
                                  const dg_prefix* prefix, int flags, void* stream);

/*
 * Parameter-free RMSNorm over the last dim (rms_norm.py:5-7 == F.rms_norm with
 * eps=None, i.e. FLT_EPSILON, computed in fp32 and rounded once to dtype).
 * x and out are M rows of N elements with row strides x_ld / out_ld.
 * Supported: N <= 8192.
 */
DG_API int dg_rms_norm(int64_t M, int N, int dtype, const void* x, int64_t x_ld,
                void* out, int64_t out_ld, void* stream);

/*
 * Token embedding and the RMSNorms that follow it, in one launch:
 * x_out[r] = rms_norm(table[ids[r]]) (gpt.py:154-155, nn.Embedding then
 * rms_norm) and, when xn_out is not NULL, xn_out[r] = rms_norm(x_out[r]) as
 * stored, the normalised input of layer 0's attention (block.py:95-97 with
 * the single-block short cut of block.py:27-28).  Both give dg_rms_norm's
 * bits for the same rows.  An id outside [0, V) gives a NaN row instead of
 * reading outside the table.  fp32 / bf16 / fp16, C <= 8192.
 */
DG_API int dg_embed_norm(int64_t M, int C, int dtype, const int64_t* ids, int64_t V,
                  const void* table, int64_t table_ld, void* x_out, int64_t x_ld,
                  void* xn_out, int64_t xn_ld, void* stream);

/*
 * Strided 4-D copy dst[i0,i1,i2,i3] = src[i0,i1,i2,i3] over shape[4], element
 * strides per tensor (a 0 src stride broadcasts).  Serves KVCache.insert_kv's
 * append (kv_cache.py:108-109) and growth copy (kv_cache.py:100-106) and
 * KVCache.prefill's batch broadcast (kv_cache.py:77-79).  Exact copy.
 */
DG_API int dg_copy4d(int dtype, const int64_t* shape, const void* src,
              const int64_t* src_st, void* dst, const int64_t* dst_st,
              void* stream);

/*
 * The layers around attention in a decode step, one launch each (the torch
 * op sequences they replace launch several).  All take M rows with element
 * row strides (*_ld), compute in fp32 and round to dtype wherever the torch
 * sequence returns a tensor, so bf16 follows the same rounding steps.
 */

/*
 * rms_norm(block_attn_res(V, w)): block.py:10-44 (stack, rms_norm(V) . w,
 * softmax over the sources, weighted sum) followed by rms_norm.py:5-7, for the
 * nsrc sources V_n = src[n] (rows of C elements, row stride src_ld[n]) in the
 * order block_attn_res stacks them (committed blocks, then the partial sum).
 * The RMSNorms give dg_rms_norm's bits for the same row.
 * Supported: C <= 2048, 1 <= nsrc <= 32.
 */
DG_API int dg_attn_res_norm(int64_t M, int C, int dtype, int nsrc, const void* const* src,
                     const int64_t* src_ld, const void* w, void* out, int64_t out_ld,
                     void* stream);

/* out = y * sigmoid(g) (mha.py:84); out may alias y. */
DG_API int dg_gate(int64_t M, int C, int dtype, const void* y, int64_t y_ld, const void* g,
            int64_t g_ld, void* out, int64_t out_ld, void* stream);

/*
 * Clamped SwiGLU (swi_glu.py:11-19) on rows of 2N interleaved (gate, linear)
 * elements: gate = min(x[2j], limit), lin = clamp(x[2j+1], -limit, limit),
 * out[j] = gate * sigmoid(alpha * gate) * (lin + 1).
 */
DG_API int dg_swiglu(int64_t M, int N, int dtype, const void* x, int64_t x_ld, void* out,
              int64_t out_ld, double alpha, double limit, void* stream);

/* Logit soft cap cap * tanh(x / cap) (gpt.py:182-186); out may alias x. */
DG_API int dg_softcap(int64_t M, int N, int dtype, const void* x, int64_t x_ld, void* out,
               int64_t out_ld, double cap, void* stream);

/*
 * lm_head + logit soft cap + greedy argmax in one launch (gpt.py:181-186 and
 * temperature.py:22-23).  logits[m, v] = cap * tanh((x[m] . w[v]) / cap)
 * (cap = 0: no cap) for the M normalised rows x (M, C) against the tied
 * embedding table w (V, C), with the matmul's result rounded to the dtype as
 * F.linear returns it and the cap computed as dg_softcap does; fp32
 * accumulation on the matrix cores (its summation order is not hipBLASLt's,
 * so the logits agree with F.linear + dg_softcap within the north-star bars,
 * not bit for bit).  With ids != NULL, ids[m] (int64) is the first maximum
 * of the logits row as stored (torch.argmax).  Supported: C a multiple of
 * 64, V in {64, 128, 256, 512, 1024}, 16-byte aligned rows; anything else
 * returns DG_EUNSUPPORTED and does nothing.
 */
DG_API int dg_lm_head(int64_t M, int C, int V, int dtype, const void* x, int64_t x_ld, const void* w,
                      int64_t w_ld, float cap, void* logits, int64_t logits_ld, int64_t* ids, void* stream);

/*
 * A layer's work after its attention in one launch: mha.py:84-85 (the gate
 * y * sigmoid(g) and c_proj), block.py:98-106 (the partial sum: the
 * attention output itself when the layer commits its input block, else
 * partial_in + attention output; the MLP's mixture over the committed
 * blocks and that partial, with its RMSNorm; the residual add) and
 * feed_forward.py:10-14 (C -> 4C, the clamped SwiGLU with alpha and limit on
 * the interleaved pairs, 2C -> C).  y, g (M, C): the attention output and
 * the gate logits; w_proj (C, C), w_up (4C, C), w_down (C, 2C); partial_in
 * NULL when the layer commits; blocks[0 .. nblk-1] the committed blocks; out
 * (M, C) the partial sum leaving the layer.  Intermediates are rounded where
 * the torch sequence rounds them (the gate as dg_gate, each product's fp32
 * sum once, the mixture as dg_attn_res_norm, the SwiGLU as dg_swiglu, the
 * residual adds); the products run on the matrix cores, so the result agrees
 * with the separate launches within the north-star bars, not bit for bit.
 * Supported: C = 64 or 128, nblk + 1 <= 32, 16-byte aligned rows; anything
 * else returns DG_EUNSUPPORTED and does nothing.
 */
DG_API int dg_block_out(int64_t M, int C, int dtype, const void* y, int64_t y_ld, const void* g, int64_t g_ld,
                        const void* w_proj, int64_t wp_ld, const void* partial_in, int64_t pin_ld, int nblk,
                        const void* const* blocks, const int64_t* blocks_ld, const void* w_mix,
                        const void* w_up, int64_t wu_ld, const void* w_down, int64_t wd_ld, float alpha,
                        float limit, void* out, int64_t out_ld, void* stream);

/*
 * dg_block_out that also writes xn = rms_norm(out) row by row, of the output
 * as stored, with dg_rms_norm's bits: the last layer's output and the head's
 * normalised input (gpt.py:180) from one launch.  Same support as
 * dg_block_out; xn rows 16-byte aligned.
 */
DG_API int dg_block_out_norm(int64_t M, int C, int dtype, const void* y, int64_t y_ld, const void* g,
                             int64_t g_ld, const void* w_proj, int64_t wp_ld, const void* partial_in,
                             int64_t pin_ld, int nblk, const void* const* blocks, const int64_t* blocks_ld,
                             const void* w_mix, const void* w_up, int64_t wu_ld, const void* w_down,
                             int64_t wd_ld, float alpha, float limit, void* out, int64_t out_ld, void* xn,
                             int64_t xn_ld, void* stream);

/*
 * The sampler's draw (temperature.py:24-25, torch.multinomial with one
 * sample, by its Exp(1) method): ids[r] = the first index of the maximum of
 * probs[r, j] / q[r, j] over j < V, q the caller's Exp(1) variates (torch's
 * exponential_ on the caller's generator, so the random stream stays
 * torch's).  The quotient is rounded to the data dtype and compared as
 * torch.argmax does (NaN above every number, first of equals wins): the
 * ids of torch.argmax(probs / q, -1).  fp32 / bf16 / fp16 / fp64.
 */
DG_API int dg_draw_argmax(int64_t M, int V, int dtype, const void* probs, int64_t p_ld, const void* q,
                   int64_t q_ld, int64_t* ids, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DGATTN_H */
