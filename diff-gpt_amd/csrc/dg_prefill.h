// Launch arguments and schedule constants shared by the MFMA prefill kernels
// (dg_attn_mfma.hip: bf16 / fp16; dg_attn_mfma_f32.hip: fp32).
#pragma once

#include "dg_common.h"

namespace dg {

struct PrefillArgs {
  const void* q;
  const void* k;
  const void* v;
  void* y;
  int64_t qb, qt, qh;
  int64_t kb, kt, kh;
  int64_t vb, vt, vh;
  int64_t yb, yt, yh;
  int H, Tq, Tk, q_offset;
  int nqb;     // query blocks per (b, h)
  int nbh;     // B*H
  int win;     // (b, h) pairs per scheduling window
  float scale_log2;  // SDPA scale * log2(e)
  float lazy_raw;    // kLazyLog2 / scale_log2: allowed growth of a row max in raw score units
  // ROPE instances: (cos, sin) pairs of query row (b, i, h) at
  // freqs + b*fb + i*ft + h*fh (D/2 pairs, contiguous), and the QK-norm flag
  const void* freqs;
  int64_t fb, ft, fh;
  int qknorm;
};

constexpr int kPrefillWindow = 64;      // (b, h) pairs per scheduling window
constexpr int kPrefillWindowLong = 32;  // ... for long rows and large batches (prefill_args)
constexpr float kLazyLog2 = 8.0f;   // probabilities stay <= 2^8 between rescales

// fp32 prefill on v_mfma_f32_32x32x2_f32 (dg_attn_mfma_f32.hip): D is 64 or
// 128; a.nqb is set by the launch.  With a.freqs set, q is rotated (and
// normalised when a.qknorm) as it is loaded (fp32 table).
int launch_prefill_f32(PrefillArgs a, int D, hipStream_t s);

}  // namespace dg
