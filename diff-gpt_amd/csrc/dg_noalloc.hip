// dg_decode_step_noalloc: the decode step of dg_decode_step with the key-split
// partials in a static device array instead of a caller workspace, for
// callers that cannot allocate device memory.
//
// The array `scratch` is a file-scope __device__ array: every GPU the library
// runs on holds one copy of it, at its own device address, until the process
// ends.  That address is looked up once per device (hipGetSymbolAddress with
// the device current) and kept in g_scratch_ptr; kernels only ever receive
// that pointer, never the array's host-side name.
//
// Contents: with key splits, the split kernel writes the (acc, m, l) partial
// of every (row, head, split) -- splits without a visible key included -- and
// the combine kernel, later on the same stream, reads them.  Nothing has to
// start at zero, and a call leaves the last call's partials behind.  Every
// call on one GPU uses the same array: calls that overlap on one GPU (two
// streams, or two host threads) race on it and must be serialised by the
// caller.
#include "dg_common.h"

#include <mutex>

// Largest key-split workspace of a decode step: up to 16 splits merge inside
// the workgroup and need none (8 for head dims past 512); more happen only
// while B*H < 256 (512) -- they aim at 4096 waves -- so B*H*splits is below
// 4096 + 256 (4096 + 512) partials of at most 512 + 2 (1024 + 2) floats:
// < 9 MB (< 19 MB) for any head_dim the library takes.  The check below
// stays as a guard.
constexpr size_t kStaticScratchBytes = size_t(20) << 20;

static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

namespace dg {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];  // device address of `scratch` per device, null until looked up

// Device address of this GPU's `scratch`, looked up on the first call made
// with `dev` current.
int device_scratch(int dev, void** out) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    DG_REQUIRE(e == hipSuccess && p != nullptr, DG_ELAUNCH,
               "decode_step_noalloc: hipGetSymbolAddress(scratch) on device %d failed: %s", dev,
               hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return DG_OK;
}

}  // namespace
}  // namespace dg

using namespace dg;

extern "C" size_t dg_decode_step_noalloc_scratch_bytes(void) { return kStaticScratchBytes; }

extern "C" int dg_decode_step_noalloc(int B, int H, int D, int dtype, const void* q, const dg_stride3* q_st,
                                      const void* k, const dg_stride3* k_st, const void* v,
                                      const dg_stride3* v_st, void* k_cache, const dg_stride3* kc_st,
                                      void* v_cache, const dg_stride3* vc_st, const void* freqs,
                                      int64_t freqs_pos_stride, int freqs_dtype, int pos, const int32_t* pos_dev,
                                      int max_pos, void* y, const dg_stride3* y_st, float scale,
                                      const dg_prefix* prefix, int flags, void* stream) {
  DG_REQUIRE(B >= 0 && H >= 0 && D >= 2 && max_pos >= 1, DG_EINVAL,
             "decode_step_noalloc: bad sizes (B=%d H=%d D=%d max_pos=%d)", B, H, D, max_pos);
  const size_t need = dg_decode_step_workspace_size(B, H, max_pos, D, dtype);
  DG_REQUIRE(need <= kStaticScratchBytes, DG_EWORKSPACE,
             "decode_step_noalloc: B=%d H=%d max_pos=%d D=%d needs %zu bytes of key-split scratch, more "
             "than the static %zu; use dg_decode_step with a workspace",
             B, H, max_pos, D, need, kStaticScratchBytes);
  if ((int64_t)B * H == 0) return DG_OK;

  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  DG_REQUIRE(e == hipSuccess, DG_ELAUNCH, "decode_step_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  DG_REQUIRE(dev >= 0 && dev < kMaxDevices, DG_EINVAL, "decode_step_noalloc: device %d out of range", dev);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (s != nullptr) {
    int sdev = -1;
    e = hipStreamGetDevice(s, &sdev);
    DG_REQUIRE(e == hipSuccess, DG_EINVAL, "decode_step_noalloc: hipStreamGetDevice: %s", hipGetErrorString(e));
    DG_REQUIRE(sdev == dev, DG_EINVAL,
               "decode_step_noalloc: the stream belongs to device %d but device %d is current", sdev, dev);
  }
  void* ws = nullptr;
  const int rc = device_scratch(dev, &ws);
  if (rc != DG_OK) return rc;
  return dg_decode_step(B, H, D, dtype, q, q_st, k, k_st, v, v_st, k_cache, kc_st, v_cache, vc_st, freqs,
                        freqs_pos_stride, freqs_dtype, pos, pos_dev, max_pos, y, y_st, scale, prefix, flags, ws,
                        kStaticScratchBytes, stream);
}
