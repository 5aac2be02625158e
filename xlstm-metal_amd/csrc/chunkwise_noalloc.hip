// Chunkwise forward for callers that cannot allocate device memory (code under
// HIP graph capture, serving loops that forbid hipMalloc): the fused
// algorithm with its gate-prep scratch in a static device array instead of a
// caller workspace.
//
// `scratch` is a file-scope __device__ array; every GPU the library runs on
// holds its own copy for the life of the process.  Host code never passes the
// array's name to a kernel (in host code it is a stand-in, not a device
// address): the first call on a device, with that device current, resolves
// the device address with hipGetSymbolAddress and keeps it per device.  The
// gate-prep kernel writes every byte of the region a call uses before the
// fused kernel reads it, so nothing has to be cleared between calls.  All
// calls on one GPU share the array: calls that overlap on one GPU (two
// streams, or two host threads enqueueing concurrently) race on it.
#include <mutex>

#include "chunkwise.h"

namespace xl {
namespace {

static __device__ __align__(256) unsigned char scratch[XL_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the stream's device, which must be current.
int scratch_address(void* stream, void** out) {
  const char* who = "xl_mlstm_chunkwise_fwd_noalloc";
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(XL_ERR_LAUNCH, "%s: hipGetDevice failed: %s", who, hipGetErrorString(e));
  if (stream) {
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice((hipStream_t)stream, &sdev);
    if (e != hipSuccess)
      return set_error(XL_ERR_INVALID_ARG, "%s: hipStreamGetDevice failed: %s", who, hipGetErrorString(e));
    if ((int)sdev != dev)
      return set_error(XL_ERR_INVALID_ARG, "%s: the stream belongs to device %d but device %d is current", who,
                       (int)sdev, dev);
  }
  if (dev < 0 || dev >= kMaxDevices) return set_error(XL_ERR_UNSUPPORTED, "%s: device ordinal %d", who, dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(XL_ERR_LAUNCH, "%s: hipGetSymbolAddress(scratch) failed on device %d: %s", who, dev,
                       hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return XL_OK;
}

}  // namespace
}  // namespace xl

extern "C" size_t xl_mlstm_chunkwise_noalloc_max_bytes(void) { return XL_NOALLOC_SCRATCH_BYTES; }

extern "C" int xl_mlstm_chunkwise_fwd_noalloc(const void* q, const void* k, const void* v, const void* i,
                                              const void* f, const float* c0, const float* n0, const float* m0,
                                              void* h, float* c_last, float* n_last, float* m_last, int B, int NH,
                                              int S, int DQK, int DV, int L, float qk_scale, float eps,
                                              int dtype_qkv, int dtype_gates, void* stream) {
  using namespace xl;
  clear_error();
  // no sequence split: the static scratch holds the gate prep only
  ChunkwiseArgs a = {q, k, v, i, f, c0, n0, m0, h, c_last, n_last, m_last, B, NH, S, DQK, DV, L,
                     qk_scale, eps, dtype_qkv, dtype_gates, nullptr, 0, stream, 1};
  int rc = chunkwise_check_args(a, XL_CHUNKWISE_FUSED);
  if (rc) return rc;
  const char* why = nullptr;
  if (!chunkwise_fused_supported(a, &why))
    return set_error(XL_ERR_UNSUPPORTED, "xl_mlstm_chunkwise_fwd_noalloc: fused algorithm unsupported here: %s", why);
  const size_t need = chunkwise_fused_workspace(B, NH, S, DQK, DV, 1);
  if (need > (size_t)XL_NOALLOC_SCRATCH_BYTES)
    return set_error(XL_ERR_UNSUPPORTED,
                     "xl_mlstm_chunkwise_fwd_noalloc: B*NH*ceil(S/64) = %lld chunks need %zu bytes of scratch, "
                     "more than the static %zu (at most %zu chunks); use xl_mlstm_chunkwise_fwd with a workspace",
                     (long long)B * NH * ((S + 63) / 64), need, (size_t)XL_NOALLOC_SCRATCH_BYTES,
                     (size_t)XL_NOALLOC_SCRATCH_BYTES / chunkwise_fused_workspace(1, 1, 64, DQK, DV, 1));
  void* ws = nullptr;
  rc = scratch_address(stream, &ws);
  if (rc) return rc;
  a.workspace = ws;
  a.workspace_bytes = XL_NOALLOC_SCRATCH_BYTES;
  return chunkwise_fused(a);
}
