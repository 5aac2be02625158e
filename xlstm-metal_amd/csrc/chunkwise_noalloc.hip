// Chunkwise forward for callers that cannot allocate device memory (code under
// HIP graph capture, serving loops that forbid hipMalloc): the fused
// algorithm with its gate-prep scratch in a static device array instead of a
// caller workspace.
//
// `scratch` is a file-scope __device__ array; every GPU the library runs on
// holds its own copy for the life of the process.  Host code never passes the
// array's name to a kernel (in host code it is a stand-in, not a device
// address): the first call on a device, with that device current, resolves
// the device address with hipGetSymbolAddress and keeps it per device, and
// creates one HIP event per device (no device memory).  The gate-prep kernel
// writes every byte of the region a call uses before the fused kernel reads
// it, so nothing has to be cleared between calls.
//
// All calls on one GPU share the array.  Outside graph capture the calls are
// ordered: a call on a stream other than the previous call's waits on an
// event recorded behind the previous call's kernels, so calls from several
// streams (or host threads) run one after another on the array.  A stream
// under capture gets no such wait (an event recorded outside a capture cannot
// be waited on inside it): replays of a captured call are ordered with work on
// the stream they are launched on only, and a replay that overlaps another
// call on the same GPU races on the array.
#include <mutex>

#include "chunkwise.h"

namespace xl {
namespace {

static __device__ __align__(256) unsigned char scratch[XL_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;

// Per-device set-up and the ordering of calls on the shared array.
struct DeviceState {
  void* scratch = nullptr;      // device address of `scratch`
  hipEvent_t done = nullptr;    // recorded behind the last call's kernels (outside capture)
  void* last_stream = nullptr;  // stream of that call
  bool has_last = false;
};
std::mutex g_scratch_mu;  // held from the set-up through the launch and the event record
DeviceState g_dev[kMaxDevices];

// Device state of the stream's device, which must be current (g_scratch_mu held).
int device_state(void* stream, DeviceState** out) {
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
  DeviceState& d = g_dev[dev];
  if (!d.scratch) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(XL_ERR_LAUNCH, "%s: hipGetSymbolAddress(scratch) failed on device %d: %s", who, dev,
                       hipGetErrorString(e));
    d.scratch = p;
  }
  if (!d.done) {
    e = hipEventCreateWithFlags(&d.done, hipEventDisableTiming);
    if (e != hipSuccess) {
      d.done = nullptr;
      return set_error(XL_ERR_LAUNCH, "%s: hipEventCreateWithFlags failed on device %d: %s", who, dev,
                       hipGetErrorString(e));
    }
  }
  *out = &d;
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
  if (!chunkwise_fused_supported(a, &why, false))
    return set_error(XL_ERR_UNSUPPORTED, "xl_mlstm_chunkwise_fwd_noalloc: fused algorithm unsupported here: %s", why);
  const size_t need = chunkwise_fused_workspace(B, NH, S, DQK, DV, 1);
  if (need > (size_t)XL_NOALLOC_SCRATCH_BYTES)
    return set_error(XL_ERR_UNSUPPORTED,
                     "xl_mlstm_chunkwise_fwd_noalloc: B*NH*ceil(S/64) = %lld chunks need %zu bytes of scratch, "
                     "more than the static %zu (at most %zu chunks); use xl_mlstm_chunkwise_fwd with a workspace",
                     (long long)B * NH * ((S + 63) / 64), need, (size_t)XL_NOALLOC_SCRATCH_BYTES,
                     (size_t)XL_NOALLOC_SCRATCH_BYTES / chunkwise_fused_workspace(1, 1, 64, DQK, DV, 1));
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  DeviceState* d = nullptr;
  rc = device_state(stream, &d);
  if (rc) return rc;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing((hipStream_t)stream, &cap);
  if (e != hipSuccess)
    return set_error(XL_ERR_INVALID_ARG, "xl_mlstm_chunkwise_fwd_noalloc: hipStreamIsCapturing failed: %s",
                     hipGetErrorString(e));
  const bool eager = cap == hipStreamCaptureStatusNone;
  if (eager && d->has_last && d->last_stream != stream) {
    e = hipStreamWaitEvent((hipStream_t)stream, d->done, 0);
    if (e != hipSuccess)
      return set_error(XL_ERR_LAUNCH, "xl_mlstm_chunkwise_fwd_noalloc: hipStreamWaitEvent failed: %s",
                       hipGetErrorString(e));
  }
  a.workspace = d->scratch;
  a.workspace_bytes = XL_NOALLOC_SCRATCH_BYTES;
  rc = chunkwise_fused(a);
  if (rc == XL_OK && eager) {
    e = hipEventRecord(d->done, (hipStream_t)stream);
    if (e != hipSuccess)
      return set_error(XL_ERR_LAUNCH, "xl_mlstm_chunkwise_fwd_noalloc: hipEventRecord failed: %s", hipGetErrorString(e));
    d->last_stream = stream;
    d->has_last = true;
  }
  return rc;
}
