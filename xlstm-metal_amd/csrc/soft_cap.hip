// soft_cap: y = cap * tanh(x / cap).
//
// Pure HBM stream (2 * numel * sizeof(T) bytes).  Each thread moves 16-byte
// vectors (4 floats or 8 halves) in a grid-stride loop; the grid is sized to
// a few waves per SIMD so loads of several iterations are in flight.
#include "common.h"

namespace xl {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <typename T>
union Vec16 {
  static constexpr int N = 16 / sizeof(T);
  u32x4 raw;
  T v[N];
};

template <typename T>
__global__ __launch_bounds__(256) void soft_cap_kernel(const T* x, T* y, int64_t numel, float cap,
                                                        float inv_cap) {
  constexpr int N = Vec16<T>::N;
  const int64_t nvec = numel / N;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const u32x4* xv = reinterpret_cast<const u32x4*>(x);
  u32x4* yv = reinterpret_cast<u32x4*>(y);
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < nvec; idx += stride) {
    Vec16<T> a, b;
    a.raw = __builtin_nontemporal_load(&xv[idx]);
#pragma unroll
    for (int j = 0; j < N; ++j) b.v[j] = from_f32<T>(cap * tanh_f32(to_f32(a.v[j]) * inv_cap));
    __builtin_nontemporal_store(b.raw, &yv[idx]);
  }
  // tail (< N elements) handled by block 0
  if (blockIdx.x == 0) {
    const int64_t t = nvec * N + threadIdx.x;
    if (t < numel) y[t] = from_f32<T>(cap * tanh_f32(to_f32(x[t]) * inv_cap));
  }
}

template <typename T>
static int launch_soft_cap(const void* x, void* y, int64_t numel, float cap, hipStream_t s) {
  constexpr int N = Vec16<T>::N;
  const int64_t nvec = numel / N;
  int64_t blocks = (nvec + 255) / 256;
  if (blocks < 1) blocks = 1;
  if (blocks > 256 * 16) blocks = 256 * 16;  // 16 WGs per CU, grid-stride beyond
  hipLaunchKernelGGL(soft_cap_kernel<T>, dim3((unsigned)blocks), dim3(256), 0, s, (const T*)x, (T*)y, numel, cap,
                     1.0f / cap);
  return check_launch("xl_soft_cap_fwd");
}

}  // namespace xl

extern "C" int xl_soft_cap_fwd(const void* x, void* y, int64_t numel, float cap, int dtype, void* stream) {
  using namespace xl;
  clear_error();
  if (numel < 0) return set_error(XL_ERR_INVALID_ARG, "xl_soft_cap_fwd: numel=%lld < 0", (long long)numel);
  if (!dtype_ok(dtype)) return set_error(XL_ERR_INVALID_ARG, "xl_soft_cap_fwd: unknown dtype %d", dtype);
  if (numel == 0) return XL_OK;
  if (!x || !y) return set_error(XL_ERR_INVALID_ARG, "xl_soft_cap_fwd: null pointer");
  if ((((uintptr_t)x) | ((uintptr_t)y)) & 15u)
    return set_error(XL_ERR_INVALID_ARG, "xl_soft_cap_fwd: x and y must be 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  if (!(cap > 0.0f)) {  // reference: cap <= 0 returns x unchanged (softcap.py:27-28)
    if (x == y) return XL_OK;
    hipError_t e = hipMemcpyAsync(y, x, (size_t)numel * dtype_size(dtype), hipMemcpyDeviceToDevice, s);
    if (e != hipSuccess) return set_error(XL_ERR_LAUNCH, "xl_soft_cap_fwd: copy failed: %s", hipGetErrorString(e));
    return XL_OK;
  }
  switch (dtype) {
    case XL_DTYPE_F32: return launch_soft_cap<float>(x, y, numel, cap, s);
    case XL_DTYPE_BF16: return launch_soft_cap<bf16_t>(x, y, numel, cap, s);
    default: return launch_soft_cap<f16_t>(x, y, numel, cap, s);
  }
}
